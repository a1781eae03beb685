"""Projection factory of the decoder layers: a plain nn.Linear for an unquantized checkpoint, a
W4Linear for an AutoAWQ one. Same two entry points and signatures as
python/tandem/layers/linear.py:10-31 (make_linear, finalize_quantized)."""

from __future__ import annotations

from typing import Any, Optional

from torch import nn


def make_linear(in_features: int, out_features: int, bias: bool = False, quant: Optional[Any] = None) -> nn.Module:
    """The projection module for one weight. ``quant`` is None (dense float weights) or a
    quantization description with a ``group_size`` attribute (``tandem_amd.loader.QuantConfig``).
    A W4Linear is created empty: it holds only the AutoAWQ tensors the loader fills, never a dense
    copy of the weight, and is usable once ``finalize_quantized`` has run. The W4A16 kernels have
    no bias term, so a biased quantized projection is refused."""
    if quant is not None:
        if bias:
            raise NotImplementedError("quantized projections with a bias")
        from tandem_amd.layers.awq import W4Linear

        return W4Linear(in_features, out_features, quant.group_size)
    return nn.Linear(in_features, out_features, bias=bias)


def finalize_quantized(model: nn.Module, device_name: Optional[str] = None) -> int:
    """Run ``finalize(device_name)`` on every module still holding AutoAWQ tensors (``awq_layout``
    set): the one-time repack into the kernels' tile layout and the choice of the device's kernel
    tables. Call it with the weights loaded and the model on its GPU. Returns how many layers it
    finalized; a second call finds none."""
    pending = [m for m in model.modules() if getattr(m, "awq_layout", False) and callable(getattr(m, "finalize", None))]
    for module in pending:
        module.finalize(device_name)
    return len(pending)

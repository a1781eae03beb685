"""Put an AutoAWQ "gemm" checkpoint into a model built from W4Linear (and nn.Linear) projections.

Behaviour kept from 12vivi/tandem (python/tandem/model_config.py:28-43 for ``QuantConfig``,
python/tandem/models/loader.py:66-105 for ``load_weights``):

- only 4-bit AWQ "gemm" checkpoints with zero points are accepted; anything else raises
  NotImplementedError, and an absent quantization_config means an unquantized model;
- the model's fused projections take their halves from the checkpoint's separate ones
  (q / k / v -> qkv_proj, gate / up -> gate_up_proj), in that order along the output features;
- a tensor the model has no use for is logged and skipped (a stored lm_head of a tied-embedding
  model silently); a model tensor the checkpoint cannot fill raises RuntimeError; a shape that does
  not fit raises ValueError; a directory without *.safetensors raises FileNotFoundError.

How this module does it: the model drives the load. ``load_weights`` first indexes the tensor names
of every shard file (reading no data), then asks, for each tensor the model owns, where its data
comes from (``plan_sources``): a checkpoint tensor of the same name, or the list of per-projection
tensors that stacked along the output dimension make it up. The output dimension is dim 0 of a
dense weight or bias and dim 1 of the AutoAWQ tensors (qweight [K, N/8], qzeros [K/G, N/8],
scales [K/G, N]), so ``fused_sources`` records the axis with the names. Every plan is checked
(sources present, stacked shape equal to the target's) before any data is copied. Loading is host
work on CPU tensors; the layers are moved to the GPU and repacked afterwards by
``finalize_quantized`` (see ``tandem_amd.model.prepare``).
"""

from __future__ import annotations

import contextlib
import glob
import logging
import os
import re
from dataclasses import dataclass
from typing import Any, Optional

import torch
from torch import nn

logger = logging.getLogger(__name__)

AWQ_TENSORS = ("qweight", "qzeros", "scales")


@dataclass(frozen=True)
class QuantConfig:
    """The ``quantization_config`` entry of a checkpoint's config.json, for weight-only AWQ."""

    method: str
    bits: int
    group_size: int

    @classmethod
    def from_dict(cls, d: Optional[dict[str, Any]]) -> Optional["QuantConfig"]:
        """None when the checkpoint is not quantized. Accepts AutoAWQ's 4-bit "gemm" packing with
        zero points (``version`` and ``zero_point`` may be absent: those are AutoAWQ's defaults) and
        raises NotImplementedError, naming what does not fit, for every other scheme."""
        if not d:
            return None
        reasons = []
        if d.get("quant_method") != "awq":
            reasons.append(f"quant_method {d.get('quant_method')!r} (only 'awq')")
        if d.get("bits") != 4:
            reasons.append(f"bits {d.get('bits')!r} (only 4)")
        if not d.get("zero_point", True):
            reasons.append("symmetric quantization (AutoAWQ zero points expected)")
        if str(d.get("version", "gemm")).lower() != "gemm":
            reasons.append(f"packing {d.get('version')!r} (only 'gemm')")
        if reasons:
            raise NotImplementedError(f"cannot load quantization_config {d}: " + "; ".join(reasons))
        return cls("awq", 4, int(d.get("group_size", 128)))


# Model tensors assembled from several checkpoint tensors: (model-name pattern, parts in stacking
# order). The attention prefix may sit anywhere in the module tree; the MLP pattern names the
# dense decoder MLP only (a mixture-of-experts layer's "mlp.experts.E.*" never matches).
_FUSED = (
    (re.compile(r"^(?P<pre>.+\.self_attn)\.qkv_proj\.(?P<t>weight|bias|qweight|qzeros|scales)$"),
     ("q_proj", "k_proj", "v_proj")),
    (re.compile(r"^(?P<pre>model\.layers\.\d+\.mlp)\.gate_up_proj\.(?P<t>weight|qweight|qzeros|scales)$"),
     ("gate_proj", "up_proj")),
)
# Checkpoint tensors that are never model state (buffers older exporters saved).
_NOT_STATE = ("rotary_emb.inv_freq", ".attn.bias", ".masked_bias")


def fused_sources(target: str) -> Optional[tuple[list[str], int]]:
    """(checkpoint names in stacking order, stacking axis) of a fused model tensor, else None."""
    for pattern, parts in _FUSED:
        hit = pattern.match(target)
        if hit:
            kind = hit.group("t")
            return [f"{hit.group('pre')}.{p}.{kind}" for p in parts], 1 if kind in AWQ_TENSORS else 0
    return None


def model_tensors(model: nn.Module) -> dict[str, torch.Tensor]:
    """What a checkpoint fills: every parameter, and the AutoAWQ buffers W4Linear registers."""
    out = dict(model.named_parameters())
    out.update((n, b) for n, b in model.named_buffers() if n.rsplit(".", 1)[-1] in AWQ_TENSORS)
    return out


def plan_sources(targets: dict[str, torch.Tensor], available: set[str]
                 ) -> tuple[dict[str, tuple[list[str], int]], list[str]]:
    """For each target: (checkpoint names, stacking axis), the same-named tensor first, else the
    fused parts. Returns (plans, targets the checkpoint cannot fill)."""
    plans, missing = {}, []
    for name in targets:
        if name in available:
            plans[name] = ([name], 0)
            continue
        fused = fused_sources(name)
        if fused is not None and all(src in available for src in fused[0]):
            plans[name] = fused
        else:
            missing.append(name)
    return plans, missing


def _stacked_shape(shapes: list[tuple[int, ...]], axis: int) -> Optional[tuple[int, ...]]:
    first = shapes[0]
    if any(len(s) != len(first) or s[:axis] + s[axis + 1:] != first[:axis] + first[axis + 1:] for s in shapes):
        return None
    return first[:axis] + (sum(s[axis] for s in shapes),) + first[axis + 1:]


def load_weights(model: nn.Module, model_path: str) -> None:
    """Fill every parameter of ``model`` and the AutoAWQ buffers of its W4Linear layers from the
    *.safetensors files in ``model_path`` (CPU tensors, cast to each target's dtype)."""
    from safetensors import safe_open

    files = sorted(glob.glob(os.path.join(model_path, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors files in {model_path}")
    with contextlib.ExitStack() as stack:
        handles = [stack.enter_context(safe_open(f, framework="pt", device="cpu")) for f in files]
        where = {name: h for h in handles for name in h.keys()}  # the last shard wins a duplicate name
        shape_of = {name: tuple(h.get_slice(name).get_shape()) for name, h in where.items()}
        targets = model_tensors(model)
        plans, missing = plan_sources(targets, set(where))
        if missing:
            raise RuntimeError(f"the checkpoint in {model_path} lacks {len(missing)} model tensors, "
                               f"e.g. {sorted(missing)[:5]}")
        for name, (srcs, axis) in plans.items():
            got = _stacked_shape([shape_of[s] for s in srcs], axis)
            if got != tuple(targets[name].shape):
                detail = ", ".join(f"{s} {shape_of[s]}" for s in srcs)
                raise ValueError(f"shape mismatch for {name}: model {tuple(targets[name].shape)}, checkpoint {detail}")
        with torch.no_grad():
            for name, (srcs, axis) in plans.items():
                dst = targets[name]
                parts = [where[s].get_tensor(s) for s in srcs]
                dst.copy_((parts[0] if len(parts) == 1 else torch.cat(parts, dim=axis)).to(dst.dtype))
        used = {s for srcs, _ in plans.values() for s in srcs}
        extra = sorted(n for n in where if n not in used and n != "lm_head.weight" and not n.endswith(_NOT_STATE))
        if extra:
            logger.warning("skipped %d checkpoint tensors the model has no place for, e.g. %s", len(extra), extra[:3])

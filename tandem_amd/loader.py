"""AutoAWQ checkpoint loading and the model wiring of the W4A16 linears.

The counterpart of the parts of 12vivi/tandem that put a real AutoAWQ checkpoint through the op:

    QuantConfig              quantization_config of config.json      python/tandem/model_config.py:28-43
    load_weights             safetensors -> parameters and AWQ        python/tandem/models/loader.py:14-105
                             buffers, fused q/k/v and gate/up

A checkpoint stores q_proj / k_proj / v_proj and gate_proj / up_proj separately; the model holds
one fused qkv_proj and gate_up_proj. Dense weights are fused along their rows; the AutoAWQ
tensors (qweight [K, N/8], qzeros [K/G, N/8], scales [K/G, N]) carry the output dimension second,
so they are fused along their columns: shard offsets are taken from the fused size (q first, k and
v sharing the remainder; gate and up halves). Loading is host work on CPU tensors; the W4Linear
layers are then moved to the GPU and repacked by ``finalize_quantized`` (``tandem_amd.model.prepare``).
The model classes, with the SwiGLU wiring of the MLP, are in ``tandem_amd.model``.
"""

from __future__ import annotations

import glob
import logging
import os
import re
from dataclasses import dataclass
from typing import Any, Optional

import torch
from torch import nn


logger = logging.getLogger(__name__)


@dataclass
class QuantConfig:
    """Weight-only quantization of a checkpoint (``quantization_config`` in config.json)."""

    method: str  # "awq"
    bits: int
    group_size: int

    @classmethod
    def from_dict(cls, d: Optional[dict[str, Any]]) -> Optional["QuantConfig"]:
        """None for an unquantized model; 4-bit AutoAWQ "gemm" with zero points, else
        NotImplementedError (python/tandem/model_config.py:35-43)."""
        if not d:
            return None
        if (d.get("quant_method") == "awq" and d.get("bits") == 4 and d.get("zero_point", True)
                and str(d.get("version", "gemm")).lower() == "gemm"):
            return cls("awq", 4, int(d.get("group_size", 128)))
        raise NotImplementedError(f"unsupported quantization_config: {d} (4-bit AWQ 'gemm' checkpoints only)")


_IGNORED = re.compile(r"(rotary_emb\.inv_freq|\.attn\.bias|\.masked_bias)$")
_AWQ_SUFFIXES = (".qweight", ".qzeros", ".scales")
# checkpoint tensors that fill a slice of a fused model tensor: (pattern, fused name, shard order)
_STACKED = (
    (re.compile(r"^(.*\.self_attn)\.(q|k|v)_proj\.(weight|bias|qweight|qzeros|scales)$"), "qkv_proj", ("q", "k", "v")),
    (re.compile(r"^(model\.layers\.\d+\.mlp)\.(gate|up)_proj\.(weight|qweight|qzeros|scales)$"), "gate_up_proj",
     ("gate", "up")),
)


def stacked_target(name: str) -> Optional[tuple[str, str, tuple[str, ...]]]:
    """Checkpoint name -> (fused tensor name, shard, all shards), or None."""
    for pattern, fused, shards in _STACKED:
        m = pattern.match(name)
        if m:
            return f"{m.group(1)}.{fused}.{m.group(3)}", m.group(2), shards
    return None


def copy_shard(dst: torch.Tensor, src: torch.Tensor, shard: str, shards: tuple[str, ...], name: str) -> None:
    """Copy one shard into its slice of the fused tensor: rows for dense tensors, columns for the
    AutoAWQ ones (python/tandem/models/loader.py:41-58)."""
    if name.endswith(_AWQ_SUFFIXES):
        dst, src = dst.t(), src.t()
    rows, total = src.shape[0], dst.shape[0]
    if shards == ("q", "k", "v"):
        start = {"q": 0, "k": total - 2 * rows, "v": total - rows}[shard]
    else:
        start = {"gate": 0, "up": rows}[shard]
    if start < 0 or start + rows > total or tuple(src.shape[1:]) != tuple(dst.shape[1:]):
        raise ValueError(f"shape mismatch for {name}: checkpoint {tuple(src.shape)} vs fused {tuple(dst.shape)}")
    with torch.no_grad():
        dst[start:start + rows].copy_(src.to(dst.dtype))


def load_weights(model: nn.Module, model_path: str) -> None:
    """Every parameter, and the AWQ buffers of quantized layers (qweight / qzeros / scales, which
    the W4Linear constructor registers), from the *.safetensors files of ``model_path``. Unknown
    checkpoint tensors are reported and skipped; a parameter or buffer left unfilled raises."""
    from safetensors import safe_open

    files = sorted(glob.glob(os.path.join(model_path, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors files in {model_path}")
    targets = dict(model.named_parameters())
    targets.update({n: b for n, b in model.named_buffers() if n.endswith(_AWQ_SUFFIXES)})
    loaded: set[str] = set()
    unexpected: list[str] = []
    shards_seen: dict[str, set[str]] = {}
    for path in files:
        with safe_open(path, framework="pt", device="cpu") as f:
            for name in f.keys():
                if _IGNORED.search(name):
                    continue
                stacked = stacked_target(name)
                if stacked is not None and stacked[0] in targets:
                    target, shard, shards = stacked
                    copy_shard(targets[target], f.get_tensor(name), shard, shards, name)
                    seen = shards_seen.setdefault(target, set())
                    seen.add(shard)
                    if seen == set(shards):
                        loaded.add(target)
                    continue
                if name not in targets:
                    if name != "lm_head.weight":  # tied-embedding checkpoints may still store it
                        unexpected.append(name)
                    continue
                tensor, dst = f.get_tensor(name), targets[name]
                if tuple(dst.shape) != tuple(tensor.shape):
                    raise ValueError(f"shape mismatch for {name}: checkpoint {tuple(tensor.shape)} vs model "
                                     f"{tuple(dst.shape)}")
                with torch.no_grad():
                    dst.copy_(tensor.to(dst.dtype))
                loaded.add(name)
    if unexpected:
        logger.warning("ignored %d unexpected checkpoint tensors, e.g. %s", len(unexpected), unexpected[:3])
    missing = sorted(set(targets) - loaded)
    if missing:
        raise RuntimeError(f"{len(missing)} parameters missing from checkpoint, e.g. {missing[:5]}")

"""RMSNorm and residual-add + RMSNorm around the W4A16 projections, on libtandem_w4.so.

The decoder layer's small per-token kernels that sit between the projections of a decode step
(python/tandem/models/llama_family.py:47-67):

    RMSNorm               the module (weight, eps)                 python/tandem/layers/norm.py:7-19
    HipOps.rms_norm       y = rms_norm(x) * w                      python/tandem/layers/ops.py:107-109
    HipOps.fused_add_rms_norm  residual <- x + residual; x <- rms_norm(residual) * w, in place
                                                                   python/tandem/layers/ops.py:111-120

Numerics are those of the reference's GPU path (FlashInfer's kernels and the Triton
fused_add_rmsnorm, python/tandem/layers/triton_ops.py:101-124): fp32 sum, the residual stored in
fp16, the output from the unrounded sum with one rounding. The reference's TorchOps (norm then
weight in fp16) differs from it by fp16 rounding only.
"""

from __future__ import annotations

import torch
from torch import nn

from tandem_amd.layers import w4_hip


def _check(who: str, x: torch.Tensor, weight: torch.Tensor) -> tuple[int, int]:
    if x.dim() != 2 or not x.is_contiguous() or x.dtype != torch.float16 or not x.is_cuda:
        raise RuntimeError(f"{who}: contiguous float16 [M, K] GPU rows expected (got {tuple(x.shape)}, {x.dtype})")
    if (weight.shape != (x.shape[1],) or weight.dtype != torch.float16 or weight.device != x.device
            or not weight.is_contiguous()):
        raise RuntimeError(f"{who}: contiguous float16 weight [{x.shape[1]}] on x's GPU expected")
    return x.shape[0], x.shape[1]


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = fp16(x * rsqrt(mean(x^2) + eps) * weight) over the last dimension (tw4_rms_norm)."""
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    m, k = _check("rms_norm", x2, weight)
    if out is None:
        y = torch.empty_like(x2)
    elif (out.shape != x.shape or out.dtype != torch.float16 or out.device != x.device or not out.is_contiguous()
          or out.data_ptr() % 16):
        raise RuntimeError(f"rms_norm: out must be a contiguous 16-byte aligned float16 tensor shaped like x "
                           f"{tuple(shape)} on x's GPU")
    else:
        y = out.view(m, k)
    if m == 0:
        return y.view(shape)
    with torch.cuda.device(x.device):
        w4_hip.check(w4_hip.library().tw4_rms_norm(x2.data_ptr(), weight.data_ptr(), y.data_ptr(), m, k, float(eps),
                                                   torch.cuda.current_stream(x.device).cuda_stream))
    return y.view(shape)


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                       eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """In place: residual <- x + residual, x <- rms_norm(residual) * weight (tw4_add_rms_norm).
    Returns (x, residual)."""
    m, k = _check("fused_add_rms_norm", x, weight)
    if residual.shape != x.shape or residual.dtype != x.dtype or not residual.is_contiguous() \
            or residual.device != x.device:
        raise RuntimeError("fused_add_rms_norm: residual must match x")
    if m == 0:
        return x, residual
    with torch.cuda.device(x.device):
        w4_hip.check(w4_hip.library().tw4_add_rms_norm(x.data_ptr(), residual.data_ptr(), weight.data_ptr(), m, k,
                                                       float(eps), torch.cuda.current_stream(x.device).cuda_stream))
    return x, residual


class HipOps:
    """The norm half of the reference's ops interface (python/tandem/layers/ops.py:62-120) on the
    HIP kernels; the attention-side ops (RoPE) belong to another path."""

    name = "hip"

    @staticmethod
    def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
        return rms_norm(x, weight, eps)

    @staticmethod
    def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                           eps: float) -> tuple[torch.Tensor, torch.Tensor]:
        return fused_add_rms_norm(x, residual, weight, eps)


class RMSNorm(nn.Module):
    """RMSNorm with a learned weight (python/tandem/layers/norm.py:7-19), on tw4_rms_norm."""

    def __init__(self, dim: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.weight, self.eps)

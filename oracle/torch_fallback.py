"""The reference's dequantize-then-matmul fallback restated in torch on the CPU. TEST INFRASTRUCTURE
ONLY: ``bench.py``'s ``cpu_baseline`` leg times it, and ``tests/`` pins it against the numpy oracle;
the product (``tandem_amd``) never imports it.

12vivi/tandem's W4Linear falls back, for shapes its kernels do not take, to dequantizing the whole
weight every call and one dense product (python/tandem/layers/awq.py:282-286):

    w = w4_dequant(...)          fp16_rne((q - z) * s), [N, K]           awq.py:89-133
    y = F.linear(x, w)           fp16 GEMM                               awq.py:284-285

Its dequantization is a Triton GPU kernel, so that fallback cannot run on a CPU as written. This
module is the same arithmetic in plain torch CPU ops, written for speed on many cores (the group
dimension broadcast rather than repeated), so that it is a fair CPU baseline:

    unpack_awq        AutoAWQ nibble order (feature 8 c + j in nibble            awq.py:38-46
                      AWQ_REVERSE_ORDER[j] of word c)
    dequant_kn        fp16_rne((q - z) * s) as [K, N] (float32 product, one      awq.py:110-119
                      rounding: bit-exact to the numpy oracle's dequant)
    fallback_linear   x @ dequant(W)^T with the product in ``dtype`` (float16     awq.py:284-285
                      like F.linear on the fp16 weight, or float32), y in fp16
"""

from __future__ import annotations

import torch

GROUP = 128
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)
_SHIFTS = torch.tensor([4 * i for i in AWQ_REVERSE_ORDER], dtype=torch.int32)


def unpack_awq(packed: torch.Tensor) -> torch.Tensor:
    """[R, C] int32 -> [R, 8 C] int32 values 0..15 (python/tandem/layers/awq.py:42-46)."""
    return ((packed.unsqueeze(-1) >> _SHIFTS) & 0xF).reshape(packed.shape[0], -1)


def dequant_kn(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """AutoAWQ tensors -> fp16 [K, N] = fp16_rne((q - z) * s): the integer difference times the fp16
    scale is exact in float32, then one cast (python/tandem/layers/awq.py:110-119)."""
    k = qweight.shape[0]
    q = unpack_awq(qweight).view(k // GROUP, GROUP, -1)
    z = unpack_awq(qzeros).unsqueeze(1)
    w = (q - z).to(torch.float32) * scales.to(torch.float32).unsqueeze(1)
    return w.view(k, -1).to(torch.float16)


def fallback_linear(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                    dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """The fallback per call: dequantize the whole weight, then one product in ``dtype``; y fp16."""
    w = dequant_kn(qweight, qzeros, scales)
    return (x.to(dtype) @ w.to(dtype)).to(torch.float16)

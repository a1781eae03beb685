"""Small-batch fp16 GEMV for decode on MI355X: y[M, N] = x[M, K] @ w[N, K]^T, M <= 8.

Drop-in for python/tandem/layers/triton_gemv.py (12vivi/tandem) on the path of a W4A16 model's
fp16 lm_head: the same ``gemv`` / ``linear`` / ``install`` / ``table_for`` / ``default_table``
functions, the same per-GPU ``CONFIGS`` keyed by (N, K, M bucket) and the same fallback to
``F.linear`` (hipBLASLt here) for shapes without an entry. The kernel is tw4_gemv_f16 of
libtandem_w4.so (hand-written HIP for gfx950, no Triton): it streams every row of w once with
coalesced 16-byte loads and reduces on v_dot2_f32_f16, so it is bound by HBM bandwidth; for the
M = 8 bucket a matrix-core form (config rows_inflight 16 or 32) multiplies 16-row tiles of w with x
on v_mfma_f32_16x16x32_f16 instead, which reads x from LDS once per 16 rows rather than once per row.

The reference's fused norm / activation prologue (triton_gemv.py:92-178, 330-415) is not part of
this build: it enabled no shape there (triton_gemv.py:316-329).
"""

from __future__ import annotations

import functools
import os

import torch
import torch.nn.functional as F
from torch import nn

from tandem_amd.layers import w4_hip

# Config per GPU and (N, K, M bucket): (rows_inflight, rows_per_wave) of tw4_gemv_f16 (rows_inflight
# 16 / 32: the matrix-core form with one / two 128-k chunks per step in flight, rows_per_wave a
# multiple of 16), the fastest of
# `python -m tandem_amd.tune --projs lm_head --kinds dense16,torch16` on the GPU. Shapes without
# an entry keep F.linear (python/tandem/layers/triton_gemv.py:221-268). Keyed by device name and by
# gfx architecture.
Config = tuple[int, int]
GFX950_DENSE: dict[tuple[int, int, int], Config] = {
    # Qwen3-8B lm_head: 190 / 185 / 188 us at M = 1 / 2 / 4 (82-84 % of 8 TB/s) vs F.linear 243-251 us;
    # M = 5 .. 8: the matrix-core form with two chunks in flight, 231 us vs F.linear 246-249 us
    # (one chunk: 234-239 us; the v_dot2 form: 270-283 us)
    (151936, 4096, 1): (4, 32),
    (151936, 4096, 2): (2, 32),
    (151936, 4096, 4): (2, 32),
    (151936, 4096, 8): (32, 16),
    # Qwen3-1.7B lm_head: 96-99 us at M = 1 .. 4, 119 us at M = 8 (the matrix-core form) vs
    # F.linear 203 us
    (151936, 2048, 1): (2, 16),
    (151936, 2048, 2): (2, 16),
    (151936, 2048, 4): (2, 16),
    (151936, 2048, 8): (16, 16),
}
CONFIGS: dict[str, dict[tuple[int, int, int], Config]] = {
    "AMD Instinct MI355X": GFX950_DENSE,
    "gfx950": GFX950_DENSE,
}

# decoder-layer projections that run per decode step (python/tandem/layers/triton_gemv.py:270)
PROJECTIONS = ("qkv_proj", "o_proj", "gate_up_proj", "down_proj")
KS = (512, 1024, 2048, 4096)  # the K the kernel is compiled for


def m_bucket(m: int) -> int:
    """CUDA-graph decode batch buckets 1, 2, 4, 8 (python/tandem/layers/triton_gemv.py:273-274)."""
    return 1 if m <= 1 else 2 if m == 2 else 4 if m <= 4 else 8


def table_for(device: torch.device, model: nn.Module) -> dict[tuple[int, int, int], Config]:
    """This GPU's table (by name, else by gfx architecture); ``TANDEM_GEMV_FORCE=1`` sends every
    projection through the kernel (python/tandem/layers/triton_gemv.py:277-282)."""
    if os.environ.get("TANDEM_GEMV_FORCE") in ("1", "2"):
        return default_table(model)
    name = torch.cuda.get_device_name(device)
    if name in CONFIGS:
        return CONFIGS[name]
    arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "").split(":")[0]
    return CONFIGS.get(arch, {})


def gemv(x: torch.Tensor, w: torch.Tensor, rows_inflight: int = 2, rows_per_wave: int = 32,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """x [M, K] (M <= 8), w [N, K] row-major, both float16 on the GPU -> [M, N] float16
    (python/tandem/layers/triton_gemv.py:180-218). Launches on the current stream."""
    if x.dim() != 2 or w.dim() != 2:
        raise ValueError(f"gemv: 2-D x and w expected (x {tuple(x.shape)}, w {tuple(w.shape)})")
    m, k = x.shape
    n, k2 = w.shape
    if k != k2 or m > 8 or m < 1 or k not in KS or x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError(f"gemv: unsupported shapes x {tuple(x.shape)} w {tuple(w.shape)}")
    if not (x.is_cuda and w.is_cuda and x.dtype == torch.float16 and w.dtype == torch.float16):
        raise RuntimeError("gemv: float16 GPU tensors expected")
    if not (x.is_contiguous() and w.is_contiguous() and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0):
        raise RuntimeError("gemv: x and w must be contiguous and 16-byte aligned")
    y = out if out is not None else torch.empty((m, n), dtype=x.dtype, device=x.device)
    w4_hip.check(w4_hip.library().tw4_gemv_f16(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k, rows_inflight,
                                               rows_per_wave, torch.cuda.current_stream(x.device).cuda_stream))
    return y


def linear(x: torch.Tensor, w: torch.Tensor, table: dict[tuple[int, int, int], Config],
           eager: bool = True) -> torch.Tensor:
    """F.linear(x, w) without bias, through the kernel where ``table`` has an entry
    (python/tandem/layers/triton_gemv.py:285-297). ``eager=False``: only inside graph capture."""
    if (x.dim() == 2 and x.shape[0] <= 8 and x.is_contiguous() and x.dtype == w.dtype == torch.float16
            and (eager or torch.cuda.is_current_stream_capturing())):
        cfg = table.get((w.shape[0], w.shape[1], m_bucket(x.shape[0])))
        if cfg is not None and x.data_ptr() % 16 == 0:
            return gemv(x, w, *cfg)
    return F.linear(x, w)


def _forward(module: nn.Linear, table: dict, x: torch.Tensor) -> torch.Tensor:
    return linear(x, module.weight, table, eager=False)


def install(model: nn.Module, table: dict[tuple[int, int, int], Config]) -> int:
    """Route the decoder projections of ``model`` through ``linear``; returns how many
    (python/tandem/layers/triton_gemv.py:304-315)."""
    if not table:
        return 0
    n = 0
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and mod.bias is None and name.rsplit(".", 1)[-1] in PROJECTIONS:
            mod.forward = functools.partial(_forward, mod, table)  # instance attribute shadows Linear.forward
            n += 1
    model.gemv_table = table  # the logits head goes through ``linear`` too
    return n


def default_table(model: nn.Module) -> dict[tuple[int, int, int], Config]:
    """A table that sends every projection shape of ``model`` the kernel supports through it
    (tests; python/tandem/layers/triton_gemv.py:418-428)."""
    table = {}
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and name.rsplit(".", 1)[-1] in PROJECTIONS:
            n, k = mod.weight.shape
            if k in KS:
                for m in (1, 2, 4, 8):
                    table[(n, k, m)] = (2, 32)
    return table

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

import os

import torch
import torch.nn.functional as F
from torch import nn

from tandem_amd.layers import w4_hip

# Config per GPU and (N, K, M bucket): (rows_inflight, rows_per_wave) of tw4_gemv_f16 (rows_inflight
# 16 / 32: the matrix-core form with one / two 128-k chunks per step in flight, rows_per_wave a
# multiple of 16), the fastest of
# `python bench.py tune --projs lm_head --kinds dense16,torch16` on the GPU. Shapes without
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

# The decoder projections a step runs through the kernel when the table has their shape (the names
# python/tandem/layers/triton_gemv.py:270 routes), and the K the kernel is compiled for.
PROJECTIONS = ("qkv_proj", "o_proj", "gate_up_proj", "down_proj")
KS = (512, 1024, 2048, 4096)
# Batch buckets of the decode graphs: a table entry for bucket b serves every M up to b.
BUCKETS = (1, 2, 4, 8)
# What ``default_table`` gives every shape: two rows in flight, 32 rows per wavefront (the v_dot2 form).
DEFAULT_CONFIG: Config = (2, 32)


def m_bucket(m: int) -> int:
    """The bucket whose entry serves a batch of m rows: the smallest of BUCKETS that holds m (M past
    the last bucket maps to it; the caller sends those to F.linear)."""
    return next((b for b in BUCKETS if m <= b), BUCKETS[-1])


def _device_keys(device: torch.device) -> list[str]:
    """Table keys of a GPU, most specific first: its marketing name, then its gfx architecture (a
    HIP runtime can report a generic name, or none under rocprofv3)."""
    arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "").split(":")[0]
    return [torch.cuda.get_device_name(device), arch]


def table_for(device: torch.device, model: nn.Module) -> dict[tuple[int, int, int], Config]:
    """The measured table of ``device``, or {} (every call then takes F.linear). With
    ``TANDEM_GEMV_FORCE`` set to 1 or 2 (the reference's test switch) every projection of ``model``
    the kernel can run gets ``DEFAULT_CONFIG`` instead (python/tandem/layers/triton_gemv.py:277-282)."""
    if os.environ.get("TANDEM_GEMV_FORCE") in ("1", "2"):
        return default_table(model)
    return next((CONFIGS[k] for k in _device_keys(device) if k in CONFIGS), {})


def gemv(x: torch.Tensor, w: torch.Tensor, rows_inflight: int = 2, rows_per_wave: int = 32,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """y [M, N] = x [M, K] @ w [N, K]^T by tw4_gemv_f16, 1 <= M <= 8, float16 GPU tensors, on the
    current stream (python/tandem/layers/triton_gemv.py:180-218). Shapes the kernel does not take
    raise ValueError; placement, dtype and alignment problems RuntimeError, before any launch.
    ``out``: a float16 [M, N] contiguous 16-byte aligned tensor on x's GPU to write into."""
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"gemv: x [M, K] and w [N, K] expected (x {tuple(x.shape)}, w {tuple(w.shape)})")
    (m, k), n = x.shape, w.shape[0]
    if not 1 <= m <= BUCKETS[-1] or k not in KS:
        raise ValueError(f"gemv: 1 <= M <= {BUCKETS[-1]} and K in {KS} (x {tuple(x.shape)}, w {tuple(w.shape)})")
    for name, t in (("x", x), ("w", w)):
        if not (t.is_cuda and t.dtype == torch.float16):
            raise RuntimeError(f"gemv: {name} must be a float16 GPU tensor")
        if not t.is_contiguous() or t.data_ptr() % 16:
            raise RuntimeError(f"gemv: {name} must be contiguous and 16-byte aligned")
    if w.device != x.device:
        raise RuntimeError("gemv: x and w must be on one GPU")
    if out is None:
        out = torch.empty((m, n), dtype=torch.float16, device=x.device)
    elif (tuple(out.shape) != (m, n) or out.dtype != torch.float16 or out.device != x.device
          or not out.is_contiguous() or out.data_ptr() % 16):
        raise RuntimeError(f"gemv: out must be a contiguous 16-byte aligned float16 [{m}, {n}] tensor on x's GPU")
    w4_hip.check(w4_hip.library().tw4_gemv_f16(x.data_ptr(), w.data_ptr(), out.data_ptr(), m, n, k, rows_inflight,
                                               rows_per_wave, torch.cuda.current_stream(x.device).cuda_stream))
    return out


def entry(x: torch.Tensor, w: torch.Tensor, table: dict[tuple[int, int, int], Config],
          eager: bool = True) -> Config | None:
    """The table's configuration for F.linear(x, w) if the kernel may run it, else None: a float16
    x of 1 .. 8 contiguous 16-byte aligned rows and a float16 w, and (``eager=False``) only while a
    HIP graph is being captured, which is how the decoder projections run in a decode step."""
    if x.dim() != 2 or not 1 <= x.shape[0] <= BUCKETS[-1]:
        return None
    if x.dtype != torch.float16 or w.dtype != torch.float16 or not x.is_contiguous() or x.data_ptr() % 16:
        return None
    if not eager and not torch.cuda.is_current_stream_capturing():
        return None
    return table.get((w.shape[0], w.shape[1], m_bucket(x.shape[0])))


def linear(x: torch.Tensor, w: torch.Tensor, table: dict[tuple[int, int, int], Config],
           eager: bool = True) -> torch.Tensor:
    """F.linear(x, w) (no bias) through tw4_gemv_f16 where ``entry`` finds a configuration, through
    F.linear (hipBLASLt) otherwise (python/tandem/layers/triton_gemv.py:285-297)."""
    cfg = entry(x, w, table, eager)
    return F.linear(x, w) if cfg is None else gemv(x, w, *cfg)


class TabledLinear(nn.Linear):
    """An nn.Linear whose forward goes through ``linear`` with the table it carries, in graph
    capture only (eager calls, e.g. prefill, keep F.linear). ``install`` turns a model's bias-free
    projections into this class in place, so their names, parameters and state dicts stay those of
    nn.Linear."""

    gemv_table: dict

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return linear(x, self.weight, self.gemv_table, eager=False)


def install(model: nn.Module, table: dict[tuple[int, int, int], Config]) -> int:
    """Route the bias-free decoder projections (PROJECTIONS) of ``model`` through the kernel by
    ``table``, and keep the table on the model for its logits head. Returns how many projections;
    an empty table changes nothing (python/tandem/layers/triton_gemv.py:304-315)."""
    if not table:
        return 0
    chosen = [mod for name, mod in model.named_modules()
              if isinstance(mod, nn.Linear) and mod.bias is None and name.rsplit(".", 1)[-1] in PROJECTIONS]
    for mod in chosen:
        mod.gemv_table = table
        mod.__class__ = TabledLinear
    model.gemv_table = table
    return len(chosen)


def default_table(model: nn.Module) -> dict[tuple[int, int, int], Config]:
    """DEFAULT_CONFIG for every (N, K, bucket) of ``model``'s projections whose K the kernel takes:
    a table that sends them all through it, for tests (python/tandem/layers/triton_gemv.py:418-428)."""
    shapes = {tuple(mod.weight.shape) for name, mod in model.named_modules()
              if isinstance(mod, nn.Linear) and name.rsplit(".", 1)[-1] in PROJECTIONS}
    return {(n, k, b): DEFAULT_CONFIG for n, k in shapes if k in KS for b in BUCKETS}

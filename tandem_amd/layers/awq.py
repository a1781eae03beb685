"""The W4A16 linear layer of an AutoAWQ model on MI355X (gfx950), and its load-time helpers.

Drop-in for python/tandem/layers/awq.py (12vivi/tandem): a caller builds ``W4Linear`` with the
constructor it knows, the loader fills the same three buffers, ``enable_silu_mul`` / ``finalize`` /
``forward`` keep their contract, and the per-GPU tables, ``pick_gemm`` and the ``TANDEM_W4_GEMM``
switch keep their meaning. Underneath, every kernel is hand-written HIP for gfx950
(libtandem_w4.so, include/tandem_w4.h): no Triton, no CUDA, no CPU path.

The checkpoint side is AutoAWQ's "gemm" packing, which the loader hands over unchanged:
    qweight  int32 [K, N/8]    output features 8 c .. 8 c + 7 of input k share word (k, c); the
                               feature 8 c + j sits in nibble AWQ_REVERSE_ORDER[j]
    qzeros   int32 [K/G, N/8]  the 4-bit zero point of each (group, feature), packed alike
    scales   fp16  [K/G, N]    the scale of each (group, feature)
with G = 128 inputs per group, and weight (n, k) = (q - z) * s of its group's zero and scale.

``finalize`` repacks once, on the GPU, into the tile layout of the MI355X kernels:
    packed [Npad, K/8] int32  (Npad = N rounded up to 16), viewed as [Npad/16][K/128][4 kb][16 r][4 s]:
           word (kb, r, s) of row tile T and group g holds the 8 consecutive weights
           k = 128 g + 32 kb + 8 s + 2 q + e (q = 0..3, e = 0..1) of row 16 T + r in nibble q + 4 e;
           one (row tile, group) block is 1 KB, read by one 64-lane wavefront with one 16-byte
           load per lane (lane 16 kb + r). Rows >= N are zero.
    scales [N, K/G] float16, zeros [N, K/G] float16 (the integer zero point, exact), both stored
           tile-major (tile_major_params): a row tile's values as [group][row], so a wavefront's
           per-group load of 16 rows' scales is one 32-byte segment
The nibble order inside a word is the reference's (python/tandem/layers/awq.py:12-20); the word
order is this build's (the reference keeps each row contiguous: [N][K/G][4 j][4 cc]).

Kernels (libtandem_w4.so): w4_gemv (M <= 4, vector ALUs), w4_mma (M <= 64, matrix cores) and
w4_gemm (any M, matrix cores, LDS-staged activations, split-K). Where the table says so, with
TANDEM_W4_GEMM=0, with TANDEM_NO_CUDA_EXT=1 or for an unaligned x: HIP dequantize to float16 +
torch.matmul (hipBLASLt).
"""

from __future__ import annotations

import os

import torch
import torch.nn.functional as F
from torch import nn

from tandem_amd.layers import w4_hip
from tandem_amd.layers.w4_tables import GFX950_DECODE, GFX950_GEMM

# Nibble of an AutoAWQ word that holds feature j = 0..7 of its 8: the packer writes features
# 0, 2, 4, 6, 1, 3, 5, 7 into nibbles 0..7, so feature j is found at this position
# (python/tandem/layers/awq.py:38-39)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


def unpack_awq(packed: torch.Tensor) -> torch.Tensor:
    """[R, C] int32 in AWQ order -> [R, 8 C] int32 values 0..15 (column c*8 + j); a layout utility
    on any device (python/tandem/layers/awq.py:42-46)."""
    shifts = torch.tensor([4 * i for i in AWQ_REVERSE_ORDER], dtype=torch.int32, device=packed.device)
    return ((packed[:, :, None] >> shifts) & 0xF).reshape(packed.shape[0], -1)


def pack_rows(q: torch.Tensor) -> torch.Tensor:
    """[N, K] values 0..15 -> tile layout [Npad, K/8] int32 (see the module docstring); a layout
    utility on any device. The counterpart of python/tandem/layers/awq.py:49-57 for this build's
    layout; finalize uses the tw4_repack_awq kernel instead."""
    n, k = q.shape
    npad = w4_hip.padded_rows(n)
    v = torch.zeros((npad, k), dtype=torch.int64, device=q.device)
    v[:n] = q.to(torch.int64)
    v = v.view(npad // 16, 16, k // 128, 4, 4, 4, 2)  # [T, r, g, kb, s, q, e]: k = 128 g + 32 kb + 8 s + 2 q + e
    v = v.permute(0, 2, 3, 1, 4, 5, 6)  # -> [T, g, kb, r, s, q, e]
    shifts = 4 * (torch.arange(4, device=q.device)[:, None] + 4 * torch.arange(2, device=q.device)[None, :])
    words = (v << shifts).sum(dim=(-1, -2))  # nibbles do not overlap: sum == or
    words = torch.where(words >= 1 << 31, words - (1 << 32), words)  # int32 bit pattern
    return words.reshape(npad, k // 8).to(torch.int32)


def tile_major_params(t: torch.Tensor) -> torch.Tensor:
    """Row-major [N, K/G] scales / zeros -> the kernels' tile-major order, same shape: row tile T
    (16 rows, or the N - 16 T left over) stored as [group][row], so one group's rows are
    contiguous (offset 16 T G + g rows_T + r). A layout utility on any device."""
    n, g = t.shape
    full = n // 16 * 16
    parts = [t[:full].reshape(n // 16, 16, g).transpose(1, 2).reshape(-1)]
    if full < n:
        parts.append(t[full:].t().reshape(-1))
    return torch.cat(parts).reshape(n, g)


def row_major_params(t: torch.Tensor) -> torch.Tensor:
    """Inverse of tile_major_params."""
    n, g = t.shape
    full = n // 16 * 16
    flat = t.reshape(-1)
    parts = [flat[:full * g].reshape(n // 16, g, 16).transpose(1, 2).reshape(full, g)]
    if full < n:
        parts.append(flat[full * g:].reshape(g, n - full).t())
    return torch.cat(parts)


def repack_awq(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group: int,
               dtype: torch.dtype = torch.float16, interleave: bool = False
               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """AWQ (qweight [K, N/8], qzeros [K/G, N/8], scales [K/G, N]) -> tile layout (packed [Npad, K/8]
    int32, scales [N, K/G] and zeros [N, K/G] in tile-major order) on the GPU
    (python/tandem/layers/awq.py:60-68).
    ``interleave``: rows in interleave_gate_up order (the reference applies interleave_gate_up to
    the repacked rows, awq.py:237-238; the tile layout takes it inside the repack kernel)."""
    if group != 128 or qweight.shape[0] % 128 or scales.shape != (qweight.shape[0] // group, 8 * qweight.shape[1]):
        raise ValueError(f"repack_awq: qweight {tuple(qweight.shape)} scales {tuple(scales.shape)} group {group}")
    if dtype != torch.float16:
        raise ValueError("repack_awq: the MI355X kernels take float16 scales and zeros")
    return w4_hip.repack(qweight, qzeros, scales, interleave=interleave)


def interleave_gate_up(t: torch.Tensor) -> torch.Tensor:
    """Rows [gate (I); up (I)] -> tiles of 16 rows [gate 8i .. 8i+7, up 8i .. 8i+7], the order in
    which the kernels' SwiGLU epilogues find gate and up of a feature in paired lanes
    (python/tandem/layers/awq.py:71-75). For row-major tensors (scales, zeros, dense
    weights, before tile_major_params); the tile-layout `packed` is interleaved by
    repack_awq(..., interleave=True)."""
    n = t.shape[0]
    return t.view(2, n // 16, 8, *t.shape[1:]).transpose(0, 1).reshape(t.shape)


def silu_and_mul(y: torch.Tensor) -> torch.Tensor:
    """[M, 2I] = [gate | up] -> silu(gate) * up (python/tandem/layers/awq.py:78-86, torch branch)."""
    gate, up = y.chunk(2, dim=-1)
    return F.silu(gate) * up


def w4_dequant(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group: int = 128,
               dtype: torch.dtype = torch.float16, block_n: int = 32, deinterleave: bool = False) -> torch.Tensor:
    """-> dense [N, K] (nn.Linear layout), bit-exact fp16_rne((q - z) s), by the HIP dequant kernel
    (python/tandem/layers/awq.py:122-133). ``deinterleave``: undo interleave_gate_up on the rows.
    ``block_n`` is accepted for signature compatibility and ignored."""
    if group != 128:
        raise ValueError("w4_dequant: group 128 only")
    if deinterleave and scales.shape[0] % 16:
        raise ValueError("w4_dequant: deinterleave needs N a multiple of 16")
    w = w4_hip.dequant(packed, scales, zeros, deinterleave=deinterleave)
    return w if dtype == torch.float16 else w.to(dtype)


# Decode kernel per GPU and (N, K, M) / (N, K, M, "silu") for M <= 16, the fastest of
# `python bench.py tune` sweeps on the GPU:
#   ("gemv", warps_k, unroll, ntile)   vector ALUs, M <= 4 (with the SwiGLU epilogue too: the
#                                      reference's SwiGLU gate_up always takes "mma")
#   ("gemvm", warps_k, unroll, ntile)  the GEMV's arithmetic (exact q - z, scale per group) on the
#                                      matrix cores, M <= 16 (x' in LDS: K = 4096 up to M = 16)
#   ("mma", warps_k, unroll, ntile)    matrix cores, M <= 64
#   ("mmak", warps_k, unroll, ntile, splits)   the same with K split over `splits` workgroups per
#                                      row-tile group (x in LDS over 1 / splits of K; the last arriver
#                                      adds the partials, w4_gemm's workspace), M <= 16
#   ("mmap", warps_k, unroll, ntile, per_cu)   the same with at most per_cu workgroups per CU, each
#                                      staging x once and streaming several row-tile groups, M <= 16
#   ("gemm", MT, NT, WARPS_N, WARPS_K, STAGES, SPLITS)   the fused GEMM (below), where it wins
# warps_k: wavefronts splitting K in a workgroup; unroll: quant groups in flight per lane and
# iteration; ntile: 16-row tiles per wavefront. Shapes without an entry use DEFAULT_KERNEL.
# Keys (N, K, M[, "silu"], "norm") name the GEMV configuration of the fused add + RMSNorm prologue
# (forward_norm), timed on its own; the plain key's entry is used where there is none.
# Tables are keyed by device name and by gfx architecture; finalize() tries the name it is given,
# then the architecture of the layer's GPU. (Same dispatch structure as
# python/tandem/layers/awq.py:136-160.)
W4Kernel = tuple
DEFAULT_KERNEL: W4Kernel = ("mma", 4, 2, 1)
MI355X = "AMD Instinct MI355X"
GFX950 = "gfx950"
W4_KERNELS: dict[str, dict[tuple, W4Kernel]] = {
    MI355X: GFX950_DECODE,
    GFX950: GFX950_DECODE,
}

# GEMM for M > 16 per GPU and (N, K) / (N, K, "silu"): ((m_max, config), ...) by increasing m_max;
# M past the last m_max uses the last entry. config = (MT, NT, WARPS_N, WARPS_K, STAGES, SPLITS) of
# w4_gemm (BM = 16 MT tokens, each wavefront 16 NT rows, WARPS_N x WARPS_K wavefronts, STAGES-deep
# LDS ring, SPLITS: split-K of every tile, or 0: of the last, partial wave of tiles only), or
# ("mma", warps_k, unroll, ntile): the streaming matrix-core kernel of the decode path, whose 16-token
# batch tiles cover M <= 64 (bandwidth-bound batches), or None: dequantize to float16 +
# torch.matmul. Shapes without an entry use DEFAULT_GEMM, which stops at M = 1024 like the measured
# gfx950 ladders before the GEMM with both tiles staged through LDS (stages 3): on the Qwen3-8B shapes
# that GEMM carries the fused path to M = 2048, and past it the dequantize + hipBLASLt pair wins (by
# ~20 % at M = 4096), since the one-off dequant is small next to the product there.
# TANDEM_W4_GEMM=0: always dequantize + torch.matmul (python/tandem/layers/awq.py:163-186).
W4Gemm = tuple
DEFAULT_GEMM: tuple[tuple[int, W4Gemm | None], ...] = (
    (64, ("mma", 8, 1, 1)), (1024, (4, 2, 4, 1, 2, 0)), (1 << 30, None))
W4_GEMM_KERNELS: dict[str, dict[tuple, tuple[tuple[int, W4Gemm | None], ...]]] = {
    MI355X: GFX950_GEMM,
    GFX950: GFX950_GEMM,
}
FUSED_GEMM = os.environ.get("TANDEM_W4_GEMM", "1") != "0"


def pick_gemm(table: tuple[tuple[int, W4Gemm | None], ...], m: int) -> W4Gemm | None:
    """First entry whose m_max >= m, else the last one (python/tandem/layers/awq.py:189-193)."""
    for m_max, cfg in table:
        if m <= m_max:
            return cfg
    return table[-1][1]


def _aligned(x: torch.Tensor) -> bool:
    return x.dim() == 2 and x.dtype == torch.float16 and x.is_contiguous() and x.data_ptr() % 16 == 0


def _hip_ok(x: torch.Tensor) -> bool:
    """Decode kernels (python/tandem/layers/awq.py:196-198), plus: on a GPU."""
    return x.is_cuda and _aligned(x) and 1 <= x.shape[0] <= 16


def _gemm_ok(x: torch.Tensor) -> bool:
    """The M > 16 GEMM (python/tandem/layers/awq.py:201-203), within its M x K < 2^31 limit (the
    reference's w4_gemm check, csrc/w4_gemv.cu:661): larger inputs take dequantize + matmul."""
    return FUSED_GEMM and x.is_cuda and _aligned(x) and x.shape[0] > 16 and x.shape[0] * x.shape[1] < 1 << 31


def _table(tables: dict, device_name: str | None, device: torch.device) -> dict:
    """None: no table, every shape takes the defaults (python/tandem/layers/awq.py:244-245).
    Else the table for `device_name`, or for the gfx architecture of `device` when the name is not
    a key: a HIP runtime may report a generic marketing name ("AMD Radeon Graphics") or, under
    rocprofv3, an empty one."""
    if device_name is None:
        return {}
    if device_name in tables:
        return tables[device_name]
    if device.type == "cuda" and torch.cuda.is_available():
        arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "").split(":")[0]
        return tables.get(arch, {})
    return {}


# Chunks (16 bytes of x) one wavefront stages in one batch: 64 lanes x 2 (kXB in tw4_decode.hip).
FUSED_NORM_CHUNKS = 128


class W4Linear(nn.Module):
    """y = x @ W^T for a bias-free projection whose W is AutoAWQ 4-bit (group 128), x and y fp16.

    Life cycle (python/tandem/layers/awq.py:206-286): constructed empty on the host with the
    AutoAWQ buffers ``qweight`` / ``qzeros`` / ``scales`` (a fused qkv or gate_up holds its parts
    side by side along the output features); filled by the loader; moved to the GPU; then
    ``finalize`` replaces the three buffers by the tile layout (``packed``, ``scales``, ``zeros``) in
    one repack kernel and picks the device's kernel tables. From then on ``forward`` dispatches by
    batch size: the (N, K, M) decode table up to M = 16, the M > 16 ladder above, dequantize +
    torch.matmul where the table says None, the switch is off or x is not 16-byte aligned.

    A SwiGLU MLP's gate_up calls ``enable_silu_mul`` before ``finalize``: the repack then interleaves
    gate and up rows by 8 and every kernel's epilogue returns silu(gate) * up, [M, out_features / 2]."""

    def __init__(self, in_features: int, out_features: int, group: int) -> None:
        super().__init__()
        if group != 128 or in_features % group or out_features % 8:
            raise ValueError(f"W4Linear({in_features}, {out_features}, group {group}): the kernels take group 128, "
                             "K a multiple of 128 and N a multiple of 8")
        self.in_features, self.out_features, self.group = in_features, out_features, group
        self.awq_layout = True
        self.silu_mul = False
        self.register_buffer("qweight", torch.empty(in_features, out_features // 8, dtype=torch.int32))
        self.register_buffer("qzeros", torch.empty(in_features // group, out_features // 8, dtype=torch.int32))
        self.register_buffer("scales", torch.empty(in_features // group, out_features, dtype=torch.float16))
        self.kernels: dict[tuple, W4Kernel] = {}
        self.gemm_kernels: dict[tuple, tuple[tuple[int, W4Gemm | None], ...]] = {}

    def enable_silu_mul(self) -> bool:
        if not self.awq_layout or self.out_features % 16:
            return False
        self.silu_mul = True
        return True

    @torch.no_grad()
    def finalize(self, device_name: str | None = None) -> None:
        packed, scales, zeros = repack_awq(self.qweight, self.qzeros, self.scales, self.group, torch.float16,
                                           interleave=self.silu_mul)
        del self._buffers["qweight"], self._buffers["qzeros"]
        self.register_buffer("packed", packed)
        self.register_buffer("scales", scales)
        self.register_buffer("zeros", zeros)
        self.awq_layout = False
        self.kernels = _table(W4_KERNELS, device_name, packed.device)
        self.gemm_kernels = _table(W4_GEMM_KERNELS, device_name, packed.device)
        # device set-up and the split-K workspace now, not inside graph capture
        if w4_hip.load() is not None:
            w4_hip.workspace(packed.device)

    def _dense(self, x: torch.Tensor) -> torch.Tensor:
        """HIP dequantize (gate_up: back in [gate | up] row order) + torch.matmul, and the same
        activation as the unfused path (python/tandem/layers/awq.py:282-286)."""
        if not x.is_cuda:
            raise RuntimeError("W4Linear: x must be on the GPU (there is no CPU path)")
        w = w4_dequant(self.packed, self.scales, self.zeros, self.group, x.dtype, deinterleave=self.silu_mul)
        y = F.linear(x, w)
        return silu_and_mul(y) if self.silu_mul else y

    def _gemm(self, ext, x: torch.Tensor, cfg) -> torch.Tensor:
        buf, locks = w4_hip.workspace(x.device)
        return ext.w4_gemm(x, self.packed, self.scales, self.zeros, buf, locks, *cfg, int(self.silu_mul))

    def kernel_for(self, m: int) -> str:
        """The kernel forward runs for a 16-byte aligned fp16 x of M rows on the GPU, by the same
        lookups as forward: e.g. "gemv(4, 2, 1)", "gemm(2, 1, 4, 2, 2, 4)" or "dequant+matmul"."""
        if m == 0:
            return "empty"
        if m <= 16:
            kind, *cfg = self.decode_entry(m)
            if kind not in ("gemm", "mmak", "mmap", "mma", "gemvm") and not (kind == "gemv" and m <= 4):
                kind, *cfg = DEFAULT_KERNEL
            return f"{kind}{tuple(cfg)}"
        key = (self.out_features, self.in_features) + (("silu",) if self.silu_mul else ())
        cfg = pick_gemm(self.gemm_kernels.get(key, DEFAULT_GEMM), m)
        if not FUSED_GEMM or cfg is None or m * self.in_features >= 1 << 31 or (cfg[0] == "mma" and m > 64):
            return "dequant+matmul"
        return f"mma{tuple(cfg[1:])}" if cfg[0] == "mma" else f"gemm{tuple(cfg)}"

    def decode_entry(self, m: int) -> W4Kernel:
        """The table entry forward uses at 1 <= M <= 16."""
        key = (self.out_features, self.in_features, m)
        return (self.kernels.get((*key, "silu")) if self.silu_mul else None) or self.kernels.get(key, DEFAULT_KERNEL)

    def norm_entry(self, m: int) -> W4Kernel:
        """The entry forward_norm uses: (N, K, M[, "silu"], "norm") where the fused-norm GEMV was
        timed on its own and beats the plain entry plus a separate norm kernel (its best
        configuration differs from the plain GEMV's: qkv at M = 1 runs 5.2 us with (4, 4, 1) against
        6.1 us with the plain table's (8, 2, 1)), else decode_entry."""
        key = (self.out_features, self.in_features, m) + (("silu",) if self.silu_mul else ()) + ("norm",)
        return self.kernels.get(key) or self.decode_entry(m)

    def forward_norm(self, x: torch.Tensor, residual: torch.Tensor | None, norm_weight: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor]:
        """self(rms_norm(x + residual) * norm_weight) and the new residual x + residual (x itself
        without a residual): the decoder layer's add + RMSNorm before qkv_proj / gate_up_proj
        (python/tandem/models/llama_family.py:58-65). Where the table runs the GEMV, the norm is
        fused into the kernel's x staging (tw4_decode_norm: the same bits as the separate norm
        kernel, one launch fewer); otherwise
        tw4_add_rms_norm / tw4_rms_norm, then forward. x and residual are consumed (the separate
        norm works in place). TANDEM_W4_FUSE_NORM=0 keeps the norm separate.

        The fusion is used where it measured faster on MI355X (the Qwen3-8B decode step at M = 1:
        1452 vs 1487 us): the GEMV, when each wavefront's slice of x is one staging batch (M x 16
        chunks per quant group x its groups <= 128 chunks). A longer slice loads its later batches
        behind the first weight chunk, whose wait then delays the next prefetch; the matrix-core
        kernel with the fused norm (tw4_decode_norm kind 1, exact as well) measured slower than the
        separate norm at M = 2 .. 8 (1786 vs 1691 us per step at M = 2), so the layer does not use it."""
        from tandem_amd.layers import norm

        m = x.shape[0] if x.dim() == 2 else 0
        if (1 <= m <= 16 and not self.awq_layout and _hip_ok(x) and os.environ.get("TANDEM_W4_FUSE_NORM", "1") != "0"
                and x.is_contiguous() and x.dtype == torch.float16):
            kind, *cfg = self.norm_entry(m)
            groups = self.in_features // self.group
            one_batch = m * 16 * -(-groups // cfg[0]) <= FUSED_NORM_CHUNKS
            if kind == "gemv" and m <= 4 and one_batch:
                ext = w4_hip.load()
                y, r_out = ext.w4_decode_norm(x, residual, norm_weight, eps, self.packed, self.scales, self.zeros,
                                              0, *cfg, int(self.silu_mul))
                return y, (r_out if residual is not None else x)
        if residual is None:
            return self(norm.rms_norm(x, norm_weight, eps)), x
        xn, residual = norm.fused_add_rms_norm(x, residual, norm_weight, eps)
        return self(xn), residual

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.awq_layout:
            raise RuntimeError("W4Linear: call finalize() (after moving the layer to the GPU) before forward")
        if x.dim() == 2 and x.shape[0] == 0:
            return x.new_empty((0, self.out_features // 2 if self.silu_mul else self.out_features))
        if _hip_ok(x):  # 1 <= M <= 16: the (N, K, M) table
            ext = w4_hip.load()
            if ext is not None:
                m = x.shape[0]
                key = (self.out_features, self.in_features, m)
                entry = (self.kernels.get((*key, "silu")) if self.silu_mul else None) or \
                    self.kernels.get(key, DEFAULT_KERNEL)
                kind, *cfg = entry
                if kind == "gemm":
                    return self._gemm(ext, x, cfg)
                if kind == "gemv" and m <= 4:  # with the SwiGLU epilogue too (tw4_gemv_act)
                    return ext.w4_gemv(x, self.packed, self.scales, self.zeros, *cfg, int(self.silu_mul))
                if kind == "gemvm":  # the GEMV's arithmetic on the matrix cores (M <= 16)
                    return ext.w4_gemv_mfma(x, self.packed, self.scales, self.zeros, *cfg, int(self.silu_mul))
                if kind == "mmak":  # the matrix-core decode kernel with K split over workgroups
                    buf, locks = w4_hip.workspace(x.device)
                    return ext.w4_mma_splitk(x, self.packed, self.scales, self.zeros, buf, locks, *cfg,
                                             int(self.silu_mul))
                if kind == "mmap":  # the matrix-core decode kernel, persistent workgroups
                    return ext.w4_mma_persist(x, self.packed, self.scales, self.zeros, *cfg, int(self.silu_mul))
                if kind != "mma":  # gemv past M = 4
                    _, *cfg = DEFAULT_KERNEL
                return ext.w4_mma(x, self.packed, self.scales, self.zeros, *cfg, int(self.silu_mul))
        elif _gemm_ok(x):  # M > 16: the GEMM, unless the table prefers dequantize + torch.matmul
            ext = w4_hip.load()
            if ext is not None:
                key = (self.out_features, self.in_features) + (("silu",) if self.silu_mul else ())
                cfg = pick_gemm(self.gemm_kernels.get(key, DEFAULT_GEMM), x.shape[0])
                if cfg is not None and cfg[0] == "mma" and x.shape[0] <= 64:  # the streaming kernel, M <= 64
                    return ext.w4_mma(x, self.packed, self.scales, self.zeros, *cfg[1:], int(self.silu_mul))
                if cfg is not None and cfg[0] != "mma":
                    return self._gemm(ext, x, cfg)
        return self._dense(x)

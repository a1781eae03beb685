"""CPU oracle for tandem's AWQ W4A16 linear path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module: as the checker the HIP path is compared against, and as the CPU baseline timed beside
it. The product (``tandem_amd``) never imports it and has no CPU fallback.

A numpy restatement of the reference's algorithm for the path (reference = 12vivi/tandem; paths are
relative to its repository root):

    unpack_awq / pack_awq      AutoAWQ "gemm" nibble packing       python/tandem/layers/awq.py:38-46,
                                                                    tests/test_awq.py:17-29
    dequant                    fp16_rne((q - z) * s), [N, K]       python/tandem/layers/awq.py:89-133
    dequant_exact              (q - z) * s without rounding        tests/test_awq.py:32-38
    dequant_exact_rows         the same for selected output        python/tandem/layers/awq.py:38-46
                               features (sampled full-size checks)
    interleave_gate_up         16-row gate/up tiles                python/tandem/layers/awq.py:71-75
    deinterleave_gate_up       its inverse (w4_dequant's           python/tandem/layers/awq.py:114-118
                               DEINTERLEAVE destination rows)
    linear                     x @ w^T in float64 (the dequantize-  python/tandem/layers/awq.py:282-285
                               then-matmul path, at high precision)
    silu / silu_and_mul        silu(gate) * up on [gate | up]      python/tandem/layers/awq.py:78-86
    swiglu_reference           float32 SwiGLU on fp16-rounded      tests/test_awq.py:80-84
                               weights
    random_awq                 the reference tests' input recipe   tests/test_awq.py:32-38
                               (numpy's generator, not CUDA's)
    rms_norm                   fp16(x rstd w), fp32 semantics      python/tandem/layers/ops.py:107-109
    add_rms_norm               s = x + r (fp32); r' = fp16(s);     python/tandem/layers/triton_ops.py:101-124,
                               y = fp16(s rstd w)                  python/tandem/layers/ops.py:111-120

What pins each function (tests/test_oracle.py): known-answer words and the test packer's inverse
for the nibble order; brute force over every (q, z) pair against exact rational arithmetic for the
dequantization, and the committed fixture plus single-entry rationals for the row-sampled form;
closed forms for the interleave and SwiGLU; explicit loops for the matmul; the recipe's ranges,
shapes and packing for random_awq; closed forms (constant rows, eps-dominated rows) and explicit
loops for the norms; and planted mistakes (swapped orders, double rounding, transposed operands, a
dropped eps or residual) that those checks must reject. Every function of this module has such a
pin: none is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

GROUP = 128

# AutoAWQ packs output columns j = 0..7 of an int32 in nibble order [0, 2, 4, 6, 1, 3, 5, 7]: nibble i
# holds column AWQ_PACK_ORDER[i], so column j sits in nibble AWQ_REVERSE_ORDER[j]
# (python/tandem/layers/awq.py:38-39; tests/test_awq.py:17).
AWQ_PACK_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


def unpack_awq(packed: np.ndarray) -> np.ndarray:
    """[R, C] int32 in AWQ order -> [R, 8 C] int32 values 0..15, column 8 c + j from nibble
    AWQ_REVERSE_ORDER[j] of word c (python/tandem/layers/awq.py:42-46)."""
    p = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    shifts = np.array([4 * i for i in AWQ_REVERSE_ORDER], dtype=np.int64)
    return ((p[:, :, None] >> shifts) & 0xF).reshape(p.shape[0], -1).astype(np.int32)


def pack_awq(values: np.ndarray) -> np.ndarray:
    """[R, 8 C] values 0..15 -> [R, C] int32 in AutoAWQ order: nibble i of word c holds column
    8 c + AWQ_PACK_ORDER[i] (the reference tests' packer, tests/test_awq.py:19-29)."""
    v = np.asarray(values).astype(np.int64)
    r, c8 = v.shape
    v = v.reshape(r, c8 // 8, 8)
    out = np.zeros((r, c8 // 8), dtype=np.int64)
    for i, col in enumerate(AWQ_PACK_ORDER):
        out |= v[:, :, col] << (4 * i)
    return out.astype(np.uint32).view(np.int32)  # top nibble >= 8 wraps: the same bit pattern


def random_awq(k: int, n: int, group: int = GROUP, seed: int = 0):
    """The reference tests' input recipe (tests/test_awq.py:32-38) on numpy's generator:
    q, z uniform in 0..15, s = U[0, 1) * 0.02 + 0.001 in fp16. Returns
    (qweight [K, N/8] int32, qzeros [K/G, N/8] int32, scales [K/G, N] fp16, q [K, N], z [K/G, N])."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(k, n), dtype=np.int32)
    z = rng.integers(0, 16, size=(k // group, n), dtype=np.int32)
    s = (rng.random((k // group, n), dtype=np.float32) * np.float32(0.02) + np.float32(0.001)).astype(np.float16)
    return pack_awq(q), pack_awq(z), s, q, z


def dequant_exact(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group: int = GROUP) -> np.ndarray:
    """w_ref [N, K] float32 = (q - z) * s, exact: a 4-bit integer times an fp16 fits float32's
    24-bit significand (tests/test_awq.py:37)."""
    q = unpack_awq(qweight).astype(np.float32)                  # [K, N]
    z = unpack_awq(qzeros).astype(np.float32)                   # [K/G, N]
    s = np.asarray(scales).astype(np.float32)                   # [K/G, N]
    k = q.shape[0]
    if k % group or z.shape[0] * group != k or s.shape != z.shape:
        raise ValueError(f"dequant: qweight {q.shape} qzeros {z.shape} scales {s.shape} group {group}")
    w = (q - np.repeat(z, group, axis=0)) * np.repeat(s, group, axis=0)
    return np.ascontiguousarray(w.T)


def dequant_exact_rows(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, rows,
                       group: int = GROUP) -> np.ndarray:
    """dequant_exact(...)[rows] without unpacking the whole matrix: output feature n is nibble
    AWQ_REVERSE_ORDER[n % 8] of word column n // 8 (python/tandem/layers/awq.py:38-46), for the
    sampled-column checks at full size (a [24576, 4096] weight unpacked whole is 400 MB)."""
    rows = np.asarray(rows, dtype=np.int64)
    shifts = 4 * np.asarray(AWQ_REVERSE_ORDER, dtype=np.int64)[rows % 8]
    qw = np.asarray(qweight).astype(np.int64)[:, rows // 8] & 0xFFFFFFFF     # [K, R]
    qz = np.asarray(qzeros).astype(np.int64)[:, rows // 8] & 0xFFFFFFFF      # [K/G, R]
    q = ((qw >> shifts) & 0xF).astype(np.float32)
    z = ((qz >> shifts) & 0xF).astype(np.float32)
    s = np.asarray(scales)[:, rows].astype(np.float32)
    if q.shape[0] % group or z.shape[0] * group != q.shape[0] or s.shape != z.shape:
        raise ValueError(f"dequant: qweight {q.shape} qzeros {z.shape} scales {s.shape} group {group}")
    w = (q - np.repeat(z, group, axis=0)) * np.repeat(s, group, axis=0)
    return np.ascontiguousarray(w.T)


def dequant(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group: int = GROUP) -> np.ndarray:
    """Dense fp16 [N, K] (nn.Linear layout) = fp16_rne((q - z) * s): float32 math, then one cast to
    fp16 with round-to-nearest-even (python/tandem/layers/awq.py:110-119, `w.to(out dtype)`)."""
    return dequant_exact(qweight, qzeros, scales, group).astype(np.float16)


def interleave_gate_up(t: np.ndarray) -> np.ndarray:
    """Rows [gate (I); up (I)] -> 16-row tiles [gate 8i .. 8i+7, up 8i .. 8i+7]
    (python/tandem/layers/awq.py:71-75)."""
    n = t.shape[0]
    return t.reshape(2, n // 16, 8, *t.shape[1:]).swapaxes(0, 1).reshape(t.shape)


def deinterleave_gate_up(t: np.ndarray) -> np.ndarray:
    """Inverse of interleave_gate_up: row n' = 16 T + r goes back to T * 8 + r (r < 8) or
    N/2 + T * 8 + r - 8 (python/tandem/layers/awq.py:114-118)."""
    n = t.shape[0]
    out = np.empty_like(t)
    rows = np.arange(n)
    r = rows % 16
    dest = np.where(r < 8, (rows // 16) * 8 + r, n // 2 + (rows // 16) * 8 + r - 8)
    out[dest] = t
    return out


def linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """y [M, N] = x [M, K] @ w [N, K]^T in float64: the dequantize-then-matmul path
    (python/tandem/layers/awq.py:282-285, F.linear) without its fp16 output rounding."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T


def silu(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def silu_and_mul(y: np.ndarray) -> np.ndarray:
    """[M, 2I] = [gate | up] -> silu(gate) * up (python/tandem/layers/awq.py:84-85)."""
    y = np.asarray(y, dtype=np.float64)
    gate, up = np.split(y, 2, axis=-1)
    return silu(gate) * up


def swiglu_reference(x: np.ndarray, w_exact: np.ndarray) -> np.ndarray:
    """SwiGLU reference on the fp16-rounded weights the kernels use (tests/test_awq.py:80-84):
    x [M, K], w_exact [2I, K] in [gate | up] row order -> [M, I]."""
    return silu_and_mul(linear(x, np.asarray(w_exact, dtype=np.float32).astype(np.float16)))


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """y = fp16(x * rsqrt(mean(x^2) + eps) * w) over the last axis, the reference GPU path's
    rmsnorm (python/tandem/layers/ops.py:107-109: fp32 math, one rounding); the mean and the
    products in float64 here."""
    x64 = np.asarray(x, dtype=np.float16).astype(np.float64)
    rstd = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    return (x64 * rstd * np.asarray(w, dtype=np.float16).astype(np.float64)).astype(np.float16)


def add_rms_norm(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float) -> tuple[np.ndarray, np.ndarray]:
    """(y, r') of the residual add + RMSNorm (python/tandem/layers/triton_ops.py:101-124):
    s = x + r in float32, r' = fp16(s), y = fp16(s * rsqrt(mean(s^2) + eps) * w) from the
    unrounded s."""
    s = np.asarray(x, dtype=np.float16).astype(np.float32) + np.asarray(r, dtype=np.float16).astype(np.float32)
    s64 = s.astype(np.float64)
    rstd = 1.0 / np.sqrt(np.mean(s64 * s64, axis=-1, keepdims=True) + eps)
    y = (s64 * rstd * np.asarray(w, dtype=np.float16).astype(np.float64)).astype(np.float16)
    return y, s.astype(np.float16)

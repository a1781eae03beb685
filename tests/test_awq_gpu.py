"""GPU parity of the MI355X W4A16 path against the CPU oracle (oracle/awq_oracle.py).

Mirrors tests/test_awq.py of 12vivi/tandem: repack and dequantization (bit-exact here), the row
interleave, every compiled configuration of the three kernels against the dequantize-then-matmul
reference, SwiGLU epilogues, split-K counters and graph replay, and the W4Linear layer. Inputs
follow the reference tests' recipe (q, z uniform in 0..15, s = U[0, 1) * 0.02 + 0.001, x ~ N(0, 1))
on numpy's seeded generator. Tolerances are the reference's (atol / rtol): 0.05 / 0.02 for the
vector-ALU GEMV and the layer, 0.02 / 0.01 for the matrix-core kernels, 0.03 / 0.02 (layer) and
0.02 / 0.01 (kernels) for SwiGLU; every comparison also reports max |err| / max |ref| and the
cosine similarity, and requires cosine >= 0.9999.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import awq_oracle as o
from parity import check_close
from tandem_amd.layers import awq, w4_hip

pytestmark = pytest.mark.gpu

DEV = "cuda"
SHAPES = ((128, 24), (256, 520), (1024, 64), (4096, 1000))  # (K, N); N % 16 != 0 exercises the padded tile
DECODE_CONFIGS = w4_hip.decode_configs()  # every compiled (warps_k, unroll, ntile)
MMA_CONFIGS = w4_hip.mma_configs()        # those and the row-tile-wide ones only w4_mma takes
GEMM_CONFIGS = w4_hip.gemm_configs()      # every compiled (MT, NT, WARPS_N, WARPS_K, STAGES)


@pytest.fixture(scope="module")
def ext():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    e = w4_hip.load()
    assert e is not None, "TANDEM_NO_CUDA_EXT=1 is set"
    return e


def gpu(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


class Case:
    """One random AWQ weight on CPU (oracle) and GPU (tile layout)."""

    def __init__(self, k: int, n: int, seed: int, interleave: bool = False):
        self.k, self.n = k, n
        self.qweight, self.qzeros, self.scales, self.q, self.z = o.random_awq(k, n, seed=seed)
        self.w_exact = o.dequant_exact(self.qweight, self.qzeros, self.scales)  # [N, K] float32
        self.w16 = self.w_exact.astype(np.float16)
        self.packed, self.s, self.zz = w4_hip.repack(gpu(self.qweight), gpu(self.qzeros), gpu(self.scales),
                                                     interleave=interleave)

    def x(self, m: int, seed: int) -> np.ndarray:
        return np.random.default_rng(seed).standard_normal((m, self.k)).astype(np.float16)


# ------------------------------------------------------------------ repack and dequantization
@pytest.mark.parametrize("k,n", [(256, 64), (1024, 384), (4096, 1024), (128, 24), (256, 520), (4096, 1000)])
def test_repack_and_dequant_bit_exact(k, n):
    """HIP repack + HIP dequant == oracle fp16_rne((q - z) s), every bit (tests/test_awq.py:41-47
    checks atol 1e-3; here the bar is equality)."""
    c = Case(k, n, seed=k + n)
    assert c.packed.shape == (w4_hip.padded_rows(n), k // 8) and c.s.shape == (n, k // 128)
    assert torch.equal(c.s.cpu(), awq.tile_major_params(torch.from_numpy(c.scales.T.copy())))
    assert torch.equal(c.zz.cpu(), awq.tile_major_params(torch.from_numpy(c.z.T.astype(np.float16).copy())))
    assert torch.equal(c.packed.cpu(), awq.pack_rows(torch.from_numpy(c.q.T.copy())))
    w = awq.w4_dequant(c.packed, c.s, c.zz)
    assert w.shape == (n, k)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), o.dequant(c.qweight, c.qzeros, c.scales).view(np.uint16))


def test_dequant_full_size_gate_up_bit_exact():
    """Qwen3-8B gate_up (K 4096, N 24576): the whole 201 MB fp16 weight, bit for bit."""
    c = Case(4096, 24576, seed=77)
    w = awq.w4_dequant(c.packed, c.s, c.zz).cpu().numpy()
    assert np.array_equal(w.view(np.uint16), c.w16.view(np.uint16))


def test_dequant_deinterleave():
    """Interleaved repack + de-interleaving dequant == plain dequant (tests/test_awq.py:50-55), and the
    interleaved tile layout holds interleave_gate_up's row order."""
    c = Case(256, 96, seed=7)
    pi, si, zi = w4_hip.repack(gpu(c.qweight), gpu(c.qzeros), gpu(c.scales), interleave=True)
    assert torch.equal(awq.w4_dequant(pi, si, zi, deinterleave=True), awq.w4_dequant(c.packed, c.s, c.zz))
    assert torch.equal(si, awq.tile_major_params(awq.interleave_gate_up(awq.row_major_params(c.s))))
    q_rows = torch.from_numpy(o.interleave_gate_up(c.q.T.copy()))
    assert torch.equal(pi.cpu(), awq.pack_rows(q_rows))


# ----------------------------------------------------------------------- per-kernel parity
def test_gemv_every_config(ext):
    """Vector-ALU kernel vs the dequantized matmul, M = 1..4, every compiled config
    (tests/test_awq.py:203-214)."""
    for k, n in SHAPES:
        c = Case(k, n, seed=3)
        for m in range(1, 5):
            x = c.x(m, seed=100 + m)
            ref = o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in DECODE_CONFIGS:
                check_close(ext.w4_gemv(xg, c.packed, c.s, c.zz, *cfg), ref, 0.05, 0.02, (k, n, m, cfg), "gemv")


def test_gemv_silu_mul(ext):
    """The GEMV with the SwiGLU epilogue (tw4_gemv_act, act = 1; the reference's GEMV has none) on
    interleaved rows, M = 1..4, every compiled config, at the GEMV's tolerance."""
    for k, n in ((128, 32), (1024, 512), (4096, 1024)):
        c = Case(k, n, seed=16, interleave=True)
        for m in range(1, 5):
            x = c.x(m, seed=800 + m)
            ref = o.swiglu_reference(x, c.w_exact)
            xg = gpu(x)
            for cfg in DECODE_CONFIGS:
                y = ext.w4_gemv(xg, c.packed, c.s, c.zz, *cfg, 1)
                assert y.shape == (m, n // 2)
                check_close(y, ref, 0.05, 0.02, (k, n, m, cfg), "gemv")


def test_gemv_mfma_every_config(ext):
    """The GEMV's arithmetic on the matrix cores (tw4_gemv_mfma), M = 1..4, every compiled config,
    plain and SwiGLU, at the GEMV's tolerance (exact q - z weights, like w4_gemv)."""
    for k, n in SHAPES:
        c = Case(k, n, seed=31)
        for m in range(1, 5):
            x = c.x(m, seed=1100 + m)
            ref = o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in DECODE_CONFIGS:
                check_close(ext.w4_gemv_mfma(xg, c.packed, c.s, c.zz, *cfg), ref, 0.05, 0.02, (k, n, m, cfg), "gemvm")
    for k, n in ((128, 32), (1024, 512), (4096, 1024)):
        c = Case(k, n, seed=32, interleave=True)
        for m in range(1, 5):
            x = c.x(m, seed=1200 + m)
            ref = o.swiglu_reference(x, c.w_exact)
            xg = gpu(x)
            for cfg in DECODE_CONFIGS:
                y = ext.w4_gemv_mfma(xg, c.packed, c.s, c.zz, *cfg, 1)
                assert y.shape == (m, n // 2)
                check_close(y, ref, 0.05, 0.02, (k, n, m, cfg), "gemvm")


def test_gemv_mfma_full_batch_tile(ext):
    """tw4_gemv_mfma at M = 5 .. 16 (the rest of its 16-column B tile), every compiled config, plain
    and SwiGLU, including a partial row tile and the largest M whose x' fits in LDS at K = 4096; an
    M whose x' does not fit is refused on the host."""
    ran = 0
    for k, n, act in ((1024, 1000, 0), (4096, 1024, 0), (4096, 512, 1)):
        c = Case(k, n, seed=33 + act, interleave=bool(act))
        for m in (5, 8, 13, 16):
            x = c.x(m, seed=1300 + m)
            ref = o.swiglu_reference(x, c.w_exact) if act else o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in DECODE_CONFIGS:
                try:
                    y = ext.w4_gemv_mfma(xg, c.packed, c.s, c.zz, *cfg, act)
                except RuntimeError as e:  # x' plus this config's reduction buffer past 160 KB of LDS
                    assert m * (2 * k + 16) + (cfg[0] - 1) * cfg[2] * 1024 > 128 * 1024 and \
                        "does not fit in LDS" in str(e), (k, n, m, cfg, str(e))
                    continue
                ran += 1
                assert y.shape == (m, n // 2 if act else n)
                check_close(y, ref, 0.05, 0.02, (k, n, m, cfg), "gemvm")
    assert ran >= 3 * 4 * len(DECODE_CONFIGS) * 3 // 4
    c = Case(12288, 64, seed=35)
    with pytest.raises(RuntimeError, match="does not fit in LDS"):
        ext.w4_gemv_mfma(gpu(c.x(8, seed=1)), c.packed, c.s, c.zz, 4, 2, 1, 0)


def _norm_inputs(m: int, k: int, seed: int):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * 2).astype(np.float16)
    r = (rng.standard_normal((m, k)) * 8).astype(np.float16)
    w = (rng.random(k) + 0.5).astype(np.float16)
    return x, r, w


@pytest.mark.parametrize("kind", ["gemv", "mma"])
def test_decode_norm_matches_separate_norm(ext, kind):
    """The fused norm prologue (tw4_decode_norm) equals tw4_add_rms_norm / tw4_rms_norm followed by
    the same kernel and config, bit for bit, and so does its residual output; every config, with
    and without the SwiGLU epilogue, with and without a residual."""
    from tandem_amd.layers import norm

    k01 = 0 if kind == "gemv" else 1
    run = (lambda xx, c, cfg, act: ext.w4_gemv(xx, c.packed, c.s, c.zz, *cfg, act)) if kind == "gemv" else \
        (lambda xx, c, cfg, act: ext.w4_mma(xx, c.packed, c.s, c.zz, *cfg, act))
    for k, n, act in ((512, 64, 0), (1024, 512, 1), (2048, 520, 0), (4096, 1024, 1)):
        c = Case(k, n, seed=21, interleave=bool(act))
        for m in ((1, 2, 3, 4) if kind == "gemv" else (1, 3, 8, 9, 16)):
            if kind == "mma" and m * (k // 8 + 1) * 16 > 80 * 1024:
                with pytest.raises(RuntimeError, match="fused norm"):
                    ext.w4_decode_norm(gpu(np.zeros((m, k), np.float16)), None, gpu(np.ones(k, np.float16)), 1e-6,
                                       c.packed, c.s, c.zz, 1, *DECODE_CONFIGS[0], act)
                continue
            x, r, w = _norm_inputs(m, k, seed=900 + m)
            xg, rg, wg = gpu(x), gpu(r), gpu(w)
            xs, rs = xg.clone(), rg.clone()
            norm.fused_add_rms_norm(xs, rs, wg, 1e-6)
            xp = norm.rms_norm(xg, wg, 1e-6)
            for cfg in DECODE_CONFIGS:
                y, r_out = ext.w4_decode_norm(xg, rg, wg, 1e-6, c.packed, c.s, c.zz, k01, *cfg, act)
                assert torch.equal(r_out, rs), (k, n, m, cfg)
                assert torch.equal(y, run(xs, c, cfg, act)), (k, n, m, cfg, act)
                y2, none = ext.w4_decode_norm(xg, None, wg, 1e-6, c.packed, c.s, c.zz, k01, *cfg, act)
                assert none is None and torch.equal(y2, run(xp, c, cfg, act)), (k, n, m, cfg, act)
            assert torch.equal(xg, gpu(x)) and torch.equal(rg, gpu(r))  # inputs untouched


def test_decode_norm_small_k_against_oracle(ext):
    """K = 128 and 384 (one or three quant groups: some wavefronts have no slice and only join the
    workgroup barrier) against the oracle's norm and product, GEMV / matrix-core tolerances."""
    for k, n in ((128, 32), (384, 48)):
        c = Case(k, n, seed=22)
        for m in (1, 4):
            x, r, w = _norm_inputs(m, k, seed=950 + m)
            a, r2 = o.add_rms_norm(x, r, w, 1e-6)
            ref = o.linear(a, c.w_exact)
            for cfg in DECODE_CONFIGS:
                for k01, atol, rtol in ((0, 0.05, 0.02), (1, 0.02, 0.01)):
                    y, r_out = ext.w4_decode_norm(gpu(x), gpu(r), gpu(w), 1e-6, c.packed, c.s, c.zz, k01, *cfg, 0)
                    assert (r_out.cpu().numpy().view(np.uint16) == r2.view(np.uint16)).all()
                    check_close(y, ref, atol, rtol, (k, n, m, cfg, k01), "norm")


def test_gemv_one_group_ring_every_remainder(ext):
    """The one-group GEMV configurations keep two groups in flight in three register sets; a
    wavefront's last pass then covers 0-4 chunks after 0, 1 or more full passes of three. K = 128 G
    with G = 3 .. 40 gives the wavefronts of warps_k 4, 8 and 16 every remainder, with and without a
    full pass first (the SHAPES above reach only some), plain, SwiGLU and with the fused norm."""
    ring = [cfg for cfg in DECODE_CONFIGS if cfg[1] == 1]
    assert ring, "no one-group configuration compiled"
    for g in (3, 5, 6, 7, 9, 10, 12, 13, 20, 24, 28, 36, 40):
        k = 128 * g
        c = Case(k, 48, seed=30 + g)
        ci = Case(k, 32, seed=60 + g, interleave=True)
        for m in (1, 3):
            x = c.x(m, seed=1200 + 10 * g + m)
            ref = o.linear(x, c.w_exact)
            ref_act = o.swiglu_reference(x, ci.w_exact)
            xn, r, w = _norm_inputs(m, k, seed=1300 + 10 * g + m)
            a, r2 = o.add_rms_norm(xn, r, w, 1e-6)
            ref_norm = o.linear(a, c.w_exact)
            for cfg in ring:
                check_close(ext.w4_gemv(gpu(x), c.packed, c.s, c.zz, *cfg), ref, 0.05, 0.02, (k, m, cfg), "gemv")
                check_close(ext.w4_gemv(gpu(x), ci.packed, ci.s, ci.zz, *cfg, 1), ref_act, 0.05, 0.02, (k, m, cfg),
                            "gemv")
                y, r_out = ext.w4_decode_norm(gpu(xn), gpu(r), gpu(w), 1e-6, c.packed, c.s, c.zz, 0, *cfg, 0)
                assert (r_out.cpu().numpy().view(np.uint16) == r2.view(np.uint16)).all()
                check_close(y, ref_norm, 0.05, 0.02, (k, m, cfg), "norm")


def test_mma_every_config(ext):
    """Matrix-core decode kernel, M = 1..16, every compiled config (tests/test_awq.py:217-229),
    the row-tile-wide ones included (a partial last group of six row tiles at N = 520 and 1000)."""
    for k, n in SHAPES:
        c = Case(k, n, seed=4)
        for m in range(1, 17):
            x = c.x(m, seed=200 + m)
            ref = o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in MMA_CONFIGS:
                check_close(ext.w4_mma(xg, c.packed, c.s, c.zz, *cfg, 0), ref, 0.02, 0.01, (k, n, m, cfg), "mma")


def _wide_ok(cfg, m) -> bool:
    mt = 1 if m <= 16 else 2 if m <= 32 else 4
    return mt == 1 or cfg[1] * mt <= 4


def test_mma_wide_batches(ext):
    """The streaming matrix-core kernel with 2 or 4 batch tiles (M 17 .. 64), every compiled config
    it accepts; the rest are refused with an error, never launched."""
    for k, n in SHAPES:
        c = Case(k, n, seed=14)
        for m in (17, 32, 33, 50, 64):
            x = c.x(m, seed=600 + m)
            ref = o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in MMA_CONFIGS:
                if not _wide_ok(cfg, m):
                    with pytest.raises(RuntimeError):
                        ext.w4_mma(xg, c.packed, c.s, c.zz, *cfg, 0)
                    continue
                check_close(ext.w4_mma(xg, c.packed, c.s, c.zz, *cfg, 0), ref, 0.02, 0.01, (k, n, m, cfg), "mma")


def test_mma_wide_silu_mul(ext):
    for k, n in ((128, 32), (4096, 1024)):
        c = Case(k, n, seed=15, interleave=True)
        for m in (24, 40, 64):
            x = c.x(m, seed=700 + m)
            ref = o.swiglu_reference(x, c.w_exact)
            xg = gpu(x)
            for cfg in MMA_CONFIGS:
                if _wide_ok(cfg, m):
                    y = ext.w4_mma(xg, c.packed, c.s, c.zz, *cfg, 1)
                    assert y.shape == (m, n // 2)
                    check_close(y, ref, 0.02, 0.01, (k, n, m, cfg), "mma")


def test_mma_silu_mul(ext):
    """SwiGLU epilogue (act = 1) on interleaved rows: y = silu(gate) * up (tests/test_awq.py:302-314)."""
    for k, n in ((128, 32), (1024, 512), (4096, 1024)):
        c = Case(k, n, seed=6, interleave=True)
        for m in range(1, 17):
            x = c.x(m, seed=300 + m)
            ref = o.swiglu_reference(x, c.w_exact)
            xg = gpu(x)
            for cfg in MMA_CONFIGS:
                y = ext.w4_mma(xg, c.packed, c.s, c.zz, *cfg, 1)
                assert y.shape == (m, n // 2)
                check_close(y, ref, 0.02, 0.01, (k, n, m, cfg), "mma")


def test_mma_row_tile_wide_configs_refuse_the_other_forms(ext):
    """The row-tile-wide configs read x from global memory: the split-K, persistent and fused-norm
    entries refuse them with an error (nothing is launched); tw4_mma with splits = 1 takes them."""
    buf, locks = w4_hip.workspace(DEV)
    c = Case(1024, 512, seed=31)
    x = c.x(4, seed=31)
    xg = gpu(x)
    nw = torch.ones(1024, dtype=torch.float16, device=DEV)
    for cfg in w4_hip.mma_wide_configs():
        assert cfg not in DECODE_CONFIGS
        with pytest.raises(RuntimeError, match="reads x from global memory"):
            ext.w4_mma_splitk(xg, c.packed, c.s, c.zz, buf, locks, *cfg, 2, 0)
        with pytest.raises(RuntimeError, match="reads x from global memory"):
            ext.w4_mma_persist(xg, c.packed, c.s, c.zz, *cfg, 1, 0)
        with pytest.raises(RuntimeError, match="reads x from global memory"):
            ext.w4_decode_norm(xg, None, nw, 1e-6, c.packed, c.s, c.zz, 1, *cfg, 0)
        with pytest.raises(RuntimeError):  # not a GEMV configuration
            ext.w4_gemv(xg, c.packed, c.s, c.zz, *cfg, 0)
        one = ext.w4_mma(xg, c.packed, c.s, c.zz, *cfg, 0)
        assert torch.equal(one, ext.w4_mma_splitk(xg, c.packed, c.s, c.zz, buf, locks, *cfg, 1, 0))
        check_close(one, o.linear(x, c.w_exact), 0.02, 0.01, (1024, 512, 4, cfg), "mma")
    torch.cuda.synchronize()
    assert int(locks.abs().sum()) == 0


def test_mma_split_k_every_config(ext):
    """The matrix-core decode kernel with K split over workgroups (tw4_mma_splitk): M = 1 .. 16,
    every compiled config, 2 .. 8 splits (uneven group ranges included), plain and SwiGLU; the
    counters are back at zero after each call."""
    buf, locks = w4_hip.workspace(DEV)
    ran = 0
    for k, n, interleave in ((256, 520, False), (1024, 64, False), (4096, 1000, False), (12288, 256, False),
                             (1024, 512, True)):
        c = Case(k, n, seed=21, interleave=interleave)
        g = k // 128
        for m in (1, 3, 8, 13, 16):
            x = c.x(m, seed=800 + m)
            ref = o.swiglu_reference(x, c.w_exact) if interleave else o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in DECODE_CONFIGS:
                for splits in (2, 3, 8):
                    if splits > g:
                        continue
                    y = ext.w4_mma_splitk(xg, c.packed, c.s, c.zz, buf, locks, *cfg, splits, int(interleave))
                    ran += 1
                    check_close(y, ref, 0.02, 0.01, (k, n, m, cfg, splits, interleave), "mmak")
    torch.cuda.synchronize()
    assert int(locks.abs().sum()) == 0
    assert ran > 3 * len(DECODE_CONFIGS)


def test_mma_persistent_matches_mma(ext):
    """The persistent form of the matrix-core decode kernel (tw4_mma_persist): workgroups that
    stream 1 to 5 row-tile groups each (N past 256 CUs x 16 rows x ntile, partial last tile, K
    not a multiple of warps_k quant groups),
    every compiled config, 1 to 4 workgroups per CU, plain and SwiGLU: bit for bit the one-pass
    kernel's output (same chunk order and reduction), and within tolerance of the oracle."""
    ran = 0
    for k, n, interleave in ((1024, 16392, False), (4096, 8200, False), (2560, 8208, False), (1024, 16384, True)):
        c = Case(k, n, seed=25, interleave=interleave)  # K = 2560: 20 groups, uneven wavefront ranges
        for m in (1, 8, 16):
            x = c.x(m, seed=900 + m)
            xg = gpu(x)
            ref = o.swiglu_reference(x, c.w_exact) if interleave else o.linear(x, c.w_exact)
            for cfg in DECODE_CONFIGS:
                one = ext.w4_mma(xg, c.packed, c.s, c.zz, *cfg, int(interleave))
                for per_cu in (1, 2, 4):
                    if per_cu > 1 and m * (2 * k + 16) > 80 * 1024:  # x fits in LDS only at one per CU
                        with pytest.raises(RuntimeError, match="persistent form stages x in LDS"):
                            ext.w4_mma_persist(xg, c.packed, c.s, c.zz, *cfg, per_cu, int(interleave))
                        continue
                    y = ext.w4_mma_persist(xg, c.packed, c.s, c.zz, *cfg, per_cu, int(interleave))
                    ran += 1
                    assert torch.equal(y, one), (k, n, m, cfg, per_cu, interleave)
            check_close(one, ref, 0.02, 0.01, (k, n, m, interleave), "mmap")
    assert ran == (4 * 3 * 3 - 4) * len(DECODE_CONFIGS)


def test_mma_split_k_deterministic_and_graph_replay(ext):
    """Split-K decode: identical bits on every call (the partials are added in split order), and
    correct on every replay of a captured graph with eager work in between."""
    buf, locks = w4_hip.workspace(DEV)
    c = Case(12288, 512, seed=22)
    x = gpu(c.x(8, seed=23))
    cfg = (4, 2, 1, 4)
    first = ext.w4_mma_splitk(x, c.packed, c.s, c.zz, buf, locks, *cfg, 0)
    for _ in range(4):
        assert torch.equal(ext.w4_mma_splitk(x, c.packed, c.s, c.zz, buf, locks, *cfg, 0), first)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = ext.w4_mma_splitk(x, c.packed, c.s, c.zz, buf, locks, *cfg, 0)
    rng = np.random.default_rng(24)
    for _ in range(3):
        xn = rng.standard_normal((8, 12288)).astype(np.float16)
        x.copy_(gpu(xn))
        graph.replay()
        torch.cuda.synchronize()
        check_close(y, o.linear(xn, c.w_exact), 0.02, 0.01, "split-K replay", "mmak")
        check_close(ext.w4_mma_splitk(x, c.packed, c.s, c.zz, buf, locks, *cfg, 0), o.linear(xn, c.w_exact),
                    0.02, 0.01, "split-K eager", "mmak")
    assert int(locks.abs().sum()) == 0


def test_gemm_every_config(ext):
    """GEMM: every compiled config, partial token and row tiles, split-K of every tile or of the last
    wave only (stages 0, the resident-x variant: the fewest splits that fit, chosen on the host;
    stages 3, both tiles through LDS by direct-to-LDS loads: enough splits to fill the GPU); the
    counters are back at zero after each call (tests/test_awq.py:232-259). A stages-0 config whose x
    slice cannot fit in LDS for the requested splits, and a stages-3 config on N % 16 != 0, are refused
    on the host, before any launch."""
    buf, locks = w4_hip.workspace(DEV)
    ran = 0
    for k, n in SHAPES:
        c = Case(k, n, seed=7)
        for m in (5, 17, 40, 64, 130):
            x = c.x(m, seed=400 + m)
            ref = o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in GEMM_CONFIGS:
                for splits in (0, 1, 3):
                    if splits > (k // 128 + cfg[3] - 1) // cfg[3]:
                        continue
                    try:
                        y = ext.w4_gemm(xg, c.packed, c.s, c.zz, buf, locks, *cfg, splits, 0)
                    except RuntimeError as e:  # refused on the host, never launched
                        assert (cfg[4] == 0 and "does not fit in LDS" in str(e)) or \
                            (cfg[4] == 3 and n % 16 and "N % 16 == 0" in str(e)) or \
                            (cfg[4] == 1 and m > 16 * cfg[0] and "> 16 mt" in str(e)), (cfg, splits, str(e))
                        continue
                    ran += 1
                    check_close(y, ref, 0.02, 0.01, (k, n, m, cfg, splits), "gemm")
    torch.cuda.synchronize()
    assert int(locks.abs().sum()) == 0
    assert ran > len(GEMM_CONFIGS) * len(SHAPES)


def test_gemm_silu_mul(ext):
    """The GEMM's SwiGLU epilogue (act = 1): [M, N / 2] (tests/test_awq.py:262-276)."""
    buf, locks = w4_hip.workspace(DEV)
    for k, n in ((128, 32), (1024, 512), (4096, 1024)):
        c = Case(k, n, seed=8, interleave=True)
        for m in (17, 64, 100):
            x = c.x(m, seed=500 + m)
            ref = o.swiglu_reference(x, c.w_exact)
            xg = gpu(x)
            for cfg in GEMM_CONFIGS:
                for splits in (0, 1, 2):
                    if splits > (k // 128 + cfg[3] - 1) // cfg[3]:
                        continue
                    try:
                        y = ext.w4_gemm(xg, c.packed, c.s, c.zz, buf, locks, *cfg, splits, 1)
                    except RuntimeError as e:
                        assert (cfg[4] == 0 and "does not fit in LDS" in str(e)) or \
                            (cfg[4] == 1 and m > 16 * cfg[0] and "> 16 mt" in str(e)), (cfg, splits, str(e))
                        continue
                    assert y.shape == (m, n // 2)
                    check_close(y, ref, 0.02, 0.01, (k, n, m, cfg, splits), "gemm")
    torch.cuda.synchronize()
    assert int(locks.abs().sum()) == 0


def test_gemm_lds_partial_bands_and_blocks(ext):
    """The stages-3 GEMM where several N blocks end in a partial one (N = 784: three 256-row blocks
    and a 16-row one) and the token bands of 8 blocks end in a partial band (M = 1100 at BM = 128:
    nine blocks), plain and SwiGLU, unsplit, auto-split and split 3 ways: the band / block remap and
    the last-tile clamp against the oracle."""
    buf, locks = w4_hip.workspace(DEV)
    lds_cfgs = [cfg for cfg in GEMM_CONFIGS if cfg[4] == 3]
    assert lds_cfgs
    for act in (0, 1):
        c = Case(1024, 784, seed=41 + act, interleave=bool(act))
        for m in (1100, 300):
            x = c.x(m, seed=4100 + m)
            ref = o.swiglu_reference(x, c.w_exact) if act else o.linear(x, c.w_exact)
            xg = gpu(x)
            for cfg in lds_cfgs:
                for splits in (1, 0, 3):
                    y = ext.w4_gemm(xg, c.packed, c.s, c.zz, buf, locks, *cfg, splits, act)
                    assert y.shape == (m, 392 if act else 784)
                    check_close(y, ref, 0.02, 0.01, (1024, 784, m, cfg, splits), "gemm s3")
    torch.cuda.synchronize()
    assert int(locks.abs().sum()) == 0


def test_gemm_split_k_deterministic(ext):
    """The last arriver adds the splits in split order: identical bits on every call."""
    buf, locks = w4_hip.workspace(DEV)
    c = Case(4096, 1024, seed=9)
    xg = gpu(c.x(33, seed=9))
    for cfg in ((2, 1, 4, 1, 2, 8), (2, 2, 4, 1, 0, 8), (4, 2, 1, 4, 1, 8)):  # LDS ring; resident x; x from L2
        first = ext.w4_gemm(xg, c.packed, c.s, c.zz, buf, locks, *cfg, 0)
        for _ in range(5):
            assert torch.equal(ext.w4_gemm(xg, c.packed, c.s, c.zz, buf, locks, *cfg, 0), first)


@pytest.mark.parametrize("cfg", [(2, 2, 4, 2, 2, 4, 0), (4, 2, 1, 4, 1, 4, 0)])  # LDS ring; x from L2
def test_gemm_split_k_graph_replay(ext, cfg):
    """Split-K inside a HIP graph: the counters are reset by the kernel, so replays stay correct
    (tests/test_awq.py:279-299)."""
    buf, locks = w4_hip.workspace(DEV)
    c = Case(1024, 512, seed=9)
    x = gpu(c.x(33, seed=10))
    ext.w4_gemm(x, c.packed, c.s, c.zz, buf, locks, *cfg)  # first launch outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = ext.w4_gemm(x, c.packed, c.s, c.zz, buf, locks, *cfg)
    rng = np.random.default_rng(11)
    for _ in range(3):
        xn = rng.standard_normal((33, 1024)).astype(np.float16)
        x.copy_(gpu(xn))
        graph.replay()
        torch.cuda.synchronize()
        check_close(y, o.linear(xn, c.w_exact), 0.02, 0.01, "replay", "gemm")
    assert int(locks.abs().sum()) == 0


def test_decode_graph_replay(ext):
    """The decode kernels under graph capture and replay, eager work in between."""
    c = Case(4096, 1024, seed=12)
    x = gpu(c.x(4, seed=12))
    ext.w4_mma(x, c.packed, c.s, c.zz, 4, 2, 1, 0)
    ext.w4_gemv(x, c.packed, c.s, c.zz, 4, 2, 1)
    ext.w4_gemv_mfma(x, c.packed, c.s, c.zz, 8, 2, 1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y1 = ext.w4_mma(x, c.packed, c.s, c.zz, 4, 2, 1, 0)
        y2 = ext.w4_gemv(x, c.packed, c.s, c.zz, 4, 2, 1)
        y3 = ext.w4_gemv_mfma(x, c.packed, c.s, c.zz, 8, 2, 1)
    rng = np.random.default_rng(13)
    for _ in range(3):
        xn = rng.standard_normal((4, 4096)).astype(np.float16)
        x.copy_(gpu(xn))
        graph.replay()
        torch.cuda.synchronize()
        ref = o.linear(xn, c.w_exact)
        check_close(y1, ref, 0.02, 0.01, "mma replay")
        check_close(y2, ref, 0.05, 0.02, "gemv replay")
        check_close(y3, ref, 0.05, 0.02, "gemv_mfma replay")
        eager = ext.w4_gemv(x, c.packed, c.s, c.zz, 4, 2, 1)
        torch.cuda.synchronize()
        assert torch.equal(y2, eager), "gemv: replay differs from the eager call"


# ----------------------------------------------------------------- full Qwen3-8B shapes
QWEN3_8B = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}
SEEDS = {"qkv": 31, "o": 32, "gate_up": 33, "down": 34}


@pytest.mark.parametrize("proj", list(QWEN3_8B))
def test_qwen3_8b_shapes(ext, proj):
    """Every kernel at the real shape vs the oracle's dequantize-then-matmul (float64)."""
    k, n = QWEN3_8B[proj]
    c = Case(k, n, seed=SEEDS[proj])
    buf, locks = w4_hip.workspace(DEV)
    for m in (1, 4):
        x = c.x(m, seed=m)
        check_close(ext.w4_gemv(gpu(x), c.packed, c.s, c.zz, 4, 2, 1), o.linear(x, c.w_exact), 0.05, 0.02, (proj, m),
                    "gemv")
    for m in (1, 8, 16):
        x = c.x(m, seed=m)
        check_close(ext.w4_mma(gpu(x), c.packed, c.s, c.zz, 4, 2, 1, 0), o.linear(x, c.w_exact), 0.02, 0.01,
                    (proj, m), "mma")
    for m, cfg in ((32, (2, 1, 4, 1, 2, 0)), (64, (4, 1, 4, 1, 2, 0)), (256, (8, 2, 4, 1, 2, 0))):
        x = c.x(m, seed=m)
        check_close(ext.w4_gemm(gpu(x), c.packed, c.s, c.zz, buf, locks, *cfg, 0), o.linear(x, c.w_exact), 0.02,
                    0.01, (proj, m, cfg), "gemm")


# --------------------------------------------------------------------------- W4Linear layer
def _layer(k, n, seed, silu_mul=False):
    c = Case(k, n, seed=seed)
    layer = awq.W4Linear(k, n, 128).to(DEV)
    layer.qweight.copy_(gpu(c.qweight))
    layer.qzeros.copy_(gpu(c.qzeros))
    layer.scales.copy_(gpu(c.scales))
    if silu_mul:
        assert layer.enable_silu_mul()
    layer.finalize(torch.cuda.get_device_name())
    return layer, c


def test_w4linear_small_and_large_batch():
    """tests/test_awq.py:87-103: decode kernels for M <= 16, the GEMM above, the unaligned-x
    fallback, and table entries (a GEMM config with split-K, or None = dequantize + matmul)."""
    k, n = 512, 256
    layer, c = _layer(k, n, seed=2)
    assert not layer.awq_layout and not hasattr(layer, "qweight") and layer.packed.shape == (n, k // 8)
    rng = np.random.default_rng(20)
    for m in (1, 3, 8, 12, 16, 37, 300):
        x = rng.standard_normal((m, k)).astype(np.float16)
        check_close(layer(gpu(x)), o.linear(x, c.w_exact), 0.05, 0.02, m, "layer")
    for m in (3, 40):  # not 16-byte aligned: dequantize + matmul
        xu = torch.empty(m * k + 1, device=DEV, dtype=torch.float16)[1:].view(m, k)
        xn = rng.standard_normal((m, k)).astype(np.float16)
        xu.copy_(gpu(xn))
        check_close(layer(xu), o.linear(xn, c.w_exact), 0.05, 0.02, ("unaligned", m), "layer")
    for cfg in ((2, 2, 4, 2, 2, 2), (4, 2, 4, 1, 2, 0), ("mma", 8, 1, 1), None):
        layer.gemm_kernels = {(n, k): ((1 << 30, cfg),)}
        x = rng.standard_normal((50, k)).astype(np.float16)
        check_close(layer(gpu(x)), o.linear(x, c.w_exact), 0.05, 0.02, cfg, "layer")
    assert layer(torch.empty(0, k, device=DEV, dtype=torch.float16)).shape == (0, n)


def test_w4linear_silu_mul():
    """tests/test_awq.py:106-118: gate_up with SwiGLU, rows interleaved at finalize; the epilogue in
    the decode kernels (M <= 16) and the GEMM (M > 16); dequantize + matmul for unaligned inputs."""
    k, n = 512, 384
    layer, c = _layer(k, n, seed=5, silu_mul=True)
    rng = np.random.default_rng(21)
    for m in (1, 3, 8, 12, 16, 37, 300):
        x = rng.standard_normal((m, k)).astype(np.float16)
        y = layer(gpu(x))
        assert y.shape == (m, n // 2)
        check_close(y, o.swiglu_reference(x, c.w_exact), 0.03, 0.02, m, "layer")
    xu = torch.empty(3 * k + 1, device=DEV, dtype=torch.float16)[1:].view(3, k)
    xn = rng.standard_normal((3, k)).astype(np.float16)
    xu.copy_(gpu(xn))
    check_close(layer(xu), o.swiglu_reference(xn, c.w_exact), 0.03, 0.02, "unaligned", "layer")


def test_w4linear_gemm_switch_off(monkeypatch):
    """TANDEM_W4_GEMM=0 sends M > 16 to dequantize + matmul (python/tandem/layers/awq.py:186)."""
    layer, c = _layer(256, 128, seed=22)
    monkeypatch.setattr(awq, "FUSED_GEMM", False)
    x = np.random.default_rng(22).standard_normal((40, 256)).astype(np.float16)
    check_close(layer(gpu(x)), o.linear(x, c.w_exact), 0.05, 0.02, "switch off", "dense")


@pytest.mark.parametrize("proj,silu", [("gate_up", True), ("gate_up", False), ("down", False), ("qkv", False),
                                       ("o", False)])
def test_w4linear_qwen3_8b_tables(proj, silu):
    """W4Linear at the real Qwen3-8B shapes through the gfx950 tables, across the M ranges where
    the tables switch kernels (gemv, gemvm, mma and its split-K and persistent forms, the GEMM with
    and without split-K, the x-from-L2 and resident-x kernels at M = 17 .. 24): every M of the
    benchmark's decode sweep, its M = 24 / 32 / 64 entries and a point inside each ladder rung."""
    k, n = QWEN3_8B[proj]
    layer, c = _layer(k, n, seed=SEEDS[proj] + 10, silu_mul=silu)
    assert layer.kernels is awq.W4_KERNELS[awq.GFX950] and layer.gemm_kernels is awq.W4_GEMM_KERNELS[awq.GFX950]
    rng = np.random.default_rng(23)
    for m in (1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 20, 24, 32, 48, 64, 96, 130):
        x = rng.standard_normal((m, k)).astype(np.float16)
        y = layer(gpu(x))
        kern = layer.kernel_for(m).split("(")[0]
        if silu:
            check_close(y, o.swiglu_reference(x, c.w_exact), 0.03, 0.02, (proj, m), kern, f"{proj}+silu")
        else:
            check_close(y, o.linear(x, c.w_exact), 0.05, 0.02, (proj, m), kern)


def test_w4linear_qwen3_0_6b_qkv_table():
    """The Qwen3-0.6B fused qkv shape (K 1024, N 4096, the reference's CPU-runnable config) through
    the gfx950 decode table's own entries (gemv at M = 1, gemvm at 2 .. 4, mma at 5 .. 8) and the
    default kernels past them, against the oracle's dequantize-then-matmul."""
    layer, c = _layer(1024, 4096, seed=61)
    rng = np.random.default_rng(29)
    for m in (1, 2, 4, 5, 8, 9, 16, 32):
        if m <= 8:
            assert (4096, 1024, m) in layer.kernels, m
        x = rng.standard_normal((m, 1024)).astype(np.float16)
        check_close(layer(gpu(x)), o.linear(x, c.w_exact), 0.05, 0.02, ("0.6b qkv", m), "layer")

"""Pins the CPU oracle (oracle/awq_oracle.py) before anything is compared against it.

Each check comes from outside the oracle's own formulas: the reference tests' packer and
known-answer nibble positions (tests/test_awq.py:19-29, 58-65 of 12vivi/tandem), exact rational
arithmetic for the dequantization over every (q, z) pair, closed-form row maps for the interleave,
explicit loops for the matmul, and committed fixtures. The last section plants plausible mistakes
in copies of oracle functions and checks that these pins reject every one of them."""

from __future__ import annotations

import os
from fractions import Fraction

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import awq_oracle as o

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- nibble order (awq.py:38-46)
def _word(nibbles) -> np.ndarray:
    v = 0
    for i, q in enumerate(nibbles):
        v |= (q & 0xF) << (4 * i)
    return np.array([[v]], dtype=np.uint32).view(np.int32)


def test_unpack_known_word():
    """Nibble i of 0x76543210 is i; AutoAWQ puts column ORDER[i] in nibble i, so columns read
    [0, 4, 1, 5, 2, 6, 3, 7] (tests/test_awq.py:26: out |= v[:, :, col] << 4 i)."""
    assert o.unpack_awq(_word(range(8))).tolist() == [[0, 4, 1, 5, 2, 6, 3, 7]]


@pytest.mark.parametrize("nibble", range(8))
@pytest.mark.parametrize("value", [1, 7, 8, 15])
def test_unpack_single_nibble(nibble, value):
    """A word with only nibble i set puts its value in column AWQ_PACK_ORDER[i], nowhere else
    (covers the sign bit: nibble 7 >= 8 makes the int32 negative)."""
    nib = [0] * 8
    nib[nibble] = value
    got = o.unpack_awq(_word(nib))[0]
    want = [0] * 8
    want[(0, 2, 4, 6, 1, 3, 5, 7)[nibble]] = value
    assert got.tolist() == want


def test_pack_matches_reference_test_packer_loop():
    """pack_awq == the reference tests' packer written out with Python ints, column by column."""
    rng = np.random.default_rng(1)
    vals = rng.integers(0, 16, size=(5, 32))
    got = o.pack_awq(vals).view(np.uint32)
    for r in range(5):
        for c in range(4):
            w = 0
            for i, col in enumerate((0, 2, 4, 6, 1, 3, 5, 7)):
                w |= int(vals[r, 8 * c + col]) << (4 * i)
            assert int(got[r, c]) == w


@settings(max_examples=50, deadline=None)
@given(st.integers(1, 6), st.integers(1, 6), st.integers(0, 2**32 - 1))
def test_pack_unpack_round_trip(rows, cols, seed):
    rng = np.random.default_rng(seed)
    vals = rng.integers(0, 16, size=(rows, 8 * cols))
    assert (o.unpack_awq(o.pack_awq(vals)) == vals).all()
    words = rng.integers(0, 2**32, size=(rows, cols), dtype=np.uint64).astype(np.uint32).view(np.int32)
    assert (o.pack_awq(o.unpack_awq(words)) == words).all()


# ------------------------------------------------------------ dequantization (awq.py:110-119)
def _fp16_of_exact(q: int, z: int, s16: np.float16) -> np.float16:
    """Round (q - z) * s to fp16 once, with round-to-nearest-even. The product has <= 15
    significant bits, so the float64 product is exact (checked against the rational product) and
    numpy's float64 -> float16 cast is the single rounding; float64 also keeps IEEE's sign of zero."""
    f64 = float(q - z) * float(s16)
    assert Fraction(f64) == Fraction(q - z) * Fraction(float(s16))
    return np.float16(f64)


SCALES = np.array([0.001, 0.0010004, 0.013, 0.02, 0.019989, 1.0, 0.5, 3.0e-3, 6.1e-5, 1.0e-4, 7.0e-3, 0.0],
                  dtype=np.float16)


def test_dequant_brute_force_every_q_z():
    """Every (q, z) in 16 x 16 with scales that force rounding (one in the subnormal product range,
    and 0): the oracle's float32-then-cast equals the exactly rounded value, bit for bit."""
    qq = np.zeros((128, 16), dtype=np.int32)
    qq[0, :] = np.arange(16)  # k = 0 of column n holds q = n
    for s16 in SCALES:
        for zi in range(16):
            zz = np.full((1, 16), zi, dtype=np.int32)
            ss = np.full((1, 16), s16, dtype=np.float16)
            w = o.dequant(o.pack_awq(qq), o.pack_awq(zz), ss)  # [N = 16, K = 128]
            for qv in range(16):
                want = _fp16_of_exact(qv, zi, s16)
                assert w[qv, 0].view(np.uint16) == want.view(np.uint16), (qv, zi, float(s16))


def test_dequant_exact_is_exact():
    """(q - z) * s in float32 equals the rational product (float32 holds 4 + 11 bits exactly)."""
    qw, qz, s, q, z = o.random_awq(256, 64, seed=3)
    w = o.dequant_exact(qw, qz, s)
    for n, k in [(0, 0), (5, 131), (63, 255), (17, 128)]:
        exact = Fraction(int(q[k, n]) - int(z[k // 128, n])) * Fraction(float(s[k // 128, n]))
        assert Fraction(float(w[n, k])) == exact


def test_dequant_layout_is_nn_linear():
    """dequant returns [N, K] (F.linear's weight layout): row n, column k of qweight's [K, N]."""
    qw, qz, s, q, z = o.random_awq(256, 16, seed=4)
    w = o.dequant(qw, qz, s)
    assert w.shape == (16, 256) and w.dtype == np.float16
    n, k = 9, 200
    assert w[n, k] == np.float16(float(q[k, n] - z[k // 128, n]) * float(s[k // 128, n]))


def test_dequant_rejects_bad_group():
    qw, qz, s, _, _ = o.random_awq(256, 16)
    with pytest.raises(ValueError):
        o.dequant(qw[:200], qz, s)


def test_dequant_exact_rows_sampled_columns():
    """dequant_exact_rows (the full-size tests' sampled output features) against the committed
    fixture's fp16 weights, the rational product at single entries, and a copy that takes the pack
    order for the reverse order (a plausible slip), which the fixture must reject."""
    data = np.load(os.path.join(GOLDEN, "awq_small.npz"))
    n = data["w_fp16"].shape[0]
    rows = np.array([0, 1, 7, 8, n - 1, 3, 3], dtype=np.int64)  # repeats and any order
    got = o.dequant_exact_rows(data["qweight"], data["qzeros"], data["scales"], rows)
    assert (got.astype(np.float16).view(np.uint16) == data["w_fp16"][rows].view(np.uint16)).all()
    qw, qz, s, q, z = o.random_awq(384, 40, seed=12)
    sel = np.array([39, 0, 17, 22])
    w = o.dequant_exact_rows(qw, qz, s, sel)
    for i, n_ in enumerate(sel):
        for k in (0, 127, 128, 383):
            exact = Fraction(int(q[k, n_]) - int(z[k // 128, n_])) * Fraction(float(s[k // 128, n_]))
            assert Fraction(float(w[i, k])) == exact
    shifts = 4 * np.asarray(o.AWQ_PACK_ORDER)[rows % 8]  # the slip: nibble PACK[j] instead of REVERSE[j]
    qq = (data["qweight"].astype(np.int64)[:, rows // 8] & 0xFFFFFFFF) >> shifts & 0xF
    zz = (data["qzeros"].astype(np.int64)[:, rows // 8] & 0xFFFFFFFF) >> shifts & 0xF
    bad = ((qq - np.repeat(zz, 128, 0)) * np.repeat(data["scales"][:, rows].astype(np.float32), 128, 0)).T
    assert not (bad.astype(np.float16).view(np.uint16) == data["w_fp16"][rows].view(np.uint16)).all()


# ---------------------------------------------------------------- interleave (awq.py:71-75)
def test_interleave_closed_form():
    """Row 16 T + 8 h + i of the interleaved tensor is source row h N/2 + 8 T + i."""
    n = 96
    t = np.arange(n)
    got = o.interleave_gate_up(t[:, None])[:, 0]
    for dst in range(n):
        tt, h, i = dst // 16, (dst // 8) % 2, dst % 8
        assert got[dst] == h * (n // 2) + 8 * tt + i
    assert (o.deinterleave_gate_up(o.interleave_gate_up(t[:, None]))[:, 0] == t).all()


# ------------------------------------------------------------------------- matmul and SwiGLU
def test_linear_matches_loops():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 8))
    w = rng.standard_normal((5, 8))
    y = o.linear(x, w)
    for m in range(3):
        for n in range(5):
            assert y[m, n] == pytest.approx(sum(x[m, k] * w[n, k] for k in range(8)), rel=1e-12)


def test_silu_and_mul_closed_form():
    y = np.array([[0.0, 2.0, -1.0, 3.0, 5.0, 7.0]])
    got = o.silu_and_mul(y)  # gate = [0, 2, -1], up = [3, 5, 7]
    want = [0.0 * 3.0, 2.0 / (1 + np.exp(-2.0)) * 5.0, -1.0 / (1 + np.exp(1.0)) * 7.0]
    assert np.allclose(got[0], want, rtol=1e-15)


def test_swiglu_reference_rounds_weights_once():
    qw, qz, s, _, _ = o.random_awq(128, 32, seed=6)
    x = np.random.default_rng(6).standard_normal((2, 128)).astype(np.float16)
    w = o.dequant_exact(qw, qz, s)
    want = o.silu_and_mul(x.astype(np.float64) @ w.astype(np.float16).astype(np.float64).T)
    assert np.allclose(o.swiglu_reference(x, w), want, rtol=0, atol=0)


def test_random_awq_recipe():
    """The reference tests' input recipe (tests/test_awq.py:32-38): q and z uniform over all of 0..15,
    scales fp16 in [0.001, 0.021), AutoAWQ-packed q and z, the group dimension K / 128."""
    qw, qz, s, q, z = o.random_awq(1024, 64, seed=3)
    assert qw.shape == (1024, 8) and qz.shape == (8, 8) and s.shape == (8, 64) and s.dtype == np.float16
    assert q.shape == (1024, 64) and z.shape == (8, 64)
    assert set(np.unique(q)) == set(range(16)) and set(np.unique(z)) == set(range(16))
    assert (o.unpack_awq(qw) == q).all() and (o.unpack_awq(qz) == z).all()
    sf = s.astype(np.float64)
    assert sf.min() >= 0.001 - 1e-6 and sf.max() < 0.021 + 1e-5 and sf.std() > 0.005
    qw2, _, s2, _, _ = o.random_awq(1024, 64, seed=3)
    assert (qw2 == qw).all() and (s2.view(np.uint16) == s.view(np.uint16)).all()  # seeded


# ---------------------------------------------------------------------------- golden fixtures
def test_golden_fixtures():
    """The committed fixtures (tests/golden/make_golden.py) still come out of the oracle."""
    data = np.load(os.path.join(GOLDEN, "awq_small.npz"))
    w = o.dequant(data["qweight"], data["qzeros"], data["scales"])
    assert (w.view(np.uint16) == data["w_fp16"].view(np.uint16)).all()
    y = o.linear(data["x"], w)
    assert np.array_equal(y, data["y_f64"])
    yi = o.swiglu_reference(data["x"], o.dequant_exact(data["qweight"], data["qzeros"], data["scales"]))
    assert np.array_equal(yi, data["swiglu_f64"])
    assert (o.unpack_awq(data["qweight"]) == data["q"]).all()


# --------------------------------------------------------- planted mistakes must be rejected
def _unpack_swapped(packed):  # uses the pack order where the reverse order belongs
    p = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    shifts = np.array([4 * i for i in o.AWQ_PACK_ORDER], dtype=np.int64)
    return ((p[:, :, None] >> shifts) & 0xF).reshape(p.shape[0], -1)


def _dequant_double_rounding(qweight, qzeros, scales):  # q*s - z*s with a rounded z*s (an FMA path)
    q = o.unpack_awq(qweight).astype(np.float32)
    z = o.unpack_awq(qzeros).astype(np.float32)
    s = scales.astype(np.float32)
    zs = (np.repeat(z, 128, 0) * np.repeat(s, 128, 0)).astype(np.float16).astype(np.float32)
    return (q * np.repeat(s, 128, 0) - zs).T.astype(np.float16)


def _dequant_no_zero(qweight, qzeros, scales):  # drops the zero point
    q = o.unpack_awq(qweight).astype(np.float32)
    return (q * np.repeat(scales.astype(np.float32), 128, 0)).T.astype(np.float16)


def _dequant_transposed(qweight, qzeros, scales):  # returns [K, N]
    return o.dequant(qweight, qzeros, scales).T.copy()


def test_planted_mistakes_are_caught():
    assert _unpack_swapped(_word(range(8))).tolist() != [[0, 4, 1, 5, 2, 6, 3, 7]]
    data = np.load(os.path.join(GOLDEN, "awq_small.npz"))
    ref = data["w_fp16"].view(np.uint16)
    for bad in (_dequant_double_rounding, _dequant_no_zero, _dequant_transposed):
        got = bad(data["qweight"], data["qzeros"], data["scales"])
        assert got.shape != ref.shape or not (got.view(np.uint16) == ref).all(), bad.__name__
    # the interleave with gate and up swapped breaks the closed form
    t = np.arange(32)[:, None]
    swapped = o.interleave_gate_up(np.concatenate([t[16:], t[:16]]))
    assert not (swapped == o.interleave_gate_up(t)).all()


# ------------------------------------------- norms (ops.py:107-120, triton_ops.py:101-124)
def _norm_constant_row_expected(c: float, w: float, eps: float) -> np.float16:
    """A row of K equal values c: mean(x^2) = c^2 for any K, so y = c / sqrt(c^2 + eps) * w."""
    return np.float16(c / np.sqrt(c * c + eps) * w)


@pytest.mark.parametrize("c", [1.0, -3.5, 0.0078125, 1000.0])
@pytest.mark.parametrize("k", [512, 4096])
def test_rms_norm_constant_row(c, k):
    w = np.full(k, 0.75, dtype=np.float16)
    y = o.rms_norm(np.full((1, k), c, dtype=np.float16), w, 1e-6)
    assert (y == _norm_constant_row_expected(c, 0.75, 1e-6)).all()


def test_rms_norm_zero_row_and_eps():
    """eps keeps a zero row finite; with x^2 << eps, y = x / sqrt(eps) * w (eps dominates)."""
    k, eps = 512, 1e-2
    w = np.ones(k, dtype=np.float16)
    assert (o.rms_norm(np.zeros((2, k), dtype=np.float16), w, eps) == 0).all()
    x = np.full((1, k), 2.0 ** -10, dtype=np.float16)
    assert o.rms_norm(x, w, eps)[0, 0] == np.float16(2.0 ** -10 / np.sqrt(2.0 ** -20 + eps))


def test_rms_norm_explicit_loops():
    rng = np.random.default_rng(5)
    k = 512
    x = rng.standard_normal((3, k)).astype(np.float16)
    w = (rng.random(k) + 0.5).astype(np.float16)
    y = o.rms_norm(x, w, 1e-6)
    for m in range(3):
        row = [float(v) for v in x[m]]
        rstd = 1.0 / np.sqrt(sum(v * v for v in row) / k + 1e-6)
        want = np.array([row[i] * rstd * float(w[i]) for i in range(k)]).astype(np.float16)
        assert (np.abs(y[m].astype(np.float32) - want.astype(np.float32))
                <= np.spacing(np.abs(want)).astype(np.float32)).all()


def test_add_rms_norm_residual_and_sum():
    """r' = fp16(fp32(x + r)) element by element; y is the norm of the fp32 sum: equal to rms_norm
    of s where s is exact in fp16, and a scale-free function of the row (powers of two)."""
    rng = np.random.default_rng(6)
    k = 1024
    x = rng.standard_normal((2, k)).astype(np.float16)
    r = rng.standard_normal((2, k)).astype(np.float16)
    w = (rng.random(k) + 0.5).astype(np.float16)
    y, r2 = o.add_rms_norm(x, r, w, 1e-6)
    for m in range(2):
        for i in range(0, k, 37):
            assert r2[m, i] == np.float16(np.float32(float(x[m, i])) + np.float32(float(r[m, i])))
    xs = (x.astype(np.float32) * 0.5).astype(np.float16)  # x / 2 and x / 2: s = x exactly
    y2, r3 = o.add_rms_norm(xs, xs, w, 0.0)
    assert (r3 == x).all() and (y2 == o.rms_norm(x, w, 0.0)).all()
    y4, _ = o.add_rms_norm(xs * np.float16(4), xs * np.float16(4), w, 0.0)  # s = 4 x
    assert (y4 == y2).all()


def _add_rms_norm_no_residual(x, r, w, eps):  # forgets to add the residual into the normalised value
    return o.rms_norm(x, w, eps), (x.astype(np.float32) + r.astype(np.float32)).astype(np.float16)


def _rms_norm_unbiased(x, w, eps):  # mean over K - 1
    x64 = x.astype(np.float64)
    rstd = 1.0 / np.sqrt((x64 * x64).sum(-1, keepdims=True) / (x.shape[-1] - 1) + eps)
    return (x64 * rstd * w.astype(np.float64)).astype(np.float16)


def _rms_norm_no_eps(x, w, eps):
    x64 = x.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        return (x64 / np.sqrt(np.mean(x64 * x64, -1, keepdims=True)) * w.astype(np.float64)).astype(np.float16)


def test_planted_norm_mistakes_are_caught():
    k = 512
    w = np.full(k, 0.75, dtype=np.float16)
    row = np.full((1, k), 1.0, dtype=np.float16)
    assert not (_rms_norm_unbiased(row, w, 1e-6) == _norm_constant_row_expected(1.0, 0.75, 1e-6)).all()
    assert not (_rms_norm_no_eps(np.zeros((1, k), dtype=np.float16), w, 1e-2) == 0).all()
    x = np.full((1, k), 0.5, dtype=np.float16)
    r = np.full((1, k), -2.0, dtype=np.float16)
    y_bad, _ = _add_rms_norm_no_residual(x, r, w, 1e-6)
    assert (y_bad == _norm_constant_row_expected(0.5, 0.75, 1e-6)).all()
    assert not (y_bad == _norm_constant_row_expected(-1.5, 0.75, 1e-6)).all()  # the true s = -1.5
    y, _ = o.add_rms_norm(x, r, w, 1e-6)
    assert (y == _norm_constant_row_expected(-1.5, 0.75, 1e-6)).all()


# ------------------------------------- the torch restatement of the fallback (CPU baseline)
def test_torch_fallback_matches_numpy_oracle():
    """oracle/torch_fallback.py (the CPU baseline's arithmetic) against the numpy oracle: the same
    unpacked nibbles, the same dequantized fp16 bits (every element), and products inside the
    fp16 GEMM tolerance of the float64 product; a copy with the pack order for the reverse order
    fails the bit check."""
    import torch

    from oracle import torch_fallback as tf

    data = np.load(os.path.join(GOLDEN, "awq_small.npz"))
    qw, qz, s = (torch.from_numpy(data[n]) for n in ("qweight", "qzeros", "scales"))
    assert (tf.unpack_awq(qw).numpy() == o.unpack_awq(data["qweight"])).all()
    w = tf.dequant_kn(qw, qz, s)
    assert (w.t().contiguous().numpy().view(np.uint16) == data["w_fp16"].view(np.uint16)).all()
    x = torch.from_numpy(data["x"])
    for dt in (torch.float16, torch.float32):
        y = tf.fallback_linear(x, qw, qz, s, dt).double().numpy()
        assert np.allclose(y, data["y_f64"], atol=0.05, rtol=0.02), dt
    saved = tf._SHIFTS
    try:
        tf._SHIFTS = torch.tensor([4 * i for i in o.AWQ_PACK_ORDER], dtype=torch.int32)
        bad = tf.dequant_kn(qw, qz, s).t().contiguous().numpy()
        assert not (bad.view(np.uint16) == data["w_fp16"].view(np.uint16)).all()
    finally:
        tf._SHIFTS = saved

"""Host-side logic that runs without a GPU: the C-ABI library and its exports, argument checks
that return before any launch, the tile layout, the W4Linear contract and dispatch tables
(python/tandem/layers/awq.py:136-286 and tests/test_awq.py of 12vivi/tandem are the models)."""

from __future__ import annotations

import csv
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import awq_oracle as o
from tandem_amd.layers import awq, linear, w4_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tandem_w4.h")


def declared_symbols() -> list[str]:
    text = open(HEADER, encoding="utf-8").read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tw4_\w+)\s*\(", text)))


# ------------------------------------------------------------------------------------ C ABI
def test_library_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) >= 9
    lib = w4_hip.library()
    for name in syms:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", w4_hip.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (tw4_\w+)", out))
    assert set(syms) == exported, (set(syms) ^ exported)


def test_config_queries():
    dec, gemm = w4_hip.decode_configs(), w4_hip.gemm_configs()
    assert len(dec) >= 8 and all(len(c) == 3 and c[0] >= 1 and c[1] >= 1 for c in dec)
    assert len(gemm) >= 8 and all(len(c) == 5 and c[4] in (0, 1, 2, 3) for c in gemm)
    # warps_k: 1 or 2 wavefronts per K step (stages 0, 2), wavefronts along M (stages 3), or the
    # wavefronts that split each unit's groups (stages 1, whose warps_n is the prefetch depth)
    assert all(c[3] in ((4, 8) if c[4] == 1 else (1, 2)) for c in gemm)
    assert {c[4] for c in gemm} == {0, 1, 2, 3}
    assert awq.DEFAULT_KERNEL[1:] in dec
    wide = w4_hip.mma_wide_configs()
    assert wide and not set(wide) & set(dec) and all(len(c) == 3 and 2 <= c[2] <= 6 for c in wide)
    assert w4_hip.mma_configs() == dec + wide
    for m_max, cfg in awq.DEFAULT_GEMM:
        if cfg is not None and cfg[0] == "mma":
            assert tuple(cfg[1:]) in dec + wide and m_max <= 64
        elif cfg is not None:
            assert cfg[:5] in gemm


def test_library_identity():
    lib = w4_hip.library()
    assert lib.tw4_arch() == b"gfx950"
    assert lib.tw4_version().startswith(b"tandem_w4 ")


def _fake(addr=4096):
    return ctypes.c_void_p(addr)


def test_argument_errors_return_before_launch():
    """Each call fails a check that comes before any HIP call; the message names the problem
    (the reference's TORCH_CHECK texts, python/tandem/csrc/w4_gemv.cu:568-579, 608, 624-625)."""
    lib = w4_hip.library()
    cases = [
        (lambda: lib.tw4_dequant(_fake(), _fake(), _fake(), _fake(), 64, 100, 0, None), "K % 128"),
        (lambda: lib.tw4_dequant(_fake(), _fake(), _fake(), _fake(), 60, 128, 0, None), "N % 8"),
        (lambda: lib.tw4_dequant(_fake(), _fake(), _fake(), _fake(), 24, 128, 1, None), "deinterleave"),
        (lambda: lib.tw4_dequant(None, _fake(), _fake(), _fake(), 64, 128, 0, None), "null"),
        (lambda: lib.tw4_repack_awq(_fake(), _fake(), _fake(), _fake(), _fake(), _fake(), 100, 64, 0, None), "K % 128"),
        (lambda: lib.tw4_repack_awq(_fake(), _fake(), _fake(), _fake(), _fake(), _fake(), 128, 24, 1, None), "interleave"),
        (lambda: lib.tw4_gemv(_fake(), _fake(), _fake(), _fake(), _fake(), 5, 64, 128, 4, 2, 1, None), "M <= 4"),
        (lambda: lib.tw4_gemv(_fake(4100), _fake(), _fake(), _fake(), _fake(), 1, 64, 128, 4, 2, 1, None), "aligned"),
        (lambda: lib.tw4_gemv(_fake(), _fake(), _fake(), _fake(), _fake(), 1, 64, 65536 + 128, 1, 4, 1, None), "K <= 65536"),
        (lambda: lib.tw4_gemv_act(_fake(), _fake(), _fake(), _fake(), _fake(), 1, 24, 128, 4, 2, 1, 1, None),
         "SwiGLU"),
        (lambda: lib.tw4_mma(_fake(), _fake(), _fake(), _fake(), _fake(), 65, 64, 128, 4, 2, 1, 0, None), "M <= 64"),
        (lambda: lib.tw4_rms_norm(_fake(), _fake(), _fake(), 1, 1000, 1e-6, None), "K % 512"),
        (lambda: lib.tw4_rms_norm(_fake(), _fake(), _fake(), 1, 16384, 1e-6, None), "K <= 8192"),
        (lambda: lib.tw4_add_rms_norm(_fake(4104), _fake(), _fake(), 1, 1024, 1e-6, None), "aligned"),
        (lambda: lib.tw4_add_rms_norm(_fake(), None, _fake(), 1, 1024, 1e-6, None), "null"),
        (lambda: lib.tw4_mma(_fake(), _fake(), _fake(), _fake(), _fake(), 4, 24, 128, 4, 2, 1, 1, None), "SwiGLU"),
        (lambda: lib.tw4_mma_splitk(_fake(), _fake(), _fake(), _fake(), _fake(), _fake(), _fake(), 1 << 20, 1024,
                                    8, 64, 1024, 4, 2, 1, 17, 0, None), "splits"),
        (lambda: lib.tw4_mma_splitk(_fake(), _fake(), _fake(), _fake(), _fake(), _fake(), _fake(), 1 << 20, 1024,
                                    8, 64, 256, 4, 2, 1, 3, 0, None), "splits"),
        (lambda: lib.tw4_mma_splitk(_fake(), _fake(), _fake(), _fake(), _fake(), _fake(), _fake(), 1 << 20, 1024,
                                    17, 64, 1024, 4, 2, 1, 2, 0, None), "M <= 16"),
        (lambda: lib.tw4_mma_splitk(_fake(), _fake(), _fake(), _fake(), _fake(), None, _fake(), 1 << 20, 1024,
                                    8, 64, 1024, 4, 2, 1, 2, 0, None), "workspace"),
        (lambda: lib.tw4_mma_persist(_fake(), _fake(), _fake(), _fake(), _fake(), 17, 64, 1024, 4, 2, 1, 1, 0, None),
         "M <= 16"),
        (lambda: lib.tw4_mma_persist(_fake(), _fake(), _fake(), _fake(), _fake(), 8, 64, 1024, 4, 2, 1, 0, 0, None),
         "per_cu"),
        (lambda: lib.tw4_mma_persist(_fake(), _fake(), _fake(), _fake(), _fake(), 8, 24, 1024, 4, 2, 1, 1, 1, None),
         "SwiGLU"),
        (lambda: lib.tw4_gemm(_fake(), _fake(), _fake(), _fake(), _fake(), _fake(), _fake(), 1 << 20, 1024,
                              32, 64, 128, 2, 1, 4, 1, 2, 17, 0, None), "splits"),
        (lambda: lib.tw4_gemm(_fake(), _fake(), _fake(), _fake(), _fake(), _fake(), _fake(), 1 << 20, 1024,
                              32, 64, 100, 2, 1, 4, 1, 2, 0, 0, None), "K % 128"),
    ]
    for call, needle in cases:
        assert call() == w4_hip.TW4_EINVAL
        assert needle in lib.tw4_last_error().decode(), (needle, lib.tw4_last_error())


# ------------------------------------------------------------------------------ tile layout
def decode_tile_layout(packed: np.ndarray, n: int, k: int) -> np.ndarray:
    """Reads the tile layout back with the formula of include/tandem_w4.h: word (kb, r, s) of
    block (T, g) holds k = 128 g + 32 kb + 8 s + 2 q + e of row 16 T + r in nibble q + 4 e."""
    words = np.asarray(packed).view(np.uint32).reshape(-1)
    g_count = k // 128
    out = np.full((len(words) * 8 // k, k), -1, dtype=np.int64)
    idx = np.arange(len(words))
    blk, within = idx // 256, idx % 256
    t, g = blk // g_count, blk % g_count
    kb, r, s = within // 64, (within // 4) % 16, within % 4
    for qq in range(4):
        for e in range(2):
            nib = (words >> (4 * (qq + 4 * e))) & 0xF
            out[16 * t + r, 128 * g + 32 * kb + 8 * s + 2 * qq + e] = nib
    assert (out >= 0).all()
    return out


@pytest.mark.parametrize("n,k", [(16, 128), (24, 256), (64, 384), (1000, 256)])
def test_pack_rows_tile_layout(n, k):
    q = torch.randint(0, 16, (n, k), dtype=torch.int32, generator=torch.Generator().manual_seed(n + k))
    packed = awq.pack_rows(q)
    assert packed.shape == (w4_hip.padded_rows(n), k // 8) and packed.dtype == torch.int32
    got = decode_tile_layout(packed.numpy(), n, k)
    assert (got[:n] == q.numpy()).all()
    assert (got[n:] == 0).all()  # padding rows


def test_pack_rows_known_positions():
    """Spot checks in the style of tests/test_awq.py:58-65, on this build's layout."""
    n, k = 32, 384
    q = torch.randint(0, 16, (n, k), dtype=torch.int32)
    packed = awq.pack_rows(q).view(n // 16, k // 128, 4, 16, 4)  # [T, g, kb, r, s]
    for t, g, kb, r, s, qq, e in ((0, 0, 0, 0, 0, 0, 0), (1, 2, 3, 15, 3, 3, 1), (0, 1, 2, 7, 1, 2, 0)):
        nib = (int(packed[t, g, kb, r, s]) >> (4 * (qq + 4 * e))) & 0xF
        assert nib == int(q[16 * t + r, 128 * g + 32 * kb + 8 * s + 2 * qq + e])


@pytest.mark.parametrize("n,g", [(16, 1), (48, 32), (24, 8), (1000, 3)])
def test_tile_major_params(n, g):
    """Scales / zeros order of include/tandem_w4.h: value (row, group) at
    16 T G + g rows_T + (row - 16 T), T = row / 16, rows_T = min(16, N - 16 T)."""
    t = torch.arange(n * g, dtype=torch.int64).view(n, g)
    tm = awq.tile_major_params(t)
    assert tm.shape == (n, g)
    flat = tm.reshape(-1)
    for row in range(n):
        tt = row // 16
        rows = min(16, n - 16 * tt)
        for gg in range(g):
            assert int(flat[16 * tt * g + gg * rows + row - 16 * tt]) == int(t[row, gg])
    assert torch.equal(awq.row_major_params(tm), t)


def test_unpack_awq_matches_oracle():
    qw, _, _, q, _ = o.random_awq(256, 64, seed=11)
    assert (awq.unpack_awq(torch.from_numpy(qw)).numpy() == q).all()


def test_interleave_matches_oracle():
    t = torch.arange(96 * 3).view(96, 3)
    assert (awq.interleave_gate_up(t).numpy() == o.interleave_gate_up(t.numpy())).all()


# ----------------------------------------------------------------------- W4Linear contract
def test_w4linear_constructor_and_buffers():
    layer = awq.W4Linear(512, 256, 128)
    assert layer.awq_layout and not layer.silu_mul
    assert layer.qweight.shape == (512, 32) and layer.qweight.dtype == torch.int32
    assert layer.qzeros.shape == (4, 32) and layer.qzeros.dtype == torch.int32
    assert layer.scales.shape == (4, 256) and layer.scales.dtype == torch.float16
    for args in ((512, 256, 64), (500, 256, 128), (512, 252, 128)):
        with pytest.raises(ValueError):
            awq.W4Linear(*args)


def test_enable_silu_mul_rules():
    assert awq.W4Linear(512, 384, 128).enable_silu_mul()
    assert not awq.W4Linear(512, 392, 128).enable_silu_mul()  # N % 16 != 0: not fusable


def test_forward_needs_finalize_and_gpu():
    layer = awq.W4Linear(256, 64, 128)
    with pytest.raises(RuntimeError):
        layer(torch.zeros(1, 256, dtype=torch.float16))
    with pytest.raises(RuntimeError):  # finalize on CPU tensors: there is no CPU repack path
        layer.finalize()


def test_cpu_input_never_reaches_a_kernel():
    ext = w4_hip.W4Extension()
    x = torch.zeros(1, 128, dtype=torch.float16)
    w = torch.zeros(16, 16, dtype=torch.int32)
    s = torch.zeros(16, 1, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        ext.w4_mma(x, w, s, s, 4, 2, 1, 0)
    with pytest.raises(RuntimeError, match="GPU"):
        w4_hip.dequant(w, s, s)


def test_pick_gemm_ladder():
    table = ((17, "a"), (32, "b"), (1 << 30, None))
    assert awq.pick_gemm(table, 17) == "a" and awq.pick_gemm(table, 18) == "b"
    assert awq.pick_gemm(table, 4096) is None
    assert awq.pick_gemm(((64, "x"),), 100) == "x"  # past the last m_max: the last entry


def test_huge_batches_take_the_dense_path(monkeypatch):
    """M x K >= 2^31 is beyond the fused GEMM's 32-bit offsets (the reference's w4_gemm refuses it,
    csrc/w4_gemv.cu:661): forward's GEMM predicate sends it to dequantize + matmul, whatever the
    ladder says, and kernel_for reports the same routing."""
    import types

    layer = awq.W4Linear(4096, 4096, 128)
    layer.awq_layout = False
    layer.gemm_kernels = {(4096, 4096): ((1 << 30, (8, 4, 4, 1, 3, 0)),)}
    assert layer.kernel_for(524287).startswith("gemm(")
    assert layer.kernel_for(524288) == "dequant+matmul"  # 524288 x 4096 = 2^31
    monkeypatch.setattr(awq, "_aligned", lambda x: True)
    fake = lambda m: types.SimpleNamespace(is_cuda=True, shape=(m, 4096))  # noqa: E731
    assert awq._gemm_ok(fake(524287)) and not awq._gemm_ok(fake(524288)) and not awq._gemm_ok(fake(16))


def test_kernel_for_follows_the_tables():
    """kernel_for names the entry forward dispatches: the decode table up to M = 16 (gemv / gemvm
    only up to M = 4, else the default matrix-core kernel), the ladder above, None as dequant + matmul."""
    layer = awq.W4Linear(256, 64, 128)
    layer.awq_layout = False
    layer.kernels = {(64, 256, 1): ("gemv", 4, 2, 1), (64, 256, 6): ("gemv", 4, 2, 1),
                     (64, 256, 8): ("mmak", 8, 1, 2, 2)}
    layer.gemm_kernels = {(64, 256): ((32, ("mma", 8, 1, 1)), (64, (2, 1, 4, 2, 2, 4)), (1 << 30, None))}
    assert layer.kernel_for(1) == "gemv(4, 2, 1)"
    assert layer.kernel_for(6) == f"{awq.DEFAULT_KERNEL[0]}{tuple(awq.DEFAULT_KERNEL[1:])}"
    assert layer.kernel_for(8) == "mmak(8, 1, 2, 2)"
    assert layer.kernel_for(20) == "mma(8, 1, 1)"
    assert layer.kernel_for(40) == "gemm(2, 1, 4, 2, 2, 4)"
    assert layer.kernel_for(100) == "dequant+matmul"


def test_tables_are_well_formed():
    assert awq.DEFAULT_KERNEL[0] in ("gemv", "mma") and len(awq.DEFAULT_KERNEL) == 4
    decode = set(w4_hip.decode_configs())
    mma = set(w4_hip.mma_configs())  # w4_mma also takes the row-tile-wide configs
    gemm = set(w4_hip.gemm_configs())
    for table in awq.W4_KERNELS.values():
        for key, cfg in table.items():
            assert key[3:] in ((), ("silu",), ("norm",), ("silu", "norm"))
            if key[-1] == "norm":  # the fused add + RMSNorm GEMV (forward_norm): a GEMV config, M <= 4
                assert cfg[0] == "gemv" and tuple(cfg[1:]) in decode and key[2] <= 4
                continue
            n, k, m = key[:3]
            assert 1 <= m <= 16 and k % 128 == 0 and n % 8 == 0
            if cfg[0] == "gemm":  # a compiled GEMM config and a split mode
                assert len(cfg) == 7 and tuple(cfg[1:6]) in gemm and 0 <= cfg[6] <= 16
            elif cfg[0] == "mmak":  # a compiled decode config and 2 .. 16 K splits (at most one per group)
                assert len(cfg) == 5 and tuple(cfg[1:4]) in decode and 2 <= cfg[4] <= min(16, k // 128)
            elif cfg[0] == "mmap":  # a compiled decode config, 1 .. 8 workgroups per CU, x in LDS
                assert len(cfg) == 5 and tuple(cfg[1:4]) in decode and 1 <= cfg[4] <= 8
                assert m * (2 * k + 16) <= 136 * 1024  # past 80 KB only for grids of at most one per CU
            else:  # a compiled decode config; gemv only where it runs (M <= 4), gemvm where x' fits LDS
                assert cfg[0] in ("gemv", "gemvm", "mma") and tuple(cfg[1:]) in (mma if cfg[0] == "mma" else decode)
                assert cfg[0] != "gemv" or m <= 4
                assert cfg[0] != "gemvm" or m * (2 * k + 16) + m * (k // 128) * 36 <= 160 * 1024
    for ladder in [awq.DEFAULT_GEMM, *[v for t in awq.W4_GEMM_KERNELS.values() for v in t.values()]]:
        m_maxes = [m for m, _ in ladder]
        assert m_maxes == sorted(m_maxes)
        for m_max, cfg in ladder:
            assert cfg is None or (len(cfg) == 6 and tuple(cfg[:5]) in gemm) or \
                (cfg[0] == "mma" and tuple(cfg[1:]) in mma and m_max <= 64 and cfg[2] * -(-m_max // 16) <= 4)


def test_norm_entry_lookup():
    """forward_norm takes the (N, K, M[, silu], norm) entry, else the plain decode entry."""
    lin = awq.W4Linear(256, 64, 128)
    lin.kernels = {(64, 256, 1): ("gemv", 8, 2, 1), (64, 256, 1, "norm"): ("gemv", 4, 4, 1),
                   (64, 256, 2): ("mma", 4, 2, 1), (64, 256, 2, "silu"): ("gemv", 4, 2, 1),
                   (64, 256, 2, "silu", "norm"): ("gemv", 4, 1, 1)}
    assert lin.decode_entry(1) == ("gemv", 8, 2, 1) and lin.norm_entry(1) == ("gemv", 4, 4, 1)
    assert lin.norm_entry(2) == ("mma", 4, 2, 1)  # no plain norm entry: the decode entry
    assert lin.norm_entry(3) == awq.DEFAULT_KERNEL
    lin.silu_mul = True
    assert lin.decode_entry(2) == ("gemv", 4, 2, 1) and lin.norm_entry(2) == ("gemv", 4, 1, 1)
    assert lin.norm_entry(1) == ("gemv", 8, 2, 1)  # the silu key has no norm entry at M = 1


def test_make_linear_and_finalize_quantized():
    class Q:
        group_size = 128

    assert isinstance(linear.make_linear(256, 64), torch.nn.Linear)
    layer = linear.make_linear(256, 64, False, Q())
    assert isinstance(layer, awq.W4Linear)
    with pytest.raises(NotImplementedError):
        linear.make_linear(256, 64, True, Q())
    calls = []

    class Fake(torch.nn.Module):
        awq_layout = True

        def finalize(self, name):
            calls.append(name)
            self.awq_layout = False

    model = torch.nn.Sequential(Fake(), torch.nn.Linear(2, 2), Fake())
    assert linear.finalize_quantized(model, "dev") == 2 and calls == ["dev", "dev"]
    assert linear.finalize_quantized(model, "dev") == 0


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=300)
    assert proc.returncode != 0 and "one GPU" in proc.stderr


# -------------------------------------------------------------- staging index math (host check)
def _x_slice(gb, ge, m):
    """x_slice of csrc/tw4_decode.hip: (c0, n16, n, magic)."""
    n16 = 16 * (ge - gb)
    return (16 * gb if n16 else 0), n16, m * n16, ((0xFFFFFFFF // n16) + 1 if n16 else 0)


def _x_pos(sl, f, one_row):
    c0, n16, n, magic = sl
    f = max(min(f, n - 1), 0)
    if one_row:
        return 0, f
    mm = (f * magic) >> 32
    return mm, f - mm * n16


@pytest.mark.parametrize("k", [128, 256, 384, 512, 1024, 4096, 12288])
def test_staging_indices_in_bounds(k):
    """Every chunk the decode kernels' x staging and the fused norm prologue load (the first batch
    and every later batch, including the unconditional loads of an empty slice) lies inside x [M, K],
    the norm weight [K] and the [M][G] group-sum table, and the umulhi division is exact; for every
    compiled warps_k and M = 1..16."""
    kx, g_count = k // 8, k // 128
    for wk in sorted({c[0] for c in w4_hip.decode_configs()}):
        gw = -(-g_count // wk)
        for m in range(1, 17):
            for wave in range(wk):
                gb = min(wave * gw, g_count)
                ge = min(gb + gw, g_count)
                sl = _x_slice(gb, ge, m)
                c0, n16, n, _ = sl
                last = max(n, 128) + 64 * 2  # the first batch always, then batches while f0 - lane < n
                for lane in range(64):
                    for f in range(lane, last, 64):
                        mm, c = _x_pos(sl, f, m == 1)
                        assert 0 <= mm < m and 0 <= c0 + c < kx, (k, wk, m, wave, f)
                        assert mm * kx + c0 + c < m * kx
                        if n and f < n:  # the exact position of a real chunk
                            assert (mm, c) == divmod(f, n16)
                            assert mm * g_count + (c0 + c) // 16 < m * g_count


def test_bench_sweep_covers_the_single_linear_configs():
    """bench.py --sweep times every single-linear (shape, M) of the benchmark configs: Qwen3-0.6B qkv
    at M = 1, Qwen3-8B's four shapes at the decode and GEMM M lists, Qwen3-1.7B's at M = 1, 4, 8."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    got = {(model, proj, k, n, m) for (model, proj, k, n), ms in bench.SWEEP for m in ms}
    want = {("Qwen3-0.6B", "qkv", 1024, 4096, 1)}
    want |= {("Qwen3-8B", p, k, n, m) for p, (k, n) in {"qkv": (4096, 6144), "o": (4096, 4096),
                                                        "gate_up": (4096, 24576), "down": (12288, 4096)}.items()
             for m in (1, 4, 8, 16, 24, 32, 64, 256, 1024, 4096)}
    want |= {("Qwen3-1.7B", p, k, n, m) for p, (k, n) in {"qkv": (2048, 4096), "o": (2048, 2048),
                                                          "gate_up": (2048, 12288), "down": (6144, 2048)}.items()
             for m in (1, 4, 8)}
    assert got == want
    # the per-call byte count of the benchmark's metric: int4 weights, fp16 scales, int4 zeros, x and y
    assert bench.call_bytes(1, 4096, 24576) == 52355072


def _bench_module():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    return bench


def test_prof_summary_targets_the_profiled_kernel(tmp_path):
    """bench.py prof --summarize headlines the kernel the command launched --launches times, never the
    load-time repack that ran once per weight copy (more often than the kernel at M = 32), and scales
    each counter by the calibration copy's reading."""
    bench = _bench_module()
    assert bench.target_kernel({"tw4::repack_weights_kernel": 80, "tw4::gemm_kernel<2,1>": 40,
                                "other": 40}, 40) == "tw4::gemm_kernel<2,1>"
    assert bench.target_kernel({"tw4::repack_weights_kernel": 80, "tw4::mma_kernel": 20}, 40) == "tw4::mma_kernel"
    rows = []
    for counter, copy_val, kern_val in (("FETCH_SIZE", 131072.0, 25000.0), ("WRITE_SIZE", 262144.0, 48.0)):
        path = tmp_path / f"{counter}.csv"
        with open(path, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
            w.writeheader()
            d = 0
            for _ in range(3):
                d += 1
                w.writerow({"Dispatch_Id": d, "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": counter,
                            "Counter_Value": copy_val})
            for _ in range(90):  # 90 repacks of the weight copies, then the 40 profiled launches
                d += 1
                w.writerow({"Dispatch_Id": d, "Kernel_Name": "tw4::repack_weights_kernel", "Counter_Name": counter,
                            "Counter_Value": 999.0})
            for _ in range(40):
                d += 1
                w.writerow({"Dispatch_Id": d, "Kernel_Name": "tw4::gemm_kernel", "Counter_Name": counter,
                            "Counter_Value": kern_val})
        rows.append(str(path))
    rec = bench.summarize_traffic(rows[0], rows[1], 256, 3, 40, 52355072)
    assert rec["kernel"] == "tw4::gemm_kernel" and rec["fetch_factor"] == 2.0 and rec["write_factor"] == 1.0
    assert rec["hbm_bytes_per_launch"] == round((25000.0 * 2 + 48.0) * 1024)


def test_bench_subcommands_parse():
    """`bench.py tune` and `bench.py prof` take their own options (help exits 0 without a GPU)."""
    for sub in ("tune", "prof", "floor"):
        proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), sub, "--help"], capture_output=True,
                              text=True, timeout=300)
        assert proc.returncode == 0 and f"bench.py {sub}" in proc.stdout, proc.stderr

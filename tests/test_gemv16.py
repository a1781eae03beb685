"""The fp16 small-batch GEMV (tandem_amd/layers/gemv16.py, tw4_gemv_f16): host logic on the CPU,
parity on the GPU against a float32 matmul of the same fp16 operands (mirrors the reference's
tests of python/tandem/layers/triton_gemv.py: every variant and M bucket against F.linear)."""

from __future__ import annotations

import ctypes

import pytest
import torch
from torch import nn

from tandem_amd.layers import gemv16, w4_hip


def test_m_bucket():
    assert [gemv16.m_bucket(m) for m in range(1, 9)] == [1, 2, 4, 4, 8, 8, 8, 8]


def test_default_table_and_install():
    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv_proj = nn.Linear(1024, 3072, bias=False)
            self.o_proj = nn.Linear(1000, 1024, bias=False)  # K not compiled: no entry
            self.other = nn.Linear(1024, 1024, bias=False)

    model = nn.Sequential(Layer())
    table = gemv16.default_table(model)
    assert set(table) == {(3072, 1024, m) for m in (1, 2, 4, 8)}
    assert all(cfg in w4_hip.gemv_f16_configs() for cfg in table.values())
    assert gemv16.install(model, table) == 2 and model.gemv_table is table
    assert gemv16.install(nn.Sequential(Layer()), {}) == 0
    # no table entry / CPU tensors: F.linear, as in the reference
    x = torch.randn(2, 1024)
    assert torch.allclose(gemv16.linear(x, model[0].other.weight, table), x @ model[0].other.weight.T)


def test_gemv_rejects_bad_shapes_before_launch():
    w = torch.zeros(64, 1024, dtype=torch.float16)
    for x in (torch.zeros(9, 1024, dtype=torch.float16), torch.zeros(1, 512, dtype=torch.float16)):
        with pytest.raises(ValueError):
            gemv16.gemv(x, w)
    with pytest.raises(RuntimeError):  # CPU tensors never reach the library
        gemv16.gemv(torch.zeros(1, 1024, dtype=torch.float16), w)


def test_c_abi_argument_errors():
    lib = w4_hip.library()
    p = ctypes.c_void_p(4096)
    assert lib.tw4_gemv_f16(p, p, p, 9, 64, 1024, 2, 32, None) == w4_hip.TW4_EINVAL
    assert "M <= 8" in lib.tw4_last_error().decode()
    assert lib.tw4_gemv_f16(p, p, p, 1, 64, 3072, 2, 32, None) == w4_hip.TW4_EINVAL
    assert "K in" in lib.tw4_last_error().decode()
    assert lib.tw4_gemv_f16(p, p, p, 1, 64, 1024, 3, 32, None) == w4_hip.TW4_ECONFIG


@pytest.mark.gpu
@pytest.mark.parametrize("k", [512, 1024, 2048, 4096])
def test_gemv_every_config(k):
    """Every compiled config and M = 1 .. 8 (buckets 1, 2, 4, 8 and the rows between), N with a
    partial last block, against float32 x @ w^T; fp16 output, so atol / rtol 1e-2."""
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(k)
    n = 1000 + k // 512
    w = (torch.randn(n, k, device=dev, generator=g) * 0.05).half()
    for m in range(1, 9):
        x = torch.randn(m, k, device=dev, generator=g).half()
        ref = x.float() @ w.float().T
        for cfg in w4_hip.gemv_f16_configs():
            y = gemv16.gemv(x, w, *cfg)
            assert y.shape == (m, n) and y.dtype == torch.float16
            err = (y.float() - ref).abs()
            assert bool((err <= 1e-2 + 1e-2 * ref.abs()).all()), (k, m, cfg, float(err.max()))


@pytest.mark.gpu
def test_lm_head_shape_through_linear():
    """The Qwen3-8B fp16 lm_head shape (151936 x 4096) through linear() with a table entry, on the
    v_dot2 form (M = 1, 3) and the matrix-core form (M = 5, 8)."""
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(1)
    w = (torch.randn(151936, 4096, device=dev, generator=g) * 0.02).half()
    table = {(151936, 4096, 1): (2, 32), (151936, 4096, 4): (2, 32), (151936, 4096, 8): (32, 32)}
    for m in (1, 3, 5, 8):  # M = 5, 8: the matrix-core form
        x = torch.randn(m, 4096, device=dev, generator=g).half()
        y = gemv16.linear(x, w, table)
        ref = x.float() @ w.float().T
        err = (y.float() - ref).abs()
        assert bool((err <= 1e-2 + 1e-2 * ref.abs()).all()), (m, float(err.max()))


@pytest.mark.gpu
def test_out_and_weight_arguments_are_checked():
    """A caller's ``out`` of the wrong shape, dtype or layout and a strided norm weight are refused
    before any launch (a too-small ``out`` would otherwise be written past its end)."""
    from tandem_amd.layers import norm

    x = torch.randn(2, 1024, device="cuda", dtype=torch.float16)
    w = torch.randn(64, 1024, device="cuda", dtype=torch.float16)
    for bad in (torch.empty(2, 32, device="cuda", dtype=torch.float16),
                torch.empty(2, 64, device="cuda", dtype=torch.float32),
                torch.empty(64, 2, device="cuda", dtype=torch.float16).t()):
        with pytest.raises(RuntimeError, match="out must be"):
            gemv16.gemv(x, w, out=bad)
    good = torch.empty(2, 64, device="cuda", dtype=torch.float16)
    assert gemv16.gemv(x, w, out=good) is good
    nw = torch.ones(2048, device="cuda", dtype=torch.float16)[::2]  # 1024 values, stride 2
    with pytest.raises(RuntimeError, match="contiguous float16 weight"):
        norm.rms_norm(x, nw, 1e-6)
    with pytest.raises(RuntimeError, match="contiguous float16 weight"):
        norm.fused_add_rms_norm(x.clone(), x.clone(), nw, 1e-6)
    with pytest.raises(RuntimeError, match="out must be"):
        norm.rms_norm(x, nw.contiguous(), 1e-6, out=torch.empty(1, 1024, device="cuda", dtype=torch.float16))
    ext = w4_hip.load()
    packed = torch.zeros(64, 128, device="cuda", dtype=torch.int32)
    s = torch.zeros(64, 8, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="contiguous float16 norm weight"):
        ext.w4_decode_norm(x, None, nw, 1e-6, packed, s, s, 0, *w4_hip.decode_configs()[0], 0)

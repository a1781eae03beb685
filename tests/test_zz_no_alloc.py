"""tw4_gemm_noalloc (the GEMM entry point that allocates nothing: split-K scratch in a static device
array) against tw4_gemm with the caller's workspace, through the C ABI: the same kernels, so the same
bits, on two calls in a row, the second with a smaller input; a split that needs more than the static
scratch is refused with an error; and under HIP graph capture with replays against eager calls."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import awq_oracle as o
from tandem_amd.layers import w4_hip

pytestmark = pytest.mark.gpu


def _weights(k, n, seed, interleave=False):
    qw, qz, s, _, _ = o.random_awq(k, n, seed=seed)
    packed, sc, zz = w4_hip.repack(*(torch.from_numpy(a).cuda() for a in (qw, qz, s)), interleave=interleave)
    return packed, sc, zz, o.dequant_exact(qw, qz, s)


def test_noalloc_matches_workspace_entry_point():
    ext = w4_hip.load()
    buf, locks = w4_hip.workspace("cuda")
    rng = np.random.default_rng(77)
    # (K, N, act, M of the first call, M of the second, config with splits). splits = 0 chooses its split
    # within a fixed budget, never from the workspace it is given, so both entry points run the same one.
    cases = [(4096, 6144, 0, 64, 33, (2, 1, 4, 2, 2, 4)),     # every tile split 4 ways
             (12288, 4096, 0, 64, 20, (2, 1, 4, 1, 2, 0)),    # the last partial wave split
             (4096, 2048, 1, 130, 17, (4, 2, 4, 1, 2, 2)),    # SwiGLU epilogue, split 2
             (4096, 1024, 0, 40, 24, (2, 2, 4, 1, 0, 0)),     # resident-x streaming form
             (12288, 4096, 0, 32, 20, (2, 4, 1, 4, 1, 4)),    # x from L2 (stages 1), split 4
             (4096, 2048, 1, 16, 9, (1, 2, 2, 8, 1, 0)),      # stages 1 at decode M, SwiGLU, auto split
             (4096, 2048, 0, 300, 130, (8, 4, 4, 1, 3, 2)),   # both tiles through LDS (stages 3), split 2
             (4096, 2048, 0, 300, 130, (8, 4, 4, 1, 3, 0)),   # stages 3, automatic split (10 ways at M 300)
             (1024, 512, 0, 300, 50, (8, 2, 4, 1, 2, 1))]     # no split
    for k, n, act, m1, m2, cfg in cases:
        packed, s, z, w = _weights(k, n, seed=k + n + act, interleave=bool(act))
        for m in (m1, m2):  # the second call is smaller: stale partials of the first must not leak in
            x = rng.standard_normal((m, k)).astype(np.float16)
            xg = torch.from_numpy(x).cuda()
            want = ext.w4_gemm(xg, packed, s, z, buf, locks, *cfg, act)
            got = ext.w4_gemm_noalloc(xg, packed, s, z, *cfg, act)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (k, n, act, m, cfg)
            ref = o.swiglu_reference(x, w) if act else o.linear(x, w)
            err = np.abs(got.float().cpu().numpy() - ref)
            assert (err <= 0.02 + 0.01 * np.abs(ref)).all(), (k, n, act, m, cfg, float(err.max()))
    assert int(locks.abs().sum()) == 0


def test_noalloc_refuses_a_split_beyond_its_scratch():
    ext = w4_hip.load()
    packed, s, z, _ = _weights(4096, 24576, seed=5)
    x = torch.randn(1024, 4096, device="cuda", dtype=torch.float16)
    # 8 x 96 tiles of 128 x 256 split 8 ways: 8 x 96 x 8 x 32768 floats, far beyond TW4_NOALLOC_FLOATS
    with pytest.raises(RuntimeError, match="static scratch"):
        ext.w4_gemm_noalloc(x, packed, s, z, 8, 4, 4, 1, 2, 8, 0)
    # still usable after: 384 tiles of 32 x 64 split 2 ways fit (1.57 M floats)
    y = ext.w4_gemm_noalloc(x[:32].contiguous(), packed, s, z, 2, 1, 4, 2, 2, 2, 0)
    buf, locks = w4_hip.workspace("cuda")
    assert torch.equal(y, ext.w4_gemm(x[:32].contiguous(), packed, s, z, buf, locks, 2, 1, 4, 2, 2, 2, 0))


def test_automatic_split_does_not_depend_on_the_workspace():
    """splits = 0 with a workspace smaller than the split it picks is refused (TW4_ESPACE), not run
    with fewer splits and other bits; with the full workspace it runs and equals the no-alloc call."""
    ext = w4_hip.load()
    packed, s, z, _ = _weights(4096, 2048, seed=21)
    x = torch.randn(300, 4096, device="cuda", dtype=torch.float16)
    buf, locks = w4_hip.workspace("cuda")
    cfg = (8, 4, 4, 1, 3, 0)  # 24 tiles of 128 x 256, 10 splits: 7.9 M partials
    with pytest.raises(RuntimeError, match="workspace too small"):
        ext.w4_gemm(x, packed, s, z, buf[:1 << 21], locks, *cfg, 0)
    want = ext.w4_gemm(x, packed, s, z, buf, locks, *cfg, 0)
    assert torch.equal(ext.w4_gemm_noalloc(x, packed, s, z, *cfg, 0), want)
    assert int(locks.abs().sum()) == 0


def test_noalloc_graph_replay():
    ext = w4_hip.load()
    packed, s, z, w = _weights(4096, 4096, seed=9)
    x = torch.randn(48, 4096, device="cuda", dtype=torch.float16)
    cfg = (2, 1, 4, 2, 2, 4)
    ext.w4_gemm_noalloc(x, packed, s, z, *cfg, 0)
    torch.cuda.synchronize()
    out = torch.empty(48, 4096, device="cuda", dtype=torch.float16)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ext.w4_gemm_noalloc(x, packed, s, z, *cfg, 0, out=out)
    rng = np.random.default_rng(10)
    for _ in range(3):
        xn = rng.standard_normal((48, 4096)).astype(np.float16)
        x.copy_(torch.from_numpy(xn).cuda())
        graph.replay()
        torch.cuda.synchronize()
        eager = ext.w4_gemm_noalloc(x, packed, s, z, *cfg, 0)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        ref = o.linear(xn, w)
        assert (np.abs(out.float().cpu().numpy() - ref) <= 0.02 + 0.01 * np.abs(ref)).all()

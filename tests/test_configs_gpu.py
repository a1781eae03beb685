"""GPU parity of the benchmark's configurations at their real sizes, through the W4Linear layer and
the gfx950 tables, against the CPU oracle (oracle/awq_oracle.py).

- Qwen3-1.7B's four projections at M = 1, 2, 4, 8 (and gate_up with the SwiGLU epilogue);
- Qwen3-8B at prefill sizes M = 1024 and 4096: the path the table picks (the fused GEMM, or
  dequantize + torch.matmul) and a forced fused-GEMM configuration at M = 4096, each checked on 512
  sampled output features against the oracle's float64 product;
- the whole Qwen3-8B linear stack (36 layers x {qkv, o, gate_up, down}) plus the fp16 lm_head
  (4096 x 151936) at M = 1, 8 and 32: the HIP-graph replay equals the eager sequence of the same
  calls bit for bit, and layer 0's outputs match the oracle.

Tolerances are the reference's layer-level ones (tests/test_awq.py:87-118 of 12vivi/tandem):
atol 0.05 / rtol 0.02, SwiGLU 0.03 / 0.02; every comparison also needs cosine >= 0.9999.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import awq_oracle as o
from parity import check_close
from tandem_amd.layers import awq, gemv16, w4_hip

pytestmark = pytest.mark.gpu

DEV = "cuda"
QWEN3_1_7B = {"qkv": (2048, 4096), "o": (2048, 2048), "gate_up": (2048, 12288), "down": (6144, 2048)}
QWEN3_8B = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}


def gpu(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def awq_layer(k: int, n: int, seed: int, silu: bool = False):
    """A W4Linear holding the oracle's random AutoAWQ tensors, finalized with the gfx950 tables."""
    qweight, qzeros, scales, _, _ = o.random_awq(k, n, seed=seed)
    layer = awq.W4Linear(k, n, 128).to(DEV)
    layer.qweight.copy_(gpu(qweight))
    layer.qzeros.copy_(gpu(qzeros))
    layer.scales.copy_(gpu(scales))
    if silu:
        assert layer.enable_silu_mul()
    layer.finalize(torch.cuda.get_device_name())
    assert layer.kernels is awq.W4_KERNELS[awq.GFX950]
    return layer, (qweight, qzeros, scales)


def sampled_reference(x: np.ndarray, awq_tensors, feats: np.ndarray, n: int, silu: bool) -> np.ndarray:
    """The oracle's float64 output at the sampled output features only: linear on the exact
    weights, or (SwiGLU) silu(gate) * up on the fp16-rounded ones (tests/test_awq.py:80-84)."""
    if not silu:
        return o.linear(x, o.dequant_exact_rows(*awq_tensors, feats))
    half = n // 2
    w = o.dequant_exact_rows(*awq_tensors, np.concatenate([feats, feats + half]))
    return o.silu_and_mul(o.linear(x, w.astype(np.float16)))


@pytest.mark.parametrize("proj,silu", [("qkv", False), ("o", False), ("gate_up", False), ("gate_up", True),
                                       ("down", False)])
def test_qwen3_1_7b_tables(proj, silu):
    """Qwen3-1.7B decode shapes at M = 1, 2, 4, 8 through the table entries (gemv, gemvm, mma,
    mmak, mmap), against the oracle's dequantize-then-matmul."""
    k, n = QWEN3_1_7B[proj]
    layer, t = awq_layer(k, n, seed=170 + k % 97 + n % 89 + silu, silu=silu)
    w_exact = o.dequant_exact(*t)
    rng = np.random.default_rng(171)
    for m in (1, 2, 4, 8):
        key = (n, k, m) + (("silu",) if silu else ())
        assert key in layer.kernels or (n, k, m) in layer.kernels, key
        x = rng.standard_normal((m, k)).astype(np.float16)
        y = layer(gpu(x)).float().cpu().numpy()
        kern = layer.kernel_for(m).split("(")[0]
        if silu:
            check_close(y, o.swiglu_reference(x, w_exact), 0.03, 0.02, (proj, m, layer.decode_entry(m)), kern,
                        f"1.7b {proj}+silu")
        else:
            check_close(y, o.linear(x, w_exact), 0.05, 0.02, (proj, m, layer.decode_entry(m)), kern, f"1.7b {proj}")


@pytest.mark.parametrize("proj,silu", [("qkv", False), ("o", False), ("gate_up", True), ("down", False)])
def test_qwen3_8b_prefill_sizes(proj, silu):
    """Qwen3-8B at M = 1024 and 4096 through the table (the fused GEMM, or dequantize + hipBLASLt
    where the table says so) and a forced fused-GEMM configuration at M = 4096, on 512 sampled
    output features against the oracle's float64 product."""
    k, n = QWEN3_8B[proj]
    layer, t = awq_layer(k, n, seed=180 + len(proj), silu=silu)
    n_out = n // 2 if silu else n
    rng = np.random.default_rng(181)
    feats = np.sort(rng.choice(n_out, size=512, replace=False))
    key = (n, k) + (("silu",) if silu else ())
    table = layer.gemm_kernels.get(key, awq.DEFAULT_GEMM)
    buf, locks = w4_hip.workspace(DEV)
    ext = w4_hip.load()
    for m in (1024, 4096):
        x = rng.standard_normal((m, k)).astype(np.float16)
        xg = gpu(x)
        ref = sampled_reference(x, t, feats, n, silu)
        runs = [("table", awq.pick_gemm(table, m), layer(xg))]
        if m == 4096:  # the fused path at prefill size: x through the LDS ring, and both tiles through LDS
            for cfg in ((8, 2, 4, 1, 2, 1), (8, 4, 4, 2, 3, 1), (16, 4, 4, 1, 3, 0)):
                runs.append(("forced gemm", cfg, ext.w4_gemm(xg, layer.packed, layer.scales, layer.zeros, buf, locks,
                                                             *cfg, int(silu))))
        for what, cfg, y in runs:
            assert y.shape == (m, n_out)
            got = y[:, torch.from_numpy(feats).to(DEV)].float().cpu().numpy()
            kern = "dequant+matmul" if cfg is None else ("mma" if cfg[0] == "mma" else f"gemm s{cfg[4]}")
            check_close(got, ref, 0.03 if silu else 0.05, 0.02, (proj, m, what, cfg), kern,
                        f"{proj}{'+silu' if silu else ''}")
        del xg, runs
    torch.cuda.synchronize()
    assert int(locks.abs().sum()) == 0


# ------------------------------------------------------------- the full decode-step stack
LAYERS = 36
HEAD = (151936, 4096)  # vocabulary x hidden, fp16


@pytest.fixture(scope="module")
def stack():
    """36 layers of random AutoAWQ weights (uniform int4 q and z, scales U[0.001, 0.02]) on the GPU,
    finalized with the gfx950 tables (gate_up with the SwiGLU epilogue, as the model runs it),
    layer 0's AutoAWQ tensors kept on the host for the oracle, and a random fp16 lm_head."""
    g = torch.Generator(device=DEV).manual_seed(1234)
    layers, host0 = [], {}
    for li in range(LAYERS):
        layer = {}
        for proj, (k, n) in QWEN3_8B.items():
            lin = awq.W4Linear(k, n, 128).to(DEV)
            lin.qweight.copy_(torch.randint(-2**31, 2**31 - 1, lin.qweight.shape, device=DEV, dtype=torch.int32,
                                            generator=g))
            lin.qzeros.copy_(torch.randint(-2**31, 2**31 - 1, lin.qzeros.shape, device=DEV, dtype=torch.int32,
                                           generator=g))
            lin.scales.copy_((torch.rand(lin.scales.shape, device=DEV, generator=g) * 0.019 + 0.001).half())
            if li == 0:
                host0[proj] = (lin.qweight.cpu().numpy(), lin.qzeros.cpu().numpy(), lin.scales.cpu().numpy())
            if proj == "gate_up":
                assert lin.enable_silu_mul()
            lin.finalize(torch.cuda.get_device_name())
            layer[proj] = lin
        layers.append(layer)
    head = (torch.randn(HEAD, device=DEV, dtype=torch.float16, generator=g) * 0.02)
    table = gemv16.table_for(torch.device(DEV), torch.nn.Module())
    torch.cuda.synchronize()
    yield layers, host0, head, table
    del layers, head
    torch.cuda.empty_cache()


@pytest.mark.parametrize("m", [1, 8, 32])
def test_full_stack_graph_equals_eager(stack, m):
    """The whole step's 144 W4A16 linears and the fp16 lm_head, captured in one HIP graph: every
    replay (with eager work and a synchronization in between) reproduces the eager outputs bit for
    bit, and layer 0's four outputs and the head's match the oracle."""
    layers, host0, head, table = stack
    rng = np.random.default_rng(300 + m)
    x_np = {k: rng.standard_normal((m, k)).astype(np.float16) for k in (4096, 12288)}
    xs = {k: gpu(v) for k, v in x_np.items()}

    def step():
        outs = [layer[proj](xs[k]) for layer in layers for proj, (k, _) in QWEN3_8B.items()]
        outs.append(gemv16.linear(xs[4096], head, table))
        return outs

    eager = [t.clone() for t in step()]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        step()  # warm-up on the capture stream
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        captured = step()
    for rep in range(3):
        for t in captured:
            t.fill_(float("nan"))  # a replay that skips an output cannot pass
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        bad = [i for i, (a, b) in enumerate(zip(captured, eager)) if not torch.equal(a, b)]
        assert not bad, (m, rep, bad[:8])
        _ = torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)  # eager work between replays
    for i, (proj, (k, n)) in enumerate(QWEN3_8B.items()):
        silu = proj == "gate_up"
        n_out = n // 2 if silu else n
        feats = np.sort(rng.choice(n_out, size=min(n_out, 1024), replace=False))
        ref = sampled_reference(x_np[k], host0[proj], feats, n, silu)
        got = eager[i][:, torch.from_numpy(feats).to(DEV)].float().cpu().numpy()
        check_close(got, ref, 0.03 if silu else 0.05, 0.02, ("layer 0", proj, m),
                    layers[0][proj].kernel_for(m).split("(")[0], f"stack {proj}", m)
    rows = np.sort(rng.choice(HEAD[0], size=2048, replace=False))
    w_rows = head[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    check_close(eager[-1][:, torch.from_numpy(rows).to(DEV)].float().cpu().numpy(), o.linear(x_np[4096], w_rows),
                0.02, 0.01, ("lm_head", m), "gemv16", "lm_head", m)

"""Benchmark of the MI355X AWQ W4A16 linear path on Qwen3-8B shapes (one GPU).

    python bench.py [--steps K] [--warmup W] [--m 1] [--layers 36] [--no-cpu] [--no-detail]
    python bench.py --sweep [--sweep-out FILE]
    python bench.py tune [--model qwen3-8b] [--ms 1,4,8,16] [--kinds gemv,mma] ...
    python bench.py prof [--proj gate_up] [--m 1] [--launches 40] ...  |  prof --summarize ...
    python bench.py floor

One step = one decode token's W4A16 linears of the whole Qwen3-8B stack: 36 layers x {qkv
(K 4096, N 6144), o (4096, 4096), gate_up (4096, 24576), down (12288, 4096)} at M = 1, launched
back to back from one HIP graph through the product's own W4Linear.forward dispatch. Every layer has
its own random int4 weights (3.6 GB of tile-layout weights, far beyond the 256 MB Infinity Cache),
so every call streams its weights from HBM; inputs are resident in HBM before timing starts.

value = whole-step algorithmic HBM bytes / time (GB/s), with the per-call byte count
    B = N K / 2 + N (K/128) 2 + N (K/128) / 2 + 2 M K + 2 M N
(int4 weights, fp16 scales, int4 zeros, fp16 x and y). The JSON line adds:
  roofline      the dominant kernel (gate_up at the benchmark's M) timed alone with HIP events
                on its own stream, against MI355X's 8 TB/s HBM peak; beside it the kernel-only
                time of the committed rocprofv3 summary (profiles/roofline_gate_up_m1.json) and the
                fraction that gives; `traffic` from that summary's FETCH_SIZE / WRITE_SIZE counters
                and the plain-read floor at the same byte count (tw4_read_probe, see read_floor)
  cpu_baseline  the reference's fallback (dequantize the whole weight every call, then one matmul;
                oracle/torch_fallback.py) in torch on this host's cores, on Qwen3-0.6B's qkv at M = 1
                (the reference's CPU-runnable config) and on one Qwen3-8B layer at the benchmark's M:
                fp16 and fp32 products, and the matmul alone on a pre-dequantized weight
  detail        per projection and M in {1, 8, 32}: us/call, GB/s, % of peak, TFLOP/s, the kernel
                that ran, its parity against dequantize + torch.matmul on the same x (max |err| /
                max |ref| and cosine; parity_vs_dense holds the worst of them), and at M = 32 that
                comparator's time
  full_stack    the whole decode step of the linears plus the fp16 lm_head (4096 x 151936, through
                layers/gemv16.py's table: the HIP fp16 GEMV where it has an entry, else F.linear),
                M in {1, 8, 32}: us per step and GB/s
  decode_step   tandem_amd.model's decode step replayed from the bucketed HIP graphs of
                tandem_amd.decode_graph: norms, SwiGLU gate_up, lm_head and a ONE-TOKEN ATTENTION
                STAND-IN (no KV cache, no RoPE: the step's launch sequence, not a full model step),
                M in {1, 8, 32}: us per step, tokens/s, GB/s of the step's weight bytes

--sweep times every single-linear configuration of the benchmark's configs instead (Qwen3-0.6B
qkv at M = 1; Qwen3-8B's four shapes at M in {1, 4, 8, 16} and {24, 32, 64, 256, 1024, 4096};
Qwen3-1.7B's four shapes at M in {1, 4, 8}): one JSON line per (shape, M) with us/call, GB/s,
TFLOP/s, % of the roofline max(B / 8 TB/s, 2 M N K / 2.5 PFLOP/s), the kernel that ran, and past
M = 16 the dequantize + torch.matmul comparator. Each shape rotates over enough weight copies
(>= 1 GB) that every call streams from HBM.

`tune` times every compiled configuration of the chosen kernels per (shape, M) and prints the
fastest (how layers/w4_tables.py was measured). `prof` is a fixed eager launch sequence for
hardware-counter runs under rocprofv3, and summarizes their CSV files (see prof_main). `floor` times
the plain-read ceiling (tw4_read_probe) at each projection's byte count (see read_floor).
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, AMD public spec
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, AMD public spec
QWEN3_8B = (("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 24576), ("down", 12288, 4096))
QWEN3_1_7B = (("qkv", 2048, 4096), ("o", 2048, 2048), ("gate_up", 2048, 12288), ("down", 6144, 2048))
SWEEP = ((("Qwen3-0.6B", "qkv", 1024, 4096), (1,)),) + tuple(
    (("Qwen3-8B", p, k, n), (1, 4, 8, 16, 24, 32, 64, 256, 1024, 4096)) for p, k, n in QWEN3_8B) + tuple(
    (("Qwen3-1.7B", p, k, n), (1, 4, 8)) for p, k, n in QWEN3_1_7B)
LM_HEAD = (4096, 151936)  # Qwen3-8B vocabulary x hidden, fp16
ROOFLINE_PROFILE = os.path.join(ROOT, "profiles", "roofline_gate_up_m1.json")


def call_bytes(m: int, k: int, n: int) -> int:
    g = k // 128
    return n * k // 2 + n * g * 2 + n * g // 2 + 2 * m * k + 2 * m * n


# ------------------------------------------------------------------------------ shared helpers
def random_linear(torch, awq, k: int, n: int, dev, g, silu: bool = False):
    """One W4Linear with random AutoAWQ weights (uniform int4 q and z, fp16 scales in [0.001, 0.02]),
    repacked by the product's finalize."""
    lin = awq.W4Linear(k, n, 128).to(dev)
    lin.qweight.copy_(torch.randint(-2**31, 2**31 - 1, lin.qweight.shape, device=dev, dtype=torch.int32, generator=g))
    lin.qzeros.copy_(torch.randint(-2**31, 2**31 - 1, lin.qzeros.shape, device=dev, dtype=torch.int32, generator=g))
    lin.scales.copy_((torch.rand(lin.scales.shape, device=dev, generator=g) * 0.019 + 0.001).half())
    if silu:
        lin.enable_silu_mul()
    lin.finalize(torch.cuda.get_device_name(dev))
    return lin


def make_layers(torch, awq, n_layers: int, dev, seed: int = 0):
    """Every projection of every layer with its own random weights."""
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = [{proj: random_linear(torch, awq, k, n, dev, g) for proj, k, n in QWEN3_8B} for _ in range(n_layers)]
    torch.cuda.synchronize()
    return layers


def graph_of(torch, fn, stream):
    """Capture fn() (after one eager warm-up) into a HIP graph on `stream`."""
    with torch.cuda.stream(stream):
        fn()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    return graph


def time_graph(torch, graph, stream, reps: int) -> float:
    """Seconds per replay, HIP events recorded on the replay stream."""
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        graph.replay()
        t0.record(stream)
        for _ in range(reps):
            graph.replay()
        t1.record(stream)
    t1.synchronize()
    return t0.elapsed_time(t1) / 1e3 / reps


def kernel_of(awq, lin, m: int) -> str:
    """Which kernel W4Linear.forward runs for M (the same lookups as the forward)."""
    return lin.kernel_for(m)


def parity_vs_dense(torch, lin, x) -> dict:
    """The fused output against the dequantize-then-fp16-matmul path on the same x (HIP dequant, then
    torch.matmul, as the reference's bench compares, benchmarks/bench_w4_gemm.py:84-92): max_rel =
    max |fused - dense| / max |dense| and the cosine similarity, in float64; outside any timed region."""
    a = lin(x).double()
    b = lin._dense(x).double()
    rel = float((a - b).abs().max() / b.abs().max().clamp_min(1e-6))
    cos = float((a * b).sum() / (a.norm() * b.norm()).clamp_min(1e-30))
    return {"max_rel_vs_dense": float(f"{rel:.3g}"), "cos_vs_dense": round(cos, 7)}


# ------------------------------------------------------------------------------------ sweep
def sweep(torch, awq, dev, stream, out_path: str) -> int:
    """Per (shape, M): us/call over C weight copies (>= 1 GB in all) replayed from one HIP graph."""
    g = torch.Generator(device=dev).manual_seed(0)
    for (model, proj, k, n), ms in SWEEP:
        copies = min(512, max(2, -(-(1 << 30) // (n * k // 2))))
        lins = [random_linear(torch, awq, k, n, dev, g) for _ in range(copies)]
        for m in ms:
            x = torch.randn(m, k, device=dev, dtype=torch.float16)
            gr = graph_of(torch, lambda: [lin(x) for lin in lins], stream)
            est = time_graph(torch, gr, stream, reps=1)  # one replay, to size the timed run to ~20 ms
            us = time_graph(torch, gr, stream, reps=max(2, min(50, int(0.02 / est)))) / copies * 1e6
            del gr
            b, f = call_bytes(m, k, n), 2 * m * k * n
            roof_us = max(b / HBM_PEAK_GBS / 1e3, f / FP16_PEAK_TFLOPS / 1e6)
            rec = {"model": model, "proj": proj, "K": k, "N": n, "M": m, "us": round(us, 2),
                   "GBps": round(b / us / 1e3, 1), "pct_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS * 100, 1),
                   "TFLOPs": round(f / us / 1e6, 2), "bound": "hbm" if b / HBM_PEAK_GBS / 1e3 >= roof_us else "mfma",
                   "pct_roofline": round(roof_us / us * 100, 1), "kernel": kernel_of(awq, lins[0], m)}
            if m > 16:  # the dequantize-then-fp16-GEMM comparator (HIP dequant + torch.matmul)
                sub = lins[:min(copies, 16)]
                dg = graph_of(torch, lambda: [lin._dense(x) for lin in sub], stream)
                rec["dequant_matmul_us"] = round(time_graph(torch, dg, stream, reps=2) / len(sub) * 1e6, 2)
                rec["speedup_vs_dequant_matmul"] = round(rec["dequant_matmul_us"] / us, 2)
                del dg
            line = json.dumps(rec)
            print(line, flush=True)
            if out_path:
                with open(out_path, "a", encoding="utf-8") as fo:
                    fo.write(line + "\n")
            del x
        del lins
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return 0


# ------------------------------------------------------------------------- plain-read floor
FLOOR_WORKGROUPS = (256, 512, 1024, 2048, 4096)
FLOOR_ORDERS = (False, True)  # grid-stride, chunked
FLOOR_DEPTHS = (1, 2, 8)      # loads issued per lane before any is used


def read_floor(torch, dev, stream, nbytes: int) -> dict:
    """The plain-read ceiling at one launch size: tw4_read_probe reading `nbytes` per launch, launches
    back to back from one HIP graph over distinct slices of a >= 1 GB buffer (the decode kernels' own
    regime), at the best of FLOOR_DEPTHS x FLOOR_ORDERS x FLOOR_WORKGROUPS; us per launch and GB/s."""
    from tandem_amd.layers import w4_hip

    per = -(-nbytes // 256) * 256
    copies = max(2, -(-(1 << 30) // per))
    buf = torch.empty(copies * per // 2, dtype=torch.float16, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    slices = [buf[i * per // 2:i * per // 2 + nbytes // 2] for i in range(copies)]
    best = None
    for depth in FLOOR_DEPTHS:
        for chunked in FLOOR_ORDERS:
            for wg in FLOOR_WORKGROUPS:
                g = graph_of(torch, lambda: [w4_hip.read_probe(v, sink, wg, chunked, depth) for v in slices], stream)
                us = time_graph(torch, g, stream, reps=max(3, 200 // copies)) / copies * 1e6
                del g
                if best is None or us < best[0]:
                    best = (us, wg, chunked, depth)
    del buf, slices
    return {"bytes": nbytes, "us": round(best[0], 3), "GBps": round(nbytes / best[0] / 1e3, 1),
            "pct_hbm_peak": round(nbytes / best[0] / 1e3 / HBM_PEAK_GBS * 100, 1), "workgroups": best[1],
            "order": "chunked" if best[2] else "grid-stride", "inflight": best[3], "launches_per_graph": copies}


def floor_main(argv=None) -> int:
    """The plain-read floor at every Qwen3-8B projection's M = 1 byte count and at 1 GB (see read_floor);
    one JSON line per size."""
    ap = argparse.ArgumentParser(prog="bench.py floor", description=floor_main.__doc__.split("\n")[0])
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="kernel-only times of a rocprofv3 --kernel-trace run of `bench.py floor`, per size and "
                         "workgroup count")
    a = ap.parse_args(argv)
    if a.summarize_trace:
        print(json.dumps(summarize_floor_trace(a.summarize_trace), indent=1))
        return 0
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    for name, nbytes in [(p, call_bytes(1, k, n)) for p, k, n in QWEN3_8B] + [("1GiB", 1 << 30)]:
        print(json.dumps({"what": name, **read_floor(torch, dev, stream, nbytes)}), flush=True)
    return 0


def summarize_floor_trace(path: str) -> list[dict]:
    """The read-probe dispatches of a `bench.py floor` kernel trace, in launch order, cut into one run
    per (size, depth, order, workgroup count) as floor_main issues them (sizes in QWEN3_8B order then 1 GiB,
    each over FLOOR_DEPTHS x FLOOR_ORDERS x FLOOR_WORKGROUPS): per run the average and minimum kernel-only
    time and GB/s."""
    with open(path, newline="", encoding="utf-8") as f:
        rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), int(r["Grid_Size_X"]),
                       r["Kernel_Name"]) for r in csv.DictReader(f) if "read_probe" in r["Kernel_Name"])
    runs: list[list[tuple[int, int, int]]] = []
    for r in rows:
        if not runs or runs[-1][-1][2] != r[2] or runs[-1][-1][3] != r[3]:
            runs.append([])
        runs[-1].append(r)
    sizes = [(p, call_bytes(1, k, n)) for p, k, n in QWEN3_8B] + [("1GiB", 1 << 30)]
    out = []
    per_size = len(FLOOR_WORKGROUPS) * len(FLOOR_ORDERS) * len(FLOOR_DEPTHS)
    for i, run in enumerate(runs):
        what, nbytes = sizes[i // per_size] if i // per_size < len(sizes) else ("?", 0)
        depth = FLOOR_DEPTHS[(i % per_size) // (len(FLOOR_WORKGROUPS) * len(FLOOR_ORDERS))]
        ns = [e - s for s, e, _, _ in run]
        avg, best = sum(ns) / len(ns), min(ns)
        out.append({"what": what, "bytes": nbytes, "workgroups": run[0][2] // 256,
                    "order": "chunked" if "chunked" in run[0][3] else "grid-stride", "inflight": depth,
                    "dispatches": len(ns),
                    "avg_us": round(avg / 1e3, 3), "min_us": round(best / 1e3, 3),
                    "avg_GBps": round(nbytes / avg, 1) if nbytes else None})
    return out


# ----------------------------------------------------------------------------- CPU baseline
def _cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        return next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), "")
    except (OSError, subprocess.SubprocessError):
        return ""


def cpu_baseline(m: int) -> dict:
    """The reference's fallback restated in torch (oracle/torch_fallback.py: unpack + fp16 dequant of the
    whole weight every call, then one product; python/tandem/layers/awq.py:282-286) on this host:
    Qwen3-0.6B's qkv (K 1024, N 4096) at M = 1 and one Qwen3-8B layer's four projections at M, each
    with the product in fp16 and in fp32 and the pre-dequantized matmul alone; 3 warm-ups, then the
    median of 10 timed calls. `value` is the 8B layer's faster variant (fp16 or fp32 product) in GB/s
    of the same algorithmic bytes as the GPU figure."""
    import numpy as np
    import torch

    from oracle import awq_oracle as o
    from oracle import torch_fallback as tf

    cores = len(os.sched_getaffinity(0))
    threads = cores  # every core this process may run on
    torch.set_num_threads(threads)

    def median_s(fn) -> float:
        for _ in range(3):
            fn()
        ts = []
        for _ in range(10):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return statistics.median(ts)

    def workload(shapes, mm, seed):
        data = []
        for i, (k, n) in enumerate(shapes):
            qw, qz, s, _, _ = o.random_awq(k, n, seed=seed + i)
            x = torch.from_numpy(np.random.default_rng(seed + i).standard_normal((mm, k)).astype(np.float16))
            data.append((x, torch.from_numpy(qw), torch.from_numpy(qz), torch.from_numpy(s)))
        return data

    t_start = time.perf_counter()
    res = {}
    for label, shapes, mm in (("qwen3_0.6b_qkv_m1", [(1024, 4096)], 1),
                              (f"qwen3_8b_layer_m{m}", [(k, n) for _, k, n in QWEN3_8B], m)):
        data = workload(shapes, mm, seed=1000)
        b = sum(call_bytes(mm, k, n) for k, n in shapes)
        rec = {}
        for variant, dt in (("fp16", torch.float16), ("fp32", torch.float32)):
            sec = median_s(lambda: [tf.fallback_linear(x, qw, qz, s, dt) for x, qw, qz, s in data])
            rec[variant] = {"ms": round(sec * 1e3, 2), "GBps": round(b / sec / 1e9, 3)}
        pre = [(x, tf.dequant_kn(qw, qz, s)) for x, qw, qz, s in data]
        sec = median_s(lambda: [x @ w for x, w in pre])
        rec["matmul_only_predequantized_fp16"] = {"ms": round(sec * 1e3, 3), "GBps": round(b / sec / 1e9, 3)}
        res[label] = rec
    layer = res[f"qwen3_8b_layer_m{m}"]
    best = min(("fp16", "fp32"), key=lambda v: layer[v]["ms"])
    main = layer[best]
    return {"value": main["GBps"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the reference's fallback (AWQ unpack + fp16 dequant of the whole weight every call, then "
                      f"one matmul) in torch on {threads} threads: one Qwen3-8B layer's qkv, o, gate_up and down at "
                      f"M={m} (value: the faster product, {best}) and Qwen3-0.6B qkv at M=1; 3 warm-ups + median "
                      f"of 10 calls "
                      f"each; host {_cpu_model()} ({cores} cores visible); "
                      f"{time.perf_counter() - t_start:.1f} s in all",
            "ms_per_call": main["ms"], "variants": res}


# ------------------------------------------------------------------------------ decode step
def decode_step(torch, dev) -> dict:
    """tandem_amd.model's Qwen3-8B decode step (embedding, 36 x {add + RMSNorm, qkv, ONE-TOKEN
    ATTENTION STAND-IN, o, add + RMSNorm, gate_up with SwiGLU, down}, final add + RMSNorm, fp16
    lm_head) replayed from tandem_amd.decode_graph's bucket graphs, random AWQ weights."""
    from tandem_amd import decode_graph, model as tmodel
    from tandem_amd.loader import QuantConfig

    cfg = tmodel.QWEN3_8B
    with torch.device(dev):
        mdl = tmodel.DecoderModel(cfg, QuantConfig("awq", 4, 128))
    mdl.half()
    tmodel.init_random(mdl, seed=7)
    tmodel.prepare(mdl, dev, torch.cuda.get_device_name(dev))
    runner = decode_graph.DecodeGraphRunner(mdl, max_bs=32, device=dev)
    h, i, v = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qkv_n = (cfg.num_heads + 2 * cfg.num_kv_heads) * cfg.head_dim
    out = {"what": "linears + norms + lm_head around a one-token attention stand-in (no KV cache, no RoPE)"}
    for bs in (1, 8, 32):
        runner.run(list(range(bs)))
        graph = runner.graphs[bs]
        cur = torch.cuda.current_stream(dev)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(3):
            graph.replay()
        t0.record(cur)
        for _ in range(20):
            graph.replay()
        t1.record(cur)
        t1.synchronize()
        us = t0.elapsed_time(t1) / 20 * 1e3
        b = cfg.num_layers * (call_bytes(bs, h, qkv_n) + call_bytes(bs, cfg.num_heads * cfg.head_dim, h)
                              + call_bytes(bs, h, 2 * i) - bs * 2 * i + call_bytes(bs, i, h)) + 2 * v * h
        out[f"m{bs}"] = {"us_per_step": round(us, 1), "tokens_per_s": round(bs / us * 1e6, 1),
                         "GBps": round(b / us / 1e3, 1), "pct_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS * 100, 1)}
    del runner, mdl
    torch.cuda.synchronize()
    return out


# -------------------------------------------------------------------------------- headline
def parse(argv=None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--m", type=int, default=1, help="tokens per call (decode batch)")
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-detail", action="store_true", help="skip the per-projection sweep")
    ap.add_argument("--sweep", action="store_true", help="time every (shape, M) of the configs; JSON line each")
    ap.add_argument("--sweep-out", default="", help="also append the sweep's JSON lines to this file")
    ap.add_argument("--step-only", action="store_true",
                    help="only the decode_step section (for profiling the whole step); prints its JSON")
    return ap.parse_args(argv)


def roofline_profile(m: int) -> dict:
    """The committed rocprofv3 summary of the dominant kernel (kernel-only time, HBM counters)."""
    if m != 1 or not os.path.exists(ROOFLINE_PROFILE):
        return {}
    with open(ROOFLINE_PROFILE, encoding="utf-8") as f:
        return json.load(f)


def main(argv=None) -> int:
    a = parse(argv)
    if a.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {a.gpus} is not supported (the W4A16 linear runs on one GPU's "
              "share of the weights; sharding splits N or K across GPUs outside this op)", file=sys.stderr)
        return 2
    import torch

    from tandem_amd.layers import awq, w4_hip

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w4_hip.load()
    if a.step_only:
        print(json.dumps({"decode_step": decode_step(torch, dev)}), flush=True)
        return 0
    if a.sweep:
        return sweep(torch, awq, dev, torch.cuda.Stream(dev), a.sweep_out)
    m = a.m
    layers = make_layers(torch, awq, a.layers, dev)
    stream = torch.cuda.Stream(dev)
    xs = {4096: torch.randn(m, 4096, device=dev, dtype=torch.float16),
          12288: torch.randn(m, 12288, device=dev, dtype=torch.float16)}

    def step():
        for layer in layers:
            for proj, k, n in QWEN3_8B:
                layer[proj](xs[k])

    step_graph = graph_of(torch, step, stream)
    step_bytes = a.layers * sum(call_bytes(m, k, n) for _, k, n in QWEN3_8B)
    step_flops = a.layers * sum(2 * m * k * n for _, k, n in QWEN3_8B)
    with torch.cuda.stream(stream):
        for _ in range(a.warmup):
            step_graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t0.record(stream)
        for _ in range(a.steps):
            step_graph.replay()
        t1.record(stream)
    torch.cuda.synchronize()
    step_s = t0.elapsed_time(t1) / 1e3 / a.steps
    value = step_bytes / step_s / 1e9

    # dominant kernel: gate_up alone, one launch per layer, HIP events on its stream
    gate_graph = graph_of(torch, lambda: [layer["gate_up"](xs[4096]) for layer in layers], stream)
    gate_s = time_graph(torch, gate_graph, stream, reps=max(10, a.steps // 4)) / a.layers
    gate_bytes = call_bytes(m, 4096, 24576)
    achieved = gate_bytes / gate_s / 1e9
    prof = roofline_profile(m)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": prof.get("hbm_bytes_per_launch"),
                "kernel": f"gate_up (K 4096, N 24576) M={m}: {kernel_of(awq, layers[0]['gate_up'], m)}",
                "us_per_launch": round(gate_s * 1e6, 3), "algorithmic_bytes_per_launch": gate_bytes}
    if prof.get("kernel_us"):
        roofline["profile_kernel_us"] = prof["kernel_us"]
        roofline["profile_frac"] = round(gate_bytes / prof["kernel_us"] / 1e3 / HBM_PEAK_GBS, 4)
        roofline["profile"] = os.path.relpath(ROOFLINE_PROFILE, ROOT)
    del gate_graph
    floor = read_floor(torch, dev, stream, gate_bytes)
    roofline["read_floor"] = {**floor, "kernel_over_floor": round(gate_s * 1e6 / floor["us"], 3)}

    detail = {}
    if not a.no_detail:
        for mm in (1, 8, 32):
            xd = {4096: torch.randn(mm, 4096, device=dev, dtype=torch.float16),
                  12288: torch.randn(mm, 12288, device=dev, dtype=torch.float16)}
            for proj, k, n in QWEN3_8B:
                g = graph_of(torch, lambda: [layer[proj](xd[k]) for layer in layers], stream)
                us = time_graph(torch, g, stream, reps=20) / a.layers * 1e6
                del g
                b, f = call_bytes(mm, k, n), 2 * mm * k * n
                rec = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1),
                       "pct_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS * 100, 1),
                       "TFLOPs": round(f / us / 1e6, 2), "kernel": kernel_of(awq, layers[0][proj], mm),
                       **parity_vs_dense(torch, layers[0][proj], xd[k])}
                if mm == 32:  # the dequantize-then-fp16-GEMM comparator (HIP dequant + torch.matmul)
                    dg = graph_of(torch, lambda: [layer[proj]._dense(xd[k]) for layer in layers[:8]], stream)
                    rec["dequant_matmul_us"] = round(time_graph(torch, dg, stream, reps=10) / 8 * 1e6, 2)
                    rec["speedup_vs_dequant_matmul"] = round(rec["dequant_matmul_us"] / us, 2)
                    del dg
                detail[f"{proj}_m{mm}"] = rec
            torch.cuda.synchronize()

    full = {}
    if not a.no_detail:
        from tandem_amd.layers import gemv16

        hk, hn = LM_HEAD
        head = (torch.randn(hn, hk, device=dev, dtype=torch.float16) * 0.02)
        table = gemv16.table_for(dev, torch.nn.Module())
        for mm in (1, 8, 32):
            xd = {4096: torch.randn(mm, 4096, device=dev, dtype=torch.float16),
                  12288: torch.randn(mm, 12288, device=dev, dtype=torch.float16)}

            def full_step():
                for layer in layers:
                    for proj, k, n in QWEN3_8B:
                        layer[proj](xd[k])
                gemv16.linear(xd[4096], head, table)

            g = graph_of(torch, full_step, stream)
            us = time_graph(torch, g, stream, reps=10) * 1e6
            del g
            b = a.layers * sum(call_bytes(mm, k, n) for _, k, n in QWEN3_8B) + 2 * hn * hk + 2 * mm * (hk + hn)
            full[f"m{mm}"] = {"us_per_step": round(us, 1), "GBps": round(b / us / 1e3, 1),
                              "pct_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS * 100, 1), "step_bytes": b,
                              "lm_head": "gemv16" if gemv16.entry(xd[4096], head, table) else "F.linear"}
        del head
        torch.cuda.synchronize()

    step = {} if a.no_detail else decode_step(torch, dev)

    cpu = None if a.no_cpu else cpu_baseline(m)
    line = {
        "metric": "W4A16 us/call + achieved HBM GB/s (% peak), Qwen3-8B shapes, M=1/8/32",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (random int4 weights / zeros, fp16 scales U[0.001, 0.02], x ~ N(0,1))",
        "config": {"workload": f"Qwen3-8B AWQ W4A16 linear stack, one decode step: {a.layers} layers x "
                               f"{{qkv, o, gate_up, down}}, M={m}, one HIP graph", "M": m, "layers": a.layers,
                   "group_size": 128, "shapes_KN": {p: [k, n] for p, k, n in QWEN3_8B},
                   "step_bytes": step_bytes, "step_flops": step_flops},
        "pct_hbm_peak": round(value / HBM_PEAK_GBS * 100, 2),
        "us_per_layer": round(step_s / a.layers * 1e6, 2),
        "roofline": roofline, "cpu_baseline": cpu,
        "parity_vs_dense": {"worst_max_rel": max((r["max_rel_vs_dense"] for r in detail.values()), default=None),
                            "min_cos": min((r["cos_vs_dense"] for r in detail.values()), default=None),
                            "what": "every detail cell's fused output against HIP dequant + torch.matmul (fp16) "
                                    "on the same x"},
        "detail": detail, "full_stack": full, "decode_step": step,
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line), flush=True)
    return 0


# ------------------------------------------------------------------------------------- tune
TUNE_MODELS = {
    "qwen3-8b": {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096),
                 "lm_head": (4096, 151936)},
    "qwen3-1.7b": {"qkv": (2048, 4096), "o": (2048, 2048), "gate_up": (2048, 12288), "down": (6144, 2048),
                   "lm_head": (2048, 151936)},
    "qwen3-0.6b": {"qkv": (1024, 4096), "lm_head": (1024, 151936)},
}
DENSE = ("lm_head",)  # fp16 projections (kinds dense16 / torch16); the others are W4A16


def tune_main(argv=None) -> int:
    """Configuration sweep of the W4A16 kernels, the counterpart of the reference's
    benchmarks/bench_w4.py and bench_w4_gemm.py, which produced its per-GPU tables:

        python bench.py tune --model qwen3-8b --ms 1,4,8,16 --kinds gemv,mma [--out sweep.jsonl]
        python bench.py tune --model qwen3-8b --ms 24,32,64,256 --kinds gemm
        python bench.py tune --model qwen3-8b --projs lm_head --ms 1,2,4,8 --kinds dense16,torch16

    For each projection shape and M, every compiled configuration of each kernel is timed the way the
    reference timed them (benchmarks/bench_gemv.py:35-56): one HIP graph replays `rounds` passes over
    `copies` weight copies whose total size (>= --footprint-mb, default 1 GB) is far beyond the 256 MB
    Infinity Cache, so each call streams its weights from HBM. One JSON record per (shape, M) gives
    us/call and GB/s of the best config of each kind and of every config."""
    import torch

    from tandem_amd.layers import w4_hip

    ap = argparse.ArgumentParser(prog="bench.py tune", description=tune_main.__doc__.split("\n\n")[0])
    ap.add_argument("--model", default="qwen3-8b", choices=sorted(TUNE_MODELS))
    ap.add_argument("--projs", default="", help="comma list of projections (default: all)")
    ap.add_argument("--ms", default="1,4,8,16")
    ap.add_argument("--kinds", default="gemv,mma", help="gemv, gemvm, gemvn, mma, mmak, mmap, gemm, dense")
    ap.add_argument("--splits", default="0,1,2,4,8")
    ap.add_argument("--per-cu", default="1,2,3,4", help="workgroups per CU of the persistent mma (kind mmap)")
    ap.add_argument("--act", action="store_true", help="time the SwiGLU epilogue (gate_up only)")
    ap.add_argument("--footprint-mb", type=float, default=1024.0)
    ap.add_argument("--out", default="")
    a = ap.parse_args(argv)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    ext = w4_hip.load()
    gen = torch.Generator(device=dev).manual_seed(0)
    stream = torch.cuda.Stream(dev)
    kinds = a.kinds.split(",")
    buf, locks = w4_hip.workspace(dev)
    out = open(a.out, "a", encoding="utf-8") if a.out else None

    def time_us(calls, rounds: int = 10, reps: int = 5) -> float:
        """Microseconds per call: a HIP graph of `rounds` passes over `calls`, replayed `reps` times."""
        graph = graph_of(torch, lambda: [c() for _ in range(rounds) for c in calls], stream)
        return time_graph(torch, graph, stream, reps) * 1e6 / (rounds * len(calls))

    def random_weights(k: int, n: int):
        """Uniform random nibbles straight in the tile layout, fp16 scales in [0.001, 0.02], integer zeros."""
        packed = torch.randint(-2**31, 2**31 - 1, (w4_hip.padded_rows(n), k // 8), dtype=torch.int32, device=dev,
                               generator=gen)
        scales = (torch.rand(n, k // 128, device=dev, generator=gen) * 0.019 + 0.001).half()
        zeros = torch.randint(0, 16, (n, k // 128), device=dev, generator=gen).half()
        return packed, scales, zeros

    def emit(proj: str, k: int, n: int, m: int, act: int, copies: int, res: dict, b: int) -> None:
        if not res:
            return
        best = min(res, key=res.get)
        rec = {"model": a.model, "proj": proj, "k": k, "n": n, "m": m, "act": act, "copies": copies,
               "best": list(best), "us": round(res[best], 3), "GBps": round(b / res[best] / 1e3, 1),
               "pct_hbm_peak": round(b / res[best] / 1e3 / HBM_PEAK_GBS * 100, 2),
               "TFLOPs": round(2 * m * k * n / res[best] / 1e6, 2),
               "best_per_kind": {kd: min((v, list(c)) for c, v in res.items() if c[0] == kd)
                                 for kd in {c[0] for c in res}},
               "all": {"/".join(map(str, c)): round(v, 2) for c, v in sorted(res.items(), key=lambda kv: kv[1])}}
        print(json.dumps(rec), flush=True)
        if out:
            out.write(json.dumps(rec) + "\n")

    def attempt(res: dict, key: tuple, calls, rounds: int = 10) -> None:
        try:
            res[key] = time_us(calls, rounds)
        except RuntimeError:  # a configuration the host checks refuse for this shape
            pass

    for proj, (k, n) in TUNE_MODELS[a.model].items():
        if (a.projs and proj not in a.projs.split(",")) or (a.act and proj != "gate_up"):
            continue
        act = int(a.act)
        if (proj in DENSE) != any(kd in kinds for kd in ("dense16", "torch16")):
            continue
        if proj in DENSE:  # fp16 weights [N, K]: the kernel of layers/gemv16.py against F.linear
            from tandem_amd.layers import gemv16

            wbytes = 2 * n * k
            copies = max(1, math.ceil(a.footprint_mb * 1e6 / wbytes))
            wd = [(torch.randn(n, k, device=dev, generator=gen) * 0.02).half() for _ in range(copies)]
            for m in (int(v) for v in a.ms.split(",")):
                x = torch.randn(m, k, device=dev, dtype=torch.float16)
                res = {}
                if "dense16" in kinds:
                    for cfg in w4_hip.gemv_f16_configs():
                        attempt(res, ("dense16", *cfg), [lambda w=w, c=cfg: gemv16.gemv(x, w, *c) for w in wd], 3)
                if "torch16" in kinds:
                    attempt(res, ("torch16",), [lambda w=w: torch.nn.functional.linear(x, w) for w in wd], 3)
                emit(proj, k, n, m, 0, copies, res, wbytes + 2 * m * k + 2 * m * n)
            del wd
            torch.cuda.empty_cache()
            continue
        copies = max(2, math.ceil(a.footprint_mb * 1e6 / call_bytes(0, k, n)))
        ws = [random_weights(k, n) for _ in range(copies)]
        for m in (int(v) for v in a.ms.split(",")):
            x = torch.randn(m, k, device=dev, dtype=torch.float16)
            res = {}
            decode = w4_hip.decode_configs()
            for cfg in w4_hip.mma_configs():  # the decode configs, then the row-tile-wide ones (mma only)
                if cfg not in decode:
                    if "mma" in kinds and m <= 64:
                        attempt(res, ("mma", *cfg), [lambda w=w, c=cfg: ext.w4_mma(x, *w, *c, act) for w in ws])
                    continue
                if "gemv" in kinds and m <= 4:
                    attempt(res, ("gemv", *cfg), [lambda w=w, c=cfg: ext.w4_gemv(x, *w, *c, act) for w in ws])
                if "gemvn" in kinds and m <= 4:  # the GEMV with the add + RMSNorm prologue (tw4_decode_norm)
                    r = torch.randn(m, k, device=dev, dtype=torch.float16)
                    nw = (torch.rand(k, device=dev) + 0.5).half()
                    attempt(res, ("gemvn", *cfg),
                            [lambda w=w, c=cfg: ext.w4_decode_norm(x, r, nw, 1e-6, *w, 0, *c, act) for w in ws])
                if "gemvm" in kinds and m <= 16:
                    attempt(res, ("gemvm", *cfg), [lambda w=w, c=cfg: ext.w4_gemv_mfma(x, *w, *c, act) for w in ws])
                if "mma" in kinds and m <= 64:
                    attempt(res, ("mma", *cfg), [lambda w=w, c=cfg: ext.w4_mma(x, *w, *c, act) for w in ws])
                if "mmap" in kinds and m <= 16:
                    for pc in (int(v) for v in a.per_cu.split(",")):
                        attempt(res, ("mmap", *cfg, pc),
                                [lambda w=w, c=cfg, q=pc: ext.w4_mma_persist(x, *w, *c, q, act) for w in ws])
                if "mmak" in kinds and m <= 16:
                    for sp in (int(v) for v in a.splits.split(",")):
                        if 2 <= sp <= k // 128:
                            attempt(res, ("mmak", *cfg, sp),
                                    [lambda w=w, c=cfg, s=sp: ext.w4_mma_splitk(x, *w, buf, locks, *c, s, act)
                                     for w in ws])
            if "gemm" in kinds:
                for cfg in w4_hip.gemm_configs():
                    for sp in (int(v) for v in a.splits.split(",")):
                        if sp <= (k // 128 + cfg[3] - 1) // cfg[3]:
                            attempt(res, ("gemm", *cfg, sp),
                                    [lambda w=w, c=cfg, s=sp: ext.w4_gemm(x, *w, buf, locks, *c, s, act) for w in ws],
                                    5)
            if "dense" in kinds:  # HIP dequantize + torch.matmul, the unfused comparator
                from tandem_amd.layers import awq

                def dense(w):
                    y = torch.nn.functional.linear(x, awq.w4_dequant(*w, deinterleave=bool(act)))
                    return awq.silu_and_mul(y) if act else y

                attempt(res, ("dense",), [lambda w=w: dense(w) for w in ws[:8]], 3)
            emit(proj, k, n, m, act, copies, res, call_bytes(m, k, n))
        del ws
        torch.cuda.empty_cache()
    if out:
        out.close()
    return 0


# ------------------------------------------------------------------------------------- prof
PROF_SHAPES = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}
COPY_KERNEL_HINT = ("copybuffer",)  # the HIP runtime's device-to-device copy (torch copy_ of one dtype)
LOAD_TIME_KERNELS = ("repack",)     # finalize's kernels: never the kernel a profile is about


def prof_main(argv=None) -> int:
    """A fixed, eager sequence of kernel launches for hardware-counter runs under rocprofv3, and the
    summaries of those runs.

        python bench.py prof [--proj gate_up] [--m 1] [--launches 40] [--copy-mib 256]

    Launches, in order: `copies` torch copies of a --copy-mib MiB float16 buffer (a plain device copy
    of known size: it reads and writes exactly that many bytes, which calibrates FETCH_SIZE and
    WRITE_SIZE), then --launches calls of W4Linear.forward for one Qwen3-8B projection at M, rotating
    over enough weight copies (>= 1 GB) that every call streams its weights from HBM. --read-gb adds a
    streaming calibration before the copies: one torch sum over a --read-gb GB float16 buffer (reads
    only), the plain-read ceiling the decode kernels are held against. A counter run reads, per
    dispatch, the HBM bytes each kernel moved:

        rocprofv3 --pmc FETCH_SIZE -d <dir> -o run --output-format csv -- python3 bench.py prof
        rocprofv3 --pmc WRITE_SIZE -d <dir> -o run --output-format csv -- python3 bench.py prof
        python bench.py prof --summarize <fetch counter_collection.csv> <write counter_collection.csv>

    The summary's kernel is the one the command targets: a tw4 kernel with exactly --launches
    dispatches, never a load-time repack. The same launches give the GEMM's matrix-core utilisation
    (M > 16; --cfg forces one GEMM configuration, mt,nt,warps_n,warps_k,stages,splits, in place of
    the table's, to compare tile and split-K choices on the same shape):

        rocprofv3 --kernel-trace --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_F16 -d <dir> -o run \\
            --output-format csv -- python3 bench.py prof --proj gate_up --m 32 [--cfg 2,1,4,2,2,1]
        python bench.py prof --proj gate_up --m 32 --summarize-mfma <counter_collection.csv>

    MfmaUtil is rocprofiler's derived counter: the SIMDs' summed SQ_VALU_MFMA_BUSY_CYCLES over
    GRBM_GUI_ACTIVE x the number of SIMDs, in percent. SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 is the fp16
    matrix-core work issued, which against 2 M N K shows the padding of the token tiles."""
    ap = argparse.ArgumentParser(prog="bench.py prof", description=prof_main.__doc__.split("\n\n")[0])
    ap.add_argument("--proj", default="gate_up", choices=sorted(PROF_SHAPES))
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--launches", type=int, default=40)
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--copies", type=int, default=3)
    ap.add_argument("--read-gb", type=float, default=0.0, help="plain-read calibration size (0: none)")
    ap.add_argument("--silu", action="store_true", help="gate_up with the SwiGLU epilogue")
    ap.add_argument("--cfg", default="", help="GEMM config mt,nt,warps_n,warps_k,stages,splits (or a ladder's "
                                              "mma rung, mma,warps_k,unroll,ntile) for every M > 16")
    ap.add_argument("--decode", default="", help="decode-table entry kind,args for M <= 16 (e.g. gemv,4,2,2 or "
                                                 "mmap,8,1,2,2), in place of the table's")
    ap.add_argument("--summarize", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--summarize-mfma", metavar="COUNTER_CSV")
    ap.add_argument("--summarize-counters", nargs="+", metavar="COUNTER_CSV",
                    help="per-dispatch medians of every counter of the profiled kernel, over one or more counter "
                         "passes of the same command, with busy shares per XCD (see summarize_counters)")
    ap.add_argument("--probe", type=int, default=0, metavar="WORKGROUPS",
                    help="after the projection's launches, as many launches of the plain-read probe "
                         "(tw4_read_probe, grid-stride) over the projection's algorithmic bytes on this many "
                         "workgroups: the same counters for a kernel that only reads (0: none)")
    ap.add_argument("--kernel", default="", help="--summarize-counters: the kernel whose name contains this "
                                                 "(e.g. read_probe), in place of the projection's")
    a = ap.parse_args(argv)
    k, n = PROF_SHAPES[a.proj]
    if a.summarize_mfma:
        print(json.dumps(summarize_mfma(a.summarize_mfma, a.m, n, k), indent=1))
        return 0
    if a.summarize_counters:
        print(json.dumps(summarize_counters(a.summarize_counters, a.launches, a.kernel), indent=1))
        return 0
    if a.summarize:
        alg = call_bytes(a.m, k, n) - (a.m * n if a.silu else 0)
        print(json.dumps(summarize_traffic(*a.summarize, a.copy_mib, a.copies, a.launches, alg), indent=1))
        return 0
    return prof_run(a)


def prof_run(a: argparse.Namespace) -> int:
    import torch

    from tandem_amd.layers import awq, w4_hip

    if not torch.cuda.is_available():
        print("bench.py prof needs the GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    w4_hip.load()
    if a.read_gb > 0:
        big = torch.ones(int(a.read_gb * 1e9) // 2, device=dev, dtype=torch.float16)
        for _ in range(3):
            big.sum(dtype=torch.float32)
        torch.cuda.synchronize()
        del big
    src = torch.ones(a.copy_mib << 19, device=dev, dtype=torch.float16)
    dst = torch.empty_like(src)
    for _ in range(a.copies):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst

    k, n = PROF_SHAPES[a.proj]
    g = torch.Generator(device=dev).manual_seed(0)
    copies = max(2, -(-(1 << 30) // (n * k // 2)))
    layers = []
    for _ in range(copies):
        lin = random_linear(torch, awq, k, n, dev, g, silu=a.silu and a.proj == "gate_up")
        if a.cfg:  # a per-layer copy: the module-level table is shared by every W4Linear
            key = (n, k) + (("silu",) if lin.silu_mul else ())
            head, *rest = a.cfg.split(",")
            cfg = ("mma", *(int(v) for v in rest)) if head == "mma" else tuple(int(v) for v in a.cfg.split(","))
            lin.gemm_kernels = {**lin.gemm_kernels, key: ((1 << 30, cfg),)}
        if a.decode:
            kind, *args = a.decode.split(",")
            key = (n, k, a.m) + (("silu",) if lin.silu_mul else ())
            lin.kernels = {**lin.kernels, key: (kind, *(int(v) for v in args))}
        layers.append(lin)
    x = torch.randn(a.m, k, device=dev, dtype=torch.float16)
    torch.cuda.synchronize()
    for i in range(a.launches):
        layers[i % copies](x)
    torch.cuda.synchronize()
    kname, probe = kernel_of(awq, layers[0], a.m), ""
    if a.probe > 0:  # the same bytes per launch, read and discarded, rotating over as many copies
        nbytes = (call_bytes(a.m, k, n) - (a.m * n if layers[0].silu_mul else 0) + 15) // 16 * 16
        del layers
        bufs = [torch.ones(nbytes // 4, device=dev, dtype=torch.int32) for _ in range(copies)]
        sink = torch.zeros(4, device=dev, dtype=torch.int32)
        for i in range(a.launches):
            w4_hip.read_probe(bufs[i % copies], sink, a.probe)
        torch.cuda.synchronize()
        probe = f", then {a.launches} read probes of {nbytes} bytes on {a.probe} workgroups"
    print(f"prof: {a.copies} copies of {a.copy_mib} MiB, {a.launches} x {a.proj} (K {k}, N {n}) M={a.m} "
          f"over {copies} weight copies ({kname}), read calibration {a.read_gb} GB{probe}", flush=True)
    return 0


def _per_kernel(path: str, counter: str) -> dict[str, list[tuple[int, float]]]:
    """counter_collection.csv -> {kernel name: [(dispatch id, counter value), ...] in dispatch order}."""
    out: dict[str, list[tuple[int, float]]] = {}
    with open(path, newline="", encoding="utf-8") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") == counter:
                out.setdefault(row["Kernel_Name"], []).append((int(row["Dispatch_Id"]), float(row["Counter_Value"])))
    for v in out.values():
        v.sort()
    return out


def _calibration(per_kernel: dict[str, list[tuple[int, float]]], copies: int) -> tuple[str, list[float]]:
    """The calibration copies: the first `copies` dispatches of the run that are copy kernels."""
    first = sorted((d, name, val) for name, v in per_kernel.items() for d, val in v
                   if any(h in name.lower() for h in COPY_KERNEL_HINT) and "tw4" not in name)[:copies]
    if len(first) < copies or len({name for _, name, _ in first}) != 1:
        raise SystemExit("the counter file does not start with the calibration copies")
    return first[0][1], [val for _, _, val in first]


def target_kernel(names_to_dispatches: dict[str, int], launches: int) -> str | None:
    """The kernel a prof command targets: a tw4 kernel with exactly `launches` dispatches that is not a
    load-time kernel; else the most-dispatched such kernel."""
    cands = {nm: d for nm, d in names_to_dispatches.items()
             if "tw4" in nm and not any(t in nm for t in LOAD_TIME_KERNELS)}
    exact = [nm for nm, d in cands.items() if d == launches]
    if exact:
        return exact[0]
    return max(cands, key=cands.get) if cands else None


def summarize_traffic(fetch_csv: str, write_csv: str, copy_mib: int, copies: int, launches: int,
                      algorithmic_bytes: int | None) -> dict:
    """Average FETCH_SIZE / WRITE_SIZE (KiB) per dispatch of each tw4 kernel, and its HBM bytes per
    launch: each counter scaled by known bytes / what the counter reads for the calibration copy."""
    fetch, write = _per_kernel(fetch_csv, "FETCH_SIZE"), _per_kernel(write_csv, "WRITE_SIZE")
    copy_name, cf = _calibration(fetch, copies)
    _, cw = _calibration(write, copies)
    known_kib = copy_mib * 1024.0
    f_fetch, f_write = known_kib / (sum(cf) / len(cf)), known_kib / (sum(cw) / len(cw))
    rows = {}
    for name, v in fetch.items():
        if "tw4" not in name:
            continue
        fk = sum(val for _, val in v) / len(v)
        w = write.get(name, [])
        wk = sum(val for _, val in w) / len(w) if w else 0.0
        rows[name] = {"dispatches": len(v), "FETCH_SIZE_KiB": round(fk, 1), "WRITE_SIZE_KiB": round(wk, 1),
                      "hbm_bytes": round((fk * f_fetch + wk * f_write) * 1024)}
    rec = {"copy_kernel": copy_name, "copy_MiB": copy_mib, "copy_FETCH_SIZE_KiB": [round(c, 1) for c in cf],
           "copy_WRITE_SIZE_KiB": [round(c, 1) for c in cw], "fetch_factor": round(f_fetch, 4),
           "write_factor": round(f_write, 4), "kernels": rows}
    main_k = target_kernel({nm: r["dispatches"] for nm, r in rows.items()}, launches)
    if main_k:
        rec["kernel"] = main_k
        rec["hbm_bytes_per_launch"] = rows[main_k]["hbm_bytes"]
        if algorithmic_bytes:
            rec["algorithmic_bytes_per_launch"] = algorithmic_bytes
            rec["traffic_over_algorithmic"] = round(rows[main_k]["hbm_bytes"] / algorithmic_bytes, 4)
    return rec


def summarize_mfma(path: str, m: int, n: int, k: int) -> dict:
    """Per tw4 kernel: average MfmaUtil (%) and fp16 MFMA work per dispatch (SQ_INSTS_VALU_MFMA_MOPS_F16
    x 512 flops) against the algorithmic 2 M N K, plus the dispatch's duration where the file has
    timestamps (a --kernel-trace run of the same command)."""
    util, mops = _per_kernel(path, "MfmaUtil"), _per_kernel(path, "SQ_INSTS_VALU_MFMA_MOPS_F16")
    dur: dict[str, list[float]] = {}
    with open(path, newline="", encoding="utf-8") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") == "MfmaUtil" and row.get("Start_Timestamp") and row.get("End_Timestamp"):
                dur.setdefault(row["Kernel_Name"], []).append(
                    (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    alg = 2 * m * n * k
    rows = {}
    for name, v in util.items():
        if "tw4" not in name or any(t in name for t in LOAD_TIME_KERNELS):
            continue
        mv = [val for _, val in mops.get(name, [])]
        flops = 512 * sum(mv) / len(mv) if mv else None
        row = {"dispatches": len(v), "MfmaUtil_pct": round(sum(val for _, val in v) / len(v), 2),
               "mfma_flops": flops, "algorithmic_flops": alg,
               "mfma_over_algorithmic": round(flops / alg, 4) if flops else None}
        if dur.get(name):
            us = sum(dur[name]) / len(dur[name])
            row["us_under_counters"] = round(us, 2)
            row["algorithmic_tflops_under_counters"] = round(alg / us / 1e6, 1)
        rows[name] = row
    return {"m": m, "n": n, "k": k, "kernels": rows}


def summarize_counters(paths: list[str], launches: int, kernel: str = "") -> dict:
    """The profiled kernel of `bench.py prof` counter runs (the tw4 kernel with exactly `launches`
    dispatches, never a load-time repack; with `kernel`, the one whose name contains it, e.g. the
    read probe of --probe): the median per dispatch of every counter in the given
    counter_collection.csv files (one per --pmc pass) and of the kernel duration, plus derived shares.
    The SQ counters and GRBM_GUI_ACTIVE are summed over the 8 XCDs, so GRBM_GUI_ACTIVE / 8 is the
    kernel's clock cycles and a busy share is cycles / (cycles x 1024 SIMDs):
      mfma_busy   SQ_VALU_MFMA_BUSY_CYCLES          (the matrix cores)
      valu_busy   SQ_ACTIVE_INST_VALU x 4            (a wave64 VALU instruction holds a SIMD 4 cycles;
                                                      SQ_INSTS_VALU counts the MFMA instructions too)
      coexec      SQ_VALU_MFMA_COEXEC_CYCLES         (VALU and matrix cores busy in the same cycle)
    and per dispatch the instructions per wavefront and the L2 hit share TCC_HIT / (TCC_HIT + TCC_MISS)."""
    import statistics as st

    vals: dict[str, list[float]] = {}
    dur: list[float] = []
    name = None
    for path in paths:
        rows: dict[str, list[dict]] = {}
        with open(path, newline="", encoding="utf-8") as f:
            for row in csv.DictReader(f):
                rows.setdefault(row["Kernel_Name"], []).append(row)
        cands = [k for k in rows if "tw4" in k and not any(t in k for t in LOAD_TIME_KERNELS)
                 and len({r["Dispatch_Id"] for r in rows[k]}) == launches]
        cands = [k for k in cands if kernel in k] if kernel else [k for k in cands if "read_probe" not in k]
        if len(cands) != 1:
            raise SystemExit(f"{path}: {len(cands)} tw4 kernels with {launches} dispatches: {cands}")
        name = cands[0]
        seen = set()
        for r in rows[name]:
            vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            if r["Dispatch_Id"] not in seen and r.get("Start_Timestamp"):
                seen.add(r["Dispatch_Id"])
                dur.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    med = {c: st.median(v) for c, v in vals.items()}
    out = {"kernel": name, "dispatches_timed": len(dur), "us_under_counters": round(st.median(dur), 2) if dur else None,
           "counters": med}
    cyc = med.get("GRBM_GUI_ACTIVE", 0) / 8
    if cyc and dur and cyc / (st.median(dur) * 1e3) > 2.6:
        # on a kernel of a few us GRBM_GUI_ACTIVE also counts around the dispatch (it implies a clock
        # above the 2.4 GHz peak): take the duration at the peak clock instead (shares are then lower bounds)
        out["cycles_basis"] = "duration x 2.4 GHz (GRBM_GUI_ACTIVE / 8 implied %.2f GHz)" % (cyc / (st.median(dur) * 1e3))
        cyc = st.median(dur) * 1e3 * 2.4
    elif cyc:
        out["cycles_basis"] = "GRBM_GUI_ACTIVE / 8"
    if cyc:
        simd = 1024 * cyc
        out["clock_GHz"] = round(cyc / (st.median(dur) * 1e3), 3) if dur else None
        for key, cnt, mul in (("mfma_busy", "SQ_VALU_MFMA_BUSY_CYCLES", 1), ("valu_busy", "SQ_ACTIVE_INST_VALU", 4),
                              ("coexec", "SQ_VALU_MFMA_COEXEC_CYCLES", 1), ("lds_busy", "SQ_ACTIVE_INST_LDS", 4)):
            if cnt in med:
                out[key] = round(med[cnt] * mul / simd, 4)
    waves = med.get("SQ_WAVES")
    if waves:
        out["per_wavefront"] = {c: round(med[c] / waves, 1) for c in
                                ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_INSTS_SALU")
                                if c in med}
    if "TCC_HIT_sum" in med and "TCC_MISS_sum" in med:
        out["l2_hit_share"] = round(med["TCC_HIT_sum"] / max(med["TCC_HIT_sum"] + med["TCC_MISS_sum"], 1), 3)
    return out


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "tune":
        sys.exit(tune_main(sys.argv[2:]))
    if len(sys.argv) > 1 and sys.argv[1] == "prof":
        sys.exit(prof_main(sys.argv[2:]))
    if len(sys.argv) > 1 and sys.argv[1] == "floor":
        sys.exit(floor_main(sys.argv[2:]))
    sys.exit(main())

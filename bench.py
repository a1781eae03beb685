"""Benchmark of the MI355X AWQ W4A16 linear path on Qwen3-8B shapes (one GPU).

    python bench.py [--steps K] [--warmup W] [--m 1] [--layers 36] [--no-cpu] [--no-detail]
    python bench.py --sweep [--sweep-out FILE]

One step = one decode token's W4A16 linears of the whole Qwen3-8B stack: 36 layers x {qkv
(K 4096, N 6144), o (4096, 4096), gate_up (4096, 24576), down (12288, 4096)} at M = 1, launched
back to back from one HIP graph through the product's own W4Linear.forward dispatch. Every layer has
its own random int4 weights (3.6 GB of tile-layout weights, far beyond the 256 MB Infinity Cache),
so every call streams its weights from HBM; inputs are resident in HBM before timing starts.

value = whole-step algorithmic HBM bytes / time (GB/s), with the per-call byte count
    B = N K / 2 + N (K/128) 2 + N (K/128) / 2 + 2 M K + 2 M N
(int4 weights, fp16 scales, int4 zeros, fp16 x and y). The JSON line adds:
  roofline      the dominant kernel (gate_up at the benchmark's M) timed alone with HIP events
                on its own stream, against MI355X's 8 TB/s HBM peak; `traffic` comes from the
                committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary when present
  cpu_baseline  the CPU oracle's dequantize-then-matmul (the reference's fallback restated in
                numpy) on a bounded sample of the same workload, on this host's cores
  detail        per projection and M in {1, 8, 32}: us/call, GB/s, % of peak, TFLOP/s, the kernel
                that ran, and at M = 32 the dequantize + torch.matmul comparator
  full_stack    the whole decode step of the linears plus the fp16 lm_head (4096 x 151936, through
                layers/gemv16.py's table: the HIP fp16 GEMV where it has an entry, else F.linear),
                M in {1, 8, 32}: us per step and GB/s
  decode_step   the model's decode step (tandem_amd.model: norms, one-token attention, SwiGLU
                gate_up, lm_head) replayed from the bucketed HIP graphs of tandem_amd.decode_graph,
                M in {1, 8, 32}: us per step, tokens/s, GB/s of the step's weight bytes

--sweep times every single-linear configuration of the benchmark's configs instead (Qwen3-0.6B
qkv at M = 1; Qwen3-8B's four shapes at M in {1, 4, 8, 16} and {24, 32, 64, 256, 1024, 4096};
Qwen3-1.7B's four shapes at M in {1, 4, 8}): one JSON line per (shape, M) with us/call, GB/s,
TFLOP/s, % of the roofline max(B / 8 TB/s, 2 M N K / 2.5 PFLOP/s), the kernel that ran, and past
M = 16 the dequantize + torch.matmul comparator. Each shape rotates over enough weight copies
(>= 1 GB) that every call streams from HBM.
"""

from __future__ import annotations

import argparse
import json
import os
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gate_up_m1.json")


def call_bytes(m: int, k: int, n: int) -> int:
    g = k // 128
    return n * k // 2 + n * g * 2 + n * g // 2 + 2 * m * k + 2 * m * n


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--m", type=int, default=1, help="tokens per call (decode batch)")
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-detail", action="store_true", help="skip the per-projection sweep")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--sweep", action="store_true", help="time every (shape, M) of the configs; JSON line each")
    ap.add_argument("--sweep-out", default="", help="also append the sweep's JSON lines to this file")
    ap.add_argument("--step-only", action="store_true",
                    help="only the decode_step section (for profiling the whole step); prints its JSON")
    return ap.parse_args()


def make_layers(torch, awq, n_layers: int, dev, seed: int = 0):
    """Random AutoAWQ weights (uniform int4 q and z, fp16 scales in [0.001, 0.02]) for every
    projection of every layer, repacked by the product's W4Linear.finalize."""
    g = torch.Generator(device=dev).manual_seed(seed)
    name = torch.cuda.get_device_name(dev)
    layers = []
    for _ in range(n_layers):
        layer = {}
        for proj, k, n in QWEN3_8B:
            lin = awq.W4Linear(k, n, 128).to(dev)
            lin.qweight.copy_(torch.randint(-2**31, 2**31 - 1, lin.qweight.shape, device=dev, dtype=torch.int32,
                                            generator=g))
            lin.qzeros.copy_(torch.randint(-2**31, 2**31 - 1, lin.qzeros.shape, device=dev, dtype=torch.int32,
                                           generator=g))
            lin.scales.copy_((torch.rand(lin.scales.shape, device=dev, generator=g) * 0.019 + 0.001).half())
            lin.finalize(name)
            layer[proj] = lin
        layers.append(layer)
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
    if m <= 16:
        key = (lin.out_features, lin.in_features, m)
        kind = (lin.kernels.get((*key, "silu")) if lin.silu_mul else None) or lin.kernels.get(key, awq.DEFAULT_KERNEL)
        if kind[0] in ("gemv", "gemvm") and m > 4:
            kind = awq.DEFAULT_KERNEL
        return f"{kind[0]}{tuple(kind[1:])}"
    key = (lin.out_features, lin.in_features) + (("silu",) if lin.silu_mul else ())
    cfg = awq.pick_gemm(lin.gemm_kernels.get(key, awq.DEFAULT_GEMM), m)
    if cfg is None or not awq.FUSED_GEMM:
        return "dequant+matmul"
    return f"mma{tuple(cfg[1:])}" if cfg[0] == "mma" else f"gemm{cfg}"


def random_linear(torch, awq, k: int, n: int, dev, g):
    """One W4Linear with random AutoAWQ weights (uniform int4 q and z, fp16 scales in [0.001, 0.02]),
    repacked by the product's finalize."""
    lin = awq.W4Linear(k, n, 128).to(dev)
    lin.qweight.copy_(torch.randint(-2**31, 2**31 - 1, lin.qweight.shape, device=dev, dtype=torch.int32, generator=g))
    lin.qzeros.copy_(torch.randint(-2**31, 2**31 - 1, lin.qzeros.shape, device=dev, dtype=torch.int32, generator=g))
    lin.scales.copy_((torch.rand(lin.scales.shape, device=dev, generator=g) * 0.019 + 0.001).half())
    lin.finalize(torch.cuda.get_device_name(dev))
    return lin


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


def cpu_baseline(budget_s: float, m: int) -> dict:
    """The CPU oracle (numpy) dequantize-then-matmul on whole Qwen3-8B projections at M, repeated
    until ~budget_s seconds; GB/s of the same algorithmic bytes as the GPU figure."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import awq_oracle as o

    cores = len(os.sched_getaffinity(0))
    threads = max(1, min(cores, 16))
    data = []
    for i, (proj, k, n) in enumerate(QWEN3_8B):
        qw, qz, s, _, _ = o.random_awq(k, n, seed=1000 + i)
        x = np.random.default_rng(i).standard_normal((m, k)).astype(np.float16)
        data.append((proj, k, n, qw, qz, s, x))
    total_bytes, done, t_total = 0, 0, 0.0
    with threadpool_limits(limits=threads):
        t0 = time.perf_counter()
        while True:
            for proj, k, n, qw, qz, s, x in data:
                t = time.perf_counter()
                o.dequant_then_linear(x, qw, qz, s)
                t_total += time.perf_counter() - t
                total_bytes += call_bytes(m, k, n)
            done += 1
            if time.perf_counter() - t0 > budget_s:
                break
    model = ""
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            model = next((line.split(":", 1)[1].strip() for line in f if line.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(total_bytes / t_total / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{done} x one Qwen3-8B layer's 4 projections at M={m} (qkv, o, gate_up, down): numpy "
                      f"AWQ unpack + fp16 dequant + float32 BLAS matmul per call, BLAS on {threads} threads "
                      f"(dequant single-threaded); {t_total:.1f} s; host {model} ({cores} cores visible)",
            "ms_per_layer": round(t_total / done * 1e3, 2)}


def decode_step(torch, dev) -> dict:
    """The whole Qwen3-8B decode step of tandem_amd.model (embedding, 36 x {add + RMSNorm, qkv,
    one-token attention, o, add + RMSNorm, gate_up with SwiGLU, down}, final add + RMSNorm, fp16
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
    out = {}
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


def main() -> int:
    a = parse()
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
    traffic = None
    if os.path.exists(TRAFFIC_FILE) and m == 1:
        with open(TRAFFIC_FILE, encoding="utf-8") as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": f"gate_up (K 4096, N 24576) M={m}: {kernel_of(awq, layers[0]['gate_up'], m)}",
                "us_per_launch": round(gate_s * 1e6, 3), "algorithmic_bytes_per_launch": gate_bytes}
    del gate_graph

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
                rec = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "pct_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS * 100, 1),
                       "TFLOPs": round(f / us / 1e6, 2), "kernel": kernel_of(awq, layers[0][proj], mm)}
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
                              "lm_head": "gemv16" if table.get((hn, hk, gemv16.m_bucket(mm))) and mm <= 8
                              else "F.linear"}
        del head
        torch.cuda.synchronize()

    step = {} if a.no_detail else decode_step(torch, dev)

    cpu = None if a.no_cpu else cpu_baseline(a.cpu_seconds, m)
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
        "roofline": roofline, "cpu_baseline": cpu, "detail": detail, "full_stack": full, "decode_step": step,
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

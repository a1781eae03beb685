"""Configuration sweep for the W4A16 kernels: the MI355X counterpart of the reference's
benchmarks/bench_w4.py and bench_w4_gemm.py, which produced its per-GPU tables.

    python -m tandem_amd.tune --model qwen3-8b --ms 1,4,8,16 --kinds gemv,mma [--out sweep.jsonl]
    python -m tandem_amd.tune --model qwen3-8b --ms 24,32,64,256 --kinds gemm
    python -m tandem_amd.tune --model qwen3-8b --projs lm_head --ms 1,2,4,8 --kinds dense16,torch16

For each projection shape and M, every compiled configuration of each kernel is timed the way
the reference timed them (benchmarks/bench_gemv.py:35-56): one HIP graph replays `rounds` passes
over `copies` weight copies whose total size (>= --footprint-mb, default 1 GB) is far beyond the
256 MB Infinity Cache, so each call streams its weights from HBM. One JSON record per (shape, M)
gives us/call and GB/s of the best config of each kind and of every config.
"""

from __future__ import annotations

import argparse
import json
import math
import sys

import torch

from tandem_amd.layers import w4_hip

MODELS = {
    "qwen3-8b": {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096),
                 "lm_head": (4096, 151936)},
    "qwen3-1.7b": {"qkv": (2048, 4096), "o": (2048, 2048), "gate_up": (2048, 12288), "down": (6144, 2048),
                   "lm_head": (2048, 151936)},
    "qwen3-0.6b": {"qkv": (1024, 4096), "lm_head": (1024, 151936)},
    # other common AWQ checkpoints (hidden, intermediate, heads / kv heads x 128)
    "qwen3-4b": {"qkv": (2560, 6144), "o": (4096, 2560), "gate_up": (2560, 19456), "down": (9728, 2560)},
    "qwen3-14b": {"qkv": (5120, 7168), "o": (5120, 5120), "gate_up": (5120, 34816), "down": (17408, 5120)},
    "llama3-8b": {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 28672), "down": (14336, 4096)},
}
DENSE = ("lm_head",)  # fp16 projections (kinds dense16 / torch16); the others are W4A16


def call_bytes(m: int, k: int, n: int) -> int:
    g = k // 128
    return n * k // 2 + n * g * 2 + n * g // 2 + 2 * m * k + 2 * m * n


def random_weights(k: int, n: int, dev, gen) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Uniform random nibbles straight in the tile layout, fp16 scales in [0.001, 0.02], integer zeros."""
    packed = torch.randint(-2**31, 2**31 - 1, (w4_hip.padded_rows(n), k // 8), dtype=torch.int32, device=dev,
                           generator=gen)
    scales = (torch.rand(n, k // 128, device=dev, generator=gen) * 0.019 + 0.001).half()
    zeros = torch.randint(0, 16, (n, k // 128), device=dev, generator=gen).half()
    return packed, scales, zeros


def time_us(calls, stream, rounds: int = 10, reps: int = 5) -> float:
    """Microseconds per call: a HIP graph of `rounds` passes over `calls`, replayed `reps` times."""
    with torch.cuda.stream(stream):
        for c in calls:
            c()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(rounds):
            for c in calls:
                c()
    with torch.cuda.stream(stream):
        graph.replay()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(reps):
            graph.replay()
        t1.record(stream)
    t1.synchronize()
    return t0.elapsed_time(t1) * 1e3 / (reps * rounds * len(calls))


def emit(a, out, proj: str, k: int, n: int, m: int, act: int, copies: int, res: dict, b: int) -> None:
    """One JSON record: the best config, us/call, GB/s of the algorithmic bytes b, every config."""
    if not res:
        return
    best = min(res, key=res.get)
    rec = {"model": a.model, "proj": proj, "k": k, "n": n, "m": m, "act": act, "copies": copies,
           "best": list(best), "us": round(res[best], 3), "GBps": round(b / res[best] / 1e3, 1),
           "pct_hbm_peak": round(b / res[best] / 1e3 / 80, 2),
           "TFLOPs": round(2 * m * k * n / res[best] / 1e6, 2),
           "best_per_kind": {kd: min((v, list(c)) for c, v in res.items() if c[0] == kd)
                             for kd in {c[0] for c in res}},
           "all": {"/".join(map(str, c)): round(v, 2) for c, v in sorted(res.items(), key=lambda kv: kv[1])}}
    print(json.dumps(rec), flush=True)
    if out:
        out.write(json.dumps(rec) + "\n")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model", default="qwen3-8b", choices=sorted(MODELS))
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
    for proj, (k, n) in MODELS[a.model].items():
        if a.projs and proj not in a.projs.split(","):
            continue
        if a.act and proj != "gate_up":
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
                        res[("dense16", *cfg)] = time_us([lambda w=w, c=cfg: gemv16.gemv(x, w, *c) for w in wd],
                                                         stream, rounds=3)
                if "torch16" in kinds:
                    res[("torch16",)] = time_us([lambda w=w: torch.nn.functional.linear(x, w) for w in wd], stream,
                                                rounds=3)
                emit(a, out, proj, k, n, m, 0, copies, res, wbytes + 2 * m * k + 2 * m * n)
            del wd
            torch.cuda.empty_cache()
            continue
        wbytes = call_bytes(0, k, n)
        copies = max(2, math.ceil(a.footprint_mb * 1e6 / wbytes))
        ws = [random_weights(k, n, dev, gen) for _ in range(copies)]
        for m in (int(v) for v in a.ms.split(",")):
            x = torch.randn(m, k, device=dev, dtype=torch.float16)
            res = {}
            if "gemv" in kinds and m <= 4:
                for cfg in w4_hip.decode_configs():
                    try:
                        us = time_us([lambda w=w, c=cfg: ext.w4_gemv(x, *w, *c, act) for w in ws], stream)
                    except RuntimeError:
                        continue
                    res[("gemv", *cfg)] = us
            if "gemvn" in kinds and m <= 4:  # the GEMV with the add + RMSNorm prologue (tw4_decode_norm)
                r = torch.randn(m, k, device=dev, dtype=torch.float16)
                nw = (torch.rand(k, device=dev) + 0.5).half()
                for cfg in w4_hip.decode_configs():
                    try:
                        us = time_us([lambda w=w, c=cfg: ext.w4_decode_norm(x, r, nw, 1e-6, *w, 0, *c, act)
                                      for w in ws], stream)
                    except RuntimeError:
                        continue
                    res[("gemvn", *cfg)] = us
            if "gemvm" in kinds and m <= 4:
                for cfg in w4_hip.decode_configs():
                    try:
                        us = time_us([lambda w=w, c=cfg: ext.w4_gemv_mfma(x, *w, *c, act) for w in ws], stream)
                    except RuntimeError:
                        continue
                    res[("gemvm", *cfg)] = us
            if "mma" in kinds and m <= 64:
                for cfg in w4_hip.decode_configs():
                    try:
                        us = time_us([lambda w=w, c=cfg: ext.w4_mma(x, *w, *c, act) for w in ws], stream)
                    except RuntimeError:  # unroll * batch tiles above 4
                        continue
                    res[("mma", *cfg)] = us
            if "mmap" in kinds and m <= 16:
                for cfg in w4_hip.decode_configs():
                    for pc in (int(v) for v in a.per_cu.split(",")):
                        try:
                            us = time_us([lambda w=w, c=cfg, q=pc: ext.w4_mma_persist(x, *w, *c, q, act)
                                          for w in ws], stream)
                        except RuntimeError:
                            continue
                        res[("mmap", *cfg, pc)] = us
            if "mmak" in kinds and m <= 16:
                for cfg in w4_hip.decode_configs():
                    for sp in (int(v) for v in a.splits.split(",")):
                        if sp < 2 or sp > k // 128:
                            continue
                        try:
                            us = time_us([lambda w=w, c=cfg, s=sp: ext.w4_mma_splitk(x, *w, buf, locks, *c, s, act)
                                          for w in ws], stream)
                        except RuntimeError:
                            continue
                        res[("mmak", *cfg, sp)] = us
            if "gemm" in kinds:
                g = k // 128
                for cfg in w4_hip.gemm_configs():
                    for sp in (int(v) for v in a.splits.split(",")):
                        if sp > (g + cfg[3] - 1) // cfg[3]:
                            continue
                        try:
                            us = time_us([lambda w=w, c=cfg, s=sp: ext.w4_gemm(x, *w, buf, locks, *c, s, act)
                                          for w in ws], stream, rounds=5)
                        except RuntimeError:
                            continue
                        res[("gemm", *cfg, sp)] = us
            if "dense" in kinds:  # HIP dequantize + torch.matmul, the unfused comparator
                from tandem_amd.layers import awq

                def dense(w):
                    y = torch.nn.functional.linear(x, awq.w4_dequant(*w, deinterleave=bool(act)))
                    return awq.silu_and_mul(y) if act else y

                res[("dense",)] = time_us([lambda w=w: dense(w) for w in ws[:8]], stream, rounds=3)
            emit(a, out, proj, k, n, m, act, copies, res, call_bytes(m, k, n))
        del ws
        torch.cuda.empty_cache()
    if out:
        out.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())

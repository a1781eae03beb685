"""A fixed, eager sequence of kernel launches for hardware-counter runs under rocprofv3.

    python -m tandem_amd.prof [--proj gate_up] [--m 1] [--launches 40] [--copy-mib 256]

Launches, in order: `copies` torch copies of a --copy-mib MiB float16 buffer (a plain device copy
of known size: it reads and writes exactly that many bytes, which calibrates FETCH_SIZE and
WRITE_SIZE), then --launches calls of W4Linear.forward for one Qwen3-8B projection at M, rotating
over enough weight copies (>= 1 GB) that every call streams its weights from HBM. A counter run
then reads, per dispatch, the HBM bytes the kernel moved:

    rocprofv3 --pmc FETCH_SIZE -d <dir> -o run --output-format csv -- python3 -m tandem_amd.prof
    rocprofv3 --pmc WRITE_SIZE -d <dir> -o run --output-format csv -- python3 -m tandem_amd.prof
    python -m tandem_amd.prof --summarize <fetch counter_collection.csv> <write counter_collection.csv>

The same launches give the GEMM's matrix-core utilisation (M > 16; --cfg forces one GEMM
configuration, mt,nt,warps_n,warps_k,stages,splits, in place of the table's, to compare tile and
split-K choices on the same shape):

    rocprofv3 --kernel-trace --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_F16 -d <dir> -o run \
        --output-format csv -- python3 -m tandem_amd.prof --proj gate_up --m 32 [--cfg 2,1,4,2,2,1]
    python -m tandem_amd.prof --proj gate_up --m 32 --summarize-mfma <counter_collection.csv>

MfmaUtil is rocprofiler's derived counter: the SIMDs' summed SQ_VALU_MFMA_BUSY_CYCLES over
GRBM_GUI_ACTIVE x the number of SIMDs, in percent. SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 is the fp16
matrix-core work issued, which against 2 M N K shows the padding of the token tiles.
"""

from __future__ import annotations

import argparse
import csv
import json
import sys

SHAPES = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}
COPY_KERNEL_HINT = ("copybuffer",)  # the HIP runtime's device-to-device copy (torch copy_ of one dtype)


def run(a: argparse.Namespace) -> int:
    import torch

    from tandem_amd.layers import awq, w4_hip

    if not torch.cuda.is_available():
        print("tandem_amd.prof needs the GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    w4_hip.load()
    src = torch.ones(a.copy_mib << 19, device=dev, dtype=torch.float16)
    dst = torch.empty_like(src)
    for _ in range(a.copies):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst

    k, n = SHAPES[a.proj]
    g = torch.Generator(device=dev).manual_seed(0)
    per_copy = n * k // 2
    copies = max(2, -(-(1 << 30) // per_copy))
    layers = []
    for _ in range(copies):
        lin = awq.W4Linear(k, n, 128).to(dev)
        lin.qweight.copy_(torch.randint(-2**31, 2**31 - 1, lin.qweight.shape, device=dev, dtype=torch.int32, generator=g))
        lin.qzeros.copy_(torch.randint(-2**31, 2**31 - 1, lin.qzeros.shape, device=dev, dtype=torch.int32, generator=g))
        lin.scales.copy_((torch.rand(lin.scales.shape, device=dev, generator=g) * 0.019 + 0.001).half())
        lin.finalize(torch.cuda.get_device_name(dev))
        if a.cfg:  # a per-layer copy: the module-level table is shared by every W4Linear
            lin.gemm_kernels = {**lin.gemm_kernels, (n, k): ((1 << 30, tuple(int(v) for v in a.cfg.split(","))),)}
        layers.append(lin)
    x = torch.randn(a.m, k, device=dev, dtype=torch.float16)
    torch.cuda.synchronize()
    for i in range(a.launches):
        layers[i % copies](x)
    torch.cuda.synchronize()
    print(f"prof: {a.copies} copies of {a.copy_mib} MiB, {a.launches} x {a.proj} (K {k}, N {n}) M={a.m} "
          f"over {copies} weight copies, gemm config {a.cfg or 'from the table'}", flush=True)
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


def summarize(fetch_csv: str, write_csv: str, copy_mib: int, copies: int, algorithmic_bytes: int | None) -> dict:
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
    if rows:
        main = max(rows, key=lambda nm: rows[nm]["dispatches"])
        rec["kernel"] = main
        rec["hbm_bytes_per_launch"] = rows[main]["hbm_bytes"]
        if algorithmic_bytes:
            rec["algorithmic_bytes_per_launch"] = algorithmic_bytes
            rec["traffic_over_algorithmic"] = round(rows[main]["hbm_bytes"] / algorithmic_bytes, 4)
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
        if "tw4" not in name:
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


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--proj", default="gate_up", choices=sorted(SHAPES))
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--launches", type=int, default=40)
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--copies", type=int, default=3)
    ap.add_argument("--cfg", default="", help="GEMM config mt,nt,warps_n,warps_k,stages,splits for every M > 16")
    ap.add_argument("--summarize", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--summarize-mfma", metavar="COUNTER_CSV")
    a = ap.parse_args(argv)
    if a.summarize_mfma:
        k, n = SHAPES[a.proj]
        print(json.dumps(summarize_mfma(a.summarize_mfma, a.m, n, k), indent=1))
        return 0
    if a.summarize:
        k, n = SHAPES[a.proj]
        g = k // 128
        alg = n * k // 2 + n * g * 2 + n * g // 2 + 2 * a.m * k + 2 * a.m * n
        print(json.dumps(summarize(*a.summarize, a.copy_mib, a.copies, alg), indent=1))
        return 0
    return run(a)


if __name__ == "__main__":
    sys.exit(main())

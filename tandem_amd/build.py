"""Build libtandem_w4.so in-tree with hipcc for gfx950 (no JIT, no torch extension).

    python -m tandem_amd.build            # compile every HIP source, link tandem_amd/lib/libtandem_w4.so

Each ``csrc/*.hip`` file is compiled on its own (in parallel) and the objects are linked into one
shared library with a plain C ABI (``include/tandem_w4.h``). The library is git-ignored and
travels with the tree to the GPU box.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
LIB_DIR = os.path.join(ROOT, "lib")
LIB = os.path.join(LIB_DIR, "libtandem_w4.so")
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops (v_pk_*_f32).
CFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-I" + os.path.join(REPO, "include"), "-Wall", "-Wno-unused-function"]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


# Per-source flags for the decode kernels (tw4_decode.hip).
# - The MFMA accumulators sit in ordinary VGPRs instead of the accumulation registers: no
#   v_accvgpr moves around each quant group's MFMAs. The persistent decode kernel on Qwen3-8B
#   gate_up at M = 8 measured 13.9 -> 13.4 us (the others level).
# - The leading kernel arguments are preloaded into user SGPRs before a wavefront starts (whole
#   arguments, 13 dwords in these kernels), so its first instructions do not wait on an s_load of
#   them. The decode kernels put what their prologue needs first and compute the grid size rather
#   than read gridDim.x, a hidden argument past the preloaded ones. This shortens the start of the
#   small decode grids: the GEMV on Qwen3-8B qkv at M = 1 measured 4.74 -> 4.39 us, the matrix-core
#   kernels 1.5-3 % and the GEMV on the matrix cores 3-6 % at M = 2-16; with the grid computed,
#   gate_up's GEMV at M = 1 10.3 -> 10.0 us. (The GEMM sources measured 1-5 % slower with the same
#   preload and argument order at M = 32: their prologues still wait on the later arguments.)
SOURCE_FLAGS = {"tw4_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def _compile(src: str, obj: str) -> tuple[str, int, str]:
    flags = CFLAGS + SOURCE_FLAGS.get(os.path.basename(src), [])
    proc = subprocess.run([HIPCC, *flags, "-c", src, "-o", obj], capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag and says so: not an error
    err = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if "packed-fp32-ops" not in line)
    return src, proc.returncode, err


def build(verbose: bool = False) -> str:
    """Compile every source and link the library; returns its path. Raises RuntimeError on failure."""
    os.makedirs(LIB_DIR, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="tw4_build_") as tmp:
        srcs = sources()
        objs = [os.path.join(tmp, os.path.basename(s)[:-4] + ".o") for s in srcs]
        with cf.ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4, 8)) as pool:
            results = list(pool.map(_compile, srcs, objs))
        failed = [(s, e) for s, rc, e in results if rc != 0]
        for s, rc, e in results:
            if verbose and e.strip():
                print(f"--- {os.path.basename(s)}\n{e}", file=sys.stderr)
        if failed:
            raise RuntimeError("hipcc failed:\n" + "\n".join(f"{os.path.basename(s)}:\n{e[-4000:]}" for s, e in failed))
        tmp_lib = LIB + ".tmp"
        proc = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp_lib, *objs],
                              capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError("link failed:\n" + proc.stdout + proc.stderr)
        os.replace(tmp_lib, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

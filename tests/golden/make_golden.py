"""Writes tests/golden/awq_small.npz: small AutoAWQ-format inputs and the oracle's outputs.

These are regression fixtures of this build (the reference repository holds no data files for the
path): inputs follow the reference tests' recipe (tests/test_awq.py:32-38 of 12vivi/tandem), outputs
come from oracle/awq_oracle.py. Re-run only when the oracle changes on purpose:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import awq_oracle as o  # noqa: E402


def main() -> None:
    k, n, m = 256, 48, 3
    qweight, qzeros, scales, q, z = o.random_awq(k, n, seed=2024)
    x = np.random.default_rng(2025).standard_normal((m, k)).astype(np.float16)
    w = o.dequant(qweight, qzeros, scales)
    y = o.linear(x, w)
    sw = o.swiglu_reference(x, o.dequant_exact(qweight, qzeros, scales))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "awq_small.npz")
    np.savez_compressed(out, qweight=qweight, qzeros=qzeros, scales=scales, q=q, z=z, x=x, w_fp16=w,
                        y_f64=y, swiglu_f64=sw)
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()

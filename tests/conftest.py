"""Test set-up: repo root on sys.path, the `gpu` marker, shared helpers.

`-m "not gpu"` runs on any machine (oracle pins, host logic, C-ABI exports); `-m gpu` needs an
MI355X and compares the HIP kernels, called through the C ABI, with the CPU oracle."""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtandem_w4.so")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The parity figures the GPU tests measured (tests/parity.py): per test, the worst
    max |err| / max |ref| and the lowest cosine similarity against the oracle. With
    TANDEM_PARITY_OUT=<file> the full table per (test, kernel family, shape, M) goes there too."""
    import parity

    lines = parity.summary(by_test=True)
    if not lines:
        return
    terminalreporter.write_sep("-", "parity against the oracle (max_rel = max|err| / max|ref|)")
    for ln in lines:
        terminalreporter.write_line(ln)
    out = os.environ.get("TANDEM_PARITY_OUT")
    if out:
        with open(out, "w", encoding="utf-8") as f:
            f.write("\n".join(parity.summary(by_test=False)) + "\n")


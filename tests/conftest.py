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

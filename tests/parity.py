"""The tolerance check every GPU parity test uses, and the record of what it measured.

check_close compares a kernel's output with the oracle's float64 (or float32 SwiGLU) reference on
the reference tests' bar: |got - ref| <= atol + rtol |ref| everywhere (tests/test_awq.py of
12vivi/tandem: 0.05 / 0.02 for the GEMV and the layer, 0.02 / 0.01 for the matrix-core kernels,
0.03 / 0.02 for the SwiGLU layer) and a cosine similarity of at least 0.9999. Each call also
records max |err| / max |ref| (the reference bench's max_rel, benchmarks/bench_w4_gemm.py:84-92)
and the cosine under a key (test, kernel family, shape, M); conftest.py prints the worst figures
per key at the end of the session, so the run's log carries the numbers and not only pass / fail.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np


@dataclass
class Record:
    test: str
    family: str
    shape: str
    m: str
    max_rel: float
    max_abs: float
    cos: float
    atol: float
    rtol: float
    count: int = 1


RECORDS: dict[tuple[str, str, str, str], Record] = {}


def _current_test() -> str:
    cur = os.environ.get("PYTEST_CURRENT_TEST", "?")
    name = cur.split("::")[-1].split(" ")[0]
    return name.split("[")[0]


def _key_of(what, family, shape, m) -> tuple[str, str, str]:
    """(family, shape, M) from explicit arguments, else from a (K, N, M, config, ...) tuple."""
    if isinstance(what, tuple) and len(what) >= 3 and all(isinstance(v, (int, np.integer)) for v in what[:3]):
        shape = shape or f"{int(what[0])}x{int(what[1])}"
        m = m if m is not None else int(what[2])
        if family is None and len(what) >= 4 and isinstance(what[3], tuple):
            cfg = what[3]
            family = cfg[0] if cfg and isinstance(cfg[0], str) else None
    elif isinstance(what, tuple) and len(what) >= 2 and isinstance(what[0], str):
        shape = shape or what[0]
        m = m if m is not None else what[1]
    return family or "", shape or "", "" if m is None else str(m)


def check_close(got, ref, atol: float, rtol: float, what, family: str | None = None, shape: str | None = None,
                m=None) -> None:
    """Assert got (torch tensor or array) is within atol + rtol |ref| of ref and has cosine >= 0.9999
    (or ref is ~0); record max_rel and cosine under (test, family, shape, M)."""
    if hasattr(got, "detach"):
        got = got.detach().float().cpu().numpy()
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    ref_max = float(np.abs(ref).max()) if ref.size else 0.0
    max_rel = max_abs / max(ref_max, 1e-6)
    denom = float(np.linalg.norm(got) * np.linalg.norm(ref))
    cos = float((got * ref).sum() / denom) if denom > 0 else 1.0
    fam, shp, mm = _key_of(what, family, shape, m)
    key = (_current_test(), fam, shp, mm)
    rec = RECORDS.get(key)
    if rec is None:
        RECORDS[key] = Record(key[0], fam, shp, mm, max_rel, max_abs, cos, atol, rtol)
    else:
        rec.max_rel, rec.max_abs = max(rec.max_rel, max_rel), max(rec.max_abs, max_abs)
        rec.cos, rec.count = min(rec.cos, cos), rec.count + 1
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (what, f"max|err| {max_abs:.4g}", f"max_rel {max_rel:.3g}", f"cos {cos:.7f}")
    assert cos >= 0.9999 or ref_max < 1e-3, (what, cos)


def summary(by_test: bool = True) -> list[str]:
    """The recorded figures as text lines: per test, the worst max_rel and the lowest cosine over all
    its comparisons (with how many), then per (test, family, shape, M) in full when by_test is False."""
    if not RECORDS:
        return []
    lines = []
    if by_test:
        agg: dict[str, list] = {}
        for r in RECORDS.values():
            a = agg.setdefault(r.test, [0, 0.0, 1.0, 0.0, r.atol, r.rtol, set(), set()])
            a[0] += r.count
            a[1], a[2], a[3] = max(a[1], r.max_rel), min(a[2], r.cos), max(a[3], r.max_abs)
            if r.family:
                a[6].add(r.family)
            if r.m:
                a[7].add(r.m)
        lines.append(f"{'test':40s} {'checks':>6s} {'max_rel':>9s} {'max|err|':>9s} {'min cos':>10s}  tol  kernels / M")
        for t, (n, mr, cs, ma, at, rt, fams, ms) in agg.items():
            ms_s = ",".join(sorted(ms, key=lambda v: (len(v), v)))[:28]
            lines.append(f"{t[:40]:40s} {n:6d} {mr:9.2e} {ma:9.2e} {cs:10.7f}  {at:g}/{rt:g}  "
                         f"{'/'.join(sorted(fams))[:24]} M {ms_s}")
        return lines
    lines.append(f"{'test':44s} {'family':8s} {'shape':12s} {'M':>5s} {'checks':>6s} {'max_rel':>9s} {'max|err|':>9s} "
                 f"{'min cos':>10s}")
    for r in RECORDS.values():
        lines.append(f"{r.test[:44]:44s} {r.family[:8]:8s} {r.shape[:12]:12s} {r.m[:5]:>5s} {r.count:6d} "
                     f"{r.max_rel:9.2e} {r.max_abs:9.2e} {r.cos:10.7f}")
    return lines

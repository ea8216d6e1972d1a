"""Row tiles, merge-path windows and hybrid tiles on skewed matrices.

Every tiled SpMV schedule comes in three forms (``Config.balance``): tiles of
T consecutive rows; merge-path windows that give each workgroup an equal
share of rows plus nonzeros and cut rows longer than a window into pieces; and
hybrid tiles, row tiles that leave rows longer than B*U nonzeros to extra
workgroups over equal nonzero ranges.
This driver times the three forms of the same schedules on matrices whose rows
range from a few nonzeros to the full width, next to the BASELINE skewed
cases, and checks every result against float64 SciPy (normwise relative
error <= 1e-10) before reporting a time.

Inputs are cold: the launches rotate over copies of every array, enough to
pass the 256 MB Infinity Cache.  Times are medians of dispatch-attached
events.  ``python -m tilegen_amd.skew --out results`` writes ``skew.json`` and
``skew.md``.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
from typing import Dict, List

import numpy as np
import scipy.sparse as sp

from . import runtime as rt
from .codegen import Config
from .matrices import baseline_operands, make_baseline
from .variant import Variant

__all__ = ["skew_matrices", "SCHEDULES", "compare", "render", "main"]

TOL = 1e-10
FORMS = ("rows", "nnz", "hybrid")
SCHEDULES = [
    Config(tile_size=64, threads_per_row=8, unroll=2, block_size=512),
    Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128),
    Config(tile_size=64, threads_per_row=1, unroll=2, block_size=256),
    Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256),   # tuned for c3a
]


def _rows_with_lengths(lengths: np.ndarray, cols: int, seed: int) -> sp.csr_matrix:
    """Distinct sorted columns per row (a full row when the length is cols),
    U(-1,1) values."""
    rng = np.random.default_rng(seed)
    indptr = np.zeros(lengths.size + 1, dtype=np.int64)
    np.cumsum(lengths, out=indptr[1:])
    indices = np.empty(int(indptr[-1]), dtype=np.int64)
    for r, L in enumerate(lengths):
        L = int(L)
        if L == cols:
            indices[indptr[r]:indptr[r + 1]] = np.arange(cols)
        elif L:
            indices[indptr[r]:indptr[r + 1]] = np.sort(rng.choice(cols, size=L, replace=False))
    return sp.csr_matrix((rng.uniform(-1.0, 1.0, indices.size), indices, indptr),
                         shape=(lengths.size, cols))


def skew_matrices(scale: float = 1.0) -> Dict[str, sp.csr_matrix]:
    """The skewed matrices compared (M = N = 100000 at scale 1)."""
    n = max(1000, int(100_000 * scale))
    ten = np.full(n, 8, dtype=np.int64)
    ten[5::max(1, n // 10)] = n
    one = np.full(n, 8, dtype=np.int64)
    one[n // 2] = n
    u = np.random.default_rng(5).uniform(size=n)
    power = np.minimum(n, np.floor(u ** (-1.0 / 1.03))).astype(np.int64)
    return {
        "ten full rows, 8 elsewhere": _rows_with_lengths(ten, n, 1),
        "one full row, 8 elsewhere": _rows_with_lengths(one, n, 2),
        "c3a's power law without its 5000 cap": _rows_with_lengths(power, n, 3),
    }


def compare(matrices: Dict[str, sp.csr_matrix], schedules=SCHEDULES, iters: int = 50,
            rotate_mb: int = 640) -> List[dict]:
    rows = []
    for label, A in matrices.items():
        M, N = A.shape
        x = baseline_operands("spmv", M, N, 1)["x"]
        want = A @ x
        host = [np.ascontiguousarray(A.indptr, dtype=np.int64),
                np.ascontiguousarray(A.indices, dtype=np.int64),
                np.ascontiguousarray(A.data, dtype=np.float64), x]
        per_copy = sum(a.nbytes for a in host) + 8 * M
        copies = min(max(2, -(-(rotate_mb << 20) // per_copy)), iters)
        sets = [[rt.DeviceBuffer(a) for a in host] + [rt.DeviceBuffer(nbytes=8 * M)]
                for _ in range(copies)]
        try:
            for cfg in schedules:
                for balance in FORMS:
                    c = Config(**{**cfg.to_dict(), "balance": balance})
                    v = Variant("spmv", c)
                    g, b, lds = v.geometry(M, N, 0, A.nnz)
                    kms, _ = rt.time_launches(v.function(), g, b, lds,
                                              [s + [M, N, A.nnz] for s in sets], 5, iters)
                    # every copy's output has been written by then (launches > copies)
                    got = sets[0][4].to_host(np.empty(M))
                    err = float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-300))
                    if not err <= TOL:
                        raise AssertionError("%s %s: rel err %.3e" % (label, c.short(), err))
                    rows.append({"matrix": label, "rows": M, "nnz": int(A.nnz),
                                 "max_row": int(np.diff(A.indptr).max()),
                                 "schedule": cfg.short(), "balance": balance,
                                 "us": float(np.median(kms)) * 1e3, "rel_err": err,
                                 "copies": copies})
                    print("[skew] %s %s %s %.2f us" % (label, cfg.short(), balance,
                                                       rows[-1]["us"]), flush=True)
        finally:
            for s in sets:
                for buf in s:
                    buf.free()
    return rows


def render(rows: List[dict], device: str) -> str:
    md = ["# Row tiles, merge-path windows and hybrid tiles (%s)" % device, "",
          "Written by `python -m tilegen_amd.skew`; SpMV kernel medians of dispatch-attached "
          "events over cold (rotated) inputs, each result within 1e-10 of float64 SciPy.", "",
          "| matrix | rows | nnz | longest row | schedule | row tiles µs | merge windows µs | "
          "hybrid tiles µs | merge / rows | hybrid / rows |",
          "|---|---:|---:|---:|---|---:|---:|---:|---:|---:|"]
    by = {}
    for r in rows:
        by.setdefault((r["matrix"], r["schedule"]), {})[r["balance"]] = r
    for (m, s), d in by.items():
        a = d["rows"]
        cells = ["%.2f" % d[f]["us"] if f in d else "-" for f in FORMS]
        ratios = ["%.2f" % (d[f]["us"] / a["us"]) if f in d else "-" for f in FORMS[1:]]
        md.append("| %s | %d | %d | %d | %s | %s |" % (
            m, a["rows"], a["nnz"], a["max_row"], s, " | ".join(cells + ratios)))
    return "\n".join(md) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Row tiles, merge windows, hybrid tiles on skew.")
    ap.add_argument("--out", default="results")
    ap.add_argument("--scale", type=float, default=1.0)
    a = ap.parse_args(argv)
    if rt.device_count() < 1:
        print("skew: no HIP device visible", file=sys.stderr)
        return 2
    dev = rt.device_info(0)
    mats = skew_matrices(a.scale)
    mats["c3a (BASELINE)"] = make_baseline("c3a", scale=a.scale)
    mats["c3b (BASELINE)"] = make_baseline("c3b", scale=a.scale)
    rows = compare(mats)
    os.makedirs(a.out, exist_ok=True)
    with open(os.path.join(a.out, "skew.json"), "w") as fh:
        json.dump({"device": dev, "rows": rows}, fh, indent=1)
    md = render(rows, "%s %s" % (dev["name"], dev["arch"]))
    with open(os.path.join(a.out, "skew.md"), "w") as fh:
        fh.write(md)
    print(md)
    return 0


if __name__ == "__main__":
    sys.exit(main())

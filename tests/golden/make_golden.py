"""Writes the golden fixtures of this directory.

ref_kats.json        inputs and expected outputs of the reference's C++
                     known-answer tests (cpp/tests/test_ref.cpp:25-116), one
                     record per TEST_CASE, transcribed as data.
manifest_stats.json  the reference corpus statistics, copied field by field
                     from the reference's data/matrices/manifest.json (seed
                     1234; nnz, mean, median, max, stddev, imbalance per class).

Run from the repository root while /root/reference is mounted:
    python tests/golden/make_golden.py [/root/reference]
The fixtures are committed; tests never read /root/reference.
"""

from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))

# cpp/tests/test_ref.cpp: each record = (test name, kernel, inputs, expected)
KATS = [
    {"case": "2x2 identity csr_spmv", "source": "cpp/tests/test_ref.cpp:25-34",
     "kernel": "spmv", "rows": 2, "cols": 2, "indptr": [0, 1, 2], "indices": [0, 1],
     "data": [1.0, 1.0], "x": [3.0, -4.0], "expected": [3.0, -4.0]},
    {"case": "dense_spmv matches hand computation", "source": "cpp/tests/test_ref.cpp:36-44",
     "kernel": "dense_spmv", "rows": 2, "cols": 2, "dense": [1.0, 2.0, 3.0, 4.0],
     "x": [5.0, 6.0], "expected": [17.0, 39.0]},
    {"case": "empty row yields zero", "source": "cpp/tests/test_ref.cpp:46-55",
     "kernel": "spmv", "rows": 3, "cols": 3, "indptr": [0, 1, 1, 2], "indices": [0, 2],
     "data": [2.0, 5.0], "x": [1.0, 1.0, 1.0], "expected": [2.0, 0.0, 5.0]},
    {"case": "all-zero-data matrix yields zero", "source": "cpp/tests/test_ref.cpp:57-64",
     "kernel": "spmv", "rows": 2, "cols": 2, "indptr": [0, 2, 3], "indices": [0, 1, 1],
     "data": [0.0, 0.0, 0.0], "x": [7.0, 9.0], "expected": [0.0, 0.0]},
    {"case": "csr_spmm small", "source": "cpp/tests/test_ref.cpp:66-77",
     "kernel": "spmm", "rows": 2, "cols": 2, "indptr": [0, 2, 3], "indices": [0, 1, 1],
     "data": [1.0, 2.0, 3.0], "K": 2, "B": [1.0, 0.0, 0.0, 1.0],
     "expected": [1.0, 2.0, 0.0, 3.0]},
    {"case": "sddmm sampled product", "source": "cpp/tests/test_ref.cpp:79-90",
     "kernel": "sddmm", "rows": 2, "cols": 2, "indptr": [0, 1, 2], "indices": [0, 1],
     "data": [1.0, 1.0], "K": 2, "U": [1.0, 2.0, 3.0, 4.0], "V": [1.0, 0.0, 0.0, 1.0],
     "expected": [1.0, 4.0]},
    {"case": "fused_spmv_axpy", "source": "cpp/tests/test_ref.cpp:92-102",
     "kernel": "fused_spmv_axpy", "rows": 2, "cols": 2, "indptr": [0, 2, 3],
     "indices": [0, 1, 1], "data": [1.0, 1.0, 1.0], "x": [1.0, 2.0], "w": [1.0, 1.0],
     "alpha": 2.0, "beta": 3.0, "expected": [9.0, 7.0]},
    {"case": "float path produces same result", "source": "cpp/tests/test_ref.cpp:104-116",
     "kernel": "spmv", "rows": 2, "cols": 2, "indptr": [0, 1, 2], "indices": [0, 1],
     "data": [1.0, 1.0], "x": [3.0, -4.0], "expected": [3.0, -4.0]},
]


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    ref = argv[0] if argv else "/root/reference"
    with open(os.path.join(HERE, "ref_kats.json"), "w") as fh:
        json.dump(KATS, fh, indent=1)
    man = os.path.join(ref, "data", "matrices", "manifest.json")
    if os.path.exists(man):
        with open(man) as fh:
            m = json.load(fh)
        keep = ["class_name", "rows", "cols", "nnz", "nnz_per_row_mean", "nnz_per_row_median",
                "nnz_per_row_max", "nnz_per_row_stddev", "imbalance_ratio"]
        out = {"seed": m["seed"], "source": "data/matrices/manifest.json",
               "matrices": [{k: e[k] for k in keep} for e in m["matrices"]]}
        with open(os.path.join(HERE, "manifest_stats.json"), "w") as fh:
            json.dump(out, fh, indent=1)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

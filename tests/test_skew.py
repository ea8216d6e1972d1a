"""Row tiles, merge-path windows and hybrid tiles (``python -m tilegen_amd.skew``)."""

from __future__ import annotations

import numpy as np
import pytest

from tilegen_amd import skew


def test_skew_matrices_have_the_stated_shapes():
    m = skew.skew_matrices(scale=0.02)
    n = 2000
    for label, A in m.items():
        assert A.shape == (n, n)
        lens = np.diff(A.indptr)
        assert lens.max() == n, label  # at least one full row
        for r in range(n):  # distinct sorted columns
            cols = A.indices[A.indptr[r]:A.indptr[r + 1]]
            assert np.all(np.diff(cols) > 0)
    assert (np.diff(m["ten full rows, 8 elsewhere"].indptr) == n).sum() == 10


def test_render_lines_up_the_three_forms():
    rows = [{"matrix": "m", "rows": 10, "nnz": 99, "max_row": 10, "schedule": "T16/TPR8/U2/V1/B128",
             "balance": b, "us": us, "rel_err": 0.0, "copies": 2}
            for b, us in (("rows", 40.0), ("nnz", 10.0), ("hybrid", 20.0))]
    md = skew.render(rows, "x")
    assert ("| m | 10 | 99 | 10 | T16/TPR8/U2/V1/B128 | 40.00 | 10.00 | 20.00 | 0.25 | 0.50 |"
            in md)


@pytest.mark.gpu
def test_skew_compare_runs(hip_ready):
    # compare() checks each result against float64 SciPy before it reports a time
    mats = dict(list(skew.skew_matrices(scale=0.02).items())[:2])
    rows = skew.compare(mats, schedules=skew.SCHEDULES[:1], iters=3, rotate_mb=8)
    assert len(rows) == 2 * len(skew.FORMS) and all(r["us"] > 0 and r["rel_err"] <= 1e-10 for r in rows)

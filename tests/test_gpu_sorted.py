"""GPU: row tiles whose first-step gathers are sorted in LDS (gather "sorted").

The sort changes only the order in which a tile's operands are fetched: every
lane reads its own operands back and sums them in the order the direct gathers
use, so a sorted variant gives the same bits as the direct variant of the same
schedule.  That is checked on the uniform BASELINE matrix at full size (c1), on
scaled power-law and dense-row matrices (rows longer than the first step take
the direct steps, the wave tier and the workgroup tier), on a matrix with
more columns than the buckets can hold one each (2^20 columns), and against the
C oracle within 1e-10.  The balanced-form suite (test_gpu_merge.py) and the
row-block views (test_gpu_views.py) run the same schedules on their edge cases.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import oracle
from tests.util import ragged, rel_2, rel_inf
from tilegen_amd.matrices import make_baseline
from tilegen_amd.schedules import SORTED_TEST_SCHEDULES, schedule_id
from tilegen_amd.variant import Variant

pytestmark = pytest.mark.gpu

TOL = 1e-10


def _matrices():
    yield "c1", make_baseline("c1")
    yield "c3a/4", make_baseline("c3a", scale=0.25)
    yield "c3b/2", make_baseline("c3b", scale=0.5)
    yield "wide", ragged(41, 3000, 1 << 20, 24, empty_every=5, long_rows=[(9, 9000)])


@pytest.mark.parametrize("cfg", SORTED_TEST_SCHEDULES,
                         ids=[schedule_id(c) for c in SORTED_TEST_SCHEDULES])
def test_sorted_gathers_give_the_direct_bits(cfg, hip_ready):
    direct = dataclasses.replace(cfg, gather="direct")
    for label, A in _matrices():
        A.indptr = A.indptr.astype(np.int64)
        A.indices = A.indices.astype(np.int64)
        x = np.random.default_rng(3).uniform(-1, 1, A.shape[1])
        print("[sorted] %s %s rows=%d nnz=%d" % (cfg.short(), label, A.shape[0], A.nnz),
              flush=True)
        got = Variant("spmv", cfg).run(A, out=np.full(A.shape[0], np.nan), x=x)
        want = Variant("spmv", direct).run(A, x=x)
        assert got.tobytes() == want.tobytes(), (cfg.short(), label)
        ref = oracle.spmv(A, x)
        assert rel_inf(got, ref) <= TOL and rel_2(got, ref) <= TOL, (cfg.short(), label)

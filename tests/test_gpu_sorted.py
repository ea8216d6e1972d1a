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
from tilegen_amd.schedules import SORTED_TEST_SCHEDULES, TUNED, schedule_id
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


def _guess_mixed(M=3000, L=16, seed=4):
    """Rows of L nonzeros except perturbed runs whose lengths still sum to a
    multiple of L, so nnz = L M (the guessed first step is made) while the rows in
    and just after each run start elsewhere than r L (they load again): pairs
    (L - 4, L + 4), (0, 2 L), (L + 3, L - 3), a run (0, 0, 3 L), one long row of
    40 L balanced by empty rows, and the last row empty."""
    import scipy.sparse as sp
    lens = np.full(M, L, dtype=np.int64)
    lens[10:12] = (L - 4, L + 4)
    lens[50:52] = (0, 2 * L)
    lens[101:103] = (L + 3, L - 3)
    lens[200:203] = (0, 0, 3 * L)
    lens[700] = 40 * L
    lens[701:740] = 0
    lens[M - 2:] = (2 * L, 0)
    assert lens.sum() == L * M
    ip = np.concatenate([[0], np.cumsum(lens)])
    rng = np.random.default_rng(seed)
    N = 5000
    idx = np.concatenate([np.sort(rng.choice(N, n, replace=False)) for n in lens])
    return sp.csr_matrix((rng.uniform(-1, 1, ip[-1]), idx, ip), shape=(M, N))


_MIXED = list(SORTED_TEST_SCHEDULES[:4]) + [TUNED["c1"]]


@pytest.mark.parametrize("cfg", _MIXED, ids=[schedule_id(c) for c in _MIXED])
def test_sorted_guess_right_for_some_rows_only(cfg, hip_ready):
    """nnz is a multiple of M, so the first step is loaded at the guessed positions;
    the perturbed rows (and a long row that leaves its lane group) load again."""
    A = _guess_mixed(L=cfg.threads_per_row * cfg.unroll if cfg.unroll % 2 == 0 else 16)
    A.indptr = A.indptr.astype(np.int64)
    A.indices = A.indices.astype(np.int64)
    x = np.random.default_rng(8).uniform(-1, 1, A.shape[1])
    direct = dataclasses.replace(cfg, gather="direct")
    print("[sorted] guess-mixed %s rows=%d nnz=%d" % (cfg.short(), A.shape[0], A.nnz), flush=True)
    got = Variant("spmv", cfg).run(A, out=np.full(A.shape[0], np.nan), x=x)
    want = Variant("spmv", direct).run(A, x=x)
    assert got.tobytes() == want.tobytes(), cfg.short()
    ref = oracle.spmv(A, x)
    assert rel_inf(got, ref) <= TOL and rel_2(got, ref) <= TOL, cfg.short()

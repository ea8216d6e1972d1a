"""GPU parity of the merge-path (balance "nnz"), hybrid (balance "hybrid") and
stream (balance "stream") SpMV and fused_spmv_axpy.

Each workgroup takes an equal share of rows plus nonzeros, finds its first and
last rows with a search of the row pointers, sums the rows that begin in its
share whole, and adds its piece of any row longer than a share to the scratch
the last piece reads back.  Hybrid tiles keep row tiles but leave rows longer
than half a nonzero range to workgroups that each take one range, with the
same piece combine.  Stream ranges give every workgroup one equal range of
nonzeros and the rows that end in it, and combine the rows cut at range edges
the same way.  The matrices put that logic at its edges: no
nonzeros, one row, rows ending exactly at the last nonzero, a row spanning
hundreds of windows (more than one wave of pieces to combine), long first and
last rows, mostly empty rows, power-law and dense-row patterns, and more
windows or ranges than the scratch holds (rows past it are summed whole).  Every result
must meet the 1e-10 normwise bar against the C oracle and float64 SciPy, and
launching again onto NaN-filled outputs must give the same bits (the piece
order is fixed and every partial slot is empty again).  Launches go through
``launch_<name>`` with device pointers.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_gpu_parity import TOL, _check, _operands
from tests.util import csr, ragged, range_edge_matrix, rel_inf
from tilegen_amd import codegen as cg
from tilegen_amd.codegen import Config
from tilegen_amd.matrices import make_baseline
from tilegen_amd.schedules import (HYBRID_TEST_SCHEDULES, MERGE_TEST_SCHEDULES,
                                   SORTED_TEST_SCHEDULES, STREAM_TEST_SCHEDULES, schedule_id)
from tilegen_amd.variant import Variant

pytestmark = pytest.mark.gpu


def _cases():
    return {
        "no_nonzeros": csr(100, 50, np.zeros(101, dtype=np.int64), [], []),
        "single": csr(1, 1, [0, 1], [0], [2.5]),
        "last_row_to_nnz_end": csr(3, 5, [0, 1, 2, 7], [0, 1, 0, 1, 2, 3, 4],
                                   [1, 2, 3, 4, 5, 6, 7]),
        "one_huge_row": ragged(4, 400, 30000, 2, long_rows=[(200, 25000)]),
        "huge_first_and_last": ragged(5, 300, 9000, 5,
                                      long_rows=[(0, 8000), (299, 7000), (150, 6)]),
        "mostly_empty": ragged(3, 3000, 500, 3, empty_every=2, long_rows=[(7, 400)]),
        "power_law": make_baseline("c3a", scale=0.05),
        "dense_rows": make_baseline("c3b", scale=0.1),
        "every_row_long": ragged(21, 200, 3000, 0, long_rows=[(r, 300 + r) for r in range(200)]),
        "uniform": make_baseline("c1", scale=0.02),
    }


def _again_onto_nan(kernel, cfg, A, first):
    """A second launch onto NaNs gives the same bits as the first."""
    ops = _operands(kernel, A, 1)
    out = Variant(kernel, cfg).run(A, out=np.full(A.shape[0], np.nan), **ops)
    assert np.array_equal(out, first)


_BALANCED = (MERGE_TEST_SCHEDULES + HYBRID_TEST_SCHEDULES + STREAM_TEST_SCHEDULES
             + SORTED_TEST_SCHEDULES)


@pytest.mark.parametrize("cfg", _BALANCED, ids=[schedule_id(c) for c in _BALANCED])
@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy"])
def test_merge_path_matches_oracle(kernel, cfg, hip_ready):
    for label, A in _cases().items():
        print("[gpu] merge %s %s %s rows=%d nnz=%d" % (kernel, cfg.short(), label,
                                                      A.shape[0], A.nnz), flush=True)
        out = _check(kernel, cfg, A, K=1, label=label)
        _again_onto_nan(kernel, cfg, A, out)


@pytest.mark.parametrize("balance", ["nnz", "hybrid", "stream"])
def test_zero_rows_launch_nothing(balance, hip_ready):
    """No rows and no nonzeros make an empty grid: the launcher returns before
    any kernel runs, and the next launch of the same variant is unaffected."""
    v = Variant("spmv", Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256,
                               balance=balance))
    out = v.run(csr(0, 4, np.zeros(1, dtype=np.int64), [], []), x=np.ones(4))
    assert out.shape == (0,)
    A = _cases()["huge_first_and_last"]
    x = _operands("spmv", A, 1)["x"]
    got = v.run(A, x=x)
    assert rel_inf(got, A @ x) <= TOL


def test_merge_path_more_windows_than_scratch(hip_ready):
    """100000 windows (two rows each) against 65536 scratch slots: the long row
    near the top is cut into pieces, the one near the bottom is summed whole by
    the window it begins in."""
    rows = 200_000
    A = ragged(31, rows, 60_000, 1, long_rows=[(10, 5000), (rows - 900, 6000)])
    cfg = Config(tile_size=2, threads_per_row=4, unroll=1, block_size=64, balance="nnz")
    G = -(-rows // 2)
    X = rows + A.nnz
    D = -(-X // G)  # items per window
    assert G > cg.MERGE_CAP
    assert (rows - 900 + int(A.indptr[rows - 900 + 1]) - 1) // D >= cg.MERGE_CAP
    assert (10 + int(A.indptr[11]) - 1) // D < cg.MERGE_CAP
    print("[gpu] merge scratch capacity rows=%d nnz=%d windows=%d" % (rows, A.nnz, G),
          flush=True)
    out = _check("spmv", cfg, A, K=1, label="past_scratch")
    _again_onto_nan("spmv", cfg, A, out)


def test_hybrid_more_ranges_than_scratch(hip_ready):
    """70357 ranges of 128 nonzeros against 65536 scratch slots: the long row
    near the top is cut into pieces combined through the scratch; the one near
    the bottom, and every row over 64 nonzeros that reaches past the last slot,
    is summed whole by the range it begins in."""
    rows = 150_000
    A = ragged(37, rows, 512, 120, long_rows=[(10, 512), (rows - 50, 512)])
    cfg = Config(tile_size=64, threads_per_row=4, unroll=1, block_size=64, balance="hybrid")
    CH = Variant("spmv", cfg).gen.geometry.nnz_chunk
    assert CH == 128 and -(-A.nnz // CH) > cg.MERGE_CAP
    ip = A.indptr
    assert 0 < (ip[11] - 1) // CH - ip[10] // CH and (ip[11] - 1) // CH < cg.MERGE_CAP
    assert ip[rows - 50] // CH < (ip[rows - 49] - 1) // CH and ip[rows - 50] // CH >= cg.MERGE_CAP
    print("[gpu] hybrid scratch capacity rows=%d nnz=%d ranges=%d" % (rows, A.nnz, -(-A.nnz // CH)),
          flush=True)
    out = _check("spmv", cfg, A, K=1, label="hybrid_past_scratch")
    _again_onto_nan("spmv", cfg, A, out)


@pytest.mark.parametrize("cfg", HYBRID_TEST_SCHEDULES, ids=[schedule_id(c) for c in
                                                           HYBRID_TEST_SCHEDULES])
@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy"])
def test_hybrid_range_edges(kernel, cfg, hip_ready):
    """Every hybrid schedule on rows placed at its own ranges' edges: rows just
    under and over the long-row length, three long rows meeting one range, rows
    on range boundaries, two-piece and four-piece rows."""
    CH = Variant(kernel, cfg).gen.geometry.nnz_chunk
    A = range_edge_matrix(CH, seed=CH)
    lens = np.diff(A.indptr)
    assert (lens == CH // 2 + 1).sum() >= 6 and (lens > 3 * CH).any()
    assert (A.indptr[:-1][lens > CH // 2] % CH == 0).any()
    print("[gpu] hybrid edges %s %s CH=%d rows=%d nnz=%d" % (kernel, cfg.short(), CH,
                                                            A.shape[0], A.nnz), flush=True)
    out = _check(kernel, cfg, A, K=1, label="range_edges")
    _again_onto_nan(kernel, cfg, A, out)


def test_merge_path_agrees_with_row_tiles(hip_ready):
    """The same schedule with row tiles, merge-path windows, hybrid tiles and
    stream ranges: all meet the bar on the BASELINE skewed cases at a tenth of
    their size, and agree with each other to it."""
    for case_id, base in (("c3a", (64, 8, 2, 512)), ("c3b", (32, 32, 2, 1024))):
        A = make_baseline(case_id, scale=0.1)
        ops = _operands("spmv", A, 1)
        T, tpr, U, B = base
        rows = Variant("spmv", Config(tile_size=T, threads_per_row=tpr, unroll=U,
                                      block_size=B)).run(A, **ops)
        for balance in ("nnz", "hybrid", "stream"):
            other = Variant("spmv", Config(tile_size=T, threads_per_row=tpr, unroll=U,
                                           block_size=B, balance=balance)).run(A, **ops)
            assert rel_inf(other, rows) <= TOL, (case_id, balance)


@pytest.mark.parametrize("cfg", MERGE_TEST_SCHEDULES[:2] + HYBRID_TEST_SCHEDULES[:2] +
                         STREAM_TEST_SCHEDULES[:2],
                         ids=[schedule_id(c) for c in MERGE_TEST_SCHEDULES[:2] +
                              HYBRID_TEST_SCHEDULES[:2] + STREAM_TEST_SCHEDULES[:2]])
@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy"])
def test_verify_api_with_balance(kernel, cfg, hip_ready, tmp_path):
    """The reference's verify() on its 257 x 257 test matrix with merge-path,
    hybrid and stream schedules: the reference tolerance, the 1e-10 normwise bar
    and indptr/indices untouched."""
    from tests.util import mixed_257
    from tilegen_amd.verify import verify
    r = verify(kernel, cfg, mixed_257(), backend="hip", workdir=str(tmp_path), K=8)
    assert r.executed and r.ok, r.message
    assert r.max_abs_err <= r.tolerance
    assert r.rel_err_inf <= TOL and r.rel_err_2 <= TOL
    assert r.structure_intact is True


def test_tune_with_balance_candidates(hip_ready, tmp_path):
    """tune() times and verifies merge-path, hybrid and stream candidates beside
    row tiles on a skewed matrix; every candidate it ran is correct and the
    winner is one of them."""
    from tilegen_amd.autotune import tune
    A = make_baseline("c3a", scale=0.05)
    inc = [MERGE_TEST_SCHEDULES[1], HYBRID_TEST_SCHEDULES[1], HYBRID_TEST_SCHEDULES[0],
           STREAM_TEST_SCHEDULES[0]]
    res = tune("spmv", A, budget=len(inc) + 1, mode="random", backend="hip", include=inc,
               iters=5, warmup=2, workdir=str(tmp_path))
    ran = [r for r in res["records"] if r.get("ms_median") is not None]
    assert len(ran) == len(inc) + 1
    assert all(r["ok"] for r in ran)
    assert res["winner"] in [r["config"] for r in ran]
    assert {r["config"].get("balance", "rows") for r in ran} == {"rows", "nnz", "hybrid",
                                                                 "stream"}


def _device_set(A, ops, out_len):
    from tilegen_amd import runtime as rt
    bufs = {"indptr": rt.DeviceBuffer(np.ascontiguousarray(A.indptr, dtype=np.int64)),
            "indices": rt.DeviceBuffer(np.ascontiguousarray(A.indices, dtype=np.int64)),
            "data": rt.DeviceBuffer(np.ascontiguousarray(A.data, dtype=np.float64)),
            "x": rt.DeviceBuffer(np.ascontiguousarray(ops["x"], dtype=np.float64)),
            "y": rt.DeviceBuffer(np.full(out_len, np.nan))}
    return bufs


@pytest.mark.parametrize("case_id", ["c3a", "c3b"])
def test_scratch_variant_on_two_streams(case_id, hip_ready):
    """The tuned skewed-row variants (stream ranges on c3a and c3b) combine row
    pieces through one module scratch per device.  Launches on two streams, enqueued back to back with no
    host synchronization in between (and two more on the null stream), are
    ordered by the launcher, so every output equals a serial launch's bits."""
    from tilegen_amd import runtime as rt
    from tilegen_amd.schedules import TUNED
    A = make_baseline(case_id, scale=0.25)
    B = make_baseline(case_id, scale=0.1)
    M, N = A.shape
    v = Variant("spmv", TUNED[case_id])
    k = _kernel("spmv", TUNED[case_id])
    assert cg.module_scratch(cg._plan(k), cg._lowering(k))
    opsA, opsB = _operands("spmv", A, 1), _operands("spmv", B, 1)
    serialA = v.run(A, **opsA)
    serialB = v.run(B, **opsB)
    assert rel_inf(serialA, _check("spmv", TUNED[case_id], A, K=1)) == 0.0
    s1, s2 = rt.stream_create(), rt.stream_create()
    sets = []
    try:
        for i in range(6):
            X, ops = (A, opsA) if i % 2 == 0 else (B, opsB)
            bufs = _device_set(X, ops, X.shape[0])
            sets.append((X, bufs))
        print("[gpu] two-stream %s launches=%d rows=%d/%d" % (case_id, len(sets), M,
                                                                B.shape[0]), flush=True)
        for i, (X, bufs) in enumerate(sets):
            stream = (s1, s2, None)[i % 3]
            vals = v.abi_values(X, bufs, {}, X.shape[0], X.shape[1], 0, int(X.nnz))
            v.launch_async(vals, stream)
        rt.synchronize()
        for i, (X, bufs) in enumerate(sets):
            got = bufs["y"].to_host()
            want = serialA if X is A else serialB
            assert np.array_equal(got, want), "launch %d (stream %d) differs" % (i, i % 3)
    finally:
        for _X, bufs in sets:
            for b in bufs.values():
                b.free()
        rt.stream_destroy(s1)
        rt.stream_destroy(s2)


def _kernel(name, cfg):
    from tilegen_amd import passes
    from tilegen_amd.dsl import standard_kernels
    return passes.run_pipeline(standard_kernels()[name], cfg, backend="hip")


def _stream_scratch_matrix(CH):
    """About 75000 ranges of CH nonzeros: a long row near the top (cut into
    pieces inside the scratch), one straddling the last range with slots, and
    one beginning past it."""
    rows, max_len, seed = 2500 * CH, 60, 41
    lengths = np.random.default_rng(seed).integers(0, max_len + 1, size=rows)
    lengths[10] = 700
    starts = np.concatenate([[0], np.cumsum(lengths)])
    edge = int(np.searchsorted(starts, cg.MERGE_CAP * CH - 300, side="right")) - 1
    return ragged(seed, rows, 4096, max_len,
                  long_rows=[(10, 700), (edge, 900), (rows - 60, 900)]), edge


@pytest.mark.parametrize("cfg", [
    Config(tile_size=64, threads_per_row=1, unroll=1, block_size=64, balance="stream"),
    Config(tile_size=64, threads_per_row=4, unroll=1, block_size=128, balance="stream"),
], ids=["one-wave", "two-waves"])
def test_stream_more_ranges_than_scratch(cfg, hip_ready):
    """More ranges than the 65536 with scratch slots: the long row near the top
    is combined through the scratch; the row straddling the last range with
    slots and the row beginning past it are summed whole, with their own loads,
    by the workgroup of the range each begins in (one wave, then two, whose sums
    are added in wave order)."""
    CH = Variant("spmv", cfg).gen.geometry.nnz_chunk
    A, edge = _stream_scratch_matrix(CH)
    rows, ip = A.shape[0], A.indptr
    assert CH == cfg.block_size and -(-A.nnz // CH) > cg.MERGE_CAP
    assert ip[10] // CH < (ip[11] - 1) // CH < cg.MERGE_CAP
    assert ip[edge] // CH < cg.MERGE_CAP <= (ip[edge + 1] - 1) // CH
    assert cg.MERGE_CAP <= ip[rows - 60] // CH < (ip[rows - 59] - 1) // CH
    print("[gpu] stream scratch capacity rows=%d nnz=%d ranges=%d" % (rows, A.nnz, -(-A.nnz // CH)),
          flush=True)
    out = _check("spmv", cfg, A, K=1, label="stream_past_scratch")
    _again_onto_nan("spmv", cfg, A, out)


def _random_skewed(seed: int):
    """A seeded random CSR matrix: random shape, Zipf row lengths with a random
    share of empty rows, and sometimes three rows thousands of nonzeros long."""
    rng = np.random.default_rng(1000 + seed)
    M, N = int(rng.integers(1, 6000)), int(rng.integers(1, 8000))
    lengths = np.minimum(rng.zipf(1.5 + rng.random(), size=M) - 1, N)
    lengths[rng.random(M) < rng.random() * 0.5] = 0
    if rng.random() < 0.5 and M > 2:
        for r in rng.integers(0, M, size=3):
            lengths[r] = min(N, int(rng.integers(500, 6000)))
    indptr = np.zeros(M + 1, dtype=np.int64)
    np.cumsum(lengths, out=indptr[1:])
    indices = np.empty(int(indptr[-1]), dtype=np.int64)
    for r in range(M):
        if lengths[r]:
            indices[indptr[r]:indptr[r + 1]] = np.sort(rng.choice(N, size=int(lengths[r]),
                                                                 replace=False))
    return csr(M, N, indptr, indices, rng.uniform(-1, 1, size=indices.size))


_SKEWED_STREAM = STREAM_TEST_SCHEDULES[:4] + STREAM_TEST_SCHEDULES[-2:]


@pytest.mark.parametrize("cfg", _SKEWED_STREAM, ids=[schedule_id(c) for c in _SKEWED_STREAM])
def test_stream_random_skewed_matrices(cfg, hip_ready):
    """24 seeded random skewed matrices (4,600 cut rows, 1,400 of them in more than
    two pieces, across the six range sizes swept, two of them from blocks of 3
    and 7 waves): every one meets the bar against the oracle and SciPy, and a
    second launch onto NaNs gives the same bits."""
    for seed in range(24):
        A = _random_skewed(seed)
        print("[gpu] stream random seed=%d %s rows=%d nnz=%d" % (seed, cfg.short(), A.shape[0],
                                                                 A.nnz), flush=True)
        out = _check("spmv", cfg, A, K=1, label="random%d" % seed)
        _again_onto_nan("spmv", cfg, A, out)

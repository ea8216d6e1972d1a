"""GPU: the launch ABI's absolute-position contract, as the reference's kernels
have it.  Those kernels walk each row by indptr alone and never read nnz
(reference tilegen/codegen.py:274 declares it, :593-643 and :646-714 never use
it), so a caller may pass a block of rows of a larger matrix -- indptr pointing
into the larger matrix's row pointers, so that indptr[0] > 0, with the larger
matrix's indices/data -- and any nnz, and still get the block's product.

Every SpMV form here (row tiles, merge-path windows, hybrid tiles, stream ranges),
fused_spmv_axpy, SpMM and SDDMM is run on such blocks, with indptr[0] odd and
even, and with nnz exact, the larger matrix's, between the two, zero and too small
(never past the arrays' length, the launch ABI's precondition):

* the result matches the C oracle on the block within 1e-10 (normwise), and is
  bit-identical for every nnz that covers the block's nonzeros (exact, the larger
  matrix's, between the two).  An undercounted nnz (zero, a third) gives the same
  product too; stream and hybrid variants then sum the rows past their grid's
  last range in another order, so only the tolerance is asserted there;
* data outside the block's positions is NaN, so any use of it would show;
* indptr/indices are byte-identical after the launch, and SDDMM writes no
  output position outside the block.

A launch given too small an nnz used to leave a scratch slot of the stream,
hybrid and merge variants full, which corrupted every later launch of that
variant; the last test makes such a call between two correct ones.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.util import ragged, rel_2, rel_inf
from tilegen_amd import runtime as rt
from tilegen_amd.schedules import (HYBRID_TEST_SCHEDULES, MERGE_TEST_SCHEDULES, NOALLOC_SCHEDULE,
                                   SORTED_TEST_SCHEDULES, STREAM_TEST_SCHEDULES, TEST_SCHEDULES,
                                   TUNED, schedule_id)
from tilegen_amd.variant import Variant

pytestmark = pytest.mark.gpu

TOL = 1e-10

SPMV_FORMS = [TUNED["c1"], TUNED["c2"], TEST_SCHEDULES[0], TEST_SCHEDULES[4],
              MERGE_TEST_SCHEDULES[1], MERGE_TEST_SCHEDULES[6], NOALLOC_SCHEDULE,
              HYBRID_TEST_SCHEDULES[6], TUNED["c3a"], TUNED["c3b"], STREAM_TEST_SCHEDULES[2],
              SORTED_TEST_SCHEDULES[0], SORTED_TEST_SCHEDULES[3]]
SCRATCH_FORMS = [TUNED["c3a"], TUNED["c3b"], STREAM_TEST_SCHEDULES[0], NOALLOC_SCHEDULE,
                 HYBRID_TEST_SCHEDULES[1], MERGE_TEST_SCHEDULES[1]]


def _big():
    """4000 x 3000: rows of 0..20, every 9th empty, and five long rows (1200 to
    2999 nonzeros) so that stream and hybrid ranges cut rows."""
    return ragged(21, 4000, 3000, 20, empty_every=9,
                  long_rows=[(5, 2500), (600, 2999), (1500, 1200), (1501, 1300), (3990, 2800)])


def _block(A, parity):
    """(r0, r1): a block of rows from near the start to near the end whose first
    position indptr[r0] has the given parity and is not 0."""
    ip = A.indptr
    r0 = next(r for r in range(3, 50) if ip[r] % 2 == parity and ip[r] > 0)
    r1 = next(r for r in range(3993, 3960, -1) if ip[r] > ip[r0])
    return r0, r1


def _hints(view_nnz, full_nnz):
    """label -> (nnz given to the launch, whether it covers the block's nonzeros).
    Every nnz stays within the arrays' length, the launch ABI's precondition
    (indices/data hold at least nnz entries: a launch may load positions below
    nnz outside the block, and uses none of them)."""
    return {"exact": (view_nnz, True), "whole matrix": (full_nnz, True),
            "between": ((view_nnz + full_nnz) // 2, True), "zero": (0, False),
            "a third": (view_nnz // 3, False)}


def _run_view(kernel, cfg, A, r0, r1, nnz_hint, ops):
    """One launch of ``kernel`` on rows [r0, r1) of A through the C ABI, indptr
    pointing into A's row pointers and indices/data A's whole arrays (NaN outside
    the block).  Returns (output, output buffer content outside the block)."""
    ip = np.ascontiguousarray(A.indptr[r0:r1 + 1], dtype=np.int64)
    pbase, pend = int(ip[0]), int(ip[-1])
    data = np.array(A.data, dtype=np.float64)
    data[:pbase] = np.nan
    data[pend:] = np.nan
    Mv, N = r1 - r0, A.shape[1]
    bufs = {"indptr": rt.DeviceBuffer(ip),
            "indices": rt.DeviceBuffer(np.ascontiguousarray(A.indices, dtype=np.int64)),
            "data": rt.DeviceBuffer(data)}
    K = 0
    scalars = {}
    if kernel in ("spmv", "fused_spmv_axpy"):
        bufs["x"] = rt.DeviceBuffer(ops["x"])
        out_name, out_len = ("y", Mv) if kernel == "spmv" else ("z", Mv)
        if kernel == "fused_spmv_axpy":
            bufs["w"] = rt.DeviceBuffer(ops["w"][r0:r1].copy())
            scalars = {"alpha": ops["alpha"], "beta": ops["beta"]}
    elif kernel == "spmm":
        K = ops["B"].shape[1]
        bufs["B"] = rt.DeviceBuffer(ops["B"])
        out_name, out_len = "C", Mv * K
    else:
        K = ops["U"].shape[1]
        bufs["U"] = rt.DeviceBuffer(np.ascontiguousarray(ops["U"][r0:r1]))
        bufs["V"] = rt.DeviceBuffer(ops["V"])
        out_name, out_len = "C", int(A.nnz)   # indexed by absolute position
    bufs[out_name] = rt.DeviceBuffer(np.full(out_len, 12345.0))
    v = Variant(kernel, cfg)
    try:
        v.device_call(v.abi_values(None, bufs, scalars, Mv, N, K, nnz_hint))
        out = bufs[out_name].to_host()
        assert bufs["indptr"].to_host().tobytes() == ip.tobytes()
        assert bufs["indices"].to_host().tobytes() == \
            np.ascontiguousarray(A.indices, dtype=np.int64).tobytes()
    finally:
        for b in bufs.values():
            b.free()
    if kernel == "sddmm":
        outside = np.concatenate([out[:pbase], out[pend:]])
        return out[pbase:pend], outside
    return out.reshape(Mv, K) if kernel == "spmm" else out, np.zeros(0)


def _ops(A, K, seed=5):
    rng = np.random.default_rng(seed)
    M, N = A.shape
    return {"x": rng.uniform(-1, 1, N), "w": rng.uniform(-1, 1, M), "alpha": 0.75,
            "beta": -1.25, "B": rng.uniform(-1, 1, (N, K)), "U": rng.uniform(-1, 1, (M, K)),
            "V": rng.uniform(-1, 1, (N, K))}


def _want(kernel, A, r0, r1, ops):
    view = A[r0:r1]
    view.indptr = view.indptr.astype(np.int64)
    view.indices = view.indices.astype(np.int64)
    sub = dict(ops)
    if kernel == "fused_spmv_axpy":
        sub["w"] = ops["w"][r0:r1]
    if kernel == "sddmm":
        sub["U"] = ops["U"][r0:r1]
    return oracle.compute(kernel, view, sub)


def _check_block(kernel, cfg, parity, K=0):
    A = _big()
    r0, r1 = _block(A, parity)
    pbase, pend = int(A.indptr[r0]), int(A.indptr[r1])
    assert pbase % 2 == parity and pbase > 0 and pend < A.nnz
    ops = _ops(A, K)
    want = _want(kernel, A, r0, r1, ops)
    first = None
    for label, (hint, covers) in _hints(pend - pbase, int(A.nnz)).items():
        print("[views] %s %s parity %d rows [%d, %d) positions [%d, %d) nnz=%d (%s)"
              % (kernel, cfg.short(), parity, r0, r1, pbase, pend, hint, label), flush=True)
        got, outside = _run_view(kernel, cfg, A, r0, r1, hint, ops)
        assert np.all(np.isfinite(got)), (cfg.short(), label)
        ri, r2 = rel_inf(got, want), rel_2(got, want)
        assert ri <= TOL and r2 <= TOL, (kernel, cfg.short(), label, ri, r2)
        if outside.size:
            assert np.all(outside == 12345.0), (cfg.short(), label)
        if first is None:
            first = got
        elif covers:
            assert got.tobytes() == first.tobytes(), (kernel, cfg.short(), label)


@pytest.mark.parametrize("parity", [1, 0], ids=["odd", "even"])
@pytest.mark.parametrize("cfg", SPMV_FORMS, ids=[schedule_id(c) for c in SPMV_FORMS])
def test_spmv_row_block_of_a_larger_matrix(cfg, parity, hip_ready):
    _check_block("spmv", cfg, parity)


@pytest.mark.parametrize("cfg", [STREAM_TEST_SCHEDULES[0], HYBRID_TEST_SCHEDULES[1],
                                 MERGE_TEST_SCHEDULES[1]], ids=["stream", "hybrid", "nnz"])
def test_fused_spmv_axpy_row_block(cfg, hip_ready):
    _check_block("fused_spmv_axpy", cfg, 1)


@pytest.mark.parametrize("parity", [1, 0], ids=["odd", "even"])
def test_spmm_and_sddmm_row_block(parity, hip_ready):
    _check_block("spmm", TUNED["c4"], parity, K=8)
    _check_block("sddmm", TUNED["c5"], parity, K=16)


@pytest.mark.parametrize("cfg", SCRATCH_FORMS, ids=[schedule_id(c) for c in SCRATCH_FORMS])
def test_undercounted_nnz_then_a_correct_launch(cfg, hip_ready):
    """A launch told a third of the nonzeros (or one) gives the full product, and
    the next launch of the same variant (the same module scratch) gives the same
    bits as a launch made before it."""
    A = _big()
    A.indptr = A.indptr.astype(np.int64)
    A.indices = A.indices.astype(np.int64)
    x = np.random.default_rng(9).uniform(-1, 1, A.shape[1])
    want = oracle.spmv(A, x)
    v = Variant("spmv", cfg)
    M, N, nnz = A.shape[0], A.shape[1], int(A.nnz)
    bufs = {"indptr": rt.DeviceBuffer(A.indptr), "indices": rt.DeviceBuffer(A.indices),
            "data": rt.DeviceBuffer(np.asarray(A.data, dtype=np.float64)),
            "x": rt.DeviceBuffer(x), "y": rt.DeviceBuffer(np.full(M, np.nan))}
    outs, under = [], []
    try:
        for label, hint in (("before", nnz), ("a third", nnz // 3), ("after", nnz),
                            ("one", 1), ("after again", nnz)):
            print("[views] %s nnz=%d (%s)" % (cfg.short(), hint, label), flush=True)
            bufs["y"].upload(np.full(M, np.nan))
            v.device_call(v.abi_values(None, bufs, {}, M, N, 0, hint))
            (outs if hint == nnz else under).append(bufs["y"].to_host())
    finally:
        for b in bufs.values():
            b.free()
    for o in outs + under:
        assert rel_inf(o, want) <= TOL and rel_2(o, want) <= TOL, cfg.short()
    for o in outs[1:]:
        assert o.tobytes() == outs[0].tobytes(), cfg.short()

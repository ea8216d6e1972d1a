"""launch_spmv_noalloc (include/tilegen_noalloc.h, libtgna.so): the SpMV entry
point that allocates nothing, against launch_spmv of the same schedule.

Two calls in a row on one device, the second with a smaller matrix, each
through the C ABI with device pointers and an output pre-filled with NaN; both
must match launch_spmv's result bit for bit (the same kernel source, its slots
passed in) and the C oracle within the 1e-10 normwise bar, leave indptr/indices
untouched, and leave the library's static scratch ready for the next call.  Sizes past the scratch's limit and bad arguments are
refused before anything is launched."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from tests.util import rel_2, rel_inf
from tilegen_amd import runtime as rt
from tilegen_amd.matrices import baseline_operands, make_baseline
from tilegen_amd.schedules import NOALLOC_SCHEDULE
from tilegen_amd.variant import Variant

pytestmark = pytest.mark.gpu

TOL = 1e-10


def _noalloc(L, bufs, M, N, nnz):
    p = lambda k: ctypes.c_void_p(bufs[k].ptr)  # noqa: E731
    rt.lib().tg_clear_error()
    return L.launch_spmv_noalloc(p("indptr"), p("indices"), p("data"), p("x"), p("y"), M, N,
                                 nnz, None)


def test_noalloc_matches_launch_spmv_on_two_calls(hip_ready):
    L = rt.noalloc_lib()
    v = Variant("spmv", NOALLOC_SCHEDULE)
    mats = [("c3a full", make_baseline("c3a")), ("c3b x0.3", make_baseline("c3b", scale=0.3))]
    assert mats[1][1].nnz < mats[0][1].nnz and mats[1][1].shape[0] < mats[0][1].shape[0]
    for label, A in mats:
        M, N = A.shape
        nnz = int(A.nnz)
        x = baseline_operands("spmv", M, N, 1)["x"]
        print("[gpu] noalloc %s rows=%d nnz=%d" % (label, M, nnz), flush=True)
        want = v.run(A, x=x)                      # the existing entry point, launch_spmv
        host = {"indptr": np.ascontiguousarray(A.indptr, dtype=np.int64),
                "indices": np.ascontiguousarray(A.indices, dtype=np.int64),
                "data": np.ascontiguousarray(A.data, dtype=np.float64), "x": x,
                "y": np.full(M, np.nan)}
        bufs = {k: rt.DeviceBuffer(a) for k, a in host.items()}
        try:
            rc = _noalloc(L, bufs, M, N, nnz)
            assert rc == 0, rt.last_error()
            rt.synchronize()
            got = bufs["y"].to_host()
            assert np.isfinite(got).all(), label
            for name, ref in (("launch_spmv", want), ("oracle", oracle.spmv(A, x))):
                ri, r2 = rel_inf(got, ref), rel_2(got, ref)
                assert ri <= TOL and r2 <= TOL, "%s vs %s: %g %g" % (label, name, ri, r2)
            print("[gpu] noalloc %s max |diff| vs launch_spmv %.3g" % (
                label, float(np.abs(got - want).max())), flush=True)
            # the same kernel source with its slots passed in: the same bits
            assert np.array_equal(got, want), label
            for k in ("indptr", "indices"):
                assert bufs[k].to_host().tobytes() == host[k].tobytes(), k
        finally:
            for b in bufs.values():
                b.free()


def test_noalloc_refuses_sizes_past_its_scratch(hip_ready):
    """Refused on the host before any launch: null pointers are never touched."""
    L = rt.noalloc_lib()
    from tilegen_amd.build import noalloc_kernel_source
    src = noalloc_kernel_source()
    cap = int(src.split("#define TG_NA_MAX_NNZ ")[1].split("LL")[0])
    rt.lib().tg_clear_error()
    assert L.launch_spmv_noalloc(None, None, None, None, None, 10, 10, cap + 1, None) == -2
    assert "exceeds" in rt.last_error()
    assert L.launch_spmv_noalloc(None, None, None, None, None, -1, 10, 0, None) == -1
    assert L.launch_spmv_noalloc(None, None, None, None, None, 0, 10, 0, None) == 0

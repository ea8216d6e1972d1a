"""HIP graphs (tg_graph_*, include/tgrt.h): calls captured into a graph and
replayed.

The tuned c3a and c3b variants (stream ranges) combine cut rows through their
module's scratch, and launch_spmv_noalloc clears its static slots with a kernel
(no memset node) before its SpMV kernel.  Every replay must give the bits of
the same call made eagerly.  Replays alternate with eager calls of the same
code, ordered by synchronization as the runtime requires, and each of those is
checked too; the output is refilled with NaN before every run, so a replay
that wrote nothing would fail."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from tests.util import rel_2, rel_inf
from tilegen_amd import runtime as rt
from tilegen_amd.matrices import baseline_operands, make_baseline
from tilegen_amd.schedules import NOALLOC_SCHEDULE, TUNED
from tilegen_amd.variant import Variant

pytestmark = pytest.mark.gpu

REPLAYS = 4
TOL = 1e-10


def _device(A, x):
    host = {"indptr": np.ascontiguousarray(A.indptr, dtype=np.int64),
            "indices": np.ascontiguousarray(A.indices, dtype=np.int64),
            "data": np.ascontiguousarray(A.data, dtype=np.float64), "x": x,
            "y": np.full(A.shape[0], np.nan)}
    return host, {k: rt.DeviceBuffer(a) for k, a in host.items()}


def _replay_and_compare(label, exec_, stream, y, want, eager):
    nan = np.full(want.size, np.nan)
    for rep in range(REPLAYS):
        y.upload(nan)
        rt.graph_launch(exec_, stream, sync=True)
        got = y.to_host()
        assert np.array_equal(got, want), "%s replay %d differs from the eager call" % (label, rep)
        # the program's own eager work between replays
        y.upload(nan)
        eager()
        assert np.array_equal(y.to_host(), want), "%s eager call after replay %d" % (label, rep)


@pytest.mark.parametrize("case_id", ["c3a", "c3b"])
def test_scratch_variant_replays_from_a_graph(case_id, hip_ready):
    A = make_baseline(case_id)
    M, N = A.shape
    nnz = int(A.nnz)
    x = baseline_operands("spmv", M, N, 1)["x"]
    v = Variant("spmv", TUNED[case_id])
    want = v.run(A, x=x)                       # launch_spmv, eager and synchronous
    ref = oracle.spmv(A, x)
    assert rel_inf(want, ref) <= TOL and rel_2(want, ref) <= TOL
    host, bufs = _device(A, x)
    s = rt.stream_create()
    exec_ = None
    try:
        vals = v.abi_values(A, bufs, {}, M, N, 0, nnz)
        v.launch_async(vals, s)                # loads the module before the capture
        rt.stream_synchronize(s)
        assert np.array_equal(bufs["y"].to_host(), want)
        print("[gpu] graph %s %s rows=%d nnz=%d" % (case_id, TUNED[case_id].short(), M, nnz),
              flush=True)
        exec_ = rt.graph_capture(s, lambda: v.launch_async(vals, s))
        _replay_and_compare(case_id, exec_, s, bufs["y"], want, lambda: v.device_call(vals))
        for k in ("indptr", "indices"):
            assert bufs[k].to_host().tobytes() == host[k].tobytes(), k
    finally:
        if exec_:
            rt.graph_destroy(exec_)
        rt.stream_destroy(s)
        for b in bufs.values():
            b.free()


def test_noalloc_replays_from_a_graph(hip_ready):
    """The entry point for callers under capture: its clear kernel and its SpMV
    kernel become two graph nodes, and replays reuse the static slots."""
    L = rt.noalloc_lib()
    A = make_baseline("c3a")
    M, N = A.shape
    nnz = int(A.nnz)
    x = baseline_operands("spmv", M, N, 1)["x"]
    ref = Variant("spmv", NOALLOC_SCHEDULE).run(A, x=x)
    host, bufs = _device(A, x)
    p = {k: ctypes.c_void_p(b.ptr) for k, b in bufs.items()}
    s = rt.stream_create()
    exec_ = None

    def call(stream):
        rt.lib().tg_clear_error()
        rc = L.launch_spmv_noalloc(p["indptr"], p["indices"], p["data"], p["x"], p["y"], M, N,
                                   nnz, stream)
        assert rc == 0, rt.last_error()

    try:
        call(s)                                # resolves the device's scratch before the capture
        rt.stream_synchronize(s)
        want = bufs["y"].to_host()
        assert rel_inf(want, ref) <= TOL and rel_2(want, ref) <= TOL
        print("[gpu] graph noalloc rows=%d nnz=%d" % (M, nnz), flush=True)
        exec_ = rt.graph_capture(s, lambda: call(s))

        def eager():
            call(None)
            rt.synchronize()

        _replay_and_compare("noalloc", exec_, s, bufs["y"], want, eager)
        for k in ("indptr", "indices"):
            assert bufs[k].to_host().tobytes() == host[k].tobytes(), k
    finally:
        if exec_:
            rt.graph_destroy(exec_)
        rt.stream_destroy(s)
        for b in bufs.values():
            b.free()

"""The rocSPARSE comparison library (bench.py --vendor): exports, and on a GPU
its three timed calls produce the right products on the same buffers."""

from __future__ import annotations

import subprocess

import numpy as np
import pytest

import oracle
from tests.util import ragged, rel_inf
from tilegen_amd import runtime as rt
from tilegen_amd import vendor

pytestmark = pytest.mark.skipif(not vendor.available(), reason="rocSPARSE not installed")


def test_vendor_library_exports():
    out = subprocess.run(["nm", "-D", "--defined-only", vendor.lib_path()], capture_output=True,
                         text=True, check=True).stdout
    for name in ("tgv_vendor_spmv_time", "tgv_vendor_spmm_time", "tgv_vendor_sddmm_time",
                 "tgv_vendor_last_error"):
        assert name in out


@pytest.mark.gpu
def test_vendor_calls_compute_the_products(hip_ready):
    A = ragged(41, 600, 500, 12, empty_every=7, long_rows=[(3, 400)])
    M, N = A.shape
    K = 16
    rng = np.random.default_rng(3)
    x, B = rng.uniform(-1, 1, N), rng.uniform(-1, 1, (N, K))
    U, V = rng.uniform(-1, 1, (M, K)), rng.uniform(-1, 1, (N, K))
    ip, ind, dat = (rt.DeviceBuffer(A.indptr.astype(np.int64)),
                    rt.DeviceBuffer(A.indices.astype(np.int64)), rt.DeviceBuffer(A.data))
    bufs = {"x": rt.DeviceBuffer(x), "y": rt.DeviceBuffer(np.zeros(M)),
            "B": rt.DeviceBuffer(B), "C": rt.DeviceBuffer(np.zeros((M, K))),
            "U": rt.DeviceBuffer(U), "V": rt.DeviceBuffer(V), "S": rt.DeviceBuffer(np.zeros(A.nnz))}
    try:
        ms, _ = vendor.spmv_time("adaptive", M, N, A.nnz, [[ip, ind, dat, bufs["x"], bufs["y"]]],
                                 1, 3)
        assert ms.size == 3 and (ms > 0).all()
        assert rel_inf(bufs["y"].to_host(), oracle.spmv(A, x)) <= 1e-12
        vendor.spmm_time("csr", M, N, K, A.nnz, [[ip, ind, dat, bufs["B"], bufs["C"]]], 1, 3)
        assert rel_inf(bufs["C"].to_host().reshape(M, K), oracle.spmm(A, B)) <= 1e-12
        vendor.sddmm_time("default", M, N, K, A.nnz, [[ip, ind, bufs["U"], bufs["V"], bufs["S"]]],
                          1, 3)
        coo = A.tocoo()
        want = np.einsum("ik,ik->i", U[coo.row], V[coo.col])  # no multiply by A's values
        assert rel_inf(bufs["S"].to_host(), want) <= 1e-12
    finally:
        for b in [ip, ind, dat] + list(bufs.values()):
            b.free()

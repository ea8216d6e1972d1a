"""More than 2^31 nonzeros: every nonzero position ``p`` is 64-bit.

The matrix has 65536 rows of 32769 nonzeros, which ends past p = 2^31, then
50000 rows of 3, all of them past 2^31, so both the workgroup-per-row path and
the lane-group path index past 2^31.  ``indices`` and ``data`` (17 GB each) are
written on the device by a fill kernel:
    indices[p] = p mod N,   data[p] = (p mod 5) - 2,
and the dense operands hold small integers.  Every partial sum is then an
integer far below 2^53, so every result is exact, whatever the summation order.
The expected values come from closed forms. The summand is periodic in p with
period Q = lcm(5, N), so a row's sum is a difference of prefix sums over one
period, the prefix sum of the whole period times the number of whole periods.
Results must match bit for bit.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tilegen_amd import runtime as rt
from tilegen_amd.schedules import MERGE_TEST_SCHEDULES, NOALLOC_SCHEDULE, TEST_SCHEDULES, TUNED
from tilegen_amd.variant import Variant
from tilegen_amd.verify import hiprtc_options

pytestmark = pytest.mark.gpu

N = 4096
K = 64
LONG_ROWS, LONG_LEN = 65536, 32769
SHORT_ROWS, SHORT_LEN = 50000, 3
Q = 5 * N  # period of (p mod 5, p mod N)

_FILL = r'''
extern "C" __global__ __launch_bounds__(256)
void fill_csr(long long* __restrict__ ind, double* __restrict__ dat, long long nnz, long long n) {
  const long long stride = (long long)gridDim.x * 256;
  for (long long p = (long long)blockIdx.x * 256 + threadIdx.x; p < nnz; p += stride) {
    ind[p] = p % n;
    dat[p] = (double)(p % 5) - 2.0;
  }
}
'''


def _indptr() -> np.ndarray:
    long_part = np.arange(LONG_ROWS + 1, dtype=np.int64) * LONG_LEN
    short_part = long_part[-1] + np.arange(1, SHORT_ROWS + 1, dtype=np.int64) * SHORT_LEN
    return np.concatenate([long_part, short_part])


def _period_prefix(f: np.ndarray) -> np.ndarray:
    """pre[r] = sum of f[0:r] for r in 0..Q (f has Q rows), int64."""
    pre = np.zeros((Q + 1,) + f.shape[1:], dtype=np.int64)
    np.cumsum(f, axis=0, out=pre[1:])
    return pre


def _range_sums(pre: np.ndarray, ip: np.ndarray) -> np.ndarray:
    """Sum of the periodic summand over [ip[i], ip[i+1]) for every row."""
    def S(P):
        whole, part = P // Q, P % Q
        return whole.reshape((-1,) + (1,) * (pre.ndim - 1)) * pre[Q] + pre[part]
    return S(ip[1:]) - S(ip[:-1])


def _d(p: np.ndarray) -> np.ndarray:
    return (p % 5) - 2


def _dense(rows: int, a: int, m: int, seed_shift: int) -> np.ndarray:
    i = np.arange(rows, dtype=np.int64)[:, None]
    k = np.arange(K, dtype=np.int64)[None, :]
    return ((i * a + k + seed_shift) % m) - m // 2


def _copy_slice(buf: rt.DeviceBuffer, start: int, count: int, itemsize: int = 8,
                dtype=np.float64) -> np.ndarray:
    out = np.empty(count, dtype=dtype)
    assert 0 <= start and start + count <= buf.nbytes // itemsize
    rt.check(rt.lib().tg_memcpy_dtoh(out.ctypes.data, buf.ptr + start * itemsize,
                                     count * itemsize), "tg_memcpy_dtoh")
    return out


@pytest.fixture(scope="module")
def huge(hip_ready):
    ip = _indptr()
    nnz = int(ip[-1])
    M = ip.size - 1
    assert nnz > (1 << 31) + SHORT_ROWS and ip[LONG_ROWS] > (1 << 31)
    code, _ = rt.rtc_compile(_FILL, "fill_csr.hip", hiprtc_options())
    blob = ctypes.create_string_buffer(code, len(code))
    mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
    rt.check(rt.lib().tg_module_load(blob, len(code), ctypes.byref(mod)), "module")
    rt.check(rt.lib().tg_module_function(mod, b"fill_csr", ctypes.byref(fn)), "fill_csr")
    bufs = {"indptr": rt.DeviceBuffer(ip),
            "indices": rt.DeviceBuffer(nbytes=8 * nnz),
            "data": rt.DeviceBuffer(nbytes=8 * nnz)}
    try:
        # grid-stride loop: every p < nnz written once, nothing past nnz
        rt.launch(fn.value, 8192, 256, 0, [bufs["indices"], bufs["data"], nnz, N])
        print("[huge] M=%d nnz=%d filled" % (M, nnz), flush=True)
        yield ip, M, nnz, bufs
    finally:
        for b in bufs.values():
            b.free()
        rt.check(rt.lib().tg_module_unload(mod), "unload")


def _structure_unchanged(bufs, ip, nnz):
    assert _copy_slice(bufs["indptr"], 0, ip.size, dtype=np.int64).tobytes() == ip.tobytes()
    for start in (0, (1 << 31) - 4096, nnz - 4096):
        got = _copy_slice(bufs["indices"], start, 4096, dtype=np.int64)
        assert np.array_equal(got, np.arange(start, start + 4096, dtype=np.int64) % N)


# row tiles, the tuned stream ranges (1024 and 2048 nonzeros), hybrid tiles and
# merge-path windows; at this size every long row from about p = 2^26 (ranges of
# 1024) or 2^27 (2048) on has pieces past the 65536 ranges with scratch slots, so
# the stream and hybrid forms also sum those rows whole, with the whole workgroup
# of the range each begins in
_SPMV_HUGE = [TUNED["c1"], TEST_SCHEDULES[0], TUNED["c3a"], TUNED["c3b"], NOALLOC_SCHEDULE,
              MERGE_TEST_SCHEDULES[1]]


@pytest.mark.parametrize("cfg", _SPMV_HUGE, ids=lambda c: c.short())
def test_spmv_past_2_31_nonzeros(huge, cfg):
    ip, M, nnz, bufs = huge
    x = (np.arange(N, dtype=np.int64) % 7) - 3
    q = np.arange(Q, dtype=np.int64)
    want = _range_sums(_period_prefix(_d(q) * x[q % N]), ip).astype(np.float64)
    bx = rt.DeviceBuffer(x.astype(np.float64))
    by = rt.DeviceBuffer(np.zeros(M))
    try:
        v = Variant("spmv", cfg)
        print("[huge] spmv %s M=%d nnz=%d" % (cfg.short(), M, nnz), flush=True)
        v.device_call(v.abi_values(None, dict(bufs, x=bx, y=by), {}, M, N, 0, nnz))
        got = by.to_host()
    finally:
        bx.free()
        by.free()
    assert np.array_equal(got, want), int(np.flatnonzero(got != want)[0])
    _structure_unchanged(bufs, ip, nnz)


def test_spmm_past_2_31_nonzeros(huge):
    ip, M, nnz, bufs = huge
    B = _dense(N, 3, 11, 0)
    q = np.arange(Q, dtype=np.int64)
    want = _range_sums(_period_prefix(_d(q)[:, None] * B[q % N]), ip).astype(np.float64)
    bB = rt.DeviceBuffer(B.astype(np.float64))
    bC = rt.DeviceBuffer(np.zeros((M, K)))
    try:
        v = Variant("spmm", TUNED["c4"])
        v.device_call(v.abi_values(None, dict(bufs, B=bB, C=bC), {}, M, N, K, nnz))
        got = bC.to_host()
    finally:
        bB.free()
        bC.free()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("cfg", [TUNED["c5"], TEST_SCHEDULES[0]], ids=lambda c: c.short())
def test_sddmm_past_2_31_nonzeros(huge, cfg):
    ip, M, nnz, bufs = huge
    U = _dense(M, 1, 9, 0)
    V = _dense(N, 5, 13, 1)
    bU = rt.DeviceBuffer(U.astype(np.float64))
    bV = rt.DeviceBuffer(V.astype(np.float64))
    bC = rt.DeviceBuffer(nbytes=8 * nnz)
    try:
        bC.fill_bytes(0)
        v = Variant("sddmm", cfg)
        v.device_call(v.abi_values(None, dict(bufs, U=bU, V=bV, C=bC), {}, M, N, K, nnz))
        # the first and last long rows, the rows either side of p = 2^31, and the short rows
        p31 = 1 << 31
        starts = [(0, 2 * LONG_LEN), (p31 - 3 * LONG_LEN, 6 * LONG_LEN),
                  (int(ip[LONG_ROWS - 1]), LONG_LEN), (int(ip[LONG_ROWS]), nnz - int(ip[LONG_ROWS]))]
        for start, count in starts:
            got = _copy_slice(bC, start, count)
            p = np.arange(start, start + count, dtype=np.int64)
            row = np.searchsorted(ip, p, side="right") - 1
            want = (_d(p) * np.einsum("ij,ij->i", U[row], V[p % N])).astype(np.float64)
            assert np.array_equal(got, want), (start, int(np.flatnonzero(got != want)[0]))
    finally:
        for b in (bU, bV, bC):
            b.free()
    _structure_unchanged(bufs, ip, nnz)

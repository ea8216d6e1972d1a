"""rocSPARSE SpMV, SpMM and SDDMM on the same inputs, for the vendor comparison.

The reference times its tuned kernels against cuSPARSE through CuPy
(reference scripts/compare_cusparse.py:80-96, results in
results/cusparse_comparison.json).  Here ``libtg_vendor.so`` (csrc/vendor.cpp)
times ``rocsparse_spmv`` / ``rocsparse_spmm`` / ``rocsparse_sddmm`` with
hipEvents around each compute call on device-resident, rotated input copies;
``rocprofv3 --kernel-trace`` gives the kernel-only durations of the same calls.
rocSPARSE's SDDMM leaves out the multiply by A's values, so its output is
``(U V^T)`` on the pattern; checks multiply it by ``data`` before comparing.
"""

from __future__ import annotations

import ctypes
import os
from typing import Dict, Sequence, Tuple

import numpy as np

from . import runtime as rt

__all__ = ["ALGS", "SPMM_ALGS", "SDDMM_ALGS", "available", "spmv_time", "spmm_time",
           "sddmm_time"]

ALGS: Dict[str, int] = {"adaptive": 2, "rowsplit": 3, "lrb": 7, "nnzsplit": 8}
SPMM_ALGS: Dict[str, int] = {"default": 0, "csr": 1, "row_split": 4, "nnz_split": 5,
                             "merge_path": 9}
SDDMM_ALGS: Dict[str, int] = {"default": 0}  # "dense" (1) refuses CSR int64 input here

_LIB = None


def lib_path() -> str:
    return os.path.join(rt.lib_dir(), "libtg_vendor.so")


def available() -> bool:
    return os.path.exists(lib_path())


def _lib():
    global _LIB
    if _LIB is None:
        rt.lib()
        L = ctypes.CDLL(lib_path())
        L.tgv_vendor_spmv_time.restype = ctypes.c_int
        L.tgv_vendor_spmv_time.argtypes = [
            ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.POINTER(ctypes.c_uint64), ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
        for name in ("tgv_vendor_spmm_time", "tgv_vendor_sddmm_time"):
            f = getattr(L, name)
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.c_int] + [ctypes.c_int64] * 4 + [
                ctypes.POINTER(ctypes.c_uint64), ctypes.c_int, ctypes.c_int, ctypes.c_int,
                ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
        L.tgv_vendor_last_error.restype = ctypes.c_char_p
        _LIB = L
    return _LIB


def spmv_time(alg: str, M: int, N: int, nnz: int, sets: Sequence[Sequence],
              warmup: int = 10, iters: int = 100) -> Tuple[np.ndarray, float]:
    """Per-call milliseconds of rocsparse_spmv (y = A x) and the event wall
    time; ``sets`` are (indptr, indices, data, x, y) DeviceBuffers per copy."""
    flat = [v for s in sets for v in rt.pack_args(s)]
    arr = (ctypes.c_uint64 * len(flat))(*flat)
    ms = (ctypes.c_float * iters)()
    wall = ctypes.c_float()
    L = _lib()
    rc = L.tgv_vendor_spmv_time(ALGS[alg], M, N, nnz, arr, len(sets), warmup, iters, ms,
                                ctypes.byref(wall))
    if rc != 0:
        raise rt.TileGenHipError("rocSPARSE %s: %s" % (alg, L.tgv_vendor_last_error().decode()),
                                 rc)
    return np.array(ms[:], dtype=np.float64), float(wall.value)


def _time_mm(fname: str, what: str, alg_id: int, M: int, N: int, K: int, nnz: int,
             sets: Sequence[Sequence], warmup: int, iters: int) -> Tuple[np.ndarray, float]:
    flat = [v for s in sets for v in rt.pack_args(s)]
    arr = (ctypes.c_uint64 * len(flat))(*flat)
    ms = (ctypes.c_float * iters)()
    wall = ctypes.c_float()
    L = _lib()
    rc = getattr(L, fname)(alg_id, M, N, K, nnz, arr, len(sets), warmup, iters, ms,
                           ctypes.byref(wall))
    if rc != 0:
        raise rt.TileGenHipError("rocSPARSE %s: %s" % (what, L.tgv_vendor_last_error().decode()),
                                 rc)
    return np.array(ms[:], dtype=np.float64), float(wall.value)


def spmm_time(alg: str, M: int, N: int, K: int, nnz: int, sets: Sequence[Sequence],
              warmup: int = 10, iters: int = 100) -> Tuple[np.ndarray, float]:
    """rocsparse_spmm (C = A B, B and C row-major); ``sets`` are (indptr,
    indices, data, B, C) DeviceBuffers per copy."""
    return _time_mm("tgv_vendor_spmm_time", "spmm " + alg, SPMM_ALGS[alg], M, N, K, nnz, sets,
                    warmup, iters)


def sddmm_time(alg: str, M: int, N: int, K: int, nnz: int, sets: Sequence[Sequence],
               warmup: int = 10, iters: int = 100) -> Tuple[np.ndarray, float]:
    """rocsparse_sddmm on A's pattern; ``sets`` are (indptr, indices, U, V, out)
    DeviceBuffers per copy."""
    return _time_mm("tgv_vendor_sddmm_time", "sddmm " + alg, SDDMM_ALGS[alg], M, N, K, nnz,
                    sets, warmup, iters)


"""CPU oracle for the CSR hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only to check or to time a baseline; the
product (``tilegen_amd``) never imports, links or runs anything here.

Two checkers, both compiled by ``oracle/Makefile``:

``port``       ``_build/liboracle.so`` from ``tg_oracle.c``: this repository's
               plain-C restatement of the reference's sequential kernels
               (reference ``cpp/src/ref.cpp:6-73``).
``reference``  ``_ref/libtilegen_ref.so``: the reference's own ``ref.cpp``
               compiled from ``/root/reference`` with ``ref_capi.cpp`` glue.
               Present wherever it was built (it travels with the tree as a
               built file; the reference sources do not).

Parity status (tests/test_oracle.py): spmv, spmm, sddmm, fused_spmv_axpy and
dense_spmv are pinned by the reference's known-answer tests
(``cpp/tests/test_ref.cpp:25-116``), brute-force dense products, SciPy and
bit-equality with ``reference``.  axpy is pinned by its closed form only.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np
import scipy.sparse as sp

HERE = os.path.dirname(os.path.abspath(__file__))
PORT_LIB = os.path.join(HERE, "_build", "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libtilegen_ref.so")

_I64P = ctypes.POINTER(ctypes.c_int64)
_F64P = ctypes.POINTER(ctypes.c_double)
_I64 = ctypes.c_int64
_F64 = ctypes.c_double

_port = None
_ref = None


def build(ref: Optional[str] = None) -> None:
    """Run oracle/Makefile (the reference library only if its sources exist)."""
    cmd = ["make", "-s", "-C", HERE]
    if ref:
        cmd.append("REF=%s" % ref)
    subprocess.run(cmd, check=True, capture_output=True, text=True)


def _p(a: np.ndarray, kind):
    return a.ctypes.data_as(kind)


def port():
    """ctypes handle of liboracle.so (built on first use if needed)."""
    global _port
    if _port is None:
        if not os.path.exists(PORT_LIB):
            build()
        L = ctypes.CDLL(PORT_LIB)
        L.oracle_csr_spmv.argtypes = [_I64, _I64P, _I64P, _F64P, _F64P, _F64P]
        L.oracle_dense_spmv.argtypes = [_I64, _I64, _F64P, _F64P, _F64P]
        L.oracle_csr_spmm.argtypes = [_I64, _I64, _I64P, _I64P, _F64P, _F64P, _F64P]
        L.oracle_sddmm.argtypes = [_I64, _I64, _I64P, _I64P, _F64P, _F64P, _F64P, _F64P]
        L.oracle_fused_spmv_axpy.argtypes = [_I64, _I64P, _I64P, _F64P, _F64P, _F64P,
                                             _F64, _F64, _F64P]
        L.oracle_axpy.argtypes = [_I64, _F64P, _F64P, _F64, _F64, _F64P]
        for f in ("oracle_csr_spmv", "oracle_dense_spmv", "oracle_csr_spmm", "oracle_sddmm",
                  "oracle_fused_spmv_axpy", "oracle_axpy"):
            getattr(L, f).restype = None
        _port = L
    return _port


def reference_available() -> bool:
    return os.path.exists(REF_LIB)


def reference():
    """ctypes handle of the reference's own ref.cpp build, or None."""
    global _ref
    if _ref is None and reference_available():
        L = ctypes.CDLL(REF_LIB)
        L.ref_create.restype = ctypes.c_void_p
        L.ref_create.argtypes = [_I64, _I64, _I64, _I64P, _I64P, _F64P]
        L.ref_destroy.argtypes = [ctypes.c_void_p]
        L.ref_destroy.restype = None
        L.ref_set_operands.argtypes = [ctypes.c_void_p, _I64, _F64P, _F64P, _F64P, _F64P]
        L.ref_set_operands.restype = None
        L.ref_run.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _F64P]
        L.ref_run.restype = ctypes.c_double
        L.ref_dense_spmv.argtypes = [_I64, _I64, _F64P, _F64P, _F64P]
        L.ref_dense_spmv.restype = None
        L.ref_fused_spmv_axpy.argtypes = [ctypes.c_void_p, _F64P, _F64, _F64, _F64P]
        L.ref_fused_spmv_axpy.restype = None
        _ref = L
    return _ref


def _csr(A: sp.csr_matrix):
    return (np.ascontiguousarray(A.indptr, dtype=np.int64),
            np.ascontiguousarray(A.indices, dtype=np.int64),
            np.ascontiguousarray(A.data, dtype=np.float64))


# --------------------------------------------------------------------------- #
# port (this repository's restatement)
# --------------------------------------------------------------------------- #
def spmv(A: sp.csr_matrix, x: np.ndarray) -> np.ndarray:
    ip, ind, dat = _csr(A)
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(A.shape[0])
    port().oracle_csr_spmv(A.shape[0], _p(ip, _I64P), _p(ind, _I64P), _p(dat, _F64P),
                           _p(x, _F64P), _p(y, _F64P))
    return y


def dense_spmv(Ad: np.ndarray, x: np.ndarray) -> np.ndarray:
    Ad = np.ascontiguousarray(Ad, dtype=np.float64)
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(Ad.shape[0])
    port().oracle_dense_spmv(Ad.shape[0], Ad.shape[1], _p(Ad, _F64P), _p(x, _F64P),
                             _p(y, _F64P))
    return y


def spmm(A: sp.csr_matrix, B: np.ndarray) -> np.ndarray:
    ip, ind, dat = _csr(A)
    B = np.ascontiguousarray(B, dtype=np.float64)
    K = B.shape[1]
    C = np.empty((A.shape[0], K))
    port().oracle_csr_spmm(A.shape[0], K, _p(ip, _I64P), _p(ind, _I64P), _p(dat, _F64P),
                           _p(B, _F64P), _p(C, _F64P))
    return C


def sddmm(A: sp.csr_matrix, U: np.ndarray, V: np.ndarray) -> np.ndarray:
    ip, ind, dat = _csr(A)
    U = np.ascontiguousarray(U, dtype=np.float64)
    V = np.ascontiguousarray(V, dtype=np.float64)
    out = np.empty(ind.size)
    port().oracle_sddmm(A.shape[0], U.shape[1], _p(ip, _I64P), _p(ind, _I64P), _p(dat, _F64P),
                        _p(U, _F64P), _p(V, _F64P), _p(out, _F64P))
    return out


def fused_spmv_axpy(A: sp.csr_matrix, x: np.ndarray, w: np.ndarray, alpha: float,
                    beta: float) -> np.ndarray:
    ip, ind, dat = _csr(A)
    x = np.ascontiguousarray(x, dtype=np.float64)
    w = np.ascontiguousarray(w, dtype=np.float64)
    z = np.empty(A.shape[0])
    port().oracle_fused_spmv_axpy(A.shape[0], _p(ip, _I64P), _p(ind, _I64P), _p(dat, _F64P),
                                  _p(x, _F64P), _p(w, _F64P), alpha, beta, _p(z, _F64P))
    return z


def axpy(x: np.ndarray, w: np.ndarray, alpha: float, beta: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    w = np.ascontiguousarray(w, dtype=np.float64)
    z = np.empty(x.size)
    port().oracle_axpy(x.size, _p(x, _F64P), _p(w, _F64P), alpha, beta, _p(z, _F64P))
    return z


def compute(kernel: str, A: sp.csr_matrix, ops: dict) -> np.ndarray:
    """Oracle result of ``kernel`` with operands named as in the ABI."""
    if kernel == "spmv":
        return spmv(A, ops["x"])
    if kernel == "spmm":
        return spmm(A, ops["B"])
    if kernel == "sddmm":
        return sddmm(A, ops["U"], ops["V"])
    if kernel == "fused_spmv_axpy":
        return fused_spmv_axpy(A, ops["x"], ops["w"], ops["alpha"], ops["beta"])
    raise ValueError(kernel)


# --------------------------------------------------------------------------- #
# reference (the reference's own ref.cpp)
# --------------------------------------------------------------------------- #
class RefMatrix:
    """A matrix held inside the reference library, for repeated calls."""

    _WHICH = {"spmv": 0, "spmm": 1, "sddmm": 2}

    def __init__(self, A: sp.csr_matrix):
        L = reference()
        if L is None:
            raise RuntimeError("oracle/_ref/libtilegen_ref.so is not built")
        self.L = L
        self.A = A
        ip, ind, dat = _csr(A)
        self.h = L.ref_create(A.shape[0], A.shape[1], int(ind.size), _p(ip, _I64P),
                              _p(ind, _I64P), _p(dat, _F64P))

    def set_operands(self, K: int = 0, x=None, B=None, U=None, V=None) -> None:
        keep = []

        def ptr(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=np.float64)
            keep.append(a)
            return _p(a, _F64P)
        self.L.ref_set_operands(self.h, K, ptr(x), ptr(B), ptr(U), ptr(V))

    def run(self, kernel: str, iters: int = 1, out_shape=None):
        """(result, seconds per call)."""
        size = int(np.prod(out_shape)) if out_shape is not None else 0
        out = np.empty(size)
        sec = self.L.ref_run(self.h, self._WHICH[kernel], int(iters),
                             _p(out, _F64P) if size else None)
        return (out.reshape(out_shape) if out_shape is not None else None), float(sec)

    def close(self) -> None:
        if self.h:
            self.L.ref_destroy(self.h)
            self.h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

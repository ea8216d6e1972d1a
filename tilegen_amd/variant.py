"""One compiled HIP variant of a standard kernel, driven through its C ABI.

``Variant(kernel_name, config)`` generates the HIP source for the schedule,
builds it (hipRTC code object + C launcher, cached) and binds the variant
library's ``launch_<name>`` exactly as the reference's harnesses bind theirs
(reference tilegen/verify.py:414-451, cpp/src/harness.cpp:130-141).  ``run``
takes host arrays, mirrors them on the device and returns the output;
``device_call`` takes DeviceBuffers that already live in HBM.
"""

from __future__ import annotations

import ctypes
import os
from typing import Dict, Optional, Sequence, Tuple

import numpy as np
import scipy.sparse as sp

from . import runtime as _rt
from .codegen import Config, generate
from .dsl import standard_kernels
from .verify import _SIGNATURES, compile_generated

__all__ = ["Variant", "operand_order"]

_WORKDIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "build", "generated")


def operand_order(kernel_name: str):
    """(dense input names, scalar names, has K) in ABI order."""
    return {
        "spmv": (["x"], [], False),
        "spmm": (["B"], [], True),
        "sddmm": (["U", "V"], [], True),
        "fused_spmv_axpy": (["x", "w"], ["alpha", "beta"], False),
        "axpy": (["x", "w"], ["alpha", "beta"], False),
    }[kernel_name]


class Variant:
    def __init__(self, kernel_name: str, config: Config, workdir: str = _WORKDIR):
        self.kernel_name = kernel_name
        self.config = config
        self.gen = generate(standard_kernels()[kernel_name], config, "hip", outdir=workdir)
        self.lib_path, self.build_log = compile_generated(self.gen, "hip", workdir)
        _rt.lib()  # the runtime first, RTLD_GLOBAL
        self.lib = ctypes.CDLL(self.lib_path)
        self.launch = getattr(self.lib, "launch_%s" % kernel_name)
        self.launch.argtypes = _SIGNATURES[kernel_name]
        self.launch.restype = None
        self.lib.tgv_function.restype = ctypes.c_void_p
        self.lib.tgv_geometry.argtypes = [ctypes.c_int64] * 4 + [
            ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32),
            ctypes.POINTER(ctypes.c_int32)]
        self.lib.tgv_geometry.restype = ctypes.c_int
        self._async = None

    # -- launch geometry / raw function (for timing harnesses) ------------ #
    def function(self) -> int:
        _rt.lib().tg_clear_error()
        fn = self.lib.tgv_function()
        if not fn:
            _rt.check_status("tgv_function")
            raise _rt.TileGenHipError("tgv_function returned null")
        return int(fn)

    def geometry(self, M: int, N: int = 0, K: int = 0, nnz: int = 0) -> Tuple[int, int, int]:
        g, b, l = ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32()
        self.lib.tgv_geometry(M, N, K, nnz, ctypes.byref(g), ctypes.byref(b), ctypes.byref(l))
        return int(g.value), int(b.value), int(l.value)

    def attrs(self) -> Dict[str, int]:
        regs, lds, scratch, mt = (ctypes.c_int() for _ in range(4))
        _rt.check(_rt.lib().tg_function_attrs(self.function(), ctypes.byref(regs),
                                              ctypes.byref(lds), ctypes.byref(scratch),
                                              ctypes.byref(mt)), "tg_function_attrs")
        return {"vgprs_or_regs": regs.value, "lds_bytes": lds.value,
                "scratch_bytes": scratch.value, "max_threads": mt.value}

    # -- argument lists ------------------------------------------------------ #
    def abi_values(self, A: Optional[sp.csr_matrix], bufs: Dict[str, object],
                   scalars: Dict[str, float], M: int, N: int, K: int, nnz: int) -> list:
        """Argument values in ABI order; arrays are DeviceBuffers or ints."""
        dense, scal, has_k = operand_order(self.kernel_name)
        out = "y" if self.kernel_name == "spmv" else ("C" if self.kernel_name in ("spmm", "sddmm")
                                                      else "z")
        vals = []
        if self.kernel_name != "axpy":
            vals += [bufs["indptr"], bufs["indices"], bufs["data"]]
        vals += [bufs[d] for d in dense]
        vals.append(bufs[out])
        vals += [scalars[s] for s in scal]
        if self.kernel_name == "axpy":
            vals.append(M)
        else:
            vals += [M, N] + ([K] if has_k else []) + [nnz]
        return vals

    def device_call(self, values: Sequence) -> None:
        """Call ``launch_<name>`` with DeviceBuffers/ints/floats (synchronous)."""
        conv = []
        for v, t in zip(values, self.launch.argtypes):
            if isinstance(v, _rt.DeviceBuffer):
                conv.append(ctypes.cast(v.ptr, t))
            else:
                conv.append(v)
        _rt.lib().tg_clear_error()
        self.launch(*conv)
        _rt.check_status("launch_%s" % self.kernel_name)

    def launch_async(self, values: Sequence, stream: Optional[int]) -> None:
        """Enqueue the kernel on ``stream`` (a tg_stream_create handle; None =
        the null stream) through the library's ``tgv_launch_async``, without
        waiting for it."""
        if self._async is None:
            fn = self.lib.tgv_launch_async
            fn.argtypes = [ctypes.c_void_p] + list(_SIGNATURES[self.kernel_name])
            fn.restype = ctypes.c_int
            self._async = fn
        conv = []
        for v, t in zip(values, self.launch.argtypes):
            conv.append(ctypes.cast(v.ptr, t) if isinstance(v, _rt.DeviceBuffer) else v)
        _rt.check(self._async(stream, *conv), "tgv_launch_async")

    def run(self, A: Optional[sp.csr_matrix], out: Optional[np.ndarray] = None,
            check_structure: bool = True, **operands) -> np.ndarray:
        """Host arrays in, output out.  ``out`` (optional) is the initial
        content of the output buffer; by default it starts zeroed like every
        reference caller's.  Raises if indptr/indices changed on the device."""
        dense, scal, has_k = operand_order(self.kernel_name)
        if self.kernel_name == "axpy":
            M = int(np.asarray(operands["x"]).size)
            N = nnz = K = 0
        else:
            M, N = A.shape
            nnz = int(A.nnz)
            K = int(np.asarray(operands[dense[0]]).shape[1]) if has_k else 0
        host: Dict[str, np.ndarray] = {}
        if A is not None and self.kernel_name != "axpy":
            host["indptr"] = np.ascontiguousarray(A.indptr, dtype=np.int64)
            host["indices"] = np.ascontiguousarray(A.indices, dtype=np.int64)
            host["data"] = np.ascontiguousarray(A.data, dtype=np.float64)
        for d in dense:
            host[d] = np.ascontiguousarray(operands[d], dtype=np.float64)
        out_name, out_shape = {
            "spmv": ("y", (M,)), "spmm": ("C", (M, K)), "sddmm": ("C", (nnz,)),
            "fused_spmv_axpy": ("z", (M,)), "axpy": ("z", (M,)),
        }[self.kernel_name]
        host[out_name] = (np.zeros(out_shape) if out is None
                          else np.ascontiguousarray(out, dtype=np.float64).reshape(out_shape).copy())
        bufs = {k: _rt.DeviceBuffer(v) for k, v in host.items()}
        try:
            vals = self.abi_values(A, bufs, {s: float(operands[s]) for s in scal}, M, N, K, nnz)
            self.device_call(vals)
            result = bufs[out_name].to_host()
            if check_structure and "indptr" in bufs:
                for key in ("indptr", "indices"):
                    if bufs[key].to_host().tobytes() != host[key].tobytes():
                        raise AssertionError("%s was modified on the device" % key)
            return result
        finally:
            for b in bufs.values():
                b.free()

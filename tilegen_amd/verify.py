"""Compile, load, run and differentially check generated kernels.

Same entry points as reference ``tilegen/verify.py`` (``compile_generated``,
``run_kernel``, ``verify``, ``VerifyResult``, ``_SIGNATURES``), with the CUDA
half replaced:

* ``backend="hip"``: the device source is compiled in-process by hipRTC for
  gfx950 (libtgrt), the C launcher that embeds the code object is compiled by
  the host C compiler into the variant's shared library, and both are cached
  under a key of sha1(device source, launcher text, hipRTC options).  The
  variant library exports ``launch_<name>`` with the reference ABI; it is
  called with device pointers from ``DeviceBuffer``.
* ``backend="cpu"``: the OpenMP C++ variant, compiled by g++ with the
  reference flags (``verify.py:238-247``, ``:298-312``).

The oracle of ``verify`` is SciPy in float64 (reference ``verify.py:338-371``)
and the pass test is the reference tolerance
``max_abs <= 8 eps max(1, max_row_nnz) max|ref| + 1e-12`` (``verify.py:503-514``).
Each result also carries the normwise relative errors (inf- and 2-norm) the
BASELINE bar is stated in and, on the HIP path, whether ``indptr``/``indices``
came back byte-identical from the device.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import shutil
import subprocess
import tempfile
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np
import scipy.sparse as sp

from . import codegen as _codegen
from . import runtime as _rt
from .dsl import standard_kernels

__all__ = [
    "VerifyResult", "compile_generated", "hip_arch", "hiprtc_options", "verify",
    "run_kernel", "cache_dir", "normwise_errors",
]

I64 = ctypes.c_longlong
I64P = ctypes.POINTER(ctypes.c_longlong)
F64P = ctypes.POINTER(ctypes.c_double)

# ctypes argtypes per kernel ABI (reference verify.py:166-173)
_SIGNATURES = {
    "spmv": [I64P, I64P, F64P, F64P, F64P, I64, I64, I64],
    "spmm": [I64P, I64P, F64P, F64P, F64P, I64, I64, I64, I64],
    "sddmm": [I64P, I64P, F64P, F64P, F64P, F64P, I64, I64, I64, I64],
    "fused_spmv_axpy": [I64P, I64P, F64P, F64P, F64P, F64P, ctypes.c_double,
                        ctypes.c_double, I64, I64, I64],
    "axpy": [F64P, F64P, F64P, ctypes.c_double, ctypes.c_double, I64],
}


# --------------------------------------------------------------------------- #
# compilation
# --------------------------------------------------------------------------- #
def hip_arch() -> str:
    """Target of hipRTC; ``TILEGEN_HIP_ARCH`` overrides the gfx950 default."""
    return os.environ.get("TILEGEN_HIP_ARCH", _codegen.HIP_ARCH)


def hiprtc_options() -> List[str]:
    opts = ["--offload-arch=%s" % hip_arch(), "-O3", "-std=c++17",
            # no packed-FP32 instructions in generated code
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    extra = os.environ.get("TILEGEN_HIPRTC_OPTS", "").split()
    return opts + extra


def cache_dir() -> str:
    d = os.environ.get("TILEGEN_CACHE_DIR") or os.path.join(
        os.path.dirname(os.path.abspath(__file__)), "_kcache")
    os.makedirs(d, exist_ok=True)
    return d


def _host_cc() -> str:
    for cc in (os.environ.get("CC"), "gcc", "cc", "clang"):
        if cc and shutil.which(cc):
            return cc
    raise RuntimeError("no C compiler found (need gcc/cc)")


def _host_cxx() -> str:
    for cc in (os.environ.get("CXX"), "g++", "clang++", "c++"):
        if cc and shutil.which(cc):
            return cc
    raise RuntimeError("no C++ compiler found (need g++/clang++)")


def _omp_flags() -> List[str]:
    return ["-O3", "-march=native", "-fopenmp"]


def _bytes_as_c(blob: bytes) -> str:
    hexes = ["0x%02x" % b for b in blob]
    return ",\n".join(",".join(hexes[i:i + 24]) for i in range(0, len(hexes), 24))


def _atomic_compile(cmd_head: List[str], src: str, out: str, tail: List[str]) -> None:
    fd, tmp = tempfile.mkstemp(prefix=".tg_", suffix=".so", dir=os.path.dirname(out))
    os.close(fd)
    try:
        res = subprocess.run(cmd_head + ["-o", tmp, src] + tail, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("host compiler failed for %s:\n%s" % (src, res.stderr))
        os.replace(tmp, out)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)


def _compile_hip(gen: "_codegen.GeneratedKernel", workdir: str) -> Tuple[str, str]:
    opts = hiprtc_options()
    key = hashlib.sha1("\0".join([gen.source, gen.host_source] + opts).encode()).hexdigest()[:20]
    stem = "%s_%s" % (gen.kernel_name, key)
    cdir = cache_dir()
    so_path = os.path.join(cdir, stem + ".so")
    co_path = os.path.join(cdir, stem + ".co")
    if os.path.exists(so_path) and os.path.exists(co_path):
        return so_path, "cached %s (hipRTC %s)" % (so_path, hip_arch())
    if os.path.exists(co_path):
        with open(co_path, "rb") as fh:
            code = fh.read()
        rtc_log = "code object from cache"
    else:
        code, rtc_log = _rt.rtc_compile(gen.source, gen.filename, opts)
        tmp = co_path + ".tmp%d" % os.getpid()
        with open(tmp, "wb") as fh:
            fh.write(code)
        os.replace(tmp, co_path)
    host = gen.host_source.replace("{CODE_SIZE}", str(len(code))).replace(
        "{CODE_OBJECT}", _bytes_as_c(code))
    os.makedirs(workdir, exist_ok=True)
    # per-process file name: concurrent builds of one variant never read a
    # launcher source another process is still writing
    host_src = os.path.join(workdir, "%s_launch.%d.c" % (gen.filename.rsplit(".", 1)[0],
                                                          os.getpid()))
    with open(host_src, "w") as fh:
        fh.write(host)
    libdir = _rt.lib_dir()
    _atomic_compile([_host_cc(), "-std=c11", "-O2", "-shared", "-fPIC",
                     "-I", _rt.include_dir()], host_src, so_path,
                    ["-L", libdir, "-ltgrt", "-Wl,-rpath," + libdir])
    return so_path, ("hipRTC compiled %s for %s (%d-byte code object, options %s); "
                     "launcher %s%s" % (gen.filename, hip_arch(), len(code), " ".join(opts),
                                        so_path, ("; log: " + rtc_log) if rtc_log.strip() else ""))


def compile_generated(gen: "_codegen.GeneratedKernel", backend: str = "cpu",
                      workdir: str = "build/generated", verbose: bool = False
                      ) -> Tuple[Optional[str], str]:
    """Build a generated variant; returns (shared_object_path, log).

    Raises RuntimeError (with the compiler's diagnostics) when compilation fails.
    """
    src = os.path.join(workdir, gen.filename)
    if not os.path.exists(src):
        gen.write(workdir)
    if backend == "hip":
        if gen.backend != "hip":
            raise RuntimeError("compile_generated(backend='hip') needs a HIP variant")
        try:
            return _compile_hip(gen, workdir)
        except _rt.TileGenHipError as exc:
            raise RuntimeError(str(exc))
    out = os.path.join(workdir, gen.filename.rsplit(".", 1)[0] + ".so")
    if os.path.exists(out) and os.path.getmtime(out) >= os.path.getmtime(src):
        return out, "cached %s" % out
    cc = _host_cxx()
    base = [cc, "-std=c++17", "-shared", "-fPIC"]
    errors = []
    for flags in (_omp_flags(), ["-O3", "-march=native"]):
        try:
            _atomic_compile(base + flags, src, out, [])
            return out, "compiled %s with: %s" % (gen.filename, " ".join(base[1:] + flags))
        except RuntimeError as exc:
            errors.append(str(exc))
    raise RuntimeError(errors[-1])


# --------------------------------------------------------------------------- #
# matrices and the float64 oracle
# --------------------------------------------------------------------------- #
def _load_matrix(matrix) -> Tuple[sp.csr_matrix, str]:
    if isinstance(matrix, str):
        with np.load(matrix, allow_pickle=False) as z:
            A = sp.csr_matrix((z["data"].astype(np.float64), z["indices"].astype(np.int64),
                               z["indptr"].astype(np.int64)),
                              shape=tuple(int(s) for s in z["shape"]))
            name = str(z["class_name"]) if "class_name" in z else os.path.basename(matrix)
        return A, name
    if isinstance(matrix, dict):
        A = sp.csr_matrix((np.asarray(matrix["data"], dtype=np.float64),
                           np.asarray(matrix["indices"], dtype=np.int64),
                           np.asarray(matrix["indptr"], dtype=np.int64)),
                          shape=tuple(matrix["shape"]))
        return A, matrix.get("class_name", "custom")
    if sp.issparse(matrix):
        return matrix.tocsr().astype(np.float64), "custom"
    raise TypeError("unsupported matrix type: %r" % type(matrix))


def _inputs_for(kernel: str, A: sp.csr_matrix, K: int, seed: int = 7):
    """Dense operands, N(0,1) from ``default_rng(seed)`` drawn in the order
    x, w, B, U, V (reference ``verify.py:338-347``)."""
    M, N = A.shape
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(N)
    w = rng.standard_normal(M)
    B = rng.standard_normal((N, K))
    U = rng.standard_normal((M, K))
    V = rng.standard_normal((N, K))
    return x, w, B, U, V, 0.7, -1.3


def _reference(kernel: str, A: sp.csr_matrix, data):
    """float64 SciPy/numpy results (reference ``verify.py:350-371``)."""
    x, w, B, U, V, alpha, beta = data
    if kernel == "spmv":
        return np.asarray(A @ x, dtype=np.float64)
    if kernel == "spmm":
        return np.asarray(A @ B, dtype=np.float64)
    if kernel == "sddmm":
        coo = A.tocoo()
        out = np.empty(coo.nnz, dtype=np.float64)
        step = 200000
        for s in range(0, coo.nnz, step):
            e = min(s + step, coo.nnz)
            out[s:e] = np.einsum("ik,ik->i", U[coo.row[s:e]], V[coo.col[s:e]]) * coo.data[s:e]
        return out
    if kernel == "fused_spmv_axpy":
        return alpha * (A @ x) + beta * w
    if kernel == "axpy":
        return alpha * x + beta * w
    raise ValueError("unknown kernel %r" % kernel)


def normwise_errors(out: np.ndarray, ref: np.ndarray) -> Tuple[float, float]:
    """(||out-ref||_inf / ||ref||_inf, ||out-ref||_2 / ||ref||_2); a zero
    reference norm gives the absolute error norm instead."""
    d = np.asarray(out, dtype=np.float64).ravel() - np.asarray(ref, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    if d.size == 0:
        return 0.0, 0.0
    ninf, n2 = float(np.abs(r).max()), float(np.linalg.norm(r))
    einf, e2 = float(np.abs(d).max()), float(np.linalg.norm(d))
    return (einf / ninf if ninf > 0 else einf), (e2 / n2 if n2 > 0 else e2)


@dataclass
class VerifyResult:
    kernel: str
    matrix_class: str
    backend: str
    rows: int = 0
    nnz: int = 0
    max_abs_err: float = 0.0
    max_rel_err: float = 0.0
    tolerance: float = 0.0
    ok: bool = False
    inject_bug: bool = False
    message: str = ""
    config: Dict[str, Any] = field(default_factory=dict)
    #: normwise relative errors (the BASELINE bar is <= 1e-10)
    rel_err_inf: float = 0.0
    rel_err_2: float = 0.0
    #: HIP only: indptr/indices byte-identical after the launch
    structure_intact: Optional[bool] = None
    #: False when no device was available and only compilation ran
    executed: bool = True

    def to_dict(self) -> Dict[str, Any]:
        return dict(self.__dict__)


def _max_row_nnz(A: sp.csr_matrix) -> int:
    counts = np.diff(A.indptr)
    return int(counts.max()) if counts.size else 0


def _call_arrays(kernel_name: str, A: sp.csr_matrix, data, K: int):
    """(arrays, output index, scalars, output array) for one launch."""
    M, N = A.shape
    nnz = int(A.nnz)
    ip = np.ascontiguousarray(A.indptr, dtype=np.int64)
    ind = np.ascontiguousarray(A.indices, dtype=np.int64)
    dat = np.ascontiguousarray(A.data, dtype=np.float64)
    x, w, B, U, V, alpha, beta = data
    if kernel_name == "spmv":
        out = np.zeros(M)
        return [ip, ind, dat, x, out], 4, (M, N, nnz), out
    if kernel_name == "spmm":
        out = np.zeros((M, K))
        return [ip, ind, dat, np.ascontiguousarray(B), out], 4, (M, N, K, nnz), out
    if kernel_name == "sddmm":
        out = np.zeros(nnz)
        return ([ip, ind, dat, np.ascontiguousarray(U), np.ascontiguousarray(V), out], 5,
                (M, N, K, nnz), out)
    if kernel_name == "fused_spmv_axpy":
        out = np.zeros(M)
        return [ip, ind, dat, x, w, out], 5, (alpha, beta, M, N, nnz), out
    if kernel_name == "axpy":
        out = np.zeros(M)
        return [x, w, out], 2, (alpha, beta, M), out
    raise ValueError("unknown kernel %r" % kernel_name)


def _host_ptr(arr: np.ndarray):
    ct = ctypes.c_longlong if arr.dtype == np.int64 else ctypes.c_double
    return arr.ctypes.data_as(ctypes.POINTER(ct))


def _run_hip(fn, arrays: List[np.ndarray], out_index: int, scalars,
             structure: Sequence[int] = (0, 1)) -> bool:
    """Mirror the arrays on the device, call the launcher, copy the output
    back into ``arrays[out_index]``; returns whether the arrays listed in
    ``structure`` came back byte-identical."""
    bufs = [_rt.DeviceBuffer(a) for a in arrays]
    try:
        _rt.lib().tg_clear_error()
        fn(*([ctypes.cast(b.ptr, _SIG_PTR[a.dtype == np.int64]) for a, b in zip(arrays, bufs)]
             + list(scalars)))
        _rt.check_status("launch")
        bufs[out_index].to_host(arrays[out_index])
        intact = True
        for s in structure:
            if s < len(arrays) and s != out_index and arrays[s].dtype == np.int64:
                back = bufs[s].to_host()
                intact = intact and back.tobytes() == arrays[s].tobytes()
        return intact
    finally:
        for b in bufs:
            b.free()


_SIG_PTR = {True: I64P, False: F64P}


def run_kernel(lib_path: str, kernel_name: str, A: sp.csr_matrix, data, K: int = 8,
               backend: str = "cpu"):
    """Load ``lib_path`` and call ``launch_<kernel_name>`` (reference
    ``verify.py:414-451``).  HIP launches get device copies of every array and
    the output is copied back; returns (out, lib, fn, (indptr, indices, data))."""
    lib = ctypes.CDLL(lib_path)
    fn = getattr(lib, "launch_%s" % kernel_name)
    fn.argtypes = _SIGNATURES[kernel_name]
    arrays, out_index, scalars, out = _call_arrays(kernel_name, A, data, K)
    if backend == "hip":
        intact = _run_hip(fn, arrays, out_index, scalars)
        run_kernel.last_structure_intact = intact
    else:
        fn(*([_host_ptr(a) for a in arrays] + list(scalars)))
    return out, lib, fn, tuple(arrays[:3])


run_kernel.last_structure_intact = None


def _hip_device_present() -> bool:
    try:
        return _rt.device_count() > 0
    except _rt.TileGenHipError:
        return False


def verify(kernel_name: str, config: "_codegen.Config", matrix, backend: str = "cpu",
           workdir: str = "build/generated", K: int = 8, seed: int = 7,
           skip_passes: Sequence[str] = ()) -> VerifyResult:
    """Generate, compile and run ``kernel_name``; compare against float64 SciPy.

    Without a visible HIP device the HIP variant is still compiled for gfx950
    (a real compile, not a text check) and the result says ``executed=False``.
    """
    kernels = standard_kernels()
    if kernel_name not in kernels:
        raise ValueError("unknown kernel %r" % kernel_name)
    A, cls = _load_matrix(matrix)
    M, N = A.shape
    nnz = int(A.nnz)
    data = _inputs_for(kernel_name, A, K, seed)
    ref = _reference(kernel_name, A, data)
    common = dict(kernel=kernel_name, matrix_class=cls, backend=backend, rows=M, nnz=nnz,
                  inject_bug=config.inject_bug, config=config.to_dict())
    try:
        gen = _codegen.generate(kernels[kernel_name], config, backend, outdir=workdir,
                                write=True, skip_passes=skip_passes)
        lib_path, log = compile_generated(gen, backend, workdir)
    except (RuntimeError, ValueError) as exc:
        return VerifyResult(ok=False, message="compile error: %s" % exc, **common)
    if backend == "hip" and not _hip_device_present():
        return VerifyResult(ok=True, executed=False,
                            message="no HIP device visible: %s; numerics not run" % log,
                            **common)
    try:
        out, _lib, _fn, _bufs = run_kernel(lib_path, kernel_name, A, data, K, backend)
    except _rt.TileGenHipError as exc:
        return VerifyResult(ok=False, message="launch error: %s" % exc, **common)
    out = np.asarray(out, dtype=np.float64).ravel()
    refv = np.asarray(ref, dtype=np.float64).ravel()
    diff = np.abs(out - refv)
    max_abs = float(diff.max()) if diff.size else 0.0
    max_rel = float((diff / np.maximum(np.abs(refv), 1e-300)).max()) if diff.size else 0.0
    eps = float(np.finfo(np.float64).eps)
    scale = float(np.abs(refv).max()) if refv.size else 0.0
    tol = float(8.0 * eps * max(1, _max_row_nnz(A)) * scale + 1e-12)
    rinf, r2 = normwise_errors(out, refv)
    intact = run_kernel.last_structure_intact if backend == "hip" else None
    ok = bool(max_abs <= tol) and intact is not False
    return VerifyResult(max_abs_err=max_abs, max_rel_err=max_rel, tolerance=tol, ok=ok,
                        message=log, rel_err_inf=rinf, rel_err_2=r2, structure_intact=intact,
                        **common)

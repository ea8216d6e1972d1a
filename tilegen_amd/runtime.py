"""ctypes binding of ``libtgrt.so`` (the C ABI in ``include/tgrt.h``).

This is the only path from Python to the GPU: hipRTC compilation, device
buffers, kernel launch and GPU-side timing all go through it.  Importing the
module is cheap and never touches a device; the library is loaded on first
use and a missing build is an error, never a silent fallback.
"""

from __future__ import annotations

import ctypes
import os
import struct
import threading
from typing import List, Optional, Sequence, Tuple

import numpy as np

__all__ = [
    "TileGenHipError", "lib", "lib_path", "include_dir", "check", "device_count",
    "device_info", "rtc_compile", "DeviceBuffer", "launch", "time_launches",
    "pack_args", "synchronize", "ArgSets", "run_launches", "stream_create", "stream_destroy",
    "stream_synchronize", "graph_capture", "graph_launch", "graph_destroy",
]

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
_REPO_DIR = os.path.dirname(_PKG_DIR)


class TileGenHipError(RuntimeError):
    """A failed HIP/hipRTC call; ``code`` is the libtgrt status."""

    def __init__(self, message: str, code: int = -1):
        super().__init__(message)
        self.code = code


def lib_dir() -> str:
    return os.environ.get("TILEGEN_LIB_DIR", os.path.join(_PKG_DIR, "_lib"))


def lib_path() -> str:
    return os.path.join(lib_dir(), "libtgrt.so")


def include_dir() -> str:
    return os.path.join(_REPO_DIR, "include")


_LIB = None
_LOCK = threading.Lock()

_c_int_p = ctypes.POINTER(ctypes.c_int)
_c_i64_p = ctypes.POINTER(ctypes.c_int64)
_c_u64_p = ctypes.POINTER(ctypes.c_uint64)
_c_f32_p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p


def _declare(L) -> None:
    sig = {
        "tg_last_error": (ctypes.c_char_p, []),
        "tg_last_status": (ctypes.c_int, []),
        "tg_clear_error": (None, []),
        "tg_fail": (ctypes.c_int, [ctypes.c_int, ctypes.c_char_p]),
        "tg_device_count": (ctypes.c_int, [_c_int_p]),
        "tg_set_device": (ctypes.c_int, [ctypes.c_int]),
        "tg_get_device": (ctypes.c_int, [_c_int_p]),
        "tg_device_props": (ctypes.c_int, [ctypes.c_int, ctypes.c_char_p, ctypes.c_int,
                                           ctypes.c_char_p, ctypes.c_int, _c_int_p, _c_i64_p,
                                           _c_int_p, _c_int_p]),
        "tg_runtime_version": (ctypes.c_int, [_c_int_p, _c_int_p, _c_int_p]),
        "tg_rtc_compile": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p,
                                          ctypes.POINTER(ctypes.c_char_p), ctypes.c_int,
                                          ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_size_t),
                                          ctypes.POINTER(_vp)]),
        "tg_host_free": (None, [_vp]),
        "tg_module_load": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
        "tg_module_unload": (ctypes.c_int, [_vp]),
        "tg_module_function": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
        "tg_code_function": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.c_char_p,
                                            ctypes.POINTER(_vp)]),
        "tg_code_release": (ctypes.c_int, [_vp, ctypes.c_size_t]),
        "tg_function_attrs": (ctypes.c_int, [_vp, _c_int_p, _c_int_p, _c_int_p, _c_int_p]),
        "tg_launch": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                     _c_u64_p, ctypes.c_int, _vp, ctypes.c_int]),
        "tg_launch_ordered": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int32,
                                             ctypes.c_int32, _c_u64_p, ctypes.c_int, _vp,
                                             ctypes.c_int]),
        "tg_time_launches": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int32,
                                            ctypes.c_int32, _c_u64_p, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp,
                                            _c_f32_p, _c_f32_p]),
        "tg_run_launches": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                           _c_u64_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           _vp]),
        "tg_malloc": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_size_t]),
        "tg_free": (ctypes.c_int, [_vp]),
        "tg_memcpy_htod": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t]),
        "tg_memcpy_dtoh": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t]),
        "tg_memcpy_dtod": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t]),
        "tg_memset": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_size_t]),
        "tg_synchronize": (ctypes.c_int, []),
        "tg_stream_create": (ctypes.c_int, [ctypes.POINTER(_vp)]),
        "tg_stream_destroy": (ctypes.c_int, [_vp]),
        "tg_stream_synchronize": (ctypes.c_int, [_vp]),
        "tg_graph_begin": (ctypes.c_int, [_vp]),
        "tg_graph_end": (ctypes.c_int, [_vp, ctypes.POINTER(_vp)]),
        "tg_graph_launch": (ctypes.c_int, [_vp, _vp, ctypes.c_int]),
        "tg_graph_destroy": (ctypes.c_int, [_vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def lib():
    """The loaded runtime (RTLD_GLOBAL, so variant launchers resolve against
    this very copy).  Raises TileGenHipError when it was never built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            path = lib_path()
            if not os.path.exists(path):
                raise TileGenHipError(
                    "libtgrt.so is not built (%s); run __graft_entry__.build() or "
                    "python -m tilegen_amd.build" % path)
            L = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
            _declare(L)
            _LIB = L
    return _LIB


_NOALLOC = None


def noalloc_lib():
    """libtgna.so (include/tilegen_noalloc.h), loaded after libtgrt.  Raises
    TileGenHipError when it was never built."""
    global _NOALLOC
    if _NOALLOC is not None:
        return _NOALLOC
    lib()
    with _LOCK:
        if _NOALLOC is None:
            path = os.path.join(lib_dir(), "libtgna.so")
            if not os.path.exists(path):
                raise TileGenHipError("libtgna.so is not built (%s); run "
                                      "__graft_entry__.build()" % path)
            L = ctypes.CDLL(path)
            L.launch_spmv_noalloc.argtypes = [_vp] * 5 + [ctypes.c_int64] * 3 + [_vp]
            L.launch_spmv_noalloc.restype = ctypes.c_int
            _NOALLOC = L
    return _NOALLOC


def last_error() -> str:
    msg = lib().tg_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = last_error()
        raise TileGenHipError("%s%s" % ("%s: " % what if what else "", msg or "error %d" % rc),
                              rc)


def check_status(what: str) -> None:
    """Raise if the last libtgrt call on this thread recorded a failure (the
    void ``launch_<name>`` entry points report this way)."""
    rc = lib().tg_last_status()
    if rc != 0:
        raise TileGenHipError("%s failed: %s" % (what, last_error()), rc)


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib().tg_device_count(ctypes.byref(n)), "tg_device_count")
    return int(n.value)


def device_info(device: int = 0) -> dict:
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(256)
    cu, clk, l2 = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    mem = ctypes.c_int64()
    check(lib().tg_device_props(device, name, 256, arch, 256, ctypes.byref(cu),
                                ctypes.byref(mem), ctypes.byref(clk), ctypes.byref(l2)),
          "tg_device_props")
    return {"name": name.value.decode(), "arch": arch.value.decode(), "cu_count": cu.value,
            "global_mem_bytes": mem.value, "clock_khz": clk.value, "l2_bytes": l2.value}


def rtc_compile(source: str, name: str, options: Sequence[str]) -> Tuple[bytes, str]:
    """Compile HIP source with hipRTC; returns (code object, log)."""
    L = lib()
    opts = (ctypes.c_char_p * max(1, len(options)))(*[o.encode() for o in options])
    code, size, log = _vp(), ctypes.c_size_t(), _vp()
    rc = L.tg_rtc_compile(source.encode(), name.encode(), opts, len(options),
                          ctypes.byref(code), ctypes.byref(size), ctypes.byref(log))
    text = ""
    if log.value:
        text = ctypes.string_at(log.value).decode("utf-8", "replace")
        L.tg_host_free(log)
    if rc != 0:
        msg = last_error()
        raise TileGenHipError("hipRTC failed for %s: %s\n%s" % (name, msg, text), rc)
    blob = ctypes.string_at(code.value, size.value)
    L.tg_host_free(code)
    return blob, text


def synchronize() -> None:
    check(lib().tg_synchronize(), "tg_synchronize")


class DeviceBuffer:
    """Device copy of a contiguous numpy array (``hipMalloc`` + H2D)."""

    def __init__(self, array: Optional[np.ndarray] = None, nbytes: int = 0):
        self.array = None if array is None else np.ascontiguousarray(array)
        self.nbytes = int(self.array.nbytes if self.array is not None else nbytes)
        p = _vp()
        check(lib().tg_malloc(ctypes.byref(p), max(1, self.nbytes)), "tg_malloc")
        self.ptr = int(p.value)
        if self.array is not None and self.nbytes:
            check(lib().tg_memcpy_htod(self.ptr, self.array.ctypes.data, self.nbytes),
                  "tg_memcpy_htod")

    def to_host(self, out: Optional[np.ndarray] = None) -> np.ndarray:
        if out is None:
            if self.array is None:
                raise ValueError("DeviceBuffer made from a byte count has no host shape: "
                                 "pass out=")
            out = np.empty_like(self.array)
        if not out.flags.c_contiguous or out.nbytes < self.nbytes:
            raise ValueError("to_host: out must be C-contiguous and hold %d bytes" % self.nbytes)
        if self.nbytes:
            check(lib().tg_memcpy_dtoh(out.ctypes.data, self.ptr, self.nbytes), "tg_memcpy_dtoh")
        return out

    def upload(self, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array)
        if a.nbytes != self.nbytes:
            raise ValueError("upload of %d bytes into a %d-byte buffer" % (a.nbytes, self.nbytes))
        if self.nbytes:
            check(lib().tg_memcpy_htod(self.ptr, a.ctypes.data, self.nbytes), "tg_memcpy_htod")

    def fill_bytes(self, value: int) -> None:
        check(lib().tg_memset(self.ptr, int(value), self.nbytes), "tg_memset")

    def free(self) -> None:
        if self.ptr:
            lib().tg_free(self.ptr)
            self.ptr = 0

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.free()
        except Exception:
            pass


def stream_create() -> int:
    """A new non-blocking stream at the default priority (free with
    ``stream_destroy``)."""
    s = ctypes.c_void_p()
    check(lib().tg_stream_create(ctypes.byref(s)), "tg_stream_create")
    return int(s.value)


def stream_destroy(stream: int) -> None:
    check(lib().tg_stream_destroy(stream), "tg_stream_destroy")


def stream_synchronize(stream: int) -> None:
    check(lib().tg_stream_synchronize(stream), "tg_stream_synchronize")


def graph_capture(stream: int, enqueue) -> int:
    """Capture what ``enqueue()`` launches on ``stream`` (a ``stream_create``
    handle) into an instantiated HIP graph and return its handle (replay with
    ``graph_launch``, free with ``graph_destroy``).  The capture is ended even
    when ``enqueue`` raises."""
    L = lib()
    check(L.tg_graph_begin(stream), "tg_graph_begin")
    exec_ = ctypes.c_void_p()
    try:
        enqueue()
    finally:
        rc = L.tg_graph_end(stream, ctypes.byref(exec_))
    check(rc, "tg_graph_end")
    return int(exec_.value)


def graph_launch(exec_: int, stream: int, sync: bool = True) -> None:
    check(lib().tg_graph_launch(exec_, stream, 1 if sync else 0), "tg_graph_launch")


def graph_destroy(exec_: int) -> None:
    check(lib().tg_graph_destroy(exec_), "tg_graph_destroy")


def pack_args(values: Sequence) -> List[int]:
    """8-byte kernel-argument slots: DeviceBuffer/int pointers and int64 as
    integers, floats as their IEEE-754 bits."""
    out = []
    for v in values:
        if isinstance(v, DeviceBuffer):
            out.append(v.ptr)
        elif isinstance(v, (float, np.floating)):
            out.append(struct.unpack("<Q", struct.pack("<d", float(v)))[0])
        else:
            out.append(int(v) & 0xFFFFFFFFFFFFFFFF)
    return out


def launch(fn: int, grid: int, block: int, lds: int, args: Sequence, sync: bool = True) -> None:
    slots = pack_args(args)
    arr = (ctypes.c_uint64 * max(1, len(slots)))(*slots)
    check(lib().tg_launch(fn, int(grid), int(block), int(lds), arr, len(slots), None,
                          1 if sync else 0), "tg_launch")


def time_launches(fn: int, grid: int, block: int, lds: int, arg_sets: Sequence[Sequence],
                  warmup: int, iters: int) -> Tuple[np.ndarray, float]:
    """Per-launch kernel durations (ms) from dispatch-attached events, and the
    event wall time over all timed launches.  Launch i uses ``arg_sets[i % n]``."""
    packed = [pack_args(s) for s in arg_sets]
    n_args = len(packed[0])
    flat = (ctypes.c_uint64 * (n_args * len(packed)))(*[v for s in packed for v in s])
    kms = (ctypes.c_float * iters)()
    wall = ctypes.c_float()
    check(lib().tg_time_launches(fn, int(grid), int(block), int(lds), flat, n_args,
                                 len(packed), int(warmup), int(iters), None, kms,
                                 ctypes.byref(wall)), "tg_time_launches")
    return np.array(kms[:], dtype=np.float64), float(wall.value)


class ArgSets:
    """Packed argument slots for rotating launches (kept alive by the caller)."""

    def __init__(self, arg_sets: Sequence[Sequence]):
        packed = [pack_args(s) for s in arg_sets]
        self.n_args = len(packed[0])
        self.n_sets = len(packed)
        self.buf = (ctypes.c_uint64 * (self.n_args * self.n_sets))(
            *[v for s in packed for v in s])


def run_launches(fn: int, grid: int, block: int, lds: int, sets: "ArgSets", iters: int) -> None:
    """Enqueue ``iters`` launches (no synchronization, no events)."""
    check(lib().tg_run_launches(fn, int(grid), int(block), int(lds), sets.buf, sets.n_args,
                                sets.n_sets, int(iters), None), "tg_run_launches")

"""Schedule autotuner (entry points of reference ``tilegen/autotune.py``).

The search space is re-derived for CDNA4 rather than copied from the CUDA
one (reference ``autotune.py:47-72``):

* block_size B in {64, 128, 256, 512, 1024}: whole 64-lane waves only;
* threads_per_row TPR in {1, 2, 4, 8, 16, 32, 64}: a lane group never
  straddles a wave, so the segmented reduction stays inside one wave's DPP;
* tile_size T: rows per workgroup; T < B/TPR would leave lane groups idle
  and T > 8*B/TPR makes a lane group walk more than 8 rows in sequence;
* unroll U in {1, 2, 4, 8}; vector_width V in {1, 2} (2 x f64 = 128 bits,
  the widest global load);
* LDS per workgroup within gfx950's 160 KiB: a tiled SpMV-shaped variant
  declares about 16 bytes per tile row (staged row pointers plus the long- and
  medium-row lists), so T <= 2048 stays far inside it.

``tune(..., backend="hip")`` times each variant with GPU events attached to
the kernel dispatch (libtgrt ``tg_time_launches``), rotating over enough
device copies of the inputs that every launch reads HBM rather than a cache
the previous launch warmed; ``backend="cpu"`` keeps the reference's host
timer around the OpenMP variant.  Every variant is verified against SciPy
before it is timed, and only verified variants can win.
"""

from __future__ import annotations

import ctypes
import dataclasses
import itertools
import json
import os
import random
import time
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import scipy.sparse as sp

from . import codegen as _codegen
from .codegen import LDS_LIMIT, Config
from .dsl import standard_kernels
from .verify import _SIGNATURES, _inputs_for, _load_matrix, _reference, compile_generated

__all__ = [
    "SEARCH_SPACE", "BASELINE", "illegal_reason", "illegal_reason_for", "enumerate_configs",
    "legal_configs", "prune_log", "tune", "write_outputs",
]

SEARCH_SPACE: Dict[str, List[int]] = {
    "tile_size": [8, 16, 32, 64, 128, 256, 512, 1024, 2048],
    "threads_per_row": [1, 2, 4, 8, 16, 32, 64],
    "unroll": [1, 2, 4, 8],
    "vector_width": [1, 2],
    "block_size": [64, 128, 256, 512, 1024],
}

# The reference's default schedule (autotune.py:55-56).  On CDNA4 it leaves
# 96 of 128 lanes idle, so the search space prunes it, but tune() still times it
# first as the naive baseline every speedup is measured against.
BASELINE = Config(tile_size=32, threads_per_row=1, unroll=1, vector_width=1, block_size=128)

_WAVE = 64
# kernels whose schedules also come with merge-path windows, hybrid tiles and
# stream ranges (Config.balance)
MERGE_KERNELS = ("spmv", "fused_spmv_axpy")
ROTATE_BYTES = 640 << 20


def _shape_reason(cfg: Config) -> Optional[str]:
    """Block, lane-group and vector checks shared by every kernel."""
    B, tpr = cfg.block_size, cfg.threads_per_row
    if B % _WAVE:
        return "block_size (%d) is not a multiple of the 64-lane wave" % B
    if B > 1024:
        return "block_size (%d) > 1024" % B
    if tpr > _WAVE or _WAVE % tpr:
        return "threads_per_row (%d) does not divide the 64-lane wave" % tpr
    if tpr > B:
        return "threads_per_row (%d) > block_size (%d)" % (tpr, B)
    if cfg.vector_width not in (1, 2):
        return "vector_width %d not supported (128-bit loads hold 2 x f64)" % cfg.vector_width
    if cfg.vector_width > cfg.unroll:
        return "vector_width (%d) > unroll (%d)" % (cfg.vector_width, cfg.unroll)
    return None


def illegal_reason(cfg: Config) -> Optional[str]:
    """Why a schedule is illegal on CDNA4, or None."""
    r = _shape_reason(cfg)
    if r is not None:
        return r
    B, tpr, T = cfg.block_size, cfg.threads_per_row, cfg.tile_size
    slots = B // tpr
    if T < slots:
        return "tile_size (%d) < lane groups per block (%d): idle lanes" % (T, slots)
    if T > 8 * slots:
        return "tile_size (%d) > 8 rows per lane group (%d groups)" % (T, slots)
    if 16 * (T + 1) > LDS_LIMIT:
        return "row pointers and row lists (%d B) exceed 160 KiB of LDS" % (16 * (T + 1))
    return None


def sddmm_group_per_row(cfg: Config, K: int) -> bool:
    """Whether the SDDMM variant takes its chunked path at this K (one lane
    group per row, K covered by one group's registers) rather than one wave
    per row."""
    tpr, V = cfg.threads_per_row, 2 if cfg.vector_width >= 2 else 1
    return K <= tpr * V * max(1, cfg.unroll) and (V == 1 or K % 2 == 0)


def illegal_reason_for(kernel: str, cfg: Config, K: int = 8) -> Optional[str]:
    """Kernel-specific pruning on top of ``illegal_reason``."""
    if kernel == "sddmm":
        r = _shape_reason(cfg)
        if r is not None:
            return r
        if cfg.threads_per_row * cfg.vector_width > max(K, 1):
            return "threads_per_row x vector_width (%d) > K (%d)" % (
                cfg.threads_per_row * cfg.vector_width, K)
        if sddmm_group_per_row(cfg, K):
            per, what = cfg.block_size // cfg.threads_per_row, "lane group"
        else:
            per, what = cfg.block_size // _WAVE, "wave"
        if cfg.tile_size < per or cfg.tile_size > 8 * per:
            return ("sddmm runs one row per %s at K=%d: tile_size must be 1..8 x %d"
                    % (what, K, per))
        return None
    r = illegal_reason(cfg)
    if r is not None:
        return r
    if cfg.balance == "stream" and _stream_reason(cfg) is not None:
        return _stream_reason(cfg)
    if kernel in ("spmv", "fused_spmv_axpy") and cfg.vector_width != 1:
        return "vector_width has no effect on %s (the vectorize pass drops it)" % kernel
    if kernel == "spmm" and cfg.threads_per_row * cfg.vector_width > max(_WAVE, 2 * K):
        return "threads_per_row x vector_width (%d) far exceeds K (%d)" % (
            cfg.threads_per_row * cfg.vector_width, K)
    return None


def _sddmm_space(K: int) -> List[Config]:
    """Tiles of 1, 2 and 4 rows per lane group (chunked path) or per wave
    (general path), whichever the variant takes at this K."""
    out = []
    for B, tpr, U, V in itertools.product([64, 128, 256, 512], [1, 2, 4, 8, 16, 32, 64],
                                          [1, 2, 4, 8], [1, 2]):
        probe = Config(threads_per_row=tpr, unroll=U, vector_width=V, block_size=B)
        per = B // tpr if sddmm_group_per_row(probe, K) else B // _WAVE
        for mult in (1, 2, 4):
            if per * mult <= 4096:
                out.append(Config(tile_size=per * mult, threads_per_row=tpr, unroll=U,
                                  vector_width=V, block_size=B))
    return out


def enumerate_configs(kernel: Optional[str] = None, K: int = 8
                      ) -> List[Tuple[Config, Optional[str]]]:
    """Every raw schedule with its prune reason (None = legal)."""
    if kernel == "sddmm":
        return [(c, illegal_reason_for(kernel, c, K)) for c in _sddmm_space(K)]
    keys = list(SEARCH_SPACE)
    out = []
    for combo in itertools.product(*(SEARCH_SPACE[k] for k in keys)):
        cfg = Config(**dict(zip(keys, combo)))
        reason = illegal_reason(cfg) if kernel is None else illegal_reason_for(kernel, cfg, K)
        out.append((cfg, reason))
    if kernel in MERGE_KERNELS:
        # the same schedules with merge-path windows and with hybrid tiles
        rows = list(out)
        for balance in ("nnz", "hybrid"):
            out += [(dataclasses.replace(c, balance=balance), r) for c, r in rows]
        # and with stream ranges, which do not use the tile size: each (TPR, U, B)
        # once, at the smallest legal tile
        out += [(dataclasses.replace(c, balance="stream"),
                 r if r is not None else _stream_reason(c)) for c, r in rows
                if c.tile_size == c.block_size // c.threads_per_row]
        # and row tiles whose first-step gathers are sorted in LDS
        out += [(dataclasses.replace(c, gather="sorted"),
                 r if r is not None else _sorted_reason(c)) for c, r in rows]
    return out


def _stream_reason(cfg: Config) -> Optional[str]:
    """Stream ranges stage their products in LDS: block x unroll nonzeros."""
    from .codegen import STREAM_MAX_CHUNK
    if cfg.block_size * cfg.unroll > STREAM_MAX_CHUNK:
        return "stream range of %d nonzeros exceeds %d" % (cfg.block_size * cfg.unroll,
                                                          STREAM_MAX_CHUNK)
    return None


def _sorted_reason(cfg: Config) -> Optional[str]:
    """A sorted tile holds its first step in registers (rows per lane group x
    unroll <= 8), its items in LDS (at most SORT_MAX_ITEMS), and those with the
    tile's row pointers and lists within one workgroup's LDS."""
    from .codegen import SORT_MAX_ITEMS, _lowering, _plan, launch_geometry
    from .dsl import standard_kernels
    from .passes import run_pipeline
    slots = cfg.block_size // cfg.threads_per_row
    rows = -(-cfg.tile_size // slots)
    if rows * cfg.unroll > 8:
        return "sorted first step of %d rows x unroll %d per lane exceeds 8" % (rows, cfg.unroll)
    if rows * cfg.unroll * cfg.block_size > SORT_MAX_ITEMS:
        return "sorted first step of %d items exceeds %d" % (
            rows * cfg.unroll * cfg.block_size, SORT_MAX_ITEMS)
    k = run_pipeline(standard_kernels()["spmv"], dataclasses.replace(cfg, gather="sorted"),
                     backend="hip")
    lds = launch_geometry(_plan(k), _lowering(k)).lds_bytes
    if lds > LDS_LIMIT:
        return "sorted tile's LDS arrays (%d B) exceed 160 KiB" % lds
    return None


def legal_configs(kernel: Optional[str] = None, K: int = 8) -> List[Config]:
    return [c for c, r in enumerate_configs(kernel, K) if r is None]


def prune_log(kernel: Optional[str] = None, K: int = 8) -> List[Dict[str, str]]:
    return [{"config": str(c.to_dict()), "reason": r}
            for c, r in enumerate_configs(kernel, K) if r is not None]


# --------------------------------------------------------------------------- #
# measurement
# --------------------------------------------------------------------------- #
def _flops_bytes(kernel: str, A: sp.csr_matrix, K: int) -> Tuple[float, float, float]:
    """(flops, reference byte model, compulsory bytes).

    The reference counts one gather per nonzero (``autotune.py:97-110``); the
    compulsory model counts every array once (x, B, U, V included).
    """
    from .matrices import compulsory_bytes, flops
    M, N = A.shape
    nnz = int(A.nnz)
    ref_model = {
        "spmv": nnz * 16.0 + (M + 1) * 8.0 + nnz * 8.0 + M * 8.0,
        "spmm": nnz * 16.0 + (M + 1) * 8.0 + nnz * K * 8.0 + M * K * 8.0,
        "sddmm": nnz * 16.0 + (M + 1) * 8.0 + 2.0 * nnz * K * 8.0 + nnz * 8.0,
        "fused_spmv_axpy": nnz * 16.0 + (M + 1) * 8.0 + nnz * 8.0 + 2 * M * 8.0,
        "axpy": 3.0 * M * 8.0,
    }[kernel]
    if kernel == "axpy":
        return 2.0 * M, ref_model, 24.0 * M
    return flops(kernel, nnz, K), ref_model, float(compulsory_bytes(kernel, M, N, nnz, K))


class _HipBench:
    """Device-resident inputs (rotated copies) for one (kernel, matrix)."""

    def __init__(self, kernel_name: str, A: sp.csr_matrix, data, K: int, rotate_bytes: int):
        from . import runtime as rt
        self.rt = rt
        self.kernel = kernel_name
        self.A, self.K = A, K
        M, N = A.shape
        self.dims = (M, N, K, int(A.nnz))
        from .verify import _call_arrays
        arrays, self.out_index, self.scalars, self.out = _call_arrays(kernel_name, A, data, K)
        self.arrays = arrays
        per_copy = sum(a.nbytes for a in arrays)
        self.copies = int(min(64, max(1, -(-rotate_bytes // max(per_copy, 1)))))
        self.sets, self.bufs = [], []
        for _ in range(self.copies):
            bufs = [rt.DeviceBuffer(a) for a in arrays]
            self.bufs.append(bufs)
            self.sets.append(list(bufs) + list(self.scalars))

    def result(self) -> np.ndarray:
        return self.bufs[0][self.out_index].to_host()

    def free(self) -> None:
        for bufs in self.bufs:
            for b in bufs:
                b.free()


def _make_caller(lib_path: str, kernel_name: str, A: sp.csr_matrix, data, K: int,
                 backend: str = "cpu", bench: Optional[_HipBench] = None):
    """Zero-argument closure over one variant with fixed buffers.

    HIP: ``caller()`` launches through ``launch_<name>`` on copy 0 and copies
    the output back; ``caller.time(warmup, iters)`` returns per-launch kernel
    milliseconds from dispatch-attached events, rotating over the copies.
    CPU: ``caller()`` calls the OpenMP launcher on host arrays.
    """
    lib = ctypes.CDLL(lib_path)
    fn = getattr(lib, "launch_%s" % kernel_name)
    fn.argtypes = _SIGNATURES[kernel_name]
    if backend == "hip":
        from . import runtime as rt
        lib.tgv_function.restype = ctypes.c_void_p
        lib.tgv_geometry.argtypes = [ctypes.c_int64] * 4 + [
            ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32),
            ctypes.POINTER(ctypes.c_int32)]
        g, b, l = ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32()
        M, N, Kd, nnz = bench.dims
        lib.tgv_geometry(M, N, Kd, nnz, ctypes.byref(g), ctypes.byref(b), ctypes.byref(l))
        geom = (g.value, b.value, l.value)
        first = bench.sets[0]

        def caller():
            conv = [ctypes.cast(v.ptr, t) if isinstance(v, rt.DeviceBuffer) else v
                    for v, t in zip(first, fn.argtypes)]
            rt.lib().tg_clear_error()
            fn(*conv)
            rt.check_status("launch_%s" % kernel_name)
            return bench.result()

        def timer(warmup: int, iters: int) -> np.ndarray:
            rt.lib().tg_clear_error()
            kfn = lib.tgv_function()
            if not kfn:
                rt.check_status("tgv_function")
            if geom[0] == 0:
                return np.zeros(iters)
            kms, _wall = rt.time_launches(kfn, geom[0], geom[1], geom[2], bench.sets,
                                          warmup, iters)
            return kms

        caller.time = timer
        caller.launch = caller
        return caller, bench.out, [lib, bench]

    arrays, _oi, scalars, out = _call_arrays_host(kernel_name, A, data, K)
    args = [a.ctypes.data_as(ctypes.POINTER(ctypes.c_longlong if a.dtype == np.int64
                                             else ctypes.c_double)) for a in arrays]
    args += list(scalars)

    def caller():
        fn(*args)
        return out

    caller.launch = caller
    return caller, out, [lib, arrays]


def _call_arrays_host(kernel_name, A, data, K):
    from .verify import _call_arrays
    return _call_arrays(kernel_name, A, data, K)


def _time_host(caller, warmup: int, iters: int) -> np.ndarray:
    for _ in range(warmup):
        caller()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        caller()
        times.append((time.perf_counter() - t0) * 1e3)
    return np.array(times)


# --------------------------------------------------------------------------- #
# search
# --------------------------------------------------------------------------- #
def _candidate_configs(kernel: str, K: int, budget: int, mode: str, rng: random.Random,
                       include: Optional[List[Config]] = None,
                       backend: str = "hip") -> List[Config]:
    pool = legal_configs(kernel, K)
    if backend == "cpu":  # the OpenMP emitter ignores balance: row tiles only
        pool = [c for c in pool if c.balance == "rows"]
    out: List[Config] = []
    seen = set()

    def add(c: Config) -> None:
        if c.hash() not in seen and illegal_reason_for(kernel, c, K) is None:
            seen.add(c.hash())
            out.append(c)

    # the naive baseline is always measured first, even where the CDNA4 space
    # prunes it (the reference default leaves lanes idle): speedups refer to it
    base = (Config(**BASELINE.to_dict()) if kernel != "sddmm" else
            Config(tile_size=4, threads_per_row=4, unroll=1, vector_width=1, block_size=256))
    seen.add(base.hash())
    out.append(base)
    for c in include or []:
        add(c)
    if mode == "coordinate":
        best = out[0]
        steps = [(key, value) for key in SEARCH_SPACE for value in SEARCH_SPACE[key]]
        if kernel in MERGE_KERNELS and backend != "cpu":
            steps += [("balance", "nnz"), ("balance", "hybrid"), ("balance", "stream")]
        for key, value in steps:
            add(Config(**{**best.to_dict(), key: value}))
            if len(out) >= budget:
                return out
        return out[:budget]
    if mode == "exhaustive":
        for c in pool:
            add(c)
        return out
    rng.shuffle(pool)
    for c in pool:
        if len(out) >= budget:
            break
        add(c)
    return out


def tune(kernel_name: str, matrix, budget: int = 40, mode: str = "random",
         backend: str = "cpu", K: int = 8, workdir: str = "build/generated", warmup: int = 5,
         iters: int = 25, seed: int = 0, include: Optional[List[Config]] = None,
         rotate_bytes: int = ROTATE_BYTES, data=None, verbose: bool = False) -> Dict[str, Any]:
    """Autotune one (kernel, matrix) pair; a dict of every variant tried.

    Record keys follow the reference (``ms_mean/min/median``, ``gflops``,
    ``bandwidth_gbs`` on the reference byte model, ``max_abs_err``,
    ``tolerance``, ``ok``, ``speedup_vs_naive``) plus ``compulsory_gbs``.
    """
    rng = random.Random(seed)
    A, cls = _load_matrix(matrix)
    if data is None:
        data = _inputs_for(kernel_name, A, K, seed)
    ref = np.asarray(_reference(kernel_name, A, data), dtype=np.float64).ravel()
    flop, ref_bytes, comp_bytes = _flops_bytes(kernel_name, A, K)
    M, N = A.shape
    nnz = int(A.nnz)
    candidates = _candidate_configs(kernel_name, K, budget, mode, rng, include, backend)
    kernels = standard_kernels()
    eps = float(np.finfo(np.float64).eps)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    row_nnz = int(np.diff(A.indptr).max()) if M else 1
    tol = float(8.0 * eps * max(1, row_nnz) * scale + 1e-12)

    bench = _HipBench(kernel_name, A, data, K, rotate_bytes) if backend == "hip" else None
    records: List[Dict[str, Any]] = []
    baseline_ms = None
    try:
        for cfg in candidates:
            rec: Dict[str, Any] = {"kernel": kernel_name, "matrix_class": cls, "rows": int(M),
                                   "nnz": nnz, "config": cfg.to_dict(), "skipped": None}
            try:
                gen = _codegen.generate(kernels[kernel_name], cfg, backend, outdir=workdir)
                lib_path, log = compile_generated(gen, backend, workdir)
            except (RuntimeError, ValueError) as exc:
                rec["skipped"] = "compile error: %s" % exc
                records.append(rec)
                continue
            caller, out, _keep = _make_caller(lib_path, kernel_name, A, data, K, backend, bench)
            outv = np.asarray(caller(), dtype=np.float64).ravel()
            max_abs = float(np.abs(outv - ref).max()) if ref.size else 0.0
            times = (caller.time(warmup, iters) if backend == "hip"
                     else _time_host(caller.launch, warmup, iters))
            ms_mean, ms_min = float(np.mean(times)), float(np.min(times))
            ms_med = float(np.median(times))
            rec.update({
                "ms_mean": ms_mean, "ms_min": ms_min, "ms_median": ms_med,
                "gflops": flop / (ms_min * 1e6) if ms_min > 0 else 0.0,
                "bandwidth_gbs": ref_bytes / (ms_min * 1e6) if ms_min > 0 else 0.0,
                "compulsory_gbs": comp_bytes / (ms_median_or(ms_med) * 1e6),
                "max_abs_err": max_abs, "tolerance": tol, "ok": bool(max_abs <= tol),
                "timer": ("hip events on the dispatch, %d rotated input copies"
                          % bench.copies) if backend == "hip" else "host perf_counter",
                "log": log,
            })
            if verbose:
                print("[tune] %-6s %-24s median %.4f ms  %.1f GB/s  ok=%s" % (
                    kernel_name, cfg.short(), ms_med, rec["compulsory_gbs"], rec["ok"]),
                    flush=True)
            if cfg.hash() == candidates[0].hash():
                baseline_ms = ms_min
            records.append(rec)
    finally:
        if bench is not None:
            bench.free()

    base = baseline_ms
    if base is None:
        measured = [r for r in records if r.get("ms_min")]
        base = measured[0]["ms_min"] if measured else None
    for r in records:
        r["speedup_vs_naive"] = (base / r["ms_min"]) if (r.get("ms_min") and base) else None
    measured = [r for r in records if r.get("ms_min") and r.get("ok")]
    winner = min(measured, key=lambda r: r["ms_median"]) if measured else None
    return {"kernel": kernel_name, "matrix_class": cls, "backend": backend,
            "mode": mode, "candidates": len(candidates),
            "baseline": candidates[0].to_dict(), "baseline_ms_min": base,
            "winner": winner["config"] if winner else None,
            "winner_metrics": winner, "records": records}


def ms_median_or(v: float) -> float:
    return v if v > 0 else float("inf")


_METRIC_FIELDS = ["ms_mean", "ms_min", "ms_median", "gflops", "bandwidth_gbs",
                  "compulsory_gbs", "max_abs_err", "tolerance", "ok", "speedup_vs_naive"]
_CSV_COLS = ["matrix_class", "kernel", "tile_size", "threads_per_row", "unroll",
             "vector_width", "block_size", "balance", "gather", "ms_mean", "ms_min", "ms_median",
             "gflops", "bandwidth_gbs", "compulsory_gbs", "max_abs_err", "ok", "speedup_vs_naive"]


def _compact(record: Optional[Dict[str, Any]]) -> Optional[Dict[str, Any]]:
    if record is None:
        return None
    return {k: record.get(k) for k in _METRIC_FIELDS if k in record}


def _flat(record: Dict[str, Any]) -> Dict[str, Any]:
    # Config.to_dict leaves the default balance and gather out
    row = {"matrix_class": record["matrix_class"], "kernel": record["kernel"],
           "balance": "rows", "gather": "direct"}
    row.update(record["config"])
    row.update({k: record.get(k) for k in _METRIC_FIELDS if k in record})
    return row


def _write_csv(path: str, rows: List[Dict[str, Any]]) -> None:
    with open(path, "w") as fh:
        fh.write(",".join(_CSV_COLS) + "\n")
        for row in rows:
            fh.write(",".join(str(row.get(c, "")) for c in _CSV_COLS) + "\n")


def write_outputs(all_results: List[Dict[str, Any]], outdir: str, env: Dict[str, Any],
                  pruned: List[Dict[str, str]], full_outdir: str = "build") -> None:
    """Compact summary (winners, top five per class) into ``outdir``; the full
    sweep into ``full_outdir`` (reference ``autotune.py:354-417`` schema)."""
    os.makedirs(outdir, exist_ok=True)
    os.makedirs(full_outdir, exist_ok=True)
    best: Dict[str, Dict[str, Any]] = {}
    flat: List[Dict[str, Any]] = []
    compact: List[Dict[str, Any]] = []
    top5: Dict[str, List[Dict[str, Any]]] = {}
    for res in all_results:
        cls = res["matrix_class"]
        compact.append({"kernel": res["kernel"], "matrix_class": cls,
                        "mode": res.get("mode"), "candidates": res.get("candidates"),
                        "baseline": res["baseline"], "baseline_ms_min": res["baseline_ms_min"],
                        "winner": res["winner"], "winner_metrics": _compact(res["winner_metrics"])})
        best.setdefault(cls, {})[res["kernel"]] = {
            "config": res["winner"], "metrics": _compact(res["winner_metrics"]),
            "baseline_ms_min": res["baseline_ms_min"]}
        for r in res["records"]:
            if r.get("ms_min") is not None:
                flat.append(_flat(r))
                if r.get("ok"):
                    top5.setdefault(cls, []).append(_flat(r))
    for cls in top5:
        top5[cls] = sorted(top5[cls], key=lambda r: r["ms_median"])[:5]
    with open(os.path.join(full_outdir, "autotune.json"), "w") as fh:
        json.dump({"hardware": env, "baseline": BASELINE.to_dict(),
                   "search_space": SEARCH_SPACE, "pruned": pruned,
                   "results": all_results}, fh, indent=2, default=str)
    _write_csv(os.path.join(full_outdir, "autotune.csv"), flat)
    with open(os.path.join(outdir, "autotune.json"), "w") as fh:
        json.dump({"hardware": env, "baseline": BASELINE.to_dict(),
                   "search_space": SEARCH_SPACE, "pruned": pruned, "results": compact,
                   "best": best, "top5": top5}, fh, indent=2, default=str)
    with open(os.path.join(outdir, "best_configs.json"), "w") as fh:
        json.dump(best, fh, indent=2, default=str)
    _write_csv(os.path.join(outdir, "autotune.csv"),
               [row for cls in sorted(top5) for row in top5[cls]])

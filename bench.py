#!/usr/bin/env python3
"""Benchmark of the TileGen HIP CSR hot path on one MI355X; prints ONE JSON line.

A step is one launch of a case's tuned HIP variant over one copy of the case's
inputs, already resident in HBM.  Launches rotate over enough input copies
(>= 640 MB in total, more than the 256 MB Infinity Cache) that every step reads
its matrix from HBM, not from a cache a previous step warmed.

With no ``--case`` the run covers every BASELINE config: c1 (the config the
headline metric is quoted on) gives the top-level keys, and ``cases`` holds one
compact entry per other config (c2, c3a, c3b, c4, c5, c5x25), each measured the
same way in the same process.  ``--case X`` runs config X alone with full
detail (the form the rocprofv3 commands under profiles/ use).

value        headline case: compulsory bytes of K steps / host wall time of the
             K steps, bracketed by device synchronizations (launch gaps
             included)
roofline     per-kernel duration from start/stop events attached to each
             dispatch (hipExtModuleLaunchKernel), averaged over the timed
             launches; achieved = compulsory bytes per launch / that duration,
             against MI355X's 8 TB/s HBM peak; traffic = bytes moved beyond L2
             per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, each scaled by a
             plain copy of known size; Infinity Cache hits count as beyond L2),
             when a summary for this kernel and case is committed in profiles/
cpu_baseline the reference's own sequential cpp/src/ref.cpp (oracle/_ref, kind
             "reference"; else this repository's C restatement, kind "port"),
             one host core, on the full case matrix for a bounded number of calls
cpu_openmp   this build's OpenMP CPU backend (the reference's ``_cpu_emit``
             design) at the reference default schedule T32/TPR1/U1/V1/B128,
             compiled on this host with g++ -O3 -march=native -fopenmp and run
             on every OpenMP thread, host perf_counter around each call
cpu_openmp_tuned
             the same backend at the case's CPU-tuned schedule
             (tilegen_amd.schedules.CPU_TUNED, from tilegen_amd.cpu_tuned)
cases        per other config: us (event-timed kernel average), gbs
             (compulsory GB/s), frac (gbs / 8000), gflops, traffic (beyond-L2
             bytes / compulsory bytes, committed PMC summary), err (normwise
             relative error against float64 SciPy), cpu_ms (ref.cpp, one core),
             omp_ms / omp_tuned_ms (OpenMP backend medians, every host thread)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SpMV achieved HBM GB/s (% of peak) + GFLOP/s, fp64 CSR; SpMM/SDDMM GFLOP/s"
PEAK_HBM_GBS = 8000.0
HEADLINE = "c1"
OTHER_CASES = ("c2", "c3a", "c3b", "c4", "c5", "c5x25")


def _log(msg: str) -> None:
    print("[bench] " + msg, file=sys.stderr, flush=True)


def _parse_config(text: str):
    from tilegen_amd.codegen import Config
    vals = {}
    for part in text.replace(",", "/").split("/"):
        part = part.strip()
        if part in ("nnz", "rows", "hybrid", "stream"):  # what a tile holds (Config.balance)
            vals["balance"] = part
            continue
        if part in ("sorted", "direct"):  # the order of a tile's gathers (Config.gather)
            vals["gather"] = part
            continue
        for key, name in (("TPR", "threads_per_row"), ("T", "tile_size"), ("U", "unroll"),
                          ("V", "vector_width"), ("B", "block_size")):
            if part.startswith(key) and part[len(key):].isdigit():
                vals[name] = int(part[len(key):])
                break
        else:
            raise SystemExit("bad --config component %r (want T128/TPR8/U2/V1/B256)" % part)
    return Config(**vals)


def _pmc_summary(kernel: str, case_id: str):
    path = os.path.join(ROOT, "profiles", "%s_%s_pmc.json" % (kernel, case_id))
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        return json.load(fh)


def _traffic(kernel: str, case_id: str):
    """Bytes moved beyond L2 per launch (FETCH_SIZE + WRITE_SIZE) from a
    committed rocprofv3 PMC summary, or None."""
    d = _pmc_summary(kernel, case_id)
    return None if d is None else d.get("beyond_l2_bytes_per_launch")


_COPY_SRC = r"""
extern "C" __global__ __launch_bounds__(256)
void tg_copy_kernel(const double* __restrict__ src, double* __restrict__ dst, long long n) {
  const long long stride = (long long)gridDim.x * 256;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    dst[i] = src[i];
}
"""


def calibrate_copy(mib: int, launches: int = 10) -> int:
    """Launch a plain copy of ``mib`` MiB ``launches`` times, so a rocprofv3
    --pmc run can relate FETCH_SIZE / WRITE_SIZE to a known byte count."""
    import ctypes
    from tilegen_amd import runtime as rt
    from tilegen_amd.verify import hiprtc_options
    code, _ = rt.rtc_compile(_COPY_SRC, "tg_copy.hip", hiprtc_options())
    blob = ctypes.create_string_buffer(code, len(code))
    mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
    rt.check(rt.lib().tg_module_load(blob, len(code), ctypes.byref(mod)), "module")
    rt.check(rt.lib().tg_module_function(mod, b"tg_copy_kernel", ctypes.byref(fn)), "function")
    n = (mib << 20) // 8
    src = rt.DeviceBuffer(np.arange(n, dtype=np.float64))
    dst = rt.DeviceBuffer(nbytes=n * 8)
    for _ in range(launches):
        rt.launch(fn.value, 4096, 256, 0, [src, dst, n])
    ok = bool(np.array_equal(dst.to_host(np.empty(n)), np.arange(n, dtype=np.float64)))
    print(json.dumps({"calibration": "tg_copy_kernel", "bytes_read": n * 8,
                      "bytes_written": n * 8, "launches": launches, "ok": ok}), flush=True)
    src.free()
    dst.free()
    return 0 if ok else 1


def _cpu_baseline(kernel, A, ops, budget_s: float):
    import oracle
    kind = "reference" if oracle.reference_available() else "port"
    if kind == "reference":
        rm = oracle.RefMatrix(A)
        K = ops[next(iter(ops))].shape[1] if kernel != "spmv" else 0
        rm.set_operands(K=K, x=ops.get("x"), B=ops.get("B"), U=ops.get("U"), V=ops.get("V"))
        _, t1 = rm.run(kernel, 1)
        iters = int(max(1, min(2000, budget_s / max(t1, 1e-6))))
        _, sec = rm.run(kernel, iters)
        rm.close()
    else:
        t0 = time.perf_counter()
        oracle.compute(kernel, A, ops)
        t1 = time.perf_counter() - t0
        iters = int(max(1, min(2000, budget_s / max(t1, 1e-6))))
        t0 = time.perf_counter()
        for _ in range(iters):
            oracle.compute(kernel, A, ops)
        sec = (time.perf_counter() - t0) / iters
    return kind, sec, iters


def _omp_threads() -> int:
    import ctypes
    try:
        return int(ctypes.CDLL("libgomp.so.1").omp_get_max_threads())
    except OSError:
        return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def _openmp_baseline(kernel, A, ops, K, ref, nbytes, nflop, budget_s: float, cfg=None):
    """Time the OpenMP variant of a schedule on the host (the reference
    default schedule unless ``cfg`` is given)."""
    from tilegen_amd.autotune import BASELINE, _make_caller, _time_host
    from tilegen_amd.codegen import generate
    from tilegen_amd.dsl import standard_kernels
    from tilegen_amd.verify import compile_generated
    cfg = cfg or BASELINE
    workdir = os.path.join(ROOT, "build", "bench_cpu")
    gen = generate(standard_kernels()[kernel], cfg, "cpu", outdir=workdir)
    so, build_log = compile_generated(gen, "cpu", workdir)
    data = (ops.get("x"), None, ops.get("B"), ops.get("U"), ops.get("V"), 1.0, 0.0)
    caller, _out, _keep = _make_caller(so, kernel, A, data, K, "cpu")
    t0 = time.perf_counter()
    got = np.asarray(caller(), dtype=np.float64).reshape(np.shape(ref))
    t1 = time.perf_counter() - t0
    err = float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300))
    if not err <= 1e-10:
        raise SystemExit("OpenMP backend check failed for %s: rel err %.3e" % (kernel, err))
    iters = int(max(5, min(2000, budget_s / max(t1, 1e-6))))
    ms = _time_host(caller.launch, 2, iters)
    med = float(np.median(ms)) * 1e-3
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": _omp_threads(),
            "kind": "openmp backend", "schedule": cfg.short(),
            "gflops": round(nflop / med / 1e9, 3), "ms_median": round(med * 1e3, 4),
            "calls": iters, "rel_err": err, "compile": build_log.split(" with: ")[-1]}


def _scipy_reference(kernel, A, ops):
    """float64 SciPy/numpy result of the case (the check of this run)."""
    if kernel == "spmv":
        return A @ ops["x"]
    if kernel == "spmm":
        return A @ ops["B"]
    coo = A.tocoo()
    out = np.empty(coo.nnz)
    step = 1 << 21
    for s in range(0, coo.nnz, step):
        e = min(s + step, coo.nnz)
        out[s:e] = np.einsum("ik,ik->i", ops["U"][coo.row[s:e]], ops["V"][coo.col[s:e]]) \
            * coo.data[s:e]
    return out


class CaseRun:
    """One BASELINE config resident on the device: its tuned variant, rotated
    input copies and the argument sets that launch over them."""

    def __init__(self, case_id: str, cfg, warm: bool):
        from tilegen_amd import runtime as rt
        from tilegen_amd.matrices import (baseline_case, baseline_operands, compulsory_bytes,
                                          flops, make_baseline)
        from tilegen_amd.profiling import bench_copies
        from tilegen_amd.variant import Variant
        t0 = time.time()
        self.case_id = case_id
        self.case = baseline_case(case_id)
        self.kernel = self.case.kernel
        self.cfg = cfg
        self.A = make_baseline(case_id)
        self.M, self.N = self.A.shape
        self.nnz = int(self.A.nnz)
        self.K = self.case.K
        self.ops = baseline_operands(self.kernel, self.M, self.N, self.K)
        self.v = Variant(self.kernel, cfg)
        self.fn = self.v.function()
        self.grid, self.block, self.lds = self.v.geometry(self.M, self.N, self.K, self.nnz)
        self.nbytes = compulsory_bytes(self.kernel, self.M, self.N, self.nnz, self.K)
        self.nflop = flops(self.kernel, self.nnz, self.K)
        self.copies = 1 if warm else bench_copies(self.nbytes)
        host = {"indptr": self.A.indptr.astype(np.int64),
                "indices": self.A.indices.astype(np.int64),
                "data": self.A.data.astype(np.float64)}
        host.update({k: np.ascontiguousarray(val, dtype=np.float64)
                     for k, val in self.ops.items()})
        self.out_name = {"spmv": "y", "spmm": "C", "sddmm": "C"}[self.kernel]
        self.out_shape = {"spmv": (self.M,), "spmm": (self.M, self.K),
                          "sddmm": (self.nnz,)}[self.kernel]
        self.sets, self.keep = [], []
        for _ in range(self.copies):
            bufs = {k: rt.DeviceBuffer(a) for k, a in host.items()}
            bufs[self.out_name] = rt.DeviceBuffer(np.zeros(self.out_shape))
            self.keep.append(bufs)
            self.sets.append(self.v.abi_values(self.A, bufs, {}, self.M, self.N, self.K,
                                               self.nnz))
        _log("%s (%s) M=%d N=%d nnz=%d K=%d, %s grid=%d block=%d, %d copies (%.0f MB) "
             "resident in %.1fs" % (case_id, self.kernel, self.M, self.N, self.nnz, self.K,
                                    cfg.short(), self.grid, self.block, self.copies,
                                    self.copies * self.nbytes / 1e6, time.time() - t0))

    def check(self):
        """One launch through the C ABI, against float64 SciPy; returns
        (reference, normwise relative error)."""
        self.v.device_call(self.sets[0])
        got = self.keep[0][self.out_name].to_host()
        ref = _scipy_reference(self.kernel, self.A, self.ops)
        err = float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300))
        _log("%s check vs float64 SciPy: normwise rel err %.3e" % (self.case_id, err))
        if not err <= 1e-10:
            raise SystemExit("%s result check failed: rel err %.3e" % (self.case_id, err))
        return ref, err

    def prime(self) -> None:
        """One untimed launch on every input copy, so each copy has been touched
        on the device (address translations warm) before a timed region that
        rotates through them; no timed step is the first use of its copy."""
        from tilegen_amd import runtime as rt
        rt.run_launches(self.fn, self.grid, self.block, self.lds, rt.ArgSets(self.sets),
                        len(self.sets))
        rt.synchronize()

    def time_events(self, warmup: int, iters: int):
        from tilegen_amd import runtime as rt
        kms, ev_wall_ms = rt.time_launches(self.fn, self.grid, self.block, self.lds, self.sets,
                                           warmup, iters)
        return kms, ev_wall_ms

    def free(self) -> None:
        for bufs in self.keep:
            for b in bufs.values():
                b.free()
        self.keep, self.sets = [], []


def _vendor_leg(run: CaseRun, alg: str, ref, warmup: int, steps: int):
    from tilegen_amd import vendor as vd
    A, ops, kernel = run.A, run.ops, run.kernel
    M, N, K, nnz = run.M, run.N, run.K, run.nnz
    for b in run.keep:  # the vendor call writes the same output buffers
        b[run.out_name].upload(np.zeros(run.out_shape))
    if kernel == "spmv":
        vsets = [[b["indptr"], b["indices"], b["data"], b["x"], b["y"]] for b in run.keep]
        vms, _ = vd.spmv_time(alg, M, N, nnz, vsets, warmup, steps)
        vref, call = ref, "rocsparse_spmv compute call"
    elif kernel == "spmm":
        vsets = [[b["indptr"], b["indices"], b["data"], b["B"], b["C"]] for b in run.keep]
        vms, _ = vd.spmm_time(alg, M, N, K, nnz, vsets, warmup, steps)
        vref, call = ref, "rocsparse_spmm compute call"
    else:
        vsets = [[b["indptr"], b["indices"], b["U"], b["V"], b["C"]] for b in run.keep]
        vms, _ = vd.sddmm_time(alg, M, N, K, nnz, vsets, warmup, steps)
        # rocSPARSE's SDDMM does not multiply by A's values
        coo = A.tocoo()
        vref = np.einsum("ik,ik->i", ops["U"][coo.row], ops["V"][coo.col])
        call = "rocsparse_sddmm call (no multiply by A's values)"
    vgot = run.keep[0][run.out_name].to_host().reshape(np.shape(vref))
    verr = float(np.abs(vgot - vref).max() / max(np.abs(vref).max(), 1e-300))
    vmed = float(np.median(vms)) * 1e-3
    _log("rocSPARSE %s: median %.2f us per call (%.0f GB/s, %.0f GFLOP/s), rel err %.2e" % (
        alg, vmed * 1e6, run.nbytes / vmed / 1e9, run.nflop / vmed / 1e9, verr))
    return {"library": "rocSPARSE", "alg": alg, "us_median": round(vmed * 1e6, 3),
            "gbs_median": round(run.nbytes / vmed / 1e9, 2),
            "gflops_median": round(run.nflop / vmed / 1e9, 2),
            "timer": "hipEvents around each " + call, "rel_err": verr}


def _cpu_legs(run: CaseRun, ref, budget_s: float):
    """(cpu_baseline, cpu_openmp, cpu_openmp_tuned) of a case on this host."""
    from tilegen_amd.schedules import CPU_TUNED
    kind, sec, iters = _cpu_baseline(run.kernel, run.A, run.ops, budget_s / 2)
    cpu = {"value": round(run.nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
           "sample": "%d sequential calls of the full %s matrix (%d rows, %d nnz), %.3f ms "
                     "per call" % (iters, run.case_id, run.M, run.nnz, sec * 1e3),
           "gflops": round(run.nflop / sec / 1e9, 3), "ms_per_call": round(sec * 1e3, 4)}
    _log("%s cpu baseline (%s): %.3f ms per call" % (run.case_id, kind, sec * 1e3))
    omp = _openmp_baseline(run.kernel, run.A, run.ops, run.K, ref, run.nbytes, run.nflop,
                           budget_s / 4)
    _log("%s cpu OpenMP backend (%d threads): median %.3f ms" % (run.case_id, omp["cores"],
                                                                omp["ms_median"]))
    omp_tuned = None
    if run.case_id in CPU_TUNED:
        omp_tuned = _openmp_baseline(run.kernel, run.A, run.ops, run.K, ref, run.nbytes,
                                     run.nflop, budget_s / 4, CPU_TUNED[run.case_id])
        omp_tuned["kind"] = "openmp backend, CPU-tuned schedule"
        _log("%s cpu OpenMP backend, tuned %s: median %.3f ms" % (
            run.case_id, omp_tuned["schedule"], omp_tuned["ms_median"]))
    return cpu, omp, omp_tuned


def _case_entry(run: CaseRun, kms, err, cpu, omp, omp_tuned):
    """The compact per-config record of ``cases``."""
    avg = float(kms.mean()) * 1e-3
    gbs = run.nbytes / avg / 1e9
    traffic = _traffic(run.kernel, run.case_id)
    return {
        "kernel": run.kernel, "sched": run.cfg.short(), "nnz": run.nnz,
        "us": round(avg * 1e6, 3), "us_med": round(float(np.median(kms)) * 1e3, 3),
        "gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
        "gflops": round(run.nflop / avg / 1e9, 1),
        "traffic": round(traffic / run.nbytes, 3) if traffic else None,
        "err": float("%.3g" % err),
        "cpu_ms": cpu["ms_per_call"] if cpu else None,
        "omp_ms": omp["ms_median"] if omp else None,
        "omp_tuned_ms": omp_tuned["ms_median"] if omp_tuned else None,
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    # untimed launches before each timed loop; 2000 of c1 are about 25 ms of
    # back-to-back work (after 40, the event-timed average of c1's tuned
    # schedule read 12.9 us against 12.4 us after 4000, its median 12.5 in both)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--case", default=None,
                    help="run this BASELINE config alone (default: c1 as the headline plus "
                         "every other config under 'cases')")
    ap.add_argument("--config", default=None,
                    help="schedule override for the headline case, e.g. T128/TPR8/U2/V1/B256 "
                         "(append /nnz for merge-path windows, /hybrid for long-row "
                         "workgroups, /stream for equal nonzero ranges, /sorted for row "
                         "tiles whose gathers are sorted in LDS)")
    ap.add_argument("--case-iters", type=int, default=200,
                    help="event-timed launches per config under 'cases'")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bound on the headline case's CPU legs")
    ap.add_argument("--case-cpu-seconds", type=float, default=3.0,
                    help="bound on each other config's CPU legs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU legs")
    ap.add_argument("--warm", action="store_true",
                    help="no input rotation (cache-warm figure, reported as such)")
    ap.add_argument("--vendor", default=None, metavar="ALG",
                    help="also time rocSPARSE on the same rotated inputs, reported as an extra "
                         "field: spmv adaptive|rowsplit|lrb|nnzsplit, spmm "
                         "default|csr|row_split|nnz_split|merge_path, sddmm default")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only launch a plain copy of MIB MiB (PMC byte-count calibration)")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print("bench.py runs on exactly one GPU: this build has no multi-GPU path "
              "(--gpus %d requested). Run with --gpus 1." % args.gpus, file=sys.stderr)
        return 2

    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)

    from tilegen_amd import runtime as rt
    from tilegen_amd.schedules import TUNED

    head_id = args.case or HEADLINE
    others = [] if args.case else list(OTHER_CASES)
    if rt.device_count() < 1:
        raise SystemExit("no HIP device visible")
    dev = rt.device_info(0)
    cfg = _parse_config(args.config) if args.config else TUNED[head_id]
    run = CaseRun(head_id, cfg, args.warm)
    _log("device %s (%s, %d CUs); variant attrs %s" % (dev["name"], dev["arch"],
                                                       dev["cu_count"], run.v.attrs()))
    ref, err = run.check()

    arg_sets = rt.ArgSets(run.sets)
    rt.run_launches(run.fn, run.grid, run.block, run.lds, arg_sets, args.warmup)
    rt.synchronize()
    t0 = time.perf_counter()
    rt.run_launches(run.fn, run.grid, run.block, run.lds, arg_sets, args.steps)
    rt.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    value = run.nbytes * args.steps / wall / 1e9

    kms, ev_wall_ms = run.time_events(args.warmup, args.steps)
    k_avg_s = float(kms.mean()) * 1e-3
    k_med_s = float(np.median(kms)) * 1e-3
    achieved = run.nbytes / k_avg_s / 1e9
    _log("%s timed %d steps: %.3f ms/step (host clock), kernel avg %.2f us median %.2f us, "
         "events wall %.3f ms/step" % (head_id, args.steps, ms_per_step, k_avg_s * 1e6,
                                        k_med_s * 1e6, ev_wall_ms / args.steps))

    vendor = _vendor_leg(run, args.vendor, ref, args.warmup, args.steps) if args.vendor else None
    cpu = omp = omp_tuned = None
    if not args.no_cpu:
        cpu, omp, omp_tuned = _cpu_legs(run, ref, args.cpu_seconds)
    run.free()

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic (seeded BASELINE config generator, U(-1,1) values)",
        "config": {
            "workload": "%s: %s" % (head_id, run.case.description),
            "case": head_id, "kernel": run.kernel, "rows": run.M, "cols": run.N,
            "nnz": run.nnz, "K": run.K, "schedule": cfg.short(), "grid": run.grid,
            "block": run.block, "input_copies": run.copies,
            "cache": "warm" if args.warm else "cold (rotated)",
            "compulsory_bytes": run.nbytes,
        },
        "gflops": round(run.nflop * args.steps / wall / 1e9, 3),
        "pct_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
        "kernel_us_avg": round(k_avg_s * 1e6, 3),
        "kernel_us_median": round(k_med_s * 1e6, 3),
        "kernel_gflops_avg": round(run.nflop / k_avg_s / 1e9, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": _traffic(run.kernel, head_id),
        },
        "cpu_baseline": cpu,
        "cpu_openmp": omp,
        "cpu_openmp_tuned": omp_tuned,
        "check_rel_err": err,
    }
    if vendor is not None:
        line["vendor"] = vendor

    if others:
        cases = {}
        for cid in others:
            crun = CaseRun(cid, TUNED[cid], args.warm)
            cref, cerr = crun.check()
            crun.prime()
            ckms, _ = crun.time_events(args.warmup, args.case_iters)
            _log("%s kernel avg %.2f us median %.2f us over %d launches" % (
                cid, float(ckms.mean()) * 1e3, float(np.median(ckms)) * 1e3, args.case_iters))
            ccpu = comp = comp_t = None
            if not args.no_cpu:
                ccpu, comp, comp_t = _cpu_legs(crun, cref, args.case_cpu_seconds)
            crun.free()
            cases[cid] = _case_entry(crun, ckms, cerr, ccpu, comp, comp_t)
        line["cases"] = cases
    line["device"] = dev["arch"].split(":")[0]
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

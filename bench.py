#!/usr/bin/env python3
"""Benchmark of the TileGen HIP CSR hot path on one MI355X; prints ONE JSON line.

A step is one launch of the case's tuned HIP variant over one copy of the
case's inputs, already resident in HBM.  Launches rotate over enough input
copies (>= 640 MB in total, more than the 256 MB Infinity Cache) that every
step reads its matrix from HBM, not from a cache a previous step warmed.

value        whole-job throughput: compulsory bytes of K steps / host wall time
             of the K steps, bracketed by device synchronizations (launch gaps
             included)
roofline     per-kernel duration from start/stop events attached to each
             dispatch (hipExtModuleLaunchKernel), averaged over the timed
             launches; achieved = compulsory bytes per launch / that duration,
             against MI355X's 8 TB/s HBM peak; traffic = HBM bytes per launch
             measured with rocprofv3 FETCH_SIZE/WRITE_SIZE (profiles/), when a
             summary for this kernel and case is committed
cpu_baseline the reference's own sequential cpp/src/ref.cpp (oracle/_ref, kind
             "reference"; else this repository's C restatement, kind "port"),
             one host core, on the full case matrix for a bounded number of calls
cpu_openmp   this build's OpenMP CPU backend (the reference's ``_cpu_emit``
             design) at the reference default schedule T32/TPR1/U1/V1/B128,
             compiled on this host with g++ -O3 -march=native -fopenmp and run
             on every OpenMP thread, host perf_counter around each call
cpu_openmp_tuned
             the same backend at the case's CPU-tuned schedule
             (tilegen_amd.schedules.CPU_TUNED, from tilegen_amd.cpu_tuned);
             null for a case without one

Cases are BASELINE.json's configs (tilegen_amd.matrices.baseline_ids()); the
default c1 is the config the headline metric is quoted on.
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
ROTATE_BYTES = 640 << 20


def _log(msg: str) -> None:
    print("[bench] " + msg, file=sys.stderr, flush=True)


def _parse_config(text: str):
    from tilegen_amd.codegen import Config
    vals = {}
    for part in text.replace(",", "/").split("/"):
        part = part.strip()
        if part in ("nnz", "rows", "hybrid"):  # what a tile holds (see Config.balance)
            vals["balance"] = part
            continue
        for key, name in (("TPR", "threads_per_row"), ("T", "tile_size"), ("U", "unroll"),
                          ("V", "vector_width"), ("B", "block_size")):
            if part.startswith(key) and part[len(key):].isdigit():
                vals[name] = int(part[len(key):])
                break
        else:
            raise SystemExit("bad --config component %r (want T128/TPR8/U2/V1/B256)" % part)
    return Config(**vals)


def _traffic(kernel: str, case_id: str):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, or None."""
    path = os.path.join(ROOT, "profiles", "%s_%s_pmc.json" % (kernel, case_id))
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        d = json.load(fh)
    return d.get("hbm_bytes_per_launch")


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
    M, N = A.shape
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
    so, log = compile_generated(gen, "cpu", workdir)
    data = (ops.get("x"), None, ops.get("B"), ops.get("U"), ops.get("V"), 1.0, 0.0)
    caller, _out, _keep = _make_caller(so, kernel, A, data, K, "cpu")
    t0 = time.perf_counter()
    got = np.asarray(caller(), dtype=np.float64).reshape(np.shape(ref))
    t1 = time.perf_counter() - t0
    err = float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300))
    iters = int(max(5, min(2000, budget_s / max(t1, 1e-6))))
    ms = _time_host(caller.launch, 2, iters)
    med = float(np.median(ms)) * 1e-3
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": _omp_threads(),
            "kind": "openmp backend", "schedule": cfg.short(),
            "sample": "%d calls of the full matrix, median %.3f ms per call" % (iters, med * 1e3),
            "gflops": round(nflop / med / 1e9, 3), "ms_median": round(med * 1e3, 4),
            "ms_min": round(float(np.min(ms)), 4), "rel_err": err,
            "compile": log.split(" with: ")[-1]}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--case", default="c1")
    ap.add_argument("--config", default=None,
                    help="schedule override, e.g. T128/TPR8/U2/V1/B256 (append /nnz for "
                         "merge-path windows, /hybrid for long-row workgroups)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bound on the CPU baseline's timed calls")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
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
    from tilegen_amd.matrices import (baseline_case, baseline_operands, compulsory_bytes,
                                      flops, make_baseline)
    from tilegen_amd.schedules import TUNED
    from tilegen_amd.variant import Variant

    case = baseline_case(args.case)
    cfg = _parse_config(args.config) if args.config else TUNED[args.case]
    t_gen = time.time()
    A = make_baseline(args.case)
    M, N = A.shape
    nnz = int(A.nnz)
    K = case.K
    ops = baseline_operands(case.kernel, M, N, K)
    _log("case %s (%s) M=%d N=%d nnz=%d K=%d generated in %.1fs" % (
        args.case, case.kernel, M, N, nnz, K, time.time() - t_gen))

    if rt.device_count() < 1:
        raise SystemExit("no HIP device visible")
    dev = rt.device_info(0)
    v = Variant(case.kernel, cfg)
    fn = v.function()
    grid, block, lds = v.geometry(M, N, K, nnz)
    attrs = v.attrs()
    _log("device %s (%s, %d CUs); variant %s grid=%d block=%d lds=%d %s" % (
        dev["name"], dev["arch"], dev["cu_count"], cfg.short(), grid, block, lds, attrs))

    nbytes = compulsory_bytes(case.kernel, M, N, nnz, K)
    nflop = flops(case.kernel, nnz, K)
    copies = 1 if args.warm else int(min(64, max(2, -(-ROTATE_BYTES // nbytes))))

    host = {"indptr": A.indptr.astype(np.int64), "indices": A.indices.astype(np.int64),
            "data": A.data.astype(np.float64)}
    host.update({k: np.ascontiguousarray(val, dtype=np.float64) for k, val in ops.items()})
    out_name = {"spmv": "y", "spmm": "C", "sddmm": "C"}[case.kernel]
    out_shape = {"spmv": (M,), "spmm": (M, K), "sddmm": (nnz,)}[case.kernel]
    sets, keep = [], []
    for c in range(copies):
        bufs = {k: rt.DeviceBuffer(a) for k, a in host.items()}
        bufs[out_name] = rt.DeviceBuffer(np.zeros(out_shape))
        keep.append(bufs)
        sets.append(v.abi_values(A, bufs, {}, M, N, K, nnz))
    _log("%d input copies resident (%.0f MB)" % (copies, copies * nbytes / 1e6))

    # one checked launch through the C ABI before timing
    v.device_call(sets[0])
    got = keep[0][out_name].to_host()
    import scipy.sparse  # noqa: F401  (float64 check of this run, not the oracle)
    if case.kernel == "spmv":
        ref = A @ ops["x"]
    elif case.kernel == "spmm":
        ref = A @ ops["B"]
    else:
        coo = A.tocoo()
        ref = np.einsum("ik,ik->i", ops["U"][coo.row], ops["V"][coo.col]) * coo.data
    err = float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300))
    _log("check vs float64 SciPy: normwise rel err %.3e" % err)
    if not err <= 1e-10:
        raise SystemExit("result check failed: rel err %.3e" % err)

    arg_sets = rt.ArgSets(sets)
    rt.run_launches(fn, grid, block, lds, arg_sets, args.warmup)
    rt.synchronize()
    t0 = time.perf_counter()
    rt.run_launches(fn, grid, block, lds, arg_sets, args.steps)
    rt.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    value = nbytes * args.steps / wall / 1e9

    kms, ev_wall_ms = rt.time_launches(fn, grid, block, lds, sets, args.warmup, args.steps)
    k_avg_s = float(kms.mean()) * 1e-3
    k_med_s = float(np.median(kms)) * 1e-3
    achieved = nbytes / k_avg_s / 1e9
    _log("timed %d steps: %.3f ms/step (host clock), kernel avg %.2f us median %.2f us, "
         "events wall %.3f ms/step" % (args.steps, ms_per_step, k_avg_s * 1e6, k_med_s * 1e6,
                                        ev_wall_ms / args.steps))

    vendor = None
    if args.vendor:
        from tilegen_amd import vendor as vd
        out_key = {"spmv": "y", "spmm": "C", "sddmm": "C"}[case.kernel]
        for b in keep:  # the vendor call writes the same output buffers
            b[out_key].upload(np.zeros(out_shape))
        if case.kernel == "spmv":
            vsets = [[b["indptr"], b["indices"], b["data"], b["x"], b["y"]] for b in keep]
            vms, _ = vd.spmv_time(args.vendor, M, N, nnz, vsets, args.warmup, args.steps)
            vref, call = ref, "rocsparse_spmv compute call"
        elif case.kernel == "spmm":
            vsets = [[b["indptr"], b["indices"], b["data"], b["B"], b["C"]] for b in keep]
            vms, _ = vd.spmm_time(args.vendor, M, N, K, nnz, vsets, args.warmup, args.steps)
            vref, call = ref, "rocsparse_spmm compute call"
        else:
            vsets = [[b["indptr"], b["indices"], b["U"], b["V"], b["C"]] for b in keep]
            vms, _ = vd.sddmm_time(args.vendor, M, N, K, nnz, vsets, args.warmup, args.steps)
            # rocSPARSE's SDDMM does not multiply by A's values
            coo = A.tocoo()
            vref = np.einsum("ik,ik->i", ops["U"][coo.row], ops["V"][coo.col])
            call = "rocsparse_sddmm call (no multiply by A's values)"
        vgot = keep[0][out_key].to_host().reshape(np.shape(vref))
        verr = float(np.abs(vgot - vref).max() / max(np.abs(vref).max(), 1e-300))
        vmed = float(np.median(vms)) * 1e-3
        vendor = {"library": "rocSPARSE", "alg": args.vendor, "us_median": round(vmed * 1e6, 3),
                  "gbs_median": round(nbytes / vmed / 1e9, 2),
                  "gflops_median": round(nflop / vmed / 1e9, 2),
                  "timer": "hipEvents around each " + call, "rel_err": verr}
        _log("rocSPARSE %s: median %.2f us per call (%.0f GB/s, %.0f GFLOP/s), rel err %.2e" % (
            args.vendor, vmed * 1e6, nbytes / vmed / 1e9, nflop / vmed / 1e9, verr))

    cpu = None
    if not args.no_cpu:
        kind, sec, iters = _cpu_baseline(case.kernel, A, ops, args.cpu_seconds)
        cpu = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
               "sample": "%d sequential calls of the full %s matrix (%d rows, %d nnz), "
                         "%.3f ms per call" % (iters, args.case, M, nnz, sec * 1e3),
               "gflops": round(nflop / sec / 1e9, 3), "ms_per_call": round(sec * 1e3, 4)}
        _log("cpu baseline (%s): %.3f ms per call" % (kind, sec * 1e3))

    omp = omp_tuned = None
    if not args.no_cpu:
        omp = _openmp_baseline(case.kernel, A, ops, K, ref, nbytes, nflop, args.cpu_seconds / 2)
        _log("cpu OpenMP backend (%d threads): %s" % (omp["cores"], omp["sample"]))
        from tilegen_amd.schedules import CPU_TUNED
        if args.case in CPU_TUNED:
            omp_tuned = _openmp_baseline(case.kernel, A, ops, K, ref, nbytes, nflop,
                                         args.cpu_seconds / 2, CPU_TUNED[args.case])
            omp_tuned["kind"] = "openmp backend, CPU-tuned schedule"
            _log("cpu OpenMP backend, tuned %s: %s" % (omp_tuned["schedule"],
                                                      omp_tuned["sample"]))

    for bufs in keep:
        for b in bufs.values():
            b.free()

    unit = "GB/s"
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": unit,
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
            "workload": "%s: %s" % (args.case, case.description),
            "case": args.case, "kernel": case.kernel, "rows": M, "cols": N, "nnz": nnz,
            "K": K, "schedule": cfg.short(), "grid": grid, "block": block,
            "input_copies": copies, "cache": "warm" if args.warm else "cold (rotated)",
            "compulsory_bytes": nbytes,
        },
        "gflops": round(nflop * args.steps / wall / 1e9, 3),
        "pct_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
        "kernel_us_avg": round(k_avg_s * 1e6, 3),
        "kernel_us_median": round(k_med_s * 1e6, 3),
        "kernel_gbs_median": round(nbytes / k_med_s / 1e9, 2),
        "kernel_gflops_avg": round(nflop / k_avg_s / 1e9, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": _traffic(case.kernel, args.case),
        },
        "cpu_baseline": cpu,
        "cpu_openmp": omp,
        "cpu_openmp_tuned": omp_tuned,
        "vendor": vendor,
        "check_rel_err": err,
        "device": "%s %s" % (dev["name"], dev["arch"]),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Summaries of rocprofv3 runs for ``profiles/`` (kernel time and HBM traffic).

Inputs are the CSV outputs of ``rocprofv3 ... --output-format csv`` runs over
committed commands (see ``commands()``):

* a kernel trace with ``--stats`` of ``bench.py`` for the case;
* two PMC runs of the same bench, one with ``FETCH_SIZE`` and one with
  ``WRITE_SIZE`` (KiB per dispatch);
* the same two counters over ``bench.py --calibrate-copy MIB``, a plain copy
  of known size, which gives the factor that turns each counter into bytes
  on this GPU.

``--bench-json`` is the JSON line of the same ``bench.py`` command run
without the profiler, whose event-timed kernel average the trace is compared
with.

``python -m tilegen_amd.profiling --case c1 --root <dir>`` (the ``-d`` directory the
rocprofv3 commands wrote under) writes
``profiles/<kernel>_<case>.md`` (human summary with the exact commands) and
``profiles/<kernel>_<case>_pmc.json`` (the measured HBM bytes per launch that
``bench.py`` reports as ``roofline.traffic``).
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
from typing import Dict, List, Optional

import numpy as np

__all__ = ["commands", "trace_stats", "pmc_values", "summarize", "valu_command", "valu_summary"]

COPY_MIB = 256
BENCH_PMC = "python3 bench.py --case {case} --no-cpu --steps 20 --warmup 2"
BENCH_TRACE = "python3 bench.py --case {case} --no-cpu"


def commands(case: str, root: str = "rocprof_out") -> Dict[str, str]:
    """The rocprofv3 command lines whose outputs ``summarize`` reads."""
    d = os.path.join(root, case)
    return {
        "trace": "rocprofv3 --kernel-trace --stats --output-format csv -d %s/trace -o trace "
                 "-- %s" % (d, BENCH_TRACE.format(case=case)),
        "fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d %s/fetch -o pmc -- %s"
                 % (d, BENCH_PMC.format(case=case)),
        "write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d %s/write -o pmc -- %s"
                 % (d, BENCH_PMC.format(case=case)),
        "copy_fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d %s/copy_fetch -o pmc "
                      "-- python3 bench.py --calibrate-copy %d" % (root, COPY_MIB),
        "copy_write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d %s/copy_write -o pmc "
                      "-- python3 bench.py --calibrate-copy %d" % (root, COPY_MIB),
    }


VALU_COUNTERS = ("SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_BUSY_CU_CYCLES SQ_WAVE_CYCLES "
                 "SQ_INSTS_VALU_FMA_F64 SQ_INSTS_VALU_FLOPS_FP64 GRBM_GUI_ACTIVE")


def valu_command(case: str, root: str = "rocprof_out") -> str:
    """One PMC pass with the VALU counters (7 counters: 6 SQ, 1 GRBM)."""
    return ("rocprofv3 --pmc %s --output-format csv -d %s/%s/valu -o pmc -- %s"
            % (VALU_COUNTERS, root, case, BENCH_PMC.format(case=case)))


def _find(d: str, suffix: str) -> Optional[str]:
    hits = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    return hits[0] if hits else None


def trace_stats(d: str, kernel: str, warmup: int = 40, steps: int = 400) -> Dict[str, float]:
    """Calls and duration statistics of ``kernel`` from a kernel-trace run of
    ``bench.py``, overall and for the bench's timed region alone (dispatch
    order: one checked launch, ``warmup``, the ``steps`` timed launches, then
    the event-timed pass)."""
    path = _find(d, "kernel_trace.csv")
    if path is None:
        raise FileNotFoundError("no kernel_trace.csv under %s" % d)
    rows = []
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if r["Kernel_Name"].startswith(kernel):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    if not rows:
        raise ValueError("kernel %s not in %s" % (kernel, path))
    rows.sort()
    a = np.array([(e - b) / 1e3 for b, e in rows])
    timed = a[1 + warmup:1 + warmup + steps]
    return {"calls": int(a.size), "avg_us": float(a.mean()), "median_us": float(np.median(a)),
            "min_us": float(a.min()), "max_us": float(a.max()),
            "timed_region_avg_us": float(timed.mean()) if timed.size else None,
            "timed_region_calls": int(timed.size), "source": path}


def pmc_values(d: str, kernel: str, counter: str) -> List[float]:
    path = _find(d, "counter_collection.csv")
    if path is None:
        raise FileNotFoundError("no counter_collection.csv under %s" % d)
    vals = []
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if r["Kernel_Name"].startswith(kernel) and r["Counter_Name"] == counter:
                vals.append(float(r["Counter_Value"]))
    if not vals:
        raise ValueError("%s for %s not in %s" % (counter, kernel, path))
    return vals


def summarize(case: str, root: str, out_dir: str, bench_json: Optional[str] = None
              ) -> Dict[str, object]:
    from .matrices import baseline_case, compulsory_bytes, make_baseline
    bc = baseline_case(case)
    kernel = "%s_kernel" % bc.kernel
    A = make_baseline(case)
    M, N = A.shape
    nbytes = compulsory_bytes(bc.kernel, M, N, int(A.nnz), bc.K)
    cmds = commands(case, root)
    d = os.path.join(root, case)
    tr = trace_stats(os.path.join(d, "trace"), kernel)
    copy_bytes = COPY_MIB << 20
    f_copy = float(np.median(pmc_values(os.path.join(root, "copy_fetch"), "tg_copy_kernel",
                                        "FETCH_SIZE"))) * 1024.0 / copy_bytes
    w_copy = float(np.median(pmc_values(os.path.join(root, "copy_write"), "tg_copy_kernel",
                                        "WRITE_SIZE"))) * 1024.0 / copy_bytes
    fetch_kib = float(np.median(pmc_values(os.path.join(d, "fetch"), kernel, "FETCH_SIZE")))
    write_kib = float(np.median(pmc_values(os.path.join(d, "write"), kernel, "WRITE_SIZE")))
    read_b = fetch_kib * 1024.0 / f_copy
    write_b = write_kib * 1024.0 / w_copy
    bench = None
    if bench_json and os.path.exists(bench_json):
        with open(bench_json) as fh:
            lines = [l for l in fh.read().splitlines() if l.startswith("{")]
        bench = json.loads(lines[-1]) if lines else None
    summary = {
        "case": case, "kernel": kernel, "schedule": bench["config"]["schedule"] if bench else None,
        "compulsory_bytes": nbytes,
        "trace": {k: v for k, v in tr.items() if k != "source"},
        "bench_event_avg_us": bench["kernel_us_avg"] if bench else None,
        "fetch_size_kib": fetch_kib, "write_size_kib": write_kib,
        "fetch_scale": 1.0 / f_copy, "write_scale": 1.0 / w_copy,
        "hbm_read_bytes_per_launch": read_b, "hbm_write_bytes_per_launch": write_b,
        "hbm_bytes_per_launch": int(round(read_b + write_b)),
        "traffic_over_compulsory": (read_b + write_b) / nbytes,
        "commands": cmds,
    }
    os.makedirs(out_dir, exist_ok=True)
    stem = os.path.join(out_dir, "%s_%s" % (bc.kernel, case))
    with open(stem + "_pmc.json", "w") as fh:
        json.dump(summary, fh, indent=1)
    lines = [
        "# %s on %s (%s)" % (kernel, case, bc.description),
        "",
        "Schedule: %s. Compulsory bytes per launch: %d." % (summary["schedule"], nbytes),
        "",
        "## Kernel time (rocprofv3 kernel trace)",
        "",
        "| calls | avg µs | median µs | min µs | max µs | timed region avg µs (%d calls) |"
        % tr["timed_region_calls"],
        "|---:|---:|---:|---:|---:|---:|",
        "| %d | %.3f | %.3f | %.3f | %.3f | %.3f |" % (
            tr["calls"], tr["avg_us"], tr["median_us"], tr["min_us"], tr["max_us"],
            tr["timed_region_avg_us"]),
        "",
        "bench.py, same command without the profiler: kernel avg %s µs from start/stop events "
        "attached to each dispatch, %s µs per step on the host clock." % (
            "%.3f" % bench["kernel_us_avg"] if bench else "—",
            "%.3f" % (bench["ms_per_step"] * 1e3) if bench else "—"),
        "(Under the profiler those dispatch events also absorb the time the profiler inserts "
        "between dispatches; the kernel-trace durations above do not.)",
        "",
        "## HBM traffic (rocprofv3 --pmc, one counter per run)",
        "",
        "| counter | KiB per dispatch (median) | copy-kernel scale | bytes per launch |",
        "|---|---:|---:|---:|",
        "| FETCH_SIZE | %.1f | %.3f | %.0f |" % (fetch_kib, 1.0 / f_copy, read_b),
        "| WRITE_SIZE | %.1f | %.3f | %.0f |" % (write_kib, 1.0 / w_copy, write_b),
        "",
        "Measured traffic %.0f B per launch = %.3f x the compulsory bytes." % (
            read_b + write_b, (read_b + write_b) / nbytes),
        "The scale factors come from a copy of %d MiB (`bench.py --calibrate-copy %d`): "
        "FETCH_SIZE read %.3f and WRITE_SIZE %.3f of the bytes actually moved." % (
            COPY_MIB, COPY_MIB, f_copy, w_copy),
        "",
        "## Commands (from the repository root on the GPU box)",
        "",
    ] + ["    " + c for c in cmds.values()] + [
        "",
        "Summary written by `python -m tilegen_amd.profiling --case %s --root %s`." % (case, root),
    ]
    with open(stem + ".md", "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return summary


def valu_summary(case: str, root: str, out_dir: str, bench_json: Optional[str] = None
                 ) -> Dict[str, object]:
    """profiles/<kernel>_<case>_valu.md: vector-ALU activity of the kernel, the
    evidence for whether a matrix-core (MFMA) formulation could help it."""
    from .matrices import baseline_case, flops, make_baseline
    bc = baseline_case(case)
    kernel = "%s_kernel" % bc.kernel
    d = os.path.join(root, case, "valu")
    med = {c: float(np.median(pmc_values(d, kernel, c))) for c in VALU_COUNTERS.split()}
    A = make_baseline(case)
    alg_flops = flops(bc.kernel, int(A.nnz), bc.K)
    us = None
    if bench_json and os.path.exists(bench_json):
        with open(bench_json) as fh:
            lines = [l for l in fh.read().splitlines() if l.startswith("{")]
        us = json.loads(lines[-1])["kernel_us_avg"] if lines else None
    # MI355X: 256 CUs x 4 SIMDs at up to 2.4 GHz; a wave64 fp64 FMA occupies a
    # SIMD for 4 cycles (78.6 TFLOP/s = 1024 SIMDs x 2.4 GHz x 16 lanes x 2).
    simd_cycles = 1024 * 2.4e9 * us * 1e-6 if us else None
    fma_share = (4.0 * med["SQ_INSTS_VALU_FMA_F64"] / simd_cycles) if simd_cycles else None
    valu_share = (med["SQ_INSTS_VALU"] / simd_cycles) if simd_cycles else None
    summary = {"case": case, "kernel": kernel, "counters": med, "algorithmic_flops": alg_flops,
               "kernel_us_avg": us, "fp64_fma_simd_share": fma_share,
               "valu_issue_share_lower_bound": valu_share,
               "fp64_tflops_achieved": (alg_flops / (us * 1e-6) / 1e12) if us else None,
               "fp64_tflops_peak": 78.6, "command": valu_command(case, root)}
    os.makedirs(out_dir, exist_ok=True)
    stem = os.path.join(out_dir, "%s_%s_valu" % (bc.kernel, case))
    with open(stem + ".json", "w") as fh:
        json.dump(summary, fh, indent=1)
    rows = ["| %s | %.4g |" % (c, med[c]) for c in VALU_COUNTERS.split()]
    text = [
        "# Vector-ALU activity of %s on %s" % (kernel, case), "",
        "| counter (median per dispatch) | value |", "|---|---:|"] + rows + [
        "",
        "Algorithmic fp64 work: %.4g flop per launch%s." % (
            alg_flops, (", %.2f TFLOP/s at the bench's %.2f µs kernel average (fp64 vector "
                        "peak 78.6)" % (summary["fp64_tflops_achieved"], us)) if us else ""),
        "SQ_INSTS_VALU_FMA_F64 counts wave64 fp64 FMA instructions; algorithmic flops / 128 = "
        "%.4g." % (alg_flops / 128.0),
        "Share of SIMD time (1024 SIMDs x 2.4 GHz x kernel time) the fp64 FMAs occupy at 4 "
        "cycles each: %s; all VALU instructions at one cycle each: %s. Only the FMA share is "
        "work a matrix-core formulation could take over." % (
            "%.3f" % fma_share if fma_share is not None else "n/a",
            "%.3f" % valu_share if valu_share is not None else "n/a"),
        "",
        "## Command (from the repository root on the GPU box)", "",
        "    " + valu_command(case, root), "",
        "Summary written by `python -m tilegen_amd.profiling --case %s --root %s --valu`."
        % (case, root),
    ]
    with open(stem + ".md", "w") as fh:
        fh.write("\n".join(text) + "\n")
    return summary


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Summarize rocprofv3 CSV output into profiles/.")
    ap.add_argument("--case", required=True)
    ap.add_argument("--root", default="rocprof_out")
    ap.add_argument("--out", default="profiles")
    ap.add_argument("--bench-json", default=None)
    ap.add_argument("--print-commands", action="store_true")
    ap.add_argument("--valu", action="store_true",
                    help="summarize the VALU counter pass (valu_command) instead")
    a = ap.parse_args(argv)
    if a.valu:
        v = valu_summary(a.case, a.root, a.out, a.bench_json)
        print(json.dumps({k: v[k] for k in ("case", "fp64_fma_simd_share",
                                             "valu_issue_share_lower_bound",
                                             "fp64_tflops_achieved")}))
        return 0
    if a.print_commands:
        for c in commands(a.case, a.root).values():
            print(c)
        return 0
    s = summarize(a.case, a.root, a.out, a.bench_json)
    print(json.dumps({k: s[k] for k in ("case", "hbm_bytes_per_launch",
                                        "traffic_over_compulsory")}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

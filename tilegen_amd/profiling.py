"""Summaries of rocprofv3 runs for ``profiles/`` (kernel time and traffic
beyond L2), one per BASELINE config, from the bench command itself.

``bench.py`` with no ``--case`` runs every BASELINE config in one process (c1
as the headline, then c2, c3a, c3b, c4, c5, c5x25).  The profiled commands
(``commands()``) are that same invocation:

* a kernel trace with ``--stats`` of ``python3 bench.py --steps K --warmup W``,
  the driver's own command line;
* two PMC runs of it without the CPU legs, one with ``FETCH_SIZE`` and one
  with ``WRITE_SIZE`` (KiB per dispatch);
* the same two counters over ``bench.py --calibrate-copy MIB``, a plain copy
  of known size, which gives the factor that turns each counter into bytes.

Every case's kernel is told apart in the CSVs by its symbol and grid size, and
two cases with the same kernel and grid (c5 and c5x25) by their order: the
bench runs the cases in a fixed order and makes a known number of dispatches
per case (one checked launch, ``W`` warmup launches, then the timed ones; the
headline case also has its host-clocked pass of ``K`` steps first).

FETCH_SIZE and WRITE_SIZE count every request that leaves the L2 (Infinity
Cache hits included), so the bytes here are bytes moved beyond L2, an upper
bound on HBM traffic, not HBM traffic itself.

``python -m tilegen_amd.profiling --root <dir> --bench-json <line>`` writes
``profiles/<kernel>_<case>.md`` and ``profiles/<kernel>_<case>_pmc.json`` for
every case (``bench.py`` reports ``beyond_l2_bytes_per_launch`` of the latter as
``roofline.traffic``), plus ``profiles/bench_cases.md``, one table of them all.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

__all__ = ["commands", "case_plan", "trace_rows", "pmc_rows", "summarize", "valu_command",
           "valu_summary"]

COPY_MIB = 256
HEADLINE = "c1"
CASE_ORDER = ("c1", "c2", "c3a", "c3b", "c4", "c5", "c5x25")
STEPS, WARMUP, CASE_ITERS = 100, 2000, 200
PMC_CASE_ITERS = 20
BENCH_TRACE = "python3 bench.py --steps %d --warmup %d" % (STEPS, WARMUP)
BENCH_PMC = "python3 bench.py --no-cpu --steps %d --warmup %d --case-iters %d" % (
    STEPS, WARMUP, PMC_CASE_ITERS)


def commands(root: str = "rocprof_out") -> Dict[str, str]:
    """The rocprofv3 command lines whose outputs ``summarize`` reads."""
    return {
        "trace": "rocprofv3 --kernel-trace --stats --output-format csv -d %s/trace -o trace "
                 "-- %s" % (root, BENCH_TRACE),
        "fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d %s/fetch -o pmc -- %s"
                 % (root, BENCH_PMC),
        "write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d %s/write -o pmc -- %s"
                 % (root, BENCH_PMC),
        "copy_fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d %s/copy_fetch -o pmc "
                      "-- python3 bench.py --calibrate-copy %d" % (root, COPY_MIB),
        "copy_write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d %s/copy_write -o pmc "
                      "-- python3 bench.py --calibrate-copy %d" % (root, COPY_MIB),
    }


VALU_COUNTERS = ("SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_BUSY_CU_CYCLES SQ_WAVE_CYCLES "
                 "SQ_INSTS_VALU_FMA_F64 SQ_INSTS_VALU_FLOPS_FP64 GRBM_GUI_ACTIVE")


def valu_command(root: str = "rocprof_out") -> str:
    """One PMC pass with the VALU counters (7 counters: 6 SQ, 1 GRBM)."""
    return ("rocprofv3 --pmc %s --output-format csv -d %s/valu -o pmc -- %s"
            % (VALU_COUNTERS, root, BENCH_PMC))


ROTATE_BYTES = 640 << 20


def bench_copies(nbytes: int) -> int:
    """Input copies bench.py rotates through (cold caches) for a case whose
    launch moves ``nbytes`` compulsory bytes: about 640 MiB of them, 2 to 64."""
    return int(min(64, max(2, -(-ROTATE_BYTES // max(int(nbytes), 1)))))


def case_plan(steps: int, warmup: int, case_iters: int
              ) -> List[Tuple[str, str, int, int, int]]:
    """(case, kernel symbol, grid work-items, dispatches, event-timed dispatches)
    of every case, in the order bench.py launches them: one checked launch;
    for the headline W warmup and K host-clocked steps, then W warmup and K
    event-timed ones; for the others one launch per input copy, W warmup and
    the event-timed ones."""
    from .codegen import _lowering, _plan
    from .dsl import standard_kernels
    from .matrices import baseline_case, compulsory_bytes, make_baseline
    from .passes import run_pipeline
    from .schedules import TUNED
    from .codegen import launch_geometry
    out = []
    for case in CASE_ORDER:
        bc = baseline_case(case)
        A = make_baseline(case)
        M, N, nnz = A.shape[0], A.shape[1], int(A.nnz)
        k = run_pipeline(standard_kernels()[bc.kernel], TUNED[case], backend="hip")
        geo = launch_geometry(_plan(k), _lowering(k))
        grid = geo.grid(M, nnz) * geo.block
        if case == HEADLINE:
            timed = steps
            n = 1 + warmup + steps + warmup + steps
        else:
            timed = case_iters
            copies = bench_copies(compulsory_bytes(bc.kernel, M, N, nnz, bc.K))
            n = 1 + copies + warmup + case_iters
        out.append((case, "%s_kernel" % bc.kernel, grid, n, timed))
    return out


def _find(d: str, suffix: str) -> Optional[str]:
    hits = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    return hits[0] if hits else None


def _split(rows: Sequence[Tuple[int, str, int, object]], plan) -> Dict[str, List[object]]:
    """Assign dispatches (start, kernel name, grid work-items, payload) to the
    cases of ``plan``: each case takes, in time order, the next ``n`` of its
    kernel and grid."""
    rows = sorted(rows, key=lambda r: r[0])
    used = [False] * len(rows)
    out = {}
    for case, sym, grid, n, _timed in plan:
        got = []
        for i, (_t, name, g, payload) in enumerate(rows):
            if not used[i] and name.startswith(sym) and g == grid:
                used[i] = True
                got.append(payload)
                if len(got) == n:
                    break
        out[case] = got
    return out


def trace_rows(d: str, plan) -> Dict[str, np.ndarray]:
    """Kernel durations (µs) of every case from a kernel-trace run."""
    path = _find(d, "kernel_trace.csv")
    if path is None:
        raise FileNotFoundError("no kernel_trace.csv under %s" % d)
    rows = []
    with open(path) as fh:
        for r in csv.DictReader(fh):
            b, e = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
            rows.append((b, r["Kernel_Name"], int(r["Grid_Size_X"]), (e - b) / 1e3))
    return {c: np.array(v, dtype=np.float64) for c, v in _split(rows, plan).items()}


def pmc_rows(d: str, plan, counter: str) -> Dict[str, np.ndarray]:
    """Per-dispatch values of ``counter`` for every case from a PMC run."""
    path = _find(d, "counter_collection.csv")
    if path is None:
        raise FileNotFoundError("no counter_collection.csv under %s" % d)
    rows = []
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Start_Timestamp"]), r["Kernel_Name"], int(r["Grid_Size"]),
                             float(r["Counter_Value"])))
    return {c: np.array(v, dtype=np.float64) for c, v in _split(rows, plan).items()}


def _copy_scale(d: str, counter: str) -> float:
    path = _find(d, "counter_collection.csv")
    if path is None:
        raise FileNotFoundError("no counter_collection.csv under %s" % d)
    vals = []
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if r["Kernel_Name"].startswith("tg_copy_kernel") and r["Counter_Name"] == counter:
                vals.append(float(r["Counter_Value"]))
    if not vals:
        raise ValueError("%s of tg_copy_kernel not in %s" % (counter, path))
    return float(np.median(vals)) * 1024.0 / (COPY_MIB << 20)


def _bench_line(path: Optional[str]) -> Optional[dict]:
    if not path or not os.path.exists(path):
        return None
    with open(path) as fh:
        lines = [l for l in fh.read().splitlines() if l.startswith("{")]
    return json.loads(lines[-1]) if lines else None


def summarize(root: str, out_dir: str, bench_json: Optional[str] = None) -> Dict[str, dict]:
    from .matrices import baseline_case, compulsory_bytes, make_baseline
    from .schedules import TUNED
    cmds = commands(root)
    plan = case_plan(STEPS, WARMUP, CASE_ITERS)
    pmc_plan = case_plan(STEPS, WARMUP, PMC_CASE_ITERS)
    tr = trace_rows(os.path.join(root, "trace"), plan)
    fetch = pmc_rows(os.path.join(root, "fetch"), pmc_plan, "FETCH_SIZE")
    write = pmc_rows(os.path.join(root, "write"), pmc_plan, "WRITE_SIZE")
    f_copy = _copy_scale(os.path.join(root, "copy_fetch"), "FETCH_SIZE")
    w_copy = _copy_scale(os.path.join(root, "copy_write"), "WRITE_SIZE")
    bench = _bench_line(bench_json)
    os.makedirs(out_dir, exist_ok=True)
    out = {}
    table = []
    for case, sym, grid, n, timed in plan:
        bc = baseline_case(case)
        A = make_baseline(case)
        M, N = A.shape
        nbytes = compulsory_bytes(bc.kernel, M, N, int(A.nnz), bc.K)
        a = tr[case]
        if a.size != n:
            raise ValueError("%s: %d %s dispatches of grid %d in the trace, expected %d"
                             % (case, a.size, sym, grid, n))
        region = a[-timed:]
        fetch_kib = float(np.median(fetch[case])) if fetch[case].size else float("nan")
        write_kib = float(np.median(write[case])) if write[case].size else float("nan")
        read_b = fetch_kib * 1024.0 / f_copy
        write_b = write_kib * 1024.0 / w_copy
        ev = None
        if bench is not None:
            ev = bench["kernel_us_avg"] if case == HEADLINE else bench["cases"][case]["us"]
        s = {"case": case, "kernel": sym, "schedule": TUNED[case].short(), "grid_items": grid,
             "compulsory_bytes": nbytes,
             "trace": {"calls": int(a.size), "avg_us": float(a.mean()),
                       "median_us": float(np.median(a)), "min_us": float(a.min()),
                       "max_us": float(a.max()), "timed_region_avg_us": float(region.mean()),
                       "timed_region_calls": int(region.size)},
             "bench_event_avg_us": ev,
             "fetch_size_kib": fetch_kib, "write_size_kib": write_kib,
             "fetch_scale": 1.0 / f_copy, "write_scale": 1.0 / w_copy,
             "beyond_l2_read_bytes_per_launch": read_b,
             "beyond_l2_write_bytes_per_launch": write_b,
             "beyond_l2_bytes_per_launch": int(round(read_b + write_b)),
             "traffic_over_compulsory": (read_b + write_b) / nbytes,
             "commands": cmds}
        out[case] = s
        stem = os.path.join(out_dir, "%s_%s" % (bc.kernel, case))
        with open(stem + "_pmc.json", "w") as fh:
            json.dump(s, fh, indent=1)
        with open(stem + ".md", "w") as fh:
            fh.write(_case_md(s, bc, root, f_copy, w_copy, timed) + "\n")
        table.append("| %s | %s | %s | %d | %.3f | %.3f | %s | %.0f | %.3f |" % (
            case, sym, s["schedule"], a.size, s["trace"]["avg_us"],
            s["trace"]["timed_region_avg_us"], "%.3f" % ev if ev is not None else "—",
            read_b + write_b, s["traffic_over_compulsory"]))
    lines = [
        "# Every BASELINE config under rocprofv3", "",
        "Kernel time from one kernel trace of the bench command, traffic beyond L2 from one "
        "FETCH_SIZE and one WRITE_SIZE run of it (each scaled by a plain copy of known size). "
        "The timed region is the bench's event-timed launches of the case; the event column is "
        "the average those launches' dispatch events gave in a run of the same command without "
        "the profiler.", "",
        "| case | kernel | schedule | calls | trace avg µs | timed region avg µs | bench events "
        "avg µs | beyond-L2 bytes per launch | / compulsory |",
        "|---|---|---|---:|---:|---:|---:|---:|---:|"] + table + [
        "", "## Commands (from the repository root on the GPU box)", ""] + [
        "    " + c for c in cmds.values()] + [
        "", "Summary written by `python -m tilegen_amd.profiling --root %s --bench-json "
        "<bench line>`." % root]
    with open(os.path.join(out_dir, "bench_cases.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return out


def _case_md(s: dict, bc, root: str, f_copy: float, w_copy: float, timed: int) -> str:
    t = s["trace"]
    ev = s["bench_event_avg_us"]
    nbytes = s["compulsory_bytes"]
    tot = s["beyond_l2_bytes_per_launch"]
    lines = [
        "# %s on %s (%s)" % (s["kernel"], s["case"], bc.description),
        "",
        "Schedule: %s. Compulsory bytes per launch: %d. Told apart in the profiles by grid "
        "size %d work-items and launch order." % (s["schedule"], nbytes, s["grid_items"]),
        "",
        "## Kernel time (rocprofv3 kernel trace of the bench command)",
        "",
        "| calls | avg µs | median µs | min µs | max µs | timed region avg µs (%d calls) |"
        % timed,
        "|---:|---:|---:|---:|---:|---:|",
        "| %d | %.3f | %.3f | %.3f | %.3f | %.3f |" % (
            t["calls"], t["avg_us"], t["median_us"], t["min_us"], t["max_us"],
            t["timed_region_avg_us"]),
        "",
        "bench.py, the same command without the profiler: kernel avg %s µs from start/stop "
        "events attached to each dispatch of the timed region." % (
            "%.3f" % ev if ev is not None else "—"),
        "",
        "## Traffic beyond L2 (rocprofv3 --pmc, one counter per run)",
        "",
        "| counter | KiB per dispatch (median) | copy-kernel scale | bytes per launch |",
        "|---|---:|---:|---:|",
        "| FETCH_SIZE | %.1f | %.3f | %.0f |" % (s["fetch_size_kib"], 1.0 / f_copy,
                                                 s["beyond_l2_read_bytes_per_launch"]),
        "| WRITE_SIZE | %.1f | %.3f | %.0f |" % (s["write_size_kib"], 1.0 / w_copy,
                                                 s["beyond_l2_write_bytes_per_launch"]),
        "",
        "Measured %d B per launch beyond L2 = %.3f x the compulsory bytes. FETCH_SIZE counts "
        "Infinity Cache hits too, so this bounds HBM traffic from above." % (
            tot, s["traffic_over_compulsory"]),
        "The scale factors come from a copy of %d MiB (`bench.py --calibrate-copy %d`): "
        "FETCH_SIZE read %.3f and WRITE_SIZE %.3f of the bytes actually moved." % (
            COPY_MIB, COPY_MIB, f_copy, w_copy),
        "",
        "## Commands (from the repository root on the GPU box)",
        "",
    ] + ["    " + c for c in s["commands"].values()] + [
        "",
        "Summary written by `python -m tilegen_amd.profiling --root %s --bench-json <bench "
        "line>`." % root,
    ]
    return "\n".join(lines)


def valu_summary(root: str, out_dir: str, bench_json: Optional[str] = None,
                 cases: Sequence[str] = ("c1", "c4", "c5")) -> Dict[str, dict]:
    """profiles/<kernel>_<case>_valu.md: vector-ALU activity of each kernel, the
    evidence for whether a matrix-core (MFMA) formulation could help it."""
    from .matrices import baseline_case, flops, make_baseline
    plan = case_plan(STEPS, WARMUP, PMC_CASE_ITERS)
    d = os.path.join(root, "valu")
    per = {c: pmc_rows(d, plan, c) for c in VALU_COUNTERS.split()}
    bench = _bench_line(bench_json)
    out = {}
    for case in cases:
        bc = baseline_case(case)
        kernel = "%s_kernel" % bc.kernel
        med = {c: float(np.median(per[c][case])) for c in VALU_COUNTERS.split()}
        A = make_baseline(case)
        alg_flops = flops(bc.kernel, int(A.nnz), bc.K)
        us = None
        if bench is not None:
            us = bench["kernel_us_avg"] if case == HEADLINE else bench["cases"][case]["us"]
        # MI355X: 256 CUs x 4 SIMDs at up to 2.4 GHz; a wave64 fp64 FMA occupies a
        # SIMD for 4 cycles (78.6 TFLOP/s = 1024 SIMDs x 2.4 GHz x 16 lanes x 2).
        simd_cycles = 1024 * 2.4e9 * us * 1e-6 if us else None
        fma_share = (4.0 * med["SQ_INSTS_VALU_FMA_F64"] / simd_cycles) if simd_cycles else None
        valu_share = (med["SQ_INSTS_VALU"] / simd_cycles) if simd_cycles else None
        summary = {"case": case, "kernel": kernel, "counters": med,
                   "algorithmic_flops": alg_flops, "kernel_us_avg": us,
                   "fp64_fma_simd_share": fma_share,
                   "valu_issue_share_lower_bound": valu_share,
                   "fp64_tflops_achieved": (alg_flops / (us * 1e-6) / 1e12) if us else None,
                   "fp64_tflops_peak": 78.6, "command": valu_command(root)}
        out[case] = summary
        stem = os.path.join(out_dir, "%s_%s_valu" % (bc.kernel, case))
        with open(stem + ".json", "w") as fh:
            json.dump(summary, fh, indent=1)
        rows = ["| %s | %.4g |" % (c, med[c]) for c in VALU_COUNTERS.split()]
        text = [
            "# Vector-ALU activity of %s on %s" % (kernel, case), "",
            "| counter (median per dispatch) | value |", "|---|---:|"] + rows + [
            "",
            "Algorithmic fp64 work: %.4g flop per launch%s." % (
                alg_flops, (", %.2f TFLOP/s at the bench's %.2f µs kernel average (fp64 "
                            "vector peak 78.6)" % (summary["fp64_tflops_achieved"], us))
                if us else ""),
            "SQ_INSTS_VALU_FMA_F64 counts wave64 fp64 FMA instructions; algorithmic flops / "
            "128 = %.4g." % (alg_flops / 128.0),
            "Share of SIMD time (1024 SIMDs x 2.4 GHz x kernel time) the fp64 FMAs occupy at 4 "
            "cycles each: %s; all VALU instructions at one cycle each: %s. Only the FMA share "
            "is work a matrix-core formulation could take over." % (
                "%.3f" % fma_share if fma_share is not None else "n/a",
                "%.3f" % valu_share if valu_share is not None else "n/a"),
            "",
            "## Command (from the repository root on the GPU box)", "",
            "    " + valu_command(root), "",
            "Summary written by `python -m tilegen_amd.profiling --root %s --valu`." % root,
        ]
        with open(stem + ".md", "w") as fh:
            fh.write("\n".join(text) + "\n")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Summarize rocprofv3 CSV output into profiles/.")
    ap.add_argument("--root", default="rocprof_out")
    ap.add_argument("--out", default="profiles")
    ap.add_argument("--bench-json", default=None)
    ap.add_argument("--print-commands", action="store_true")
    ap.add_argument("--valu", action="store_true",
                    help="summarize the VALU counter pass (valu_command) instead")
    a = ap.parse_args(argv)
    if a.print_commands:
        for c in list(commands(a.root).values()) + [valu_command(a.root)]:
            print(c)
        return 0
    if a.valu:
        v = valu_summary(a.root, a.out, a.bench_json)
        print(json.dumps({c: {k: s[k] for k in ("fp64_fma_simd_share",
                                                "valu_issue_share_lower_bound",
                                                "fp64_tflops_achieved")}
                          for c, s in v.items()}))
        return 0
    s = summarize(a.root, a.out, a.bench_json)
    print(json.dumps({c: {"avg_us": v["trace"]["avg_us"],
                          "traffic_over_compulsory": round(v["traffic_over_compulsory"], 3)}
                      for c, v in s.items()}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

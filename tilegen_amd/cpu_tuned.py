"""CPU-tuned OpenMP schedules for the BASELINE cases.

The CPU baseline beside every bench line has two OpenMP legs: the reference's
default schedule T32/TPR1/U1/V1/B128 and a CPU-tuned winner.  This driver
finds the winners the way the reference tunes its CPU backend
(``autotune.tune`` with ``backend="cpu"``: random search, budget 40, seed 0,
every candidate compiled with ``g++ -O3 -march=native -fopenmp``, verified
against float64 SciPy and timed with ``perf_counter`` around the ctypes
call), on the host it runs on, which for the committed table is the GPU
box's.  ``python -m tilegen_amd.cpu_tuned --out results`` writes
``cpu_tuned.json`` and ``cpu_tuned.md``; ``schedules.CPU_TUNED`` holds the
winners and ``bench.py`` times them.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
from typing import List, Sequence

from .autotune import tune
from .codegen import Config
from .env import physical_cores
from .matrices import baseline_case, baseline_ids, make_baseline

__all__ = ["run", "render", "main"]


def run(cases: Sequence[str], budget: int = 40, seed: int = 0, log=print) -> List[dict]:
    out = []
    for case_id in cases:
        case = baseline_case(case_id)
        A = make_baseline(case_id)
        res = tune(case.kernel, A, budget=budget, mode="random", backend="cpu",
                   K=max(1, case.K), seed=seed, warmup=2, iters=10)
        w, m = res["winner"], res["winner_metrics"]
        base = next(r for r in res["records"] if r.get("ms_median") is not None)
        row = {"case": case_id, "kernel": case.kernel, "winner": w,
               "ms_median": m["ms_median"] if m else None,
               "default_ms_median": base["ms_median"],
               "candidates": sum(1 for r in res["records"] if r.get("ms_median") is not None)}
        out.append(row)
        log("[cpu_tuned] %s %s: %s %.4f ms (default %.4f ms, %d timed)" % (
            case_id, case.kernel, Config(**w).short() if w else "none",
            row["ms_median"] or 0.0, row["default_ms_median"], row["candidates"]))
    return out


def render(rows: List[dict], host: str) -> str:
    md = ["# CPU-tuned OpenMP schedules (%s)" % host, "",
          "Written by `python -m tilegen_amd.cpu_tuned`: random search, budget 40, seed 0, "
          "each candidate verified against float64 SciPy; median ms of 10 calls.", "",
          "| case | kernel | winner | ms | default T32/TPR1/U1/V1/B128 ms |",
          "|---|---|---|---:|---:|"]
    for r in rows:
        md.append("| %s | %s | %s | %.4f | %.4f |" % (
            r["case"], r["kernel"], Config(**r["winner"]).short() if r["winner"] else "none",
            r["ms_median"] or 0.0, r["default_ms_median"]))
    return "\n".join(md) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="CPU-tuned OpenMP schedules per BASELINE case.")
    ap.add_argument("--out", default="results")
    ap.add_argument("--cases", default=",".join(baseline_ids()))
    ap.add_argument("--budget", type=int, default=40)
    a = ap.parse_args(argv)
    rows = run(a.cases.split(","), a.budget, log=lambda m: print(m, flush=True))
    host = "%d logical cores, OMP_NUM_THREADS=%s" % (os.cpu_count() or 0,
                                                     os.environ.get("OMP_NUM_THREADS", "unset"))
    os.makedirs(a.out, exist_ok=True)
    with open(os.path.join(a.out, "cpu_tuned.json"), "w") as fh:
        json.dump({"host": host, "physical_cores": physical_cores(), "rows": rows}, fh,
                  indent=1)
    with open(os.path.join(a.out, "cpu_tuned.md"), "w") as fh:
        fh.write(render(rows, host))
    print(render(rows, host))
    return 0


if __name__ == "__main__":
    sys.exit(main())

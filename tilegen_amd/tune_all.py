"""Autotune every kernel over the matrix corpus and write the result files.

Restates the reference's ``scripts/autotune.py:1-90`` on this backend: for
each corpus class and each standard kernel, ``autotune.tune`` (random mode,
budget 40 by default, the CDNA4 search space) times the candidates with HIP
dispatch events on rotated device-resident inputs and verifies each against
float64 SciPy before it may win; ``write_outputs`` writes the compact summary
(``autotune.json``, ``autotune.csv``, ``best_configs.json``) into ``--out``
and the full sweep into ``--full-out``, in the reference's layout.

``python -m tilegen_amd.tune_all --out results``
"""

from __future__ import annotations

import argparse
import os
import sys
from typing import List, Optional, Sequence

from .autotune import prune_log, tune, write_outputs
from .codegen import Config
from .env import probe
from .matrices import build_corpus, corpus_classes

__all__ = ["ALL_KERNELS", "run", "main"]

ALL_KERNELS = ["spmv", "spmm", "sddmm", "fused_spmv_axpy", "axpy"]


def run(matrix_dir: str, backend: str, kernels: Sequence[str] = ALL_KERNELS,
        classes: Optional[Sequence[str]] = None, budget: int = 40, mode: str = "random",
        iters: int = 25, warmup: int = 5, workdir: str = "build/generated", log=print,
        verbose: bool = False) -> List[dict]:
    classes = list(classes or corpus_classes())
    if any(not os.path.exists(os.path.join(matrix_dir, c + ".npz")) for c in classes):
        log("[tune_all] generating corpus into %s" % matrix_dir)
        build_corpus(matrix_dir)
    out = []
    for cls in classes:
        path = os.path.join(matrix_dir, cls + ".npz")
        for kernel in kernels:
            res = tune(kernel, path, budget=budget, mode=mode, backend=backend, iters=iters,
                       warmup=warmup, workdir=workdir, verbose=verbose)
            out.append(res)
            w, m = res["winner"], res["winner_metrics"]
            if w:
                log("%-16s %-16s winner %s  median %.4f ms  %.2fx vs "
                    "T32/TPR1/U1/V1/B128" % (cls, kernel, Config(**w).short(),
                                             m["ms_median"], m["speedup_vs_naive"] or 0.0))
            else:
                log("%-16s %-16s no legal, verified variant" % (cls, kernel))
    return out


def render_markdown(results: List[dict], backend: str) -> str:
    """Winner per (class, kernel): schedule, median ms, GFLOP/s, compulsory
    GB/s, speedup over the reference default schedule."""
    lines = ["# Autotune winners (%s backend)" % backend, "",
             "The CDNA4 space, searched as each row's `search` column says (random: a seeded "
             "sample of the legal schedules; exhaustive: every legal schedule); every candidate "
             "verified against float64 SciPy before it may win; timed with HIP dispatch events "
             "on rotated inputs. Written by `python -m tilegen_amd.tune_all`.", "",
             "| class | kernel | search | winner | median ms | GFLOP/s | GB/s (compulsory) "
             "| vs T32/TPR1/U1/V1/B128 | measured |", "|---|---|---|---|---:|---:|---:|---:|---:|"]
    for r in results:
        w, m = r["winner"], r["winner_metrics"]
        mode = r.get("mode") or "random"
        if not w:
            lines.append("| %s | %s | %s | none | | | | | |" % (r["matrix_class"], r["kernel"],
                                                              mode))
            continue
        n = sum(1 for x in r["records"] if x.get("ms_min") is not None)
        lines.append("| %s | %s | %s | %s | %.4f | %.1f | %.0f | %.2fx | %d |" % (
            r["matrix_class"], r["kernel"], mode, Config(**w).short(), m["ms_median"],
            m["gflops"], m["compulsory_gbs"], m["speedup_vs_naive"] or 0.0, n))
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Autotune every kernel over the corpus.")
    ap.add_argument("--budget", type=int, default=40)
    ap.add_argument("--mode", default="random", choices=["random", "coordinate", "exhaustive"])
    ap.add_argument("--out", default="results")
    ap.add_argument("--full-out", default="build")
    ap.add_argument("--matrix-dir", default="build/matrices")
    ap.add_argument("--backend", default=None, help="hip|cpu (default: probe)")
    ap.add_argument("--kernels", default=",".join(ALL_KERNELS))
    ap.add_argument("--classes", default=None)
    ap.add_argument("--iters", type=int, default=25)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--verbose", action="store_true",
                    help="print one line per candidate as it is timed")
    a = ap.parse_args(argv)
    env = probe()
    backend = a.backend or env["backend"]
    results = run(a.matrix_dir, backend, a.kernels.split(","),
                  a.classes.split(",") if a.classes else None, a.budget, a.mode, a.iters,
                  a.warmup, log=lambda m: print(m, flush=True), verbose=a.verbose)
    write_outputs(results, a.out, env, prune_log(), full_outdir=a.full_out)
    with open(os.path.join(a.out, "autotune_summary.md"), "w") as fh:
        fh.write(render_markdown(results, backend))
    print("wrote %s/autotune.json, autotune.csv, best_configs.json, autotune_summary.md" % a.out)
    return 0


if __name__ == "__main__":
    sys.exit(main())

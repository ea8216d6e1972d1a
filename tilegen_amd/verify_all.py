"""Differential test of every (kernel, schedule, corpus class) triple.

Restates the method of the reference's ``scripts/verify_all.py:1-120`` on this
backend: the five standard kernels x three schedules (the reference's own
list, ``verify_all.py:27-31``) x the six corpus classes, plus one variant with
``inject_bug=True`` per class, each through ``verify()`` against float64
SciPy.  On the HIP backend the SpMV-shaped kernels (spmv, fused_spmv_axpy)
also run in the three load-balanced forms this build adds (``Config.balance``
"nnz" for merge-path windows, "hybrid" for row tiles plus long-row workgroups
and "stream" for equal nonzero ranges) and as row tiles with sorted gathers
(``Config.gather="sorted"``), counted apart from the reference's triples.  The result file has
the reference's ``results/correctness.json``
layout (``summary`` + per-triple ``results``), with the normwise errors and
the indptr/indices byte check of this build added to each record.

``python -m tilegen_amd.verify_all --out results`` (backend from
``env.probe()``: ``hip`` on an MI355X, else the OpenMP ``cpu`` backend).
Exit status 0 when every normal triple passes and every injected bug is
caught.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
from typing import Any, Dict, Optional, Sequence

from .codegen import Config
from .env import probe
from .matrices import build_corpus, corpus_classes
from .schedules import TUNED
from .verify import verify

__all__ = ["KERNELS", "CONFIGS", "BALANCE_CONFIGS", "SORTED_CONFIGS", "BUG_CONFIG", "run",
           "main"]

KERNELS = ["spmv", "spmm", "sddmm", "fused_spmv_axpy", "axpy"]
CONFIGS = [
    Config(tile_size=32, threads_per_row=1, unroll=1, vector_width=1, block_size=128),
    Config(tile_size=64, threads_per_row=1, unroll=4, vector_width=1, block_size=256),
    Config(tile_size=128, threads_per_row=8, unroll=2, vector_width=2, block_size=512),
]
BUG_CONFIG = Config(tile_size=32, threads_per_row=1, unroll=1, inject_bug=True)
# HIP only: merge-path windows, hybrid tiles and stream ranges of the SpMV-shaped
# kernels
BALANCE_KERNELS = ("spmv", "fused_spmv_axpy")
BALANCE_CONFIGS = [
    Config(tile_size=64, threads_per_row=4, unroll=4, vector_width=1, block_size=256,
           balance=b) for b in ("nnz", "hybrid", "stream")
] + [
    Config(tile_size=16, threads_per_row=8, unroll=2, vector_width=1, block_size=128,
           balance=b) for b in ("nnz", "hybrid", "stream")
]
# HIP only: row tiles whose first-step gathers are sorted by column in LDS (a small
# tile and the tuned c1 schedule)
SORTED_CONFIGS = [
    Config(tile_size=64, threads_per_row=4, unroll=4, vector_width=1, block_size=256,
           gather="sorted"),
    TUNED["c1"],
]


def run(matrix_dir: str, backend: str, classes: Optional[Sequence[str]] = None,
        kernels: Sequence[str] = KERNELS, configs: Sequence[Config] = CONFIGS,
        workdir: str = "build/generated", log=print,
        balance_configs: Optional[Sequence[Config]] = None) -> Dict[str, Any]:
    """Every normal triple, the forms this build adds (HIP backend;
    ``balance_configs`` defaults to BALANCE_CONFIGS + SORTED_CONFIGS there and to
    none on the CPU backend, whose emitter has row tiles with direct gathers only),
    and one injected bug per class."""
    if balance_configs is None:
        balance_configs = BALANCE_CONFIGS + SORTED_CONFIGS if backend == "hip" else []
    classes = list(classes or corpus_classes())
    missing = [c for c in classes if not os.path.exists(os.path.join(matrix_dir, c + ".npz"))]
    if missing:
        log("[verify_all] generating corpus into %s" % matrix_dir)
        build_corpus(matrix_dir)
    results = []
    for cls in classes:
        path = os.path.join(matrix_dir, cls + ".npz")
        for kernel in kernels:
            for cfg in configs:
                results.append(verify(kernel, cfg, path, backend=backend, workdir=workdir))
            if kernel in BALANCE_KERNELS:
                for cfg in balance_configs:
                    results.append(verify(kernel, cfg, path, backend=backend,
                                          workdir=workdir))
        results.append(verify("spmv", BUG_CONFIG, path, backend=backend, workdir=workdir))
    normal = [r for r in results if not r.inject_bug]
    balanced = [r for r in normal if (r.config or {}).get("balance", "rows") != "rows"]
    sorted_ = [r for r in normal if (r.config or {}).get("gather", "direct") != "direct"]
    buggy = [r for r in results if r.inject_bug]
    executed = all(getattr(r, "executed", True) for r in results)
    summary = {
        "backend": backend,
        "executed": executed,
        "total_triples": len(results),
        "normal_triples": len(normal),
        "normal_passed": sum(1 for r in normal if r.ok),
        "balance_triples": len(balanced),
        "balance_passed": sum(1 for r in balanced if r.ok),
        "sorted_triples": len(sorted_),
        "sorted_passed": sum(1 for r in sorted_ if r.ok),
        "bug_triples": len(buggy),
        "bug_caught": sum(1 for r in buggy if not r.ok),
        "max_abs_err": max((r.max_abs_err for r in normal), default=0.0),
        "max_rel_err": max((r.max_rel_err for r in normal), default=0.0),
        "max_rel_err_inf": max((r.rel_err_inf for r in normal), default=0.0),
        "max_rel_err_2": max((r.rel_err_2 for r in normal), default=0.0),
        "structure_intact": all(r.structure_intact is not False for r in results),
        "all_normal_passed": all(r.ok for r in normal),
        "all_bugs_caught": all(not r.ok for r in buggy),
    }
    return {"summary": summary, "results": [r.to_dict() for r in results]}


def render_table(payload: Dict[str, Any]) -> str:
    rows = payload["results"]
    s = payload["summary"]
    lines = ["| class | kernel | schedule | ok | rows | nnz | max abs err | normwise rel err (inf) |"
             " injected bug |", "|---|---|---|---|---:|---:|---:|---:|---|"]
    for r in rows:
        c = r.get("config") or {}
        sched = "T%s/TPR%s/U%s/V%s/B%s" % (c.get("tile_size"), c.get("threads_per_row"),
                                          c.get("unroll"), c.get("vector_width"),
                                          c.get("block_size"))
        if c.get("balance", "rows") != "rows":
            sched += "/" + c["balance"]
        if c.get("gather", "direct") != "direct":
            sched += "/" + c["gather"]
        lines.append("| %s | %s | %s | %s | %d | %d | %.3e | %.3e | %s |" % (
            r["matrix_class"], r["kernel"], sched, "PASS" if r["ok"] else "FAIL", r["rows"],
            r["nnz"], r["max_abs_err"], r.get("rel_err_inf", 0.0),
            "yes" if r["inject_bug"] else ""))
    head = [
        "# Differential test, %s backend" % s["backend"], "",
        "normal triples passed: %d / %d (of which load-balanced forms: %d / %d, sorted-gather "
        "tiles: %d / %d); injected bugs caught: %d / %d; max abs err %.3e; "
        "max normwise relative error %.3e (inf-norm), %.3e (2-norm); indptr/indices intact: %s."
        % (s["normal_passed"], s["normal_triples"], s.get("balance_passed", 0),
           s.get("balance_triples", 0), s.get("sorted_passed", 0), s.get("sorted_triples", 0),
           s["bug_caught"], s["bug_triples"],
           s["max_abs_err"], s["max_rel_err_inf"], s["max_rel_err_2"], s["structure_intact"]),
        "", "Written by `python -m tilegen_amd.verify_all`.", ""]
    return "\n".join(head + lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Verify every kernel x schedule x corpus class.")
    ap.add_argument("--out", default="results")
    ap.add_argument("--matrix-dir", default="build/matrices")
    ap.add_argument("--backend", default=None, help="hip|cpu (default: probe)")
    ap.add_argument("--classes", default=None)
    a = ap.parse_args(argv)
    env = probe()
    backend = a.backend or env["backend"]
    classes = a.classes.split(",") if a.classes else None
    payload = run(a.matrix_dir, backend, classes, log=lambda m: print(m, flush=True))
    payload["summary"]["hardware"] = env
    os.makedirs(a.out, exist_ok=True)
    with open(os.path.join(a.out, "correctness.json"), "w") as fh:
        json.dump(payload, fh, indent=1, default=str)
    with open(os.path.join(a.out, "correctness_summary.md"), "w") as fh:
        fh.write(render_table(payload))
    s = payload["summary"]
    print("normal triples passed : %d / %d" % (s["normal_passed"], s["normal_triples"]))
    print("injected bugs caught  : %d / %d" % (s["bug_caught"], s["bug_triples"]))
    print("max abs err (normal)  : %.3e" % s["max_abs_err"])
    print("max normwise rel err  : %.3e" % s["max_rel_err_inf"])
    ok = s["all_normal_passed"] and s["all_bugs_caught"] and s["executed"]
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())

"""Pass ablation: what each pass contributes to a tuned kernel, per case.

Follows the method of the reference's ``scripts/ablate_passes.py:1-23``:

1. emit the kernel with the full pipeline and with exactly one pass skipped
   (``generate(..., skip_passes=[name])``);
2. diff the emitted code with comment lines removed (the header holds the
   pass log, which always differs);
3. an identical body is ``no change``: 1.00x by definition, never timed;
4. a changed body is verified against float64 SciPy (the reference
   tolerance of ``verify``, plus the 1e-10 normwise bar), then full and
   ablated variants are timed interleaved ``repeats`` times; the cell is the
   median of ``ablated_ms / full_ms`` with its min and max.

For the HIP backend the compared code is the device kernel plus its C
launcher (the launch geometry lives in the launcher), and the timer is the
dispatch-attached HIP events of ``tg_time_launches`` over rotated input
copies (cold HBM, as in ``bench.py``).  The static effect on the other
backend's code is reported beside it, as the reference reports the CUDA code
effect when it times on the CPU (``ablate_passes.py:478-496``).

``fused_spmv_axpy`` without ``loop_fusion`` writes the temporary ``t`` and
has a different ABI, so that cell is ``invalid`` rather than timed
(``ablate_passes.py:356-373``).

``python -m tilegen_amd.ablation --out results`` writes
``pass_ablation.json`` and ``pass_ablation.md``.
"""

from __future__ import annotations

import argparse
import difflib
import hashlib
import json
import os
import statistics
import time
from typing import Any, Callable, Dict, List, Optional, Sequence

import numpy as np

from . import passes as _passes
from .codegen import Config, generate
from .dsl import standard_kernels

__all__ = ["code_body", "code_diff", "ablate", "write_outputs", "DEFAULT_CASES"]

#: BASELINE cases each kernel is ablated on by default.
DEFAULT_CASES = {
    "spmv": ["c1", "c2", "c3a", "c3b"],
    "fused_spmv_axpy": ["c1", "c2", "c3a", "c3b"],
    "spmm": ["c4"],
    "sddmm": ["c5"],
}


def code_body(gen) -> str:
    """Emitted code only: device source plus launcher, ``//`` lines dropped."""
    text = gen.source + "\n" + (gen.host_source or "")
    return "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))


def code_diff(full, ablated) -> Dict[str, Any]:
    a, b = code_body(full), code_body(ablated)
    diff = list(difflib.unified_diff(a.splitlines(), b.splitlines(), lineterm=""))
    added = sum(1 for l in diff if l.startswith("+") and not l.startswith("+++"))
    removed = sum(1 for l in diff if l.startswith("-") and not l.startswith("---"))
    return {"identical": a == b,
            "full_sha": hashlib.sha1(a.encode()).hexdigest()[:12],
            "ablated_sha": hashlib.sha1(b.encode()).hexdigest()[:12],
            "added_lines": added, "removed_lines": removed}


def _stats(ms: Sequence[float]) -> Dict[str, Any]:
    s = sorted(float(v) for v in ms)
    n = len(s)
    if n == 0:
        return {"ms_median": None, "ms_min": None, "ms_max": None, "runs": 0}
    return {"ms_median": statistics.median(s), "ms_mean": statistics.mean(s),
            "ms_min": s[0], "ms_max": s[-1],
            "ms_std": statistics.stdev(s) if n > 1 else 0.0,
            "ms_p10": s[int(0.10 * (n - 1))], "ms_p90": s[int(0.90 * (n - 1))], "runs": n}


class _Prepared:
    """One compiled variant with a checked first launch and a timer."""

    def __init__(self, kernel_name, gen, A, data, K, ref, tol, backend, workdir, bench):
        from .autotune import _make_caller, _time_host
        from .verify import compile_generated, normwise_errors
        lib_path, self.log = compile_generated(gen, backend, workdir)
        if lib_path is None:
            raise RuntimeError("compilation skipped: %s" % self.log)
        self.caller, _out, self.keep = _make_caller(lib_path, kernel_name, A, data, K,
                                                    backend, bench)
        out = np.asarray(self.caller(), dtype=np.float64).ravel()
        self.max_abs_err = float(np.abs(out - ref).max()) if ref.size else 0.0
        self.rel_inf, self.rel_2 = normwise_errors(out, ref)
        self.verified = bool(self.max_abs_err <= tol and self.rel_inf <= 1e-10
                             and self.rel_2 <= 1e-10)
        if backend == "hip":
            self.time: Callable[[int, int], np.ndarray] = self.caller.time
        else:
            self.time = lambda warmup, iters: _time_host(self.caller.launch, warmup, iters)


def _tolerance(A, ref: np.ndarray) -> float:
    eps = float(np.finfo(np.float64).eps)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    row_nnz = int(np.diff(A.indptr).max()) if A.shape[0] else 1
    return float(8.0 * eps * max(1, row_nnz) * scale + 1e-12)


def ablate(kernels: Sequence[str] = ("spmv", "fused_spmv_axpy"),
           cases: Optional[Dict[str, List[str]]] = None, backend: str = "hip",
           repeats: int = 5, warmup: int = 10, iters: int = 100,
           configs: Optional[Dict[str, Config]] = None, matrices: Optional[Dict[str, Any]] = None,
           K: Optional[int] = None, rotate_bytes: int = 640 << 20, seed: int = 7,
           workdir: str = "build/ablation", log: Callable[[str], None] = print
           ) -> Dict[str, Any]:
    """Ablate every pass for each kernel on each case; returns the payload that
    ``write_outputs`` renders.  ``matrices`` maps case name to a CSR matrix and
    overrides the BASELINE generator (tests use small ones); ``configs`` maps
    case name to its schedule (default: the tuned schedule of that case)."""
    from .autotune import _HipBench
    from .matrices import baseline_case, make_baseline
    from .schedules import TUNED
    from .verify import _inputs_for, _reference

    if backend not in ("hip", "cpu"):
        raise ValueError("backend must be 'hip' or 'cpu'")
    if repeats < 2:
        raise ValueError("repeats must be >= 2 to report a spread")
    if iters < 10:
        raise ValueError("iters must be >= 10")
    other = "cpu" if backend == "hip" else "hip"
    ks = standard_kernels()
    os.makedirs(workdir, exist_ok=True)
    rows: List[Dict[str, Any]] = []
    for kernel_name in kernels:
        for case in (cases or DEFAULT_CASES)[kernel_name]:
            A = matrices[case] if matrices and case in matrices else make_baseline(case)
            k_dim = K if K is not None else (baseline_case(case).K if not matrices else 8)
            cfg = (configs or {}).get(case) or TUNED[case]
            data = _inputs_for(kernel_name, A, k_dim, seed)
            ref = np.asarray(_reference(kernel_name, A, data), dtype=np.float64).ravel()
            tol = _tolerance(A, ref)
            kobj = ks[kernel_name]
            full_gen = generate(kobj, cfg, backend, outdir=workdir, write=False)
            full_other = generate(kobj, cfg, other, outdir=workdir, write=False)
            bench = _HipBench(kernel_name, A, data, k_dim, rotate_bytes) if backend == "hip" else None
            log("[%s] %s schedule %s backend %s" % (case, kernel_name, cfg.short(), backend))
            try:
                full = _Prepared(kernel_name, full_gen, A, data, k_dim, ref, tol, backend,
                                 workdir, bench)
                if not full.verified:
                    raise RuntimeError("%s/%s full pipeline failed verification: max_abs=%g "
                                       "tol=%g rel_inf=%g" % (kernel_name, case, full.max_abs_err,
                                                              tol, full.rel_inf))
                for pname in _passes.PASS_NAMES:
                    abl_gen = generate(kobj, cfg, backend, outdir=workdir, write=False,
                                       skip_passes=[pname])
                    abl_other = generate(kobj, cfg, other, outdir=workdir, write=False,
                                         skip_passes=[pname])
                    row: Dict[str, Any] = {
                        "kernel": kernel_name, "case": case, "pass": pname,
                        "config": cfg.to_dict(), "code_diff": code_diff(full_gen, abl_gen),
                        "other_backend": other,
                        "other_code_diff": code_diff(full_other, abl_other),
                        "full": None, "ablated": None, "contribution": None}
                    rows.append(row)
                    if row["code_diff"]["identical"]:
                        row.update(status="no_change", verified=True,
                                   contribution={"median": 1.0, "min": 1.0, "max": 1.0,
                                                 "std": 0.0})
                        log("    without %-16s no change (identical code)" % pname)
                        continue
                    if abl_gen.abi_args != full_gen.abi_args:
                        row.update(status="invalid", verified=False,
                                   reason="ABI changes without %s: %s" % (
                                       pname, abl_gen.abi_signature))
                        log("    without %-16s INVALID (ABI changes)" % pname)
                        continue
                    abl = _Prepared(kernel_name, abl_gen, A, data, k_dim, ref, tol, backend,
                                    workdir, bench)
                    if not abl.verified:
                        row.update(status="invalid", verified=False,
                                   reason="ablated kernel failed verification (max_abs=%g, "
                                          "rel_inf=%g)" % (abl.max_abs_err, abl.rel_inf))
                        log("    without %-16s INVALID (reference mismatch)" % pname)
                        continue
                    f_runs, a_runs, ratios = [], [], []
                    for _ in range(repeats):
                        f = _stats(full.time(warmup, iters))
                        a = _stats(abl.time(warmup, iters))
                        f_runs.append(f)
                        a_runs.append(a)
                        ratios.append(a["ms_median"] / f["ms_median"] if f["ms_median"] else 1.0)
                    row.update(status="ok", verified=True, full=f_runs, ablated=a_runs,
                               contribution={"median": statistics.median(ratios),
                                             "mean": statistics.mean(ratios),
                                             "min": min(ratios), "max": max(ratios),
                                             "std": statistics.stdev(ratios)})
                    log("    without %-16s %5.2fx (%.2f-%.2f)  code +%d/-%d  full %.4f ms" % (
                        pname, row["contribution"]["median"], min(ratios), max(ratios),
                        row["code_diff"]["added_lines"], row["code_diff"]["removed_lines"],
                        statistics.median(r["ms_median"] for r in f_runs)))
            finally:
                if bench is not None:
                    bench.free()
    timer = ("HIP events attached to each dispatch (tg_time_launches), rotated input copies"
             if backend == "hip" else "time.perf_counter around the OpenMP launcher")
    return {"backend": backend, "timer": timer, "warmup": warmup, "iterations": iters,
            "repeats": repeats, "passes": list(_passes.PASS_NAMES),
            "method": ("Diff emitted code first (comment lines dropped); identical bodies are "
                       "'no change' and are not timed. Changed cases are verified against "
                       "float64 SciPy and timed with interleaved full/ablated runs; "
                       "contribution = ablated_ms / full_ms."),
            "rows": rows}


def _cell(row: Optional[Dict[str, Any]]) -> str:
    if row is None:
        return "-"
    if row["status"] == "no_change":
        return "no change"
    if row["status"] != "ok":
        return "**invalid**"
    c = row["contribution"]
    return "%.2fx (%.2f-%.2f)" % (c["median"], c["min"], c["max"])


def _find(rows, kernel, pname, case):
    return next((r for r in rows if r["kernel"] == kernel and r["pass"] == pname
                 and r["case"] == case), None)


def render_markdown(payload: Dict[str, Any]) -> str:
    rows = payload["rows"]
    kernels = list(dict.fromkeys(r["kernel"] for r in rows))
    md = ["# Pass ablation (%s backend)" % payload["backend"].upper(), "",
          "Each kernel is emitted with the full pipeline and with exactly one pass skipped. "
          "The code bodies (device kernel and launcher, comment lines dropped) are diffed; "
          "identical bodies are **no change** and are not timed. Changed cases are verified "
          "against float64 SciPy and timed with %d interleaved full/ablated comparisons of "
          "%d warmup + %d timed launches; a cell is `median (min-max)` of "
          "ablated_ms / full_ms. Timer: %s. Schedules: the tuned schedule of each case."
          % (payload["repeats"], payload["warmup"], payload["iterations"], payload["timer"]),
          ""]
    for k in kernels:
        cases = list(dict.fromkeys(r["case"] for r in rows if r["kernel"] == k))
        md += ["## %s" % k, "",
               "| pass | changed | %s | mean (changed) |" % " | ".join(cases),
               "|---|---|%s---|" % ("---|" * len(cases))]
        for p in payload["passes"]:
            cells, measured, changed = [], [], 0
            for c in cases:
                r = _find(rows, k, p, c)
                if r is not None and not r["code_diff"]["identical"]:
                    changed += 1
                    if r["status"] == "ok":
                        measured.append(r["contribution"]["median"])
                cells.append(_cell(r))
            mean = "%.2fx" % statistics.mean(measured) if measured else "-"
            md.append("| `%s` | %d/%d | %s | %s |" % (p, changed, len(cases), " | ".join(cells),
                                                     mean))
        md.append("")
    other = rows[0]["other_backend"] if rows else "cpu"
    md += ["## Static code effect on the %s backend" % other, "",
           "Cells diff the %s backend's emitted code for the same schedule; `+a/-r` counts "
           "added/removed lines outside comments." % other, ""]
    for k in kernels:
        cases = list(dict.fromkeys(r["case"] for r in rows if r["kernel"] == k))
        md += ["### %s" % k, "", "| pass | %s |" % " | ".join(cases),
               "|---|%s" % ("---|" * len(cases))]
        for p in payload["passes"]:
            cells = []
            for c in cases:
                r = _find(rows, k, p, c)
                d = r["other_code_diff"] if r else None
                cells.append("-" if d is None else "no change" if d["identical"] else
                             "changed (+%d/-%d)" % (d["added_lines"], d["removed_lines"]))
            md.append("| `%s` | %s |" % (p, " | ".join(cells)))
        md.append("")
    md.append("`changed` counts cases whose emitted code differs when the pass is skipped; "
              "`no change` means the pass is a no-op for that kernel and schedule.")
    return "\n".join(md).rstrip() + "\n"


def write_outputs(payload: Dict[str, Any], outdir: str) -> Dict[str, str]:
    os.makedirs(outdir, exist_ok=True)
    jp = os.path.join(outdir, "pass_ablation.json")
    mp = os.path.join(outdir, "pass_ablation.md")
    with open(jp, "w") as fh:
        json.dump(payload, fh, indent=1)
    with open(mp, "w") as fh:
        fh.write(render_markdown(payload))
    return {"json": jp, "md": mp}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Ablate each pass on the tuned schedules.")
    ap.add_argument("--backend", default="hip", choices=["hip", "cpu"])
    ap.add_argument("--kernels", default="spmv,fused_spmv_axpy")
    ap.add_argument("--cases", default=None,
                    help="comma list applied to every kernel (default: per-kernel BASELINE cases)")
    ap.add_argument("--repeats", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--out", default="results")
    ap.add_argument("--workdir", default="build/ablation")
    a = ap.parse_args(argv)
    kernels = [k for k in a.kernels.split(",") if k]
    cases = None
    if a.cases:
        cl = [c for c in a.cases.split(",") if c]
        cases = {k: cl for k in kernels}
    t0 = time.time()
    payload = ablate(kernels, cases, a.backend, a.repeats, a.warmup, a.iters,
                     workdir=a.workdir, log=lambda s: print(s, flush=True))
    paths = write_outputs(payload, a.out)
    print("wrote %s and %s in %.1f s" % (paths["json"], paths["md"], time.time() - t0))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

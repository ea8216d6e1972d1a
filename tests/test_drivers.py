"""verify_all / tune_all drivers (reference scripts/verify_all.py,
scripts/autotune.py) on the CPU backend over a tiny matrix file; the HIP runs
are the same code with backend="hip"."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from tests.util import ragged
from tilegen_amd import tune_all, verify_all


def _write_tiny(d):
    A = ragged(5, 120, 120, 9, empty_every=6, long_rows=[(7, 60)])  # square: axpy pairs x (N) with w (M)
    np.savez(os.path.join(d, "tiny.npz"), indptr=A.indptr.astype(np.int64),
             indices=A.indices.astype(np.int64), data=A.data, shape=np.array(A.shape),
             class_name=np.array("tiny"))


def test_verify_all_cpu(tmp_path):
    _write_tiny(str(tmp_path))
    payload = verify_all.run(str(tmp_path), "cpu", classes=["tiny"],
                             workdir=str(tmp_path / "gen"), log=lambda m: None)
    s = payload["summary"]
    assert s["normal_triples"] == len(verify_all.KERNELS) * len(verify_all.CONFIGS)
    assert s["balance_triples"] == 0   # the OpenMP emitter has row tiles only
    assert s["all_normal_passed"] and s["all_bugs_caught"] and s["bug_triples"] == 1
    assert s["max_rel_err_inf"] <= 1e-10
    md = verify_all.render_table(payload)
    assert md.count("| tiny |") == s["total_triples"] and "| yes |" in md


@pytest.mark.gpu
def test_verify_all_hip_balance_forms(tmp_path, hip_ready):
    """On the HIP backend spmv also runs in its merge-path, hybrid and stream forms
    and as row tiles with sorted gathers."""
    _write_tiny(str(tmp_path))
    payload = verify_all.run(str(tmp_path), "hip", classes=["tiny"], kernels=["spmv"],
                             workdir=str(tmp_path / "gen"), log=lambda m: None)
    s = payload["summary"]
    assert s["executed"] and s["balance_triples"] == len(verify_all.BALANCE_CONFIGS)
    assert s["sorted_triples"] == s["sorted_passed"] == len(verify_all.SORTED_CONFIGS)
    assert s["normal_triples"] == (len(verify_all.CONFIGS) + len(verify_all.BALANCE_CONFIGS) +
                                   len(verify_all.SORTED_CONFIGS))
    assert s["all_normal_passed"] and s["all_bugs_caught"]
    md = verify_all.render_table(payload)
    assert md.count("/hybrid |") == 2 and md.count("/nnz |") == 2
    assert md.count("/stream |") == 2 and md.count("/sorted |") == 2


def test_tune_all_cpu(tmp_path):
    _write_tiny(str(tmp_path))
    res = tune_all.run(str(tmp_path), "cpu", kernels=["spmv", "spmm"], classes=["tiny"],
                       budget=2, iters=2, warmup=1, workdir=str(tmp_path / "gen"),
                       log=lambda m: None)
    assert [r["kernel"] for r in res] == ["spmv", "spmm"]
    assert all(r["winner"] is not None for r in res)
    from tilegen_amd.autotune import prune_log, write_outputs
    write_outputs(res, str(tmp_path / "out"), {"backend": "cpu"}, prune_log(),
                  full_outdir=str(tmp_path / "full"))
    best = json.load(open(tmp_path / "out" / "best_configs.json"))
    assert set(best["tiny"]) == {"spmv", "spmm"}

"""verify() and tune() on the CPU backend (reference tests/test_verify.py:21-50,
tests/test_autotune.py:30-80), plus the HIP path up to a real gfx950 compile
where no GPU is present."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from tests.util import csr
from tilegen_amd import runtime
from tilegen_amd.autotune import (BASELINE, SEARCH_SPACE, enumerate_configs, illegal_reason,
                                  illegal_reason_for, legal_configs, prune_log, tune,
                                  write_outputs)
from tilegen_amd.codegen import Config, generate
from tilegen_amd.dsl import standard_kernels
from tilegen_amd.verify import compile_generated, normwise_errors, verify


def test_injected_bug_is_caught(tmp_path):
    A = csr(4, 4, [0, 2, 3, 5, 6], [0, 1, 2, 1, 2, 3], [1.0, 2.0, 3.0, 4.0, 5.0, 6.0])
    good = verify("spmv", Config(unroll=1), A, backend="cpu", workdir=str(tmp_path))
    assert good.ok, good.message
    bad = verify("spmv", Config(unroll=1, inject_bug=True), A, backend="cpu",
                 workdir=str(tmp_path))
    assert not bad.ok and bad.max_abs_err > bad.tolerance


def test_empty_row_corner_case(tmp_path):
    A = csr(3, 3, [0, 1, 1, 3], [0, 1, 2], [2.0, 4.0, 5.0])
    r = verify("spmv", Config(unroll=2), A, backend="cpu", workdir=str(tmp_path))
    assert r.ok, r.message


def test_all_zero_data_corner_case(tmp_path):
    A = csr(2, 2, [0, 2, 3], [0, 1, 1], [0.0, 0.0, 0.0])
    r = verify("spmv", Config(unroll=4), A, backend="cpu", workdir=str(tmp_path))
    assert r.ok and r.max_abs_err == 0.0


@pytest.mark.parametrize("kernel", ["spmv", "spmm", "sddmm", "fused_spmv_axpy", "axpy"])
@pytest.mark.parametrize("cfg", [Config(unroll=1), Config(tile_size=2, unroll=3, vector_width=2)])
def test_cpu_backend_all_kernels(kernel, cfg, tmp_path):
    A = csr(3, 3, [0, 2, 3, 3], [0, 1, 2], [1.0, 2.0, 3.0])
    r = verify(kernel, cfg, A, backend="cpu", workdir=str(tmp_path))
    assert r.ok, "%s: %s" % (kernel, r.message)
    assert r.rel_err_inf <= 1e-12 and r.executed
    assert "-fopenmp" in r.message  # the OpenMP build succeeded (no silent serial retry)


def test_verify_reports_compile_errors(tmp_path, monkeypatch):
    monkeypatch.setenv("CXX", "false")
    A = csr(2, 2, [0, 1, 2], [0, 1], [1.0, 1.0])
    r = verify("spmv", Config(unroll=3, tile_size=7), A, backend="cpu", workdir=str(tmp_path))
    assert not r.ok and r.message.startswith("compile error")


def test_hip_compile_only_without_device(tmp_path):
    """hipRTC needs no GPU: verify compiles the real gfx950 code object and,
    without a device, says numerics were not run."""
    if runtime.device_count() > 0:
        pytest.skip("a HIP device is visible; the GPU tests cover this path")
    A = csr(3, 3, [0, 2, 3, 3], [0, 1, 2], [1.0, 2.0, 3.0])
    r = verify("sddmm", Config(tile_size=4, threads_per_row=4, unroll=2, vector_width=2,
                               block_size=256), A, backend="hip", workdir=str(tmp_path))
    assert r.ok and not r.executed
    assert "hipRTC compiled" in r.message or "cached" in r.message


def test_hip_compile_error_is_reported(tmp_path):
    gen = generate(standard_kernels()["spmv"], Config(), "hip", outdir=str(tmp_path))
    gen.source = gen.source.replace("acc[r] = ok[u] ? acc[r] + ", "acc[r] = ok[u] ? undefined_symbol + ")
    assert "undefined_symbol" in gen.source
    with pytest.raises(RuntimeError) as err:
        compile_generated(gen, "hip", str(tmp_path))
    assert "undefined_symbol" in str(err.value)


def test_normwise_errors():
    assert normwise_errors(np.array([1.0, 2.0]), np.array([1.0, 2.0])) == (0.0, 0.0)
    ri, r2 = normwise_errors(np.array([1.0, 2.5]), np.array([1.0, 2.0]))
    assert ri == pytest.approx(0.25) and r2 == pytest.approx(0.5 / np.sqrt(5.0))


# --------------------------------------------------------------------------- #
# autotune
# --------------------------------------------------------------------------- #
def _tiny():
    return {"indptr": np.array([0, 2, 3, 4, 6], dtype=np.int64),
            "indices": np.array([0, 1, 2, 2, 1, 3], dtype=np.int64),
            "data": np.array([1.0, 2.0, 3.0, 4.0, 5.0, 6.0]), "shape": (4, 4),
            "class_name": "tiny"}


def test_illegal_configs_pruned_with_reasons():
    pruned = [(c, r) for c, r in enumerate_configs() if r is not None]
    assert pruned and all(isinstance(r, str) and r for _c, r in pruned)
    assert illegal_reason(Config(threads_per_row=8, block_size=4)) is not None
    assert illegal_reason(Config(block_size=96)) is not None  # not whole waves
    assert illegal_reason(Config(threads_per_row=3, block_size=192)) is not None
    assert illegal_reason(Config(vector_width=2, unroll=1)) is not None
    assert illegal_reason(Config(tile_size=16, threads_per_row=1, block_size=128)) is not None
    assert illegal_reason(Config(tile_size=128, threads_per_row=8, unroll=2, block_size=256)) \
        is None
    assert "idle lanes" in illegal_reason(BASELINE)  # pruned, but always timed first
    assert all(illegal_reason(c) is None for c in legal_configs())
    assert len(prune_log()) == len(pruned)
    assert illegal_reason_for("spmv", Config(tile_size=128, threads_per_row=8, unroll=2,
                                             vector_width=2, block_size=256)) is not None
    assert set(SEARCH_SPACE["block_size"]) <= {64, 128, 256, 512, 1024}


def test_sddmm_space_follows_the_row_mapping():
    """Chunked path (one group's registers cover K): tiles are multiples of the
    lane groups per block; otherwise one wave per row: multiples of the waves."""
    from tilegen_amd.autotune import sddmm_group_per_row
    cs = legal_configs("sddmm", 64)
    assert cs
    for c in cs:
        per = c.block_size // (c.threads_per_row if sddmm_group_per_row(c, 64) else 64)
        assert c.tile_size % per == 0 and per <= c.tile_size <= 8 * per
    assert any(sddmm_group_per_row(c, 64) for c in cs)
    assert any(not sddmm_group_per_row(c, 64) for c in cs)
    tuned = Config(tile_size=16, threads_per_row=16, unroll=2, vector_width=2, block_size=256)
    assert sddmm_group_per_row(tuned, 64) and illegal_reason_for("sddmm", tuned, 64) is None
    assert not sddmm_group_per_row(tuned, 65)  # odd K: no 128-bit path, wave per row
    assert illegal_reason_for("sddmm", tuned, 130) is None  # wave per row: 4 rows per wave
    small = Config(tile_size=4, threads_per_row=16, unroll=2, vector_width=2, block_size=256)
    assert "lane group" in illegal_reason_for("sddmm", small, 64)  # 16 groups, 4 rows


def test_tune_smoke_cpu(tmp_path):
    res = tune("spmv", _tiny(), budget=3, backend="cpu", workdir=str(tmp_path), warmup=1,
               iters=3)
    assert res["winner"] is not None and res["records"]
    m = res["winner_metrics"]
    for key in ["ms_mean", "ms_min", "ms_median", "gflops", "bandwidth_gbs", "max_abs_err",
                "ok", "speedup_vs_naive", "compulsory_gbs"]:
        assert key in m
    assert res["baseline"] == BASELINE.to_dict() and res["baseline_ms_min"] is not None


def test_write_outputs_schema(tmp_path):
    res = tune("spmv", _tiny(), budget=2, backend="cpu", workdir=str(tmp_path / "gen"),
               warmup=1, iters=2)
    full = tmp_path / "full"
    write_outputs([res], str(tmp_path), {"backend": "cpu"}, prune_log(), full_outdir=str(full))
    for name in ["autotune.json", "autotune.csv", "best_configs.json"]:
        assert os.path.exists(str(tmp_path / name))
    data = json.load(open(str(tmp_path / "autotune.json")))
    assert {"results", "pruned", "hardware", "best", "top5"} <= set(data)
    assert all("records" not in r for r in data["results"])
    assert "tiny" in data["best"] and "spmv" in data["best"]["tiny"]
    assert 0 < len(data["top5"]["tiny"]) <= 5
    raw = json.load(open(str(full / "autotune.json")))
    assert raw["results"][0]["records"]
    assert data["results"][0]["mode"] == "random" and data["results"][0]["candidates"] == 2


def test_write_outputs_tells_sorted_from_direct(tmp_path):
    """A sorted-gather schedule and its direct twin share T/TPR/U/V/B: the CSV rows
    carry the gather form (and the balance form) so they stay apart."""
    metrics = {"ms_mean": 1.0, "ms_min": 1.0, "ms_median": 1.0, "gflops": 1.0,
               "bandwidth_gbs": 1.0, "compulsory_gbs": 1.0, "max_abs_err": 0.0,
               "tolerance": 1.0, "ok": True, "speedup_vs_naive": 1.0}
    direct = Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256)
    twins = [direct, Config(**{**direct.to_dict(), "gather": "sorted"}),
             Config(**{**direct.to_dict(), "balance": "stream"})]
    recs = [dict(metrics, kernel="spmv", matrix_class="m", config=c.to_dict()) for c in twins]
    res = {"kernel": "spmv", "matrix_class": "m", "backend": "hip", "mode": "exhaustive",
           "candidates": 3, "baseline": direct.to_dict(), "baseline_ms_min": 1.0,
           "winner": twins[1].to_dict(), "winner_metrics": recs[1], "records": recs}
    full = tmp_path / "full"
    write_outputs([res], str(tmp_path), {"backend": "hip"}, [], full_outdir=str(full))
    lines = open(str(full / "autotune.csv")).read().splitlines()
    head = lines[0].split(",")
    forms = [(r.split(",")[head.index("balance")], r.split(",")[head.index("gather")])
             for r in lines[1:]]
    assert forms == [("rows", "direct"), ("rows", "sorted"), ("stream", "direct")]
    from tilegen_amd.tune_all import render_markdown
    md = render_markdown([res], "hip")
    assert "| m | spmv | exhaustive | T64/TPR4/U4/V1/B256/sorted |" in md


def test_bench_openmp_leg_on_cpu():
    """bench.py's cpu_openmp leg: the OpenMP backend at the reference default
    schedule, checked against the float64 result it is given."""
    import bench
    from tilegen_amd.autotune import BASELINE
    from tests.util import ragged
    A = ragged(11, 300, 200, 12, empty_every=7)
    x = np.random.default_rng(0).uniform(-1, 1, A.shape[1])
    ref = A @ x
    r = bench._openmp_baseline("spmv", A, {"x": x}, 1, ref, 10**9, 10**8, 0.05)
    assert r["kind"] == "openmp backend" and r["schedule"] == BASELINE.short()
    assert r["rel_err"] <= 1e-12 and r["cores"] >= 1 and r["value"] > 0
    assert "-fopenmp" in r["compile"]


@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy"])
def test_sorted_space_matches_the_emitter(kernel):
    """Row tiles with sorted first-step gathers are in the SpMV search space
    exactly where the emitter accepts them: every legal one generates, every one
    pruned for the sort's limits is refused by the emitter too."""
    from tilegen_amd.schedules import TUNED
    sorted_ = [(c, r) for c, r in enumerate_configs(kernel) if c.gather == "sorted"]
    legal = [c for c, r in sorted_ if r is None]
    limited = [c for c, r in sorted_ if r is not None and r.startswith("sorted")]
    assert len(legal) > 100 and limited
    k = standard_kernels()[kernel]
    for c in legal:
        generate(k, c, "hip", write=False)
    for c in limited:
        with pytest.raises(ValueError, match="sorted"):
            generate(k, c, "hip", write=False)
    # the tuned c1 tile (240 rows) lies between the space's power-of-two tile sizes;
    # the same limits accept it
    from tilegen_amd.autotune import _sorted_reason
    assert TUNED["c1"].gather == "sorted" and _sorted_reason(TUNED["c1"]) is None
    generate(k, TUNED["c1"], "hip", write=False)


def test_tune_includes_tuned_schedules_outside_the_space():
    """c1's and c2's tuned schedules lie between the space's powers of two; they are
    legal, and ``include`` puts them among the candidates right after the baseline."""
    import random
    from tilegen_amd.autotune import _candidate_configs
    from tilegen_amd.schedules import TUNED
    extra = [TUNED["c1"], TUNED["c2"]]
    legal = {c.hash() for c, r in enumerate_configs("spmv") if r is None}
    assert all(c.hash() not in legal for c in extra)   # not in the space itself
    assert all(illegal_reason_for("spmv", c) is None for c in extra)
    cands = _candidate_configs("spmv", 8, 6, "random", random.Random(0), extra, "hip")
    assert [c.hash() for c in cands[1:3]] == [c.hash() for c in extra]
    assert cands[0].hash() == BASELINE.hash()

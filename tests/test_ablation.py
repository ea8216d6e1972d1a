"""Pass ablation (reference scripts/ablate_passes.py): code diff first, no-op
passes are never timed, ABI-changing ablations are invalid, changed cases are
verified and timed interleaved."""

from __future__ import annotations

import pytest

from tests.util import ragged
from tilegen_amd.ablation import ablate, code_diff, render_markdown, write_outputs
from tilegen_amd.codegen import Config, generate
from tilegen_amd.dsl import standard_kernels
from tilegen_amd.passes import PASS_NAMES

CFG = Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128)


def test_code_diff_ignores_comment_header():
    k = standard_kernels()["spmv"]
    full = generate(k, CFG, "hip", write=False)
    same = generate(k, CFG, "hip", write=False, skip_passes=["vectorize"])
    assert full.source != same.source  # the pass log in the header differs
    assert code_diff(full, same)["identical"]
    changed = code_diff(full, generate(k, CFG, "hip", write=False, skip_passes=["unroll"]))
    assert not changed["identical"] and changed["added_lines"] > 0


def _payload(backend, tmp_path, kernels=("spmv", "fused_spmv_axpy")):
    A = ragged(3, 400, 300, 12, empty_every=7, long_rows=[(5, 200)])
    return ablate(kernels, {k: ["small"] for k in kernels}, backend=backend, repeats=2,
                  warmup=1, iters=10, configs={"small": CFG}, matrices={"small": A},
                  workdir=str(tmp_path), log=lambda s: None)


def _check_rows(payload, kernels):
    rows = payload["rows"]
    assert len(rows) == len(kernels) * len(PASS_NAMES)
    for r in rows:
        if r["code_diff"]["identical"]:
            assert r["status"] == "no_change" and r["full"] is None
            assert r["contribution"]["median"] == 1.0
    by = {(r["kernel"], r["pass"]): r for r in rows}
    for k in kernels:
        for p in ("tiling", "unroll", "thread_mapping"):
            r = by[(k, p)]
            assert not r["code_diff"]["identical"], (k, p)
            assert r["status"] == "ok" and r["verified"], (k, p, r.get("reason"))
            assert len(r["full"]) == 2 and r["contribution"]["min"] > 0
        for p in ("canonicalize", "vectorize", "dead_code_elim"):
            assert by[(k, p)]["status"] == "no_change", (k, p)
    if "fused_spmv_axpy" in kernels:
        r = by[("fused_spmv_axpy", "loop_fusion")]
        assert r["status"] == "invalid" and "ABI" in r["reason"]


def test_cpu_ablation(tmp_path):
    payload = _payload("cpu", tmp_path)
    _check_rows(payload, ("spmv", "fused_spmv_axpy"))
    paths = write_outputs(payload, str(tmp_path / "out"))
    md = open(paths["md"]).read()
    assert "| `unroll` | 1/1 |" in md and "**invalid**" in md
    assert "Static code effect on the hip backend" in md
    assert render_markdown(payload) == md


@pytest.mark.gpu
def test_hip_ablation(tmp_path, hip_ready):
    payload = _payload("hip", tmp_path, kernels=("spmv",))
    _check_rows(payload, ("spmv",))
    assert payload["timer"].startswith("HIP events")

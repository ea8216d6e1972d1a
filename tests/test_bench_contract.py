"""bench.py's output contract: one JSON line with the driver's keys, the
roofline and CPU-baseline objects, and a clear refusal of more than one GPU."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KEYS = ["metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
        "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config", "roofline",
        "cpu_baseline"]


def _bench(*args, timeout=300):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + list(args),
                          capture_output=True, text=True, timeout=timeout, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2")
    assert r.returncode != 0 and "one GPU" in r.stderr and r.stdout.strip() == ""


def test_config_parser_and_traffic_lookup():
    sys.path.insert(0, ROOT)
    import bench
    cfg = bench._parse_config("T128/TPR8/U2/V1/B256")
    assert (cfg.tile_size, cfg.threads_per_row, cfg.unroll, cfg.vector_width,
            cfg.block_size) == (128, 8, 2, 1, 256)
    with pytest.raises(SystemExit):
        bench._parse_config("T128/X9")
    t = bench._traffic("spmv", "c1")
    assert t is None or t > 28_000_008  # measured HBM bytes exceed the compulsory ones


@pytest.mark.gpu
@pytest.mark.timeout(500)
def test_bench_json_line(hip_ready):
    """The default run: c1 as the headline plus every other BASELINE config."""
    r = _bench("--steps", "20", "--warmup", "2", "--cpu-seconds", "1", "--case-cpu-seconds",
               "0.3", "--case-iters", "10", timeout=480)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.strip()]
    assert len(lines) == 1
    assert len(lines[0]) < 3600, len(lines[0])  # a driver's tail holds it whole
    out = json.loads(lines[0])
    assert sorted(out["cases"]) == sorted(["c2", "c3a", "c3b", "c4", "c5", "c5x25"])
    for cid, c in out["cases"].items():
        assert c["err"] <= 1e-10 and c["us"] > 0 and c["gflops"] > 0, cid
        assert abs(c["frac"] - c["gbs"] / 8000.0) < 1e-3, cid
        assert c["cpu_ms"] > 0 and c["omp_ms"] > 0, cid
    for k in KEYS:
        assert k in out, k
    assert out["n_gpus"] == 1 and out["steps"] == 20 and out["unit"] == "GB/s"
    assert out["config"]["workload"].startswith("c1:") and out["dtype"] == "f64"
    roof = out["roofline"]
    assert roof["bound"] == "hbm" and roof["peak"] == 8000.0 and roof["unit"] == "GB/s"
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    cpu = out["cpu_baseline"]
    assert cpu["kind"] in ("reference", "port") and cpu["cores"] == 1 and cpu["value"] > 0
    assert out["check_rel_err"] <= 1e-10


def test_cpu_tuned_schedules_are_row_tiles_of_known_cases():
    """Every CPU-tuned schedule names a BASELINE case and is a plain row-tile
    schedule (the OpenMP backend ignores the GPU-only balance)."""
    from tilegen_amd.matrices import baseline_ids
    from tilegen_amd.schedules import CPU_TUNED
    for case_id, cfg in CPU_TUNED.items():
        assert case_id in baseline_ids()
        assert cfg.balance == "rows"

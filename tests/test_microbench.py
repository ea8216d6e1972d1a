"""The hardware microbenchmarks (gather ceiling, streaming-read floor)."""

from __future__ import annotations

import pytest

from tilegen_amd import microbench, runtime
from tilegen_amd.verify import hiprtc_options


def test_probe_kernels_compile():
    for src in (microbench._GATHER_SRC, microbench._STREAM_SRC):
        code, _ = runtime.rtc_compile(src, "microbench.hip", hiprtc_options())
        assert len(code) > 0


def test_render_tables():
    g = [{"kernel": "mb_gather", "lanes_or_uniform": 64, "us": 10.0, "gathers_per_s": 2e11,
          "gather_instr_per_s": 3e9}]
    s = [{"mb": 27, "bytes": 27 << 20, "us": 5.0, "gb_per_s": 5600.0, "workgroups": 4096,
          "copies": 47}]
    md = microbench.render(g, s, "MI355X gfx950")
    assert "| mb_gather | 64 | 10.00 | 200.0 | 3.00 |" in md
    assert "| 27 | 5.00 | 5600 | 4096 |" in md


@pytest.mark.gpu
def test_probes_run(hip_ready):
    g = microbench.gather_probe(workgroups=512, iters=3)
    assert len(g) == 8 and all(r["us"] > 0 and r["gathers_per_s"] > 0 for r in g)
    s = microbench.stream_probe(sizes_mb=(8,), rotate_mb=32, iters=5)
    assert s[0]["copies"] == 4 and 0 < s[0]["gb_per_s"] < 20000


def test_rowgather_kernel_compiles_and_renders():
    code, _ = runtime.rtc_compile(microbench._ROWGATHER_SRC, "rg.hip", hiprtc_options())
    assert len(code) > 0
    rg = [{"table_mb": 51.2, "cold": True, "copies": 13, "rows_gathered": 1600000,
           "us": 100.0, "g_rows_per_s": 16.0, "gathered_gb_per_s": 8192.0,
           "written_gb_per_s": 512.0}]
    assert "| 51.2 | cold (13 copies) | 100.00 | 16.00 | 8192 | 512 |" in microbench.render(
        [], [], "x", rg)


@pytest.mark.gpu
def test_rowgather_probe_runs(hip_ready):
    r = microbench.rowgather_probe(table_rows=(6_250,), n_groups=2_000, per=8, rotate_mb=8,
                                   iters=3)
    assert len(r) == 2 and all(x["us"] > 0 for x in r)


def test_flat_kernel_compiles_and_renders():
    code, _ = runtime.rtc_compile(microbench._FLAT_SRC, "flat.hip", hiprtc_options())
    assert len(code) > 0
    fl = [{"cold": True, "copies": 47, "gather": True, "block": 128, "nnz": 1600000,
           "us": 11.5, "streamed_bytes": 26400000, "streamed_gb_per_s": 2295.7,
           "g_gathers_per_s": 139.1},
          {"cold": False, "copies": 1, "gather": False, "block": 256, "nnz": 1600000,
           "us": 4.0, "streamed_bytes": 26400000, "streamed_gb_per_s": 6600.0,
           "g_gathers_per_s": 0.0}]
    fl[1]["case"] = "c2"
    md = microbench.render([], [], "x", flat=fl)
    assert "| c1 | cold (47 copies) | yes | 128 | 11.50 | 2296 | 139.1 |" in md
    assert "| c2 | warm | no | 256 | 4.00 | 6600 | - |" in md


@pytest.mark.gpu
def test_flat_probe_runs(hip_ready):
    # the probe checks its own output against numpy before reporting a time
    r = microbench.flat_probe(rotate_mb=64, iters=3, blocks=(256,))
    assert len(r) == 4 and all(x["us"] > 0 for x in r)
    assert [x["gather"] for x in r] == [True, False, True, False]
    # c2's nonzero count is not a multiple of 16: the probe leaves the tail out
    r2 = microbench.flat_probe(rotate_mb=64, iters=3, blocks=(256,), case="c2")
    assert r2[0]["nnz"] % 16 == 0 and r2[0]["case"] == "c2"

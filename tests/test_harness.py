"""tilegen_bench, the native host harness (reference cpp/src/harness.cpp):
TGM1 input, launch_<name> through dlopen, JSON output with the reference's keys,
and its exit codes.  CPU-backend runs here; the HIP run is marked gpu."""

from __future__ import annotations

import json
import os
import subprocess

import pytest

from tests.util import ragged
from tilegen_amd.codegen import Config, generate
from tilegen_amd.dsl import standard_kernels
from tilegen_amd.matrices import export_matrix_bin
from tilegen_amd.verify import compile_generated

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "tilegen_amd", "_lib", "tilegen_bench")
REF_KEYS = ["kernel", "config", "backend", "matrix", "rows", "cols", "nnz", "ms_mean", "ms_min",
            "gflops", "bandwidth_gbs", "max_abs_err", "max_rel_err"]


def _run(*args):
    return subprocess.run([BENCH] + [str(a) for a in args], capture_output=True, text=True,
                          timeout=120)


@pytest.fixture(scope="module")
def matrix_bin(tmp_path_factory):
    d = tmp_path_factory.mktemp("tgm1")
    path = str(d / "m.bin")
    export_matrix_bin(path, ragged(5, 300, 250, 20, empty_every=9, long_rows=[(3, 240)]))
    return path


def _lib(kernel, backend, tmp_path, cfg=None):
    cfg = cfg or Config(tile_size=32, threads_per_row=4, unroll=2, vector_width=2,
                        block_size=256)
    gen = generate(standard_kernels()[kernel], cfg, backend, outdir=str(tmp_path))
    so, _ = compile_generated(gen, backend, str(tmp_path))
    return so


@pytest.mark.parametrize("kernel", ["spmv", "spmm", "sddmm"])
def test_cpu_backend_json(kernel, matrix_bin, tmp_path):
    so = _lib(kernel, "cpu", tmp_path)
    r = _run("--kernel", kernel, "--matrix", matrix_bin, "--lib", so, "--backend", "cpu",
             "--K", 8, "--iters", 3, "--warmup", 1, "--config", '{"tile_size": 32}')
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    for key in REF_KEYS:
        assert key in out
    assert out["rows"] == 300 and out["cols"] == 250 and out["config"] == {"tile_size": 32}
    assert out["max_abs_err"] < 1e-12, out
    assert out["timer"] == "host clock around launch"


def test_exit_codes(matrix_bin, tmp_path):
    assert _run("--kernel", "spmv").returncode == 2
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"NOPE" + b"\0" * 40)
    so = _lib("spmv", "cpu", tmp_path)
    assert _run("--kernel", "spmv", "--matrix", str(bad), "--lib", so, "--backend",
                "cpu").returncode == 2
    assert _run("--kernel", "spmm", "--matrix", matrix_bin, "--lib", so, "--backend",
                "cpu").returncode == 3  # launch_spmm not exported by an spmv variant
    assert _run("--kernel", "spmv", "--matrix", matrix_bin, "--lib",
                str(tmp_path / "missing.so"), "--backend", "cpu").returncode == 3
    assert _run("--kernel", "axpy", "--matrix", matrix_bin, "--lib", so).returncode == 2


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", ["spmv", "spmm", "sddmm"])
def test_hip_backend_device_buffers(kernel, matrix_bin, tmp_path, hip_ready):
    so = _lib(kernel, "hip", tmp_path)
    r = _run("--kernel", kernel, "--matrix", matrix_bin, "--lib", so, "--backend", "hip",
             "--K", 64, "--iters", 10, "--warmup", 2, "--rotate", 3)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["max_abs_err"] < 1e-12, out
    assert out["timer"] == "dispatch events (tg_time_launches)" and out["ms_min"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("balance", ["nnz", "hybrid", "stream"])
def test_hip_harness_balance_modes(balance, matrix_bin, tmp_path, hip_ready):
    """The harness takes its grid from tgv_geometry, which counts the hybrid
    tiles' range workgroups and, for stream ranges, one workgroup per range of
    64 nonzeros; with windows and ranges of a few rows, the 240-nonzero row is
    cut into pieces, and the result still matches."""
    so = _lib("spmv", "hip", tmp_path, Config(tile_size=2, threads_per_row=4, unroll=1,
                                              block_size=64, balance=balance))
    r = _run("--kernel", "spmv", "--matrix", matrix_bin, "--lib", so, "--backend", "hip",
             "--iters", 10, "--warmup", 2, "--rotate", 3)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["max_abs_err"] < 1e-12, out

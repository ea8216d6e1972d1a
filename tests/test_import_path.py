"""The ``tilegen`` import path: every module path and name the reference's
own callers import (scripts/*.py and tests/*.py of TileGen) resolves, to the
same objects as ``tilegen_amd``, and the reference scripts' calls run on the
CPU backend through it."""

from __future__ import annotations

import importlib

import pytest

# (module, names) as the reference's callers import them
REFERENCE_IMPORTS = [
    # scripts/ablate_passes.py:40-51, scripts/compare_cusparse.py:24-34
    ("tilegen.autotune", ["BASELINE", "_make_caller", "prune_log", "tune"]),
    ("tilegen.codegen", ["Config", "generate"]),
    ("tilegen.dsl", ["standard_kernels"]),
    ("tilegen.env", ["probe"]),
    ("tilegen.matrices", ["build_corpus", "corpus_classes"]),
    ("tilegen.verify", ["_inputs_for", "_load_matrix", "_reference", "compile_generated"]),
    # scripts/autotune.py:16-18, scripts/verify_all.py:16-19
    ("tilegen.autotune", ["write_outputs"]),
    ("tilegen.verify", ["verify"]),
    # tests/test_autotune.py:10-19
    ("tilegen.autotune", ["enumerate_configs", "illegal_reason", "legal_configs"]),
    # tests/test_dsl.py:7-29
    ("tilegen.dsl", ["CSR", "Index", "assign", "dense_tensor", "kernel", "reduce_sum",
                     "scalar_tensor", "sparse_tensor"]),
    ("tilegen.ir", ["Format"]),
    # tests/test_env_matrices.py:10-17
    ("tilegen.matrices", ["load_csr_npz", "make_matrix", "matrix_stats"]),
    # tests/test_passes.py:5-17
    ("tilegen.codegen", ["emit_cpu"]),
]

# CUDA-only names of the reference and the HIP name that replaces each
HIP_COUNTERPARTS = {
    ("tilegen.verify", "cuda_arch"): ("tilegen.verify", "hip_arch"),
    ("tilegen.codegen", "emit_cuda"): ("tilegen.codegen", "emit_hip"),
}


@pytest.mark.parametrize("module,names", REFERENCE_IMPORTS)
def test_reference_import_resolves(module, names):
    mod = importlib.import_module(module)
    impl = importlib.import_module(module.replace("tilegen.", "tilegen_amd.", 1))
    assert mod is impl
    for n in names:
        assert getattr(mod, n) is getattr(impl, n), (module, n)


def test_from_tilegen_import_passes():
    from tilegen import passes
    import tilegen_amd.passes
    assert passes is tilegen_amd.passes and callable(passes.run_pipeline)


@pytest.mark.parametrize("cuda_name,hip_name", sorted(HIP_COUNTERPARTS.items()))
def test_cuda_names_have_hip_counterparts(cuda_name, hip_name):
    assert not hasattr(importlib.import_module(cuda_name[0]), cuda_name[1])
    assert callable(getattr(importlib.import_module(hip_name[0]), hip_name[1]))


def test_config_is_one_class_under_both_names():
    from tilegen.codegen import Config as A
    from tilegen_amd.codegen import Config as B
    assert A is B and isinstance(A(), B)


def test_reference_scripts_calls_run_on_cpu(tmp_path):
    """What scripts/verify_all.py and scripts/gen_demo.py do, through the
    ``tilegen`` names, on the CPU backend."""
    from tilegen.codegen import Config, generate
    from tilegen.dsl import standard_kernels
    from tilegen.env import probe
    from tilegen.matrices import make_matrix
    from tilegen.verify import verify
    assert probe()["backend"] in ("hip", "cpu")
    cfg = Config(tile_size=64, threads_per_row=1, unroll=4, vector_width=1, block_size=256)
    for name in ("spmv", "spmm", "sddmm"):
        gen = generate(standard_kernels()[name], cfg, backend="cpu", outdir=str(tmp_path))
        assert gen.filename.startswith(name + "_") and "launch_%s" % name in gen.source
    A = make_matrix("banded")
    sub = A[:3000, :3000].tocsr()
    for name in ("spmv", "sddmm"):
        r = verify(name, cfg, sub, backend="cpu", workdir=str(tmp_path), K=8)
        assert r.ok and r.max_abs_err <= r.tolerance, (name, r.message)
    bug = verify("spmv", Config(inject_bug=True), sub, backend="cpu", workdir=str(tmp_path))
    assert not bug.ok

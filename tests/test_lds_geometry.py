"""The LDS figure of a HIP variant (``launch_geometry(...).lds_bytes``): it adds up
every ``__shared__`` array the emitted kernel declares, it agrees with the group
segment size hipRTC's code object reports, and the emitter and the schedule space
refuse what does not fit a gfx950 workgroup's 160 KiB.  CPU only (hipRTC
cross-compiles)."""

from __future__ import annotations

import dataclasses
import os
import random
import re
import subprocess

import pytest

from tilegen_amd.autotune import enumerate_configs
from tilegen_amd.codegen import LDS_LIMIT, Config, generate
from tilegen_amd.dsl import standard_kernels

_ELEM = {"unsigned long long": 8, "tg_i64": 8, "double": 8, "unsigned": 4, "int": 4}
_DECL = re.compile(r"__shared__\s+(unsigned long long|tg_i64|double|unsigned|int)\s+\w+"
                   r"(?:\[(\d+)\])?\s*;")


def _declared(source: str) -> int:
    """The kernel text's own __shared__ declarations, summed and rounded to 16."""
    decls = _DECL.findall(source)
    assert source.count("__shared__") == len(decls), "an LDS declaration the test cannot read"
    total = sum(_ELEM[t] * int(n or 1) for t, n in decls)
    return (total + 15) // 16 * 16


def _sample(kernel: str, n: int, seed: int):
    legal = [c for c, r in enumerate_configs(kernel) if r is None]
    forms = {}
    for c in legal:
        forms.setdefault((c.balance, c.gather), []).append(c)
    rng = random.Random(seed)
    out = []
    for key in sorted(forms):          # every form, n schedules of each
        cs = forms[key]
        out += rng.sample(cs, min(n, len(cs)))
    return out


@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy", "spmm", "sddmm", "axpy"])
def test_geometry_lds_is_the_declared_arrays(kernel):
    k = standard_kernels()[kernel]
    for cfg in _sample(kernel, 12, 7):
        gen = generate(k, cfg, "hip", write=False)
        assert gen.geometry.lds_bytes == _declared(gen.source), cfg.short()
        assert "static lds = %d B" % gen.geometry.lds_bytes in gen.source


_COMPILED = [
    ("spmv", Config(tile_size=240, threads_per_row=4, unroll=4, block_size=960, gather="sorted")),
    ("spmv", Config(tile_size=256, threads_per_row=1, unroll=4, block_size=256, balance="stream")),
    ("spmv", Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256, balance="hybrid")),
    ("spmv", Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256, balance="nnz")),
    ("spmv", Config(tile_size=64, threads_per_row=32, unroll=4, block_size=256)),
    ("spmm", Config(tile_size=16, threads_per_row=8, unroll=2, vector_width=2, block_size=64)),
    ("sddmm", Config(tile_size=16, threads_per_row=8, unroll=4, vector_width=2, block_size=128)),
]


def test_geometry_lds_bounds_the_code_object(tmp_path):
    """The figure is the code object's group segment size or at most 15 bytes more
    (the compiler rounds its packed block to 8 or 16 bytes)."""
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not os.path.exists(readelf):
        pytest.skip("llvm-readelf not available")
    from tilegen_amd.verify import compile_generated
    for kernel, cfg in _COMPILED:
        gen = generate(standard_kernels()[kernel], cfg, "hip", outdir=str(tmp_path))
        so, _ = compile_generated(gen, "hip", str(tmp_path))
        notes = subprocess.run([readelf, "--notes", so[:-3] + ".co"], capture_output=True,
                               text=True).stdout
        seg = [int(v) for v in re.findall(r"\.group_segment_fixed_size:\s+(\d+)", notes)]
        assert len(seg) == 1, (cfg.short(), notes[:300])
        assert seg[0] <= gen.geometry.lds_bytes <= seg[0] + 15, (cfg.short(), seg,
                                                                 gen.geometry.lds_bytes)


def test_sorted_tiles_over_the_lds_limit_are_pruned_and_refused():
    """A 2048-row sorted tile on 1024 lanes holds 8192 items and 2049 row pointers:
    168,144 B, over 160 KiB.  The space prunes it with that reason and the emitter
    refuses it with a ValueError instead of leaving it to hipRTC."""
    over = [(c, r) for c, r in enumerate_configs("spmv")
            if c.gather == "sorted" and r is not None and "LDS" in r]
    assert sorted(c.short() for c, _ in over) == [
        "T2048/TPR1/U4/V1/B1024/sorted", "T2048/TPR2/U2/V1/B1024/sorted",
        "T2048/TPR4/U1/V1/B1024/sorted"]
    assert all("168144 B" in r for _, r in over)
    k = standard_kernels()["spmv"]
    for c, _ in over:
        with pytest.raises(ValueError, match="168144 B of LDS"):
            generate(k, c, "hip", write=False)
        # the direct twin, without the sort's arrays, fits
        direct = dataclasses.replace(c, gather="direct")
        assert generate(k, direct, "hip", write=False).geometry.lds_bytes <= LDS_LIMIT
    # every legal schedule of every kernel fits
    for kernel in ("spmv", "fused_spmv_axpy", "spmm", "sddmm", "axpy"):
        kk = standard_kernels()[kernel]
        for cfg in _sample(kernel, 4, 3):
            assert generate(kk, cfg, "hip", write=False).geometry.lds_bytes <= LDS_LIMIT

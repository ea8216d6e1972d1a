"""Pass pipeline and emitters (reference tests/test_passes.py:24-158 and the
emitter checks of tests/test_verify.py:53-89), for the HIP and CPU backends.
No GPU: HIP sources are checked as text and compiled by hipRTC for gfx950."""

from __future__ import annotations

import os
import re

import numpy as np

import pytest

from tilegen_amd import passes
from tilegen_amd.codegen import (Config, abi_of, emit_cpu, emit_hip, emit_hip_host,
                                 generate, launch_geometry, _lowering, _plan)
from tilegen_amd.dsl import (CSR, Index, assign, dense_tensor, kernel, reduce_sum,
                             scalar_tensor, sparse_tensor, standard_kernels)


def _run(k, cfg=None, backend="cpu", skip=()):
    return passes.run_pipeline(k, cfg or Config(), backend=backend, skip=skip)


def _code(src: str) -> str:
    return "\n".join(l for l in src.splitlines() if not l.lstrip().startswith("//"))


def test_pass_names_and_order():
    assert passes.PASS_NAMES == ["canonicalize", "loop_fusion", "tiling", "thread_mapping",
                                 "unroll", "vectorize", "dead_code_elim"]
    assert passes.optimize is passes.run_pipeline


def test_fusion_collapses_two_loop_nests():
    out = _run(standard_kernels()["fused_spmv_axpy"])
    assert len(out.stmts) == 1
    fusion = [e for e in out.pass_log if e["pass"] == "loop_fusion"]
    assert fusion and "fused" in fusion[0]["action"]
    reads = [n.tensor.name for st in out.stmts for n in st.rhs.walk() if hasattr(n, "tensor")]
    assert "t" not in reads


def test_fusion_refused_on_true_dependency():
    i, j, kk = Index("i"), Index("j"), Index("kk")
    A = sparse_tensor("A", CSR, shape=("M", "N"))
    x = dense_tensor("x", shape=("N",))
    w = dense_tensor("w", shape=("M",))
    t = dense_tensor("t", shape=("M",))
    z = dense_tensor("z", shape=("M",))
    alpha, beta = scalar_tensor("alpha"), scalar_tensor("beta")
    k = kernel("dependent", [assign(t[i], reduce_sum(j, A[i, j] * x[j])),
                             assign(z[kk], alpha * t[kk] + beta * w[kk])])
    out = _run(k)
    assert len(out.stmts) == 2
    fusion = [e for e in out.pass_log if e["pass"] == "loop_fusion"]
    assert fusion and "refused" in fusion[0]["action"]


def test_canonicalize_folds_and_reports_no_change_second_time():
    i = Index("i")
    x = dense_tensor("x", shape=("M",))
    z = dense_tensor("z", shape=("M",))
    k = kernel("c", [assign(z[i], (1.0 * x[i]) + (2.0 + 3.0) * 0.0 + 0.0)])
    once = passes.canonicalize(k)
    assert "no change" not in once.pass_log[-1]["action"]
    twice = passes.canonicalize(once)
    assert "no change" in twice.pass_log[-1]["action"]
    k2 = standard_kernels()["spmv"]
    assert "no change" in passes.canonicalize(passes.canonicalize(k2)).pass_log[-1]["action"]


def test_dead_code_elim_drops_unread_temporary():
    i, j = Index("i"), Index("j")
    A = sparse_tensor("A", CSR, shape=("M", "N"))
    x = dense_tensor("x", shape=("N",))
    y = dense_tensor("y", shape=("M",))
    t = dense_tensor("t", shape=("M",))
    k = kernel("dce", [assign(y[i], reduce_sum(j, A[i, j] * x[j])), assign(t[i], x[i] * 2.0)])
    out = passes.dead_code_elim(k)
    assert "removed 0" in out.pass_log[-1]["action"]  # both are outputs


def test_lowering_transforms_recorded_in_schedule():
    cfg = Config(tile_size=64, threads_per_row=8, unroll=4, vector_width=2, block_size=512)
    spmm = _run(standard_kernels()["spmm"], cfg, "hip")
    low = _lowering(spmm)
    assert (low.tile, low.threads_per_row, low.unroll, low.vector_width, low.block_size) == \
        (64, 8, 4, 2, 512)
    assert low.tiled and low.parallel
    spmv = _run(standard_kernels()["spmv"], cfg, "hip")
    assert _lowering(spmv).vector_width == 1  # the spmv gather is not vectorized
    vec = [e for e in spmv.pass_log if e["pass"] == "vectorize"][0]
    assert "skipped" in vec["action"]
    tm = [e for e in spmv.pass_log if e["pass"] == "thread_mapping"][0]
    assert "wave64" in tm["action"] and "8 lanes per row" in tm["action"]


def test_pipeline_idempotent_on_canonical_ir():
    cfg = Config(tile_size=64, unroll=2, threads_per_row=4)
    for name in ("spmv", "spmm", "sddmm", "fused_spmv_axpy"):
        once = _run(standard_kernels()[name], cfg, "hip")
        twice = _run(once, cfg, "hip")
        d1, d2 = once.to_dict(), twice.to_dict()
        d1.pop("pass_log")
        d2.pop("pass_log")
        assert d1 == d2, name


# --------------------------------------------------------------------------- #
# ABI
# --------------------------------------------------------------------------- #
EXPECTED_ABI = {
    # reference verify.py:166-173 / tilegen_launch.h
    "spmv": "void launch_spmv(const int64_t* indptr, const int64_t* indices, const double* data, "
            "const double* x, double* y, int64_t M, int64_t N, int64_t nnz)",
    "spmm": "void launch_spmm(const int64_t* indptr, const int64_t* indices, const double* data, "
            "const double* B, double* C, int64_t M, int64_t N, int64_t K, int64_t nnz)",
    "sddmm": "void launch_sddmm(const int64_t* indptr, const int64_t* indices, "
             "const double* data, const double* U, const double* V, double* C, int64_t M, "
             "int64_t N, int64_t K, int64_t nnz)",
    "fused_spmv_axpy": "void launch_fused_spmv_axpy(const int64_t* indptr, "
                       "const int64_t* indices, const double* data, const double* x, "
                       "const double* w, double* z, double alpha, double beta, int64_t M, "
                       "int64_t N, int64_t nnz)",
    "axpy": "void launch_axpy(const double* x, const double* w, double* z, double alpha, "
            "double beta, int64_t M)",
}


@pytest.mark.parametrize("name", sorted(EXPECTED_ABI))
def test_abi_signature_matches_reference(name):
    k = _run(standard_kernels()[name], Config(), "hip")
    sig, _args, _info = abi_of(k)
    assert sig == EXPECTED_ABI[name]


def test_abi_matches_header():
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = " ".join(open(os.path.join(here, "include", "tilegen_launch.h")).read().split())
    for name in ("spmv", "spmm", "sddmm"):
        assert " ".join(EXPECTED_ABI[name].split()) in text.replace("( ", "(").replace(
            "void launch_%s(" % name, "void launch_%s(" % name)


# --------------------------------------------------------------------------- #
# HIP emitter structure
# --------------------------------------------------------------------------- #
def _hip(name, cfg, skip=()):
    return emit_hip(_run(standard_kernels()[name], cfg, "hip", skip), cfg)


def test_hip_markers():
    src = _hip("spmv", Config(tile_size=32, threads_per_row=4, unroll=4, block_size=256))
    for marker in ('extern "C" __global__', "__launch_bounds__(256)", "spmv_kernel",
                   "tg_segsum<4>", "#pragma unroll", "__shared__ tg_i64 s_ptr[33]",
                   "__builtin_nontemporal_load", "tg_i64x2"):
        assert marker in src, marker
    assert "__shfl_down_sync" not in src and "cuda" not in src.lower()


def test_hip_no_reduction_when_one_lane_per_row():
    src = _hip("spmv", Config(tile_size=128, threads_per_row=1, unroll=2, block_size=128))
    body = _code(src).split("tg_uniform(tg_i64 v)")[1]
    assert "acc[r] = tg_segsum" not in body
    # only the wave path for medium rows and the workgroup path for long rows
    # reduce across lanes
    assert body.count("tg_segsum<") == 2
    assert "macc = tg_segsum<64>(macc);" in body and "cacc = tg_segsum<64>(cacc);" in body


def test_hip_long_rows_leave_the_lane_group_only_when_tiled():
    # narrow lane groups: rows over 2 steps go to a wave, over 4 wave steps to
    # the workgroup
    cfg = Config(tile_size=64, threads_per_row=4, unroll=2, block_size=256)
    tiled = _hip("spmv", cfg)
    # over 2 steps of 4 lanes x 2 nonzeros and over twice the tile's average row,
    # or over 8 steps outright
    assert "coop[r] = len > 16 && (len * t_rows > 2 * t_nnz || len > 64);" in tiled
    assert "const tg_i64 t_nnz = s_ptr[64] - s_ptr[0];" in tiled
    assert "if (re[r] - rs[r] > 512) s_long[atomicAdd(&s_nlong, 1)] = lr;" in tiled
    assert "else s_med[atomicAdd(&s_nmed, 1)] = lr;" in tiled
    assert "for (int k = wv; k < n_med; k += 4)" in tiled  # medium rows spread over the waves
    untiled = _hip("spmv", cfg, skip=("tiling",))
    assert "s_long[" not in untiled and "s_med[" not in untiled
    # lane groups of 32 or more go straight to the workgroup after 8 steps
    wide = _hip("spmv", Config(tile_size=32, threads_per_row=32, unroll=2, block_size=1024))
    assert "coop[r] = re[r] - rs[r] > 512;" in wide and "s_med[" not in wide
    assert "if (lane == 0) s_long[atomicAdd(&s_nlong, 1)] = lr;" in wide


def test_skipping_tiling_changes_hip_and_cpu_code():
    cfg = Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256)
    k = standard_kernels()["spmv"]
    assert _code(_hip("spmv", cfg)) != _code(_hip("spmv", cfg, skip=("tiling",)))
    assert "s_ptr" not in _hip("spmv", cfg, skip=("tiling",))
    assert _code(emit_cpu(_run(k, cfg), cfg)) != _code(emit_cpu(_run(k, cfg, skip=("tiling",)),
                                                                cfg))


def test_skipping_thread_mapping_changes_hip_code():
    cfg = Config(tile_size=32, threads_per_row=4, unroll=1, block_size=128)
    full = _hip("spmv", cfg)
    ablated = _hip("spmv", cfg, skip=("thread_mapping",))
    assert "tg_segsum<4>(acc[r])" in full
    assert "tg_segsum<4>(acc[r])" not in ablated
    assert _code(full) != _code(ablated)


def test_noop_passes_emit_identical_hip_code():
    cfg = Config(tile_size=32, threads_per_row=1, unroll=1, block_size=256)
    full = _code(_hip("spmv", cfg))
    for name in ("canonicalize", "loop_fusion", "vectorize", "dead_code_elim"):
        assert _code(_hip("spmv", cfg, skip=(name,))) == full, name


def test_hip_vectorize_changes_spmm_and_sddmm():
    for name in ("spmm", "sddmm"):
        v1 = _hip(name, Config(tile_size=8, threads_per_row=16, unroll=2, vector_width=1,
                               block_size=256))
        v2 = _hip(name, Config(tile_size=8, threads_per_row=16, unroll=2, vector_width=2,
                               block_size=256))
        assert "vec_ok" in v2 and "tg_f64x2" in _code(v2).split("void %s_kernel" % name)[1]
        assert "vec_ok" not in v1


def test_hip_wave_uniform_spmm_path():
    src = _hip("spmm", Config(tile_size=4, threads_per_row=64, unroll=4, block_size=256))
    assert "__builtin_amdgcn_readfirstlane(threadIdx.x / 64)" in src
    assert "tg_uniform(indptr[row])" in src


def test_hip_injected_bug_stops_one_row_short():
    good = _hip("spmv", Config(tile_size=32, threads_per_row=4, unroll=2))
    bad = emit_hip(_run(standard_kernels()["spmv"],
                        Config(tile_size=32, threads_per_row=4, unroll=2, inject_bug=True),
                        "hip"), Config(tile_size=32, threads_per_row=4, unroll=2,
                                       inject_bug=True))
    assert "const tg_i64 row_end = M;" in good
    assert "const tg_i64 row_end = (M - 1);" in bad


def test_launch_geometry_covers_every_row():
    for cfg, rows_per_block in (
            (Config(tile_size=32, threads_per_row=4, unroll=4, block_size=256), 32),
            # tile_size 1 = no Tile transform: one row per lane group
            (Config(tile_size=1, threads_per_row=4, unroll=1, block_size=128), 32),
            (Config(tile_size=256, threads_per_row=1, unroll=4, block_size=256), 256)):
        k = _run(standard_kernels()["spmv"], cfg, "hip")
        geo = launch_geometry(_plan(k), _lowering(k))
        assert geo.rows_per_block == rows_per_block
        assert geo.grid(1000) * geo.rows_per_block >= 1000
        host = emit_hip_host(k, cfg)
        assert "(rows + %d - 1) / %d" % (rows_per_block, rows_per_block) in host
    sd = _run(standard_kernels()["sddmm"], Config(tile_size=8, threads_per_row=4,
                                                   block_size=256), "hip")
    assert launch_geometry(_plan(sd), _lowering(sd)).rows_per_block == 8
    # untiled SDDMM: one row per lane group, as for SpMV
    untiled = _run(standard_kernels()["sddmm"], Config(threads_per_row=4, block_size=256),
                   "hip", skip=("tiling",))
    assert launch_geometry(_plan(untiled), _lowering(untiled)).rows_per_block == 64


@pytest.mark.parametrize("bad", [Config(block_size=96), Config(threads_per_row=3),
                                 Config(block_size=2048), Config(tile_size=5000),
                                 Config(unroll=32)])
def test_hip_rejects_illegal_schedules(bad):
    with pytest.raises(ValueError):
        _hip("spmv", bad)


def test_generate_names_and_writes(tmp_path):
    gen = generate(standard_kernels()["sddmm"], Config(), "hip", outdir=str(tmp_path))
    assert os.path.exists(tmp_path / gen.filename)
    assert gen.filename.startswith("sddmm_%s_" % Config().hash()) and gen.filename.endswith(".hip")
    assert gen.abi_signature.startswith("void launch_sddmm")
    assert "{CODE_OBJECT}" in gen.host_source and "launch_sddmm" in gen.host_source
    assert gen.device_symbol == "sddmm_kernel"
    cpu = generate(standard_kernels()["axpy"], Config(), "cpu", outdir=str(tmp_path))
    assert cpu.filename.endswith(".cpp") and cpu.abi_signature.startswith("void launch_axpy")
    with pytest.raises(ValueError):
        generate(standard_kernels()["spmv"], Config(), "cuda", outdir=str(tmp_path))


def test_config_hash_closed_form():
    import hashlib
    c = Config(tile_size=64, threads_per_row=8, unroll=2, vector_width=1, block_size=128)
    assert c.hash() == hashlib.sha1(b"64|8|2|1|128|f64|0").hexdigest()[:10]
    assert Config().hash() != Config(inject_bug=True).hash()


# --------------------------------------------------------------------------- #
# CPU emitter (the OpenMP baseline)
# --------------------------------------------------------------------------- #
def test_cpu_tiling_and_unroll_change_source():
    k = standard_kernels()["spmv"]
    base = emit_cpu(_run(k, Config(tile_size=1)), Config(tile_size=1))
    tiled = emit_cpu(_run(k, Config(tile_size=64)), Config(tile_size=64))
    assert "i_o" not in base and "i_o" in tiled
    one = emit_cpu(_run(k, Config(unroll=1)), Config(unroll=1))
    four = emit_cpu(_run(k, Config(unroll=4)), Config(unroll=4))
    assert four.count("acc += ") > one.count("acc += ")
    assert "#pragma omp parallel for schedule(dynamic, 256)" in base


def test_cpu_simd_pragma_sits_on_its_loop():
    cfg = Config(tile_size=32, unroll=2, vector_width=2)
    src = emit_cpu(_run(standard_kernels()["spmm"], cfg), cfg)
    lines = [l.strip() for l in src.splitlines()]
    i = lines.index("#pragma omp simd")
    assert lines[i + 1].startswith("for (")


def test_spmm_sddmm_long_rows_relative_to_the_tile():
    """SpMM/SDDMM share a row with the workgroup only when it dwarfs its tile
    (more than 2x the average row) or is long outright; uniformly long rows
    stay with their lane groups."""
    spmm = _hip("spmm", Config(tile_size=16, threads_per_row=16, unroll=2, vector_width=2,
                               block_size=64))
    assert "((re - rs) > 32 && ((re - rs) * t_rows > 2 * t_nnz || (re - rs) > 128))" in spmm
    sddmm = _hip("sddmm", Config(tile_size=16, threads_per_row=8, unroll=4, vector_width=2,
                                 block_size=128))
    assert "((len) > 64 && ((len) * t_rows > 2 * t_nnz || (len) > 128))" in sddmm
    assert "s_tnnz = t_end > row0 ? indptr[t_end] - indptr[row0] : 0;" in sddmm



# --------------------------------------------------------------------------- #
# SpMM long-row combine: the emitted fixed-order tree over the lane groups'
# partial C-row slices, executed here on integers
# --------------------------------------------------------------------------- #
_TREE = re.compile(r"for \(int e = threadIdx\.x; e < (\d+); e \+= (\d+)\) "
                   r"s_part\[e\] \+= s_part\[e \+ (\d+)\];")


def _tree_groups(src):
    """Each combine (one per vector width) as its list of (limit, offset)."""
    groups, cur = [], None
    for line in src.splitlines():
        if "fixed-order tree over the lane groups' partial slices" in line:
            cur = []
            groups.append(cur)
            continue
        m = _TREE.search(line)
        if m and cur is not None:
            cur.append((int(m.group(1)), int(m.group(3))))
    return groups


def _run_tree(steps, slots, cols, seed=0):
    """Execute the tree with the lanes' parallel semantics (every read sees
    the level's input); returns the first ``cols`` entries and the exact sums."""
    rng = np.random.default_rng(seed)
    part = [int(v) for v in rng.integers(-2**40, 2**40, size=slots * cols)]
    want = [sum(part[s * cols + c] for s in range(slots)) for c in range(cols)]
    for limit, off in steps:
        assert limit + off <= slots * cols
        assert limit <= off, "a level reads what it writes"
        part = [part[e] + part[e + off] if e < limit else part[e] for e in range(len(part))]
    return part[:cols], want


@pytest.mark.parametrize("block,tpr", [(64, 64), (192, 64), (320, 8), (448, 16), (576, 32),
                                       (960, 64), (1024, 8), (384, 4), (704, 1)])
def test_spmm_long_row_tree_sums_every_slice(block, tpr):
    """Block sizes whose lane-group count is not a power of two (3, 5, 7 ...
    waves) keep every slice: the tree folds the upper ceil(n/2) slices onto the
    lower floor(n/2) at each level."""
    cfg = Config(tile_size=2 * (block // tpr), threads_per_row=tpr, unroll=1, vector_width=2,
                 block_size=block)
    groups = _tree_groups(_hip("spmm", cfg))
    assert len(groups) == 2  # 128-bit and scalar paths
    slots = block // tpr
    for steps, cols in zip(groups, (2 * tpr, tpr)):
        got, want = _run_tree(steps, slots, cols)
        assert got == want, (block, tpr, cols)


def test_tree_simulation_catches_a_dropped_slice():
    """The power-of-two halving (n //= 2) loses the middle slice of 3."""
    cols, slots = 4, 3
    halving = [(1 * cols, 1 * cols)]  # 3 // 2 = 1 level
    got, want = _run_tree(halving, slots, cols)
    assert got != want


@pytest.mark.parametrize("dtype", ["f32", "float", "f16"])
def test_hip_refuses_non_f64_accumulator(dtype):
    cfg = Config(tile_size=32, threads_per_row=4, unroll=2, block_size=256, dtype=dtype)
    with pytest.raises(ValueError, match="float64 only"):
        _hip("spmv", cfg)
    with pytest.raises(ValueError, match="float64 only"):
        generate(standard_kernels()["spmm"], cfg, "hip", write=False)
    # the CPU backend declares its accumulator in that type, as the reference does
    if dtype != "f16":
        src = generate(standard_kernels()["spmv"], cfg, "cpu", write=False).source
        assert "float acc" in src


def test_hip_verify_reports_non_f64_as_compile_error(tmp_path):
    from tilegen_amd.verify import verify
    from tests.util import mixed_257
    r = verify("spmv", Config(dtype="f32"), mixed_257(), backend="hip", workdir=str(tmp_path))
    assert not r.ok and "float64 only" in r.message


@pytest.mark.parametrize("balance,ordered", [("rows", False), ("nnz", True), ("hybrid", True),
                                             ("stream", True)])
def test_scratch_modules_launch_in_order(balance, ordered):
    """Merge-path, hybrid and stream modules share one scratch per device: their
    launchers order each launch after the previous one on any stream."""
    cfg = Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256, balance=balance)
    for name in ("spmv", "fused_spmv_axpy"):
        k = _run(standard_kernels()[name], cfg, "hip")
        host = emit_hip_host(k, cfg)
        async_fn = host.split("int tgv_launch_async(")[1].split("\n}\n")[0]
        assert ("tg_launch_ordered(tg_code, fn," in async_fn) == ordered
        assert ("return tg_launch(fn," in async_fn) == (not ordered)
        assert ("tg_mp_part" in emit_hip(k, cfg)) == ordered


@pytest.mark.parametrize("balance", ["nnz", "hybrid", "stream"])
def test_scratch_argument_form_of_scratch_modules(balance):
    """scratch_arg: the same kernel with its slots as a last parameter and no
    module array; refused for variants that combine nothing."""
    cfg = Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256, balance=balance)
    k = _run(standard_kernels()["spmv"], cfg, "hip")
    mod, arg = emit_hip(k, cfg), emit_hip(k, cfg, scratch_arg=True)
    assert "__device__ unsigned long long tg_mp_part[" in mod
    assert "tg_mp_part" not in arg
    assert "unsigned long long* __restrict__ tg_part)" in arg
    assert "unsigned long long* const tg_part = tg_mp_part;" in mod
    assert "tg_mp_commit(tg_part," in arg

    def code(t):  # the lines that do not name where the slots come from
        t = t.replace(", unsigned long long* __restrict__ tg_part)", ")")
        return [l for l in t.splitlines()
                if "tg_mp_part" not in l and not l.lstrip().startswith("//")]
    assert code(mod) == code(arg)
    rows = Config(tile_size=64, threads_per_row=4)
    with pytest.raises(ValueError, match="scratch_arg"):
        emit_hip(_run(standard_kernels()["spmv"], rows, "hip"), rows, scratch_arg=True)


def test_noalloc_kernel_source_geometry():
    from tilegen_amd.build import noalloc_kernel_source
    from tilegen_amd.codegen import MERGE_CAP
    from tilegen_amd.schedules import NOALLOC_SCHEDULE
    src = noalloc_kernel_source()
    cfg = NOALLOC_SCHEDULE
    chunk = 2 * cfg.block_size * cfg.unroll
    assert "#define TG_NA_CHUNK %d " % chunk in src
    assert "#define TG_NA_SLOTS %d " % (2 * MERGE_CAP) in src
    assert "#define TG_NA_MAX_NNZ %dLL" % (MERGE_CAP * chunk) in src
    assert "#define TG_NA_BLOCK %d" % cfg.block_size in src
    assert "__device__ unsigned long long tg_mp_part[" not in src


def test_stream_tile_through_passes_and_ir():
    """balance="stream" lowers to Tile(i, T, by=stream): the tiling pass logs the
    nonzero split, the IR round-trips it, and the schedule's name and hash carry
    it without touching a reference schedule's."""
    from tilegen_amd.ir import Kernel, Tile
    cfg = Config(tile_size=128, threads_per_row=4, unroll=4, block_size=512, balance="stream")
    k = _run(standard_kernels()["spmv"], cfg, "hip")
    tiles = [t for t in k.schedule if isinstance(t, Tile)]
    assert len(tiles) == 1 and tiles[0].by == "stream"
    assert "by=stream" in k.pretty()
    log = [r for r in k.pass_log if r["pass"] == "tiling"][0]["action"]
    assert "equal range of nonzeros" in log
    again = Kernel.from_dict(k.to_dict())
    assert [t for t in again.schedule if isinstance(t, Tile)][0].by == "stream"
    assert cfg.short().endswith("/stream") and cfg.to_dict()["balance"] == "stream"
    plain = Config(tile_size=128, threads_per_row=4, unroll=4, block_size=512)
    assert cfg.hash() != plain.hash() and "balance" not in plain.to_dict()
    gen = generate(standard_kernels()["spmv"], cfg, "hip", write=False)
    assert gen.geometry.stream and gen.geometry.nnz_chunk == 2048
    assert "grid = floor(nnz / 2048) + 1" in gen.source


def test_lane_group_rows_load_before_any_gather():
    """A lane group owning several rows of its tile (1 < R, R U <= 8, as c2's
    schedule) issues every row's first-step loads, then every row's gathers outside any
    per-lane condition (positions outside a row gather x[0] and are masked,
    under a uniform ghi > glo: the tile holds nonzeros), then the sums; one row
    per lane group (c1's schedule) keeps the single guarded step."""
    from tilegen_amd.schedules import TUNED
    src = generate(standard_kernels()["spmv"], TUNED["c2"], "hip", write=False).source
    loads = src.index("// first step of every row: every row's loads")
    guard = src.index("if (ghi > glo) {", loads)
    gather = src.index("fxv[r][u] = x[cu];", guard)
    sums = src.index("acc[r] = fok[r][u] ?", gather)
    rest = src.index("// remaining steps", sums)
    assert loads < guard < gather < sums < rest
    # the loads sit in the per-lane guarded block, the gathers do not
    assert src.count("if (q < re[r] && rs[r] < re[r])", loads, guard) == 1
    assert "if (q < re[r]" not in src[guard:sums]
    one = generate(standard_kernels()["spmv"],
                   Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128), "hip",
                   write=False).source
    assert "every row's loads" not in one
    assert "// first step of every row in flight before any accumulation" in one
    # past R U = 8 the operands of every row would not fit in registers: one step per row
    big = generate(standard_kernels()["spmv"],
                   Config(tile_size=256, threads_per_row=64, unroll=4, block_size=256), "hip",
                   write=False).source
    assert "every row's loads" not in big

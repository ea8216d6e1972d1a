"""GPU parity: every HIP variant against the C oracle and float64 SciPy.

All launches go through the variant library's C ABI ``launch_<name>`` with
device pointers.  The bar: normwise relative error <= 1e-10 (inf- and 2-norm)
against both checkers, the reference tolerance from verify(), and indptr /
indices byte-identical after the launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from tests.util import csr, mixed_257, ragged, rel_2, rel_inf
from tilegen_amd.codegen import Config
from tilegen_amd.matrices import make_baseline
from tilegen_amd.schedules import (ODD_BLOCK_SCHEDULES, TEST_KERNELS, TEST_SCHEDULES,
                                   schedule_id)
from tilegen_amd import runtime as rt
from tilegen_amd.variant import Variant, operand_order
from tilegen_amd.verify import _inputs_for, _reference, verify

pytestmark = pytest.mark.gpu

TOL = 1e-10  # normwise relative error bar


def _operands(kernel, A, K, seed=7):
    x, w, B, U, V, alpha, beta = _inputs_for(kernel, A, K, seed)
    return {"x": x, "w": w, "B": B, "U": U, "V": V, "alpha": alpha, "beta": beta}


def _oracle(kernel, A, ops):
    if kernel == "axpy":
        return oracle.axpy(ops["x"], ops["w"], ops["alpha"], ops["beta"])
    return oracle.compute(kernel, A, ops)


def _check(kernel, cfg, A, K, label=""):
    ops = _operands(kernel, A, K)
    v = Variant(kernel, cfg)
    if kernel == "axpy":
        out = v.run(None, x=ops["x"], w=ops["w"], alpha=ops["alpha"], beta=ops["beta"])
    else:
        out = v.run(A, **ops)
    want = _oracle(kernel, A, ops)
    sci = _reference(kernel, A, (ops["x"], ops["w"], ops["B"], ops["U"], ops["V"],
                                 ops["alpha"], ops["beta"]))
    for name, ref in (("oracle", want), ("scipy", sci)):
        ri, r2 = rel_inf(out, ref), rel_2(out, ref)
        assert ri <= TOL and r2 <= TOL, "%s %s %s vs %s: rel_inf=%g rel_2=%g" % (
            kernel, cfg.short(), label, name, ri, r2)
    return out


@pytest.mark.parametrize("kernel", TEST_KERNELS)
@pytest.mark.parametrize("cfg", TEST_SCHEDULES, ids=[schedule_id(c) for c in TEST_SCHEDULES])
def test_verify_matches_float64_reference(kernel, cfg, hip_ready, tmp_path):
    r = verify(kernel, cfg, mixed_257(), backend="hip", workdir=str(tmp_path), K=8)
    assert r.executed, r.message
    assert r.ok, "%s %s: %s" % (kernel, cfg.short(), r.message)
    assert r.max_abs_err <= r.tolerance
    assert r.rel_err_inf <= TOL and r.rel_err_2 <= TOL
    if kernel != "axpy":
        assert r.structure_intact is True


@pytest.mark.parametrize("kernel", TEST_KERNELS)
@pytest.mark.parametrize("cfg", TEST_SCHEDULES, ids=[schedule_id(c) for c in TEST_SCHEDULES])
def test_matches_oracle_k64(kernel, cfg, hip_ready):
    _check(kernel, cfg, mixed_257(), K=64)


@pytest.mark.parametrize("kernel", ["spmm", "sddmm"])
@pytest.mark.parametrize("K", [1, 7, 63, 130, 1024, 2049])
def test_odd_and_wide_K(kernel, K, hip_ready):
    """K not a multiple of the vector width (scalar fallback) and K wider than
    one pass of the lanes, up to many passes (1024, and 2049 odd)."""
    for cfg in (Config(tile_size=8, threads_per_row=32, unroll=4, vector_width=2,
                       block_size=256),
                Config(tile_size=4, threads_per_row=4, unroll=2, vector_width=2,
                       block_size=256),
                Config(tile_size=16, threads_per_row=8, unroll=4, vector_width=2,
                       block_size=128)):
        _check(kernel, cfg, mixed_257(), K=K, label="K=%d" % K)


@pytest.mark.parametrize("kernel", TEST_KERNELS)
def test_injected_bug_is_caught(kernel, hip_ready, tmp_path):
    cfg = Config(tile_size=32, threads_per_row=4, unroll=2, vector_width=1, block_size=256,
                 inject_bug=True)
    r = verify(kernel, cfg, mixed_257(), backend="hip", workdir=str(tmp_path), K=8)
    assert r.executed and "compile error" not in r.message, r.message
    assert not r.ok, "%s: injected bug not detected" % kernel
    assert r.max_abs_err > r.tolerance


@pytest.mark.parametrize("balance", ["nnz", "hybrid", "stream"])
@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy"])
def test_injected_bug_is_caught_in_balanced_forms(kernel, balance, hip_ready, tmp_path):
    """The reference's bug injection (the last row is never written) in the
    merge-path, hybrid and stream forms: verify() must fail it."""
    cfg = Config(tile_size=32, threads_per_row=4, unroll=2, vector_width=1, block_size=256,
                 inject_bug=True, balance=balance)
    r = verify(kernel, cfg, mixed_257(), backend="hip", workdir=str(tmp_path), K=8)
    assert r.executed and "compile error" not in r.message, r.message
    assert not r.ok, "%s %s: injected bug not detected" % (kernel, balance)
    assert r.max_abs_err > r.tolerance


@pytest.mark.parametrize("kernel", TEST_KERNELS)
@pytest.mark.parametrize("cfg", ODD_BLOCK_SCHEDULES,
                         ids=[schedule_id(c) for c in ODD_BLOCK_SCHEDULES])
def test_block_sizes_not_a_power_of_two(kernel, cfg, hip_ready):
    """3, 5 and 7 waves per workgroup; rows long enough to leave their lane
    group, so SpMM's long-row tree combines 3, 28, 40 and 96 slices."""
    long_rows = ragged(8, 2500, 2500, 6, empty_every=7,
                       long_rows=[(5, 2000), (150, 700), (2499, 129)])
    for label, A in (("mixed_257", mixed_257()), ("long_rows", long_rows)):
        print("[gpu] odd-block %s %s %s" % (kernel, cfg.short(), label), flush=True)
        _check(kernel, cfg, A, K=64, label=label)


SPMV_CFGS = [
    Config(tile_size=128, threads_per_row=8, unroll=2, block_size=256),
    Config(tile_size=64, threads_per_row=64, unroll=4, block_size=256),
    Config(tile_size=256, threads_per_row=1, unroll=3, block_size=256),
    Config(tile_size=32, threads_per_row=16, unroll=1, block_size=64),
]


@pytest.mark.parametrize("cfg", SPMV_CFGS, ids=[schedule_id(c) for c in SPMV_CFGS])
def test_edge_cases_spmv(cfg, hip_ready):
    cases = {
        "no_nonzeros": csr(100, 50, np.zeros(101, dtype=np.int64), [], []),
        "single": csr(1, 1, [0, 1], [0], [2.5]),
        "one_long_row": ragged(3, 300, 40000, 0, long_rows=[(150, 25000)]),
        "long_and_short": ragged(4, 2000, 6000, 9, empty_every=5,
                                 long_rows=[(0, 5000), (1999, 3001), (777, 1)]),
        "last_row_to_nnz_end": csr(3, 5, [0, 1, 2, 7], [0, 1, 0, 1, 2, 3, 4],
                                   [1, 2, 3, 4, 5, 6, 7]),
    }
    for label, A in cases.items():
        _check("spmv", cfg, A, K=1, label=label)


def test_zero_rows(hip_ready):
    A = sp.csr_matrix((np.zeros(0), np.zeros(0, dtype=np.int64), np.zeros(1, dtype=np.int64)),
                      shape=(0, 4))
    v = Variant("spmv", Config(tile_size=128, threads_per_row=8, unroll=2, block_size=256))
    out = v.run(A, x=np.ones(4))
    assert out.shape == (0,)


def test_spmm_overwrites_output(hip_ready):
    """C is output-only: prior contents (even NaN) never leak into the result."""
    A = mixed_257()
    ops = _operands("spmm", A, 64)
    v = Variant("spmm", Config(tile_size=8, threads_per_row=32, unroll=4, vector_width=2,
                               block_size=256))
    out = v.run(A, out=np.full((A.shape[0], 64), np.nan), B=ops["B"])
    assert np.isfinite(out).all()
    assert rel_inf(out, oracle.spmm(A, ops["B"])) <= TOL


def test_sddmm_empty_rows_and_long_rows(hip_ready):
    A = ragged(9, 500, 700, 40, empty_every=3, long_rows=[(10, 600)])
    for cfg in (Config(tile_size=4, threads_per_row=4, unroll=2, vector_width=2, block_size=256),
                Config(tile_size=1, threads_per_row=64, unroll=1, vector_width=1, block_size=64)):
        _check("sddmm", cfg, A, K=64)


SKEW_CFGS = [
    Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128),
    Config(tile_size=64, threads_per_row=1, unroll=1, block_size=64),     # long = 8 nonzeros
    Config(tile_size=32, threads_per_row=4, unroll=3, block_size=256),
    Config(tile_size=16, threads_per_row=64, unroll=4, block_size=1024),
    # workgroups of 3 and 5 waves: the waves' partial sums of a listed row are added in
    # wave order over a count that is not a power of two; T96/TPR4/U2/B192 also takes the
    # multi-row first step (two rows per lane group)
    Config(tile_size=96, threads_per_row=4, unroll=2, block_size=192),
    Config(tile_size=40, threads_per_row=8, unroll=2, block_size=320),
]


@pytest.mark.parametrize("cfg", SKEW_CFGS, ids=[schedule_id(c) for c in SKEW_CFGS])
@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy"])
def test_skewed_rows_workgroup_path(kernel, cfg, hip_ready):
    """Rows longer than 8 lane-group steps go to the whole workgroup: one
    enormous row, many long rows in one tile, long rows at the matrix end."""
    cases = {
        "power_law_small": make_baseline("c3a", scale=0.05),
        "every_row_long": ragged(21, 200, 3000, 0, long_rows=[(r, 300 + r) for r in range(200)]),
        "mixed": ragged(22, 3000, 8000, 6, empty_every=4,
                        long_rows=[(0, 7000), (1, 9), (1500, 4000), (2998, 2500), (2999, 33)]),
    }
    for label, A in cases.items():
        _check(kernel, cfg, A, K=1, label=label)


CHUNK_CFGS = [
    Config(tile_size=16, threads_per_row=16, unroll=2, vector_width=2, block_size=256),
    Config(tile_size=8, threads_per_row=64, unroll=1, vector_width=1, block_size=128),
    Config(tile_size=64, threads_per_row=4, unroll=8, vector_width=2, block_size=256),
    Config(tile_size=32, threads_per_row=1, unroll=16, vector_width=2, block_size=64),
    # workgroups of 3 and 5 waves, whose lane groups share out listed rows' chunks
    Config(tile_size=24, threads_per_row=8, unroll=4, vector_width=2, block_size=192),
    Config(tile_size=80, threads_per_row=4, unroll=8, vector_width=2, block_size=320),
]


@pytest.mark.parametrize("cfg", CHUNK_CFGS, ids=[schedule_id(c) for c in CHUNK_CFGS])
def test_sddmm_chunked_path(cfg, hip_ready):
    """K covered by one lane group's registers: lane groups own adjacent rows,
    chunks of TPR nonzeros with broadcast column indices.  Dense 4x4 blocks
    (rows sharing columns), rows of different lengths in one wave, rows longer
    than several chunks, empty rows, K below the register capacity."""
    cases = {
        "blocked": make_baseline("c5", scale=0.01),
        "ragged": ragged(31, 700, 900, 37, empty_every=5, long_rows=[(3, 500), (4, 65)]),
    }
    for label, A in cases.items():
        for K in (64, 40, 2):
            _check("sddmm", cfg, A, K=K, label="%s K=%d" % (label, K))


SPMM_SKEW_CFGS = [
    Config(tile_size=16, threads_per_row=16, unroll=2, vector_width=2, block_size=64),
    Config(tile_size=32, threads_per_row=8, unroll=2, vector_width=2, block_size=128),
    Config(tile_size=8, threads_per_row=64, unroll=4, vector_width=2, block_size=256),
    Config(tile_size=256, threads_per_row=4, unroll=1, vector_width=1, block_size=1024),
    # lane-group counts that are not powers of two (3 and 40): the long rows' partial
    # C-row slices are added by a tree over an odd count
    Config(tile_size=12, threads_per_row=64, unroll=1, vector_width=1, block_size=192),
    Config(tile_size=40, threads_per_row=8, unroll=2, vector_width=2, block_size=320),
]


@pytest.mark.parametrize("cfg", SPMM_SKEW_CFGS, ids=[schedule_id(c) for c in SPMM_SKEW_CFGS])
def test_spmm_skewed_rows_workgroup_path(cfg, hip_ready):
    """Rows longer than 16*U nonzeros go to the whole workgroup (strided shares,
    fixed-order LDS tree): one enormous row, every row long, long rows at the
    matrix end; K = 64 (128-bit path), 7 (scalar path) and 130 (several
    K-slices)."""
    cases = {
        "power_law_small": make_baseline("c3a", scale=0.03),
        "every_row_long": ragged(23, 96, 2000, 0, long_rows=[(r, 100 + 3 * r) for r in range(96)]),
        "mixed": ragged(24, 1500, 4000, 6, empty_every=4,
                        long_rows=[(0, 3500), (1, 17), (750, 2000), (1498, 900), (1499, 33)]),
    }
    for label, A in cases.items():
        for K in (64, 7, 130):
            _check("spmm", cfg, A, K=K, label="%s K=%d" % (label, K))


SDDMM_WIDE_CFGS = [
    Config(tile_size=16, threads_per_row=4, unroll=2, vector_width=2, block_size=256),
    Config(tile_size=8, threads_per_row=16, unroll=1, vector_width=1, block_size=128),
    Config(tile_size=64, threads_per_row=64, unroll=2, vector_width=2, block_size=1024),
    Config(tile_size=12, threads_per_row=16, unroll=1, vector_width=1, block_size=192),
]


@pytest.mark.parametrize("cfg", SDDMM_WIDE_CFGS, ids=[schedule_id(c) for c in SDDMM_WIDE_CFGS])
def test_sddmm_wide_k_skewed_rows(cfg, hip_ready):
    """K wider than one lane group's registers (one wave per row): rows that
    dwarf their tile are shared by every wave of the workgroup."""
    cases = {
        "power_law_small": make_baseline("c3a", scale=0.03),
        "mixed": ragged(25, 1200, 3000, 5, empty_every=4,
                        long_rows=[(0, 2500), (1, 300), (600, 1200), (1199, 700)]),
    }
    for label, A in cases.items():
        for K in (130, 257):
            _check("sddmm", cfg, A, K=K, label="%s K=%d" % (label, K))


class _View(rt.DeviceBuffer):
    """A device pointer into another buffer (a caller's sub-buffer); the base
    buffer owns the memory."""

    def __init__(self, base: rt.DeviceBuffer, offset: int, nbytes: int):
        self.array, self.nbytes, self.ptr, self._base = None, nbytes, base.ptr + offset, base

    def free(self) -> None:
        self.ptr = 0


GUARD = -7.25e300


def _guarded(arr: np.ndarray):
    """``arr`` placed 8 bytes into an allocation (so only 8-byte aligned), with
    one guard element on each side; returns (base, view)."""
    a = np.ascontiguousarray(arr).ravel()
    dt = a.dtype
    guard = np.array([GUARD], dtype=np.float64).view(dt) if dt.itemsize == 8 else None
    base = rt.DeviceBuffer(np.concatenate([guard, a, guard]))
    return base, _View(base, 8, a.nbytes)


OFFSET_CASES = [
    ("spmv", Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128)),
    ("spmv", Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256)),
    ("spmv", Config(tile_size=4, threads_per_row=64, unroll=2, block_size=256)),
    ("fused_spmv_axpy", Config(tile_size=128, threads_per_row=4, unroll=2, block_size=256)),
    ("spmm", Config(tile_size=16, threads_per_row=16, unroll=2, vector_width=2, block_size=64)),
    ("spmm", Config(tile_size=4, threads_per_row=64, unroll=2, vector_width=2, block_size=256)),
    ("sddmm", Config(tile_size=16, threads_per_row=8, unroll=4, vector_width=2, block_size=128)),
    ("sddmm", Config(tile_size=8, threads_per_row=16, unroll=2, vector_width=2, block_size=128)),
    ("axpy", Config(tile_size=64, threads_per_row=1, unroll=4, vector_width=2, block_size=256)),
    # the balanced forms: pair loads of ranges and pieces, commits of cut rows
    ("spmv", Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256, balance="hybrid")),
    ("spmv", Config(tile_size=128, threads_per_row=4, unroll=4, block_size=512, balance="stream")),
    ("spmv", Config(tile_size=64, threads_per_row=1, unroll=1, block_size=64, balance="stream")),
    ("fused_spmv_axpy", Config(tile_size=256, threads_per_row=4, unroll=4, block_size=1024,
                               balance="stream")),
]


@pytest.mark.parametrize("kernel,cfg", OFFSET_CASES,
                         ids=["%s-%s" % (k, schedule_id(c)) for k, c in OFFSET_CASES])
def test_operands_at_8_byte_offsets(kernel, cfg, hip_ready):
    """Every array argument (indptr, indices, data, dense operands, output)
    starts 8 bytes into its allocation, as a caller's sub-buffer can: the
    128-bit paths must notice and fall back, results must stay at the bar, and
    the guard elements either side of every array must be untouched."""
    A = ragged(26, 700, 900, 40, empty_every=6, long_rows=[(3, 800), (699, 500)])
    K = 64 if kernel in ("spmm", "sddmm") else 0
    ops = _operands(kernel, A, max(K, 1))
    M, N = A.shape
    host = {}
    if kernel != "axpy":
        host.update(indptr=A.indptr.astype(np.int64), indices=A.indices.astype(np.int64),
                    data=A.data.astype(np.float64))
    dense, scal, _ = operand_order(kernel)
    for d in dense:
        host[d] = np.asarray(ops[d], dtype=np.float64)
    out_name, out_shape = {"spmv": ("y", (M,)), "fused_spmv_axpy": ("z", (M,)),
                           "axpy": ("z", (M,)), "spmm": ("C", (M, K)),
                           "sddmm": ("C", (A.nnz,))}[kernel]
    host[out_name] = np.zeros(out_shape)
    if kernel == "axpy":
        host["x"], host["w"] = host["x"][:M], host["w"][:M]
    pairs = {k: _guarded(v) for k, v in host.items()}
    try:
        v = Variant(kernel, cfg)
        vals = v.abi_values(A, {k: p[1] for k, p in pairs.items()},
                            {s: float(ops[s]) for s in scal}, M, N, K, A.nnz)
        v.device_call(vals)
        for k, (base, _view) in pairs.items():
            full = base.to_host()
            assert full[:1].view(np.float64)[0] == GUARD, (k, "guard before")
            assert full[-1:].view(np.float64)[0] == GUARD, (k, "guard after")
            if k != out_name:
                assert full[1:-1].tobytes() == host[k].tobytes(), (k, "input modified")
        out = pairs[out_name][0].to_host()[1:-1].reshape(out_shape)
    finally:
        for base, view in pairs.values():
            view.free()
            base.free()
    if kernel == "axpy":
        want = oracle.axpy(host["x"], host["w"], ops["alpha"], ops["beta"])
    else:
        want = oracle.compute(kernel, A, {k: host.get(k, ops[k]) for k in ops})
    assert rel_inf(out, want) <= TOL and rel_2(out, want) <= TOL


@pytest.mark.parametrize("kernel", ["spmv", "spmm", "sddmm", "fused_spmv_axpy"])
def test_matrices_without_nonzeros(kernel, hip_ready):
    """No nonzeros at all (every row empty) and no rows: SpMV/SpMM outputs are
    all zero even when the output buffer starts with NaNs (written, not
    accumulated), SDDMM's output is empty, and verify() passes."""
    cfgs = (Config(tile_size=16, threads_per_row=8, unroll=2, vector_width=2, block_size=128),
            Config(tile_size=32, threads_per_row=1, unroll=1, vector_width=1, block_size=128))
    empty = csr(100, 50, np.zeros(101, dtype=np.int64), [], [])
    norows = csr(0, 50, np.zeros(1, dtype=np.int64), [], [])
    for A in (empty, norows):
        M, N = A.shape
        ops = _operands(kernel, A, 8)
        for cfg in cfgs:
            v = Variant(kernel, cfg)
            shape = {"spmv": (M,), "fused_spmv_axpy": (M,), "spmm": (M, 8), "sddmm": (0,)}[kernel]
            dense = {k: ops[k] for k in operand_order(kernel)[0] + operand_order(kernel)[1]}
            out = v.run(A, out=np.full(shape, np.nan), **dense)
            assert out.shape == tuple(shape)
            want = _oracle(kernel, A, ops).reshape(shape)
            assert np.array_equal(out, want), (kernel, cfg.short(), M)
            r = verify(kernel, cfg, A, backend="hip", K=8)
            assert r.ok, r.message


def _nonfinite_cases():
    from tilegen_amd.schedules import (HYBRID_TEST_SCHEDULES, MERGE_TEST_SCHEDULES,
                                       STREAM_TEST_SCHEDULES, TUNED)
    rows = [Config(tile_size=32, threads_per_row=1, unroll=1, block_size=128),
            Config(tile_size=64, threads_per_row=4, unroll=4, block_size=256),
            Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128),
            Config(tile_size=8, threads_per_row=64, unroll=2, block_size=256)]
    return (rows + MERGE_TEST_SCHEDULES[:3] + HYBRID_TEST_SCHEDULES[:3] +
            STREAM_TEST_SCHEDULES[:3] + [TUNED["c3a"], TUNED["c3b"]])


@pytest.mark.parametrize("cfg", _nonfinite_cases(), ids=[schedule_id(c) for c in
                                                          _nonfinite_cases()])
@pytest.mark.parametrize("kernel", ["spmv", "fused_spmv_axpy"])
def test_nonfinite_x_reaches_only_rows_that_use_it(kernel, cfg, hip_ready):
    """x[0] = NaN and x[5] = +Inf.  Lanes past a row's end gather x[0] so that
    every gather of a step is issued before any is used; their products must
    be dropped, not multiplied by zero (0 * NaN is NaN).  So exactly the rows
    that reference column 0 or 5 are non-finite, with SciPy's NaN/Inf pattern,
    and every other row meets the bar."""
    A = ragged(41, 3000, 2000, 40, empty_every=9,
               long_rows=[(17, 1900), (1500, 1300), (2999, 700)])
    ops = _operands(kernel, A, 1)
    x = ops["x"].copy()
    x[0], x[5] = np.nan, np.inf
    ops["x"] = x
    out = Variant(kernel, cfg).run(A, **ops)
    sci = _reference(kernel, A, (x, ops["w"], ops["B"], ops["U"], ops["V"],
                                 ops["alpha"], ops["beta"]))
    uses = np.zeros(A.shape[0], dtype=bool)
    coo = A.tocoo()
    uses[coo.row[(coo.col == 0) | (coo.col == 5)]] = True
    assert 0 < uses.sum() < A.shape[0] // 2
    assert np.array_equal(np.isnan(out), np.isnan(sci)), cfg.short()
    assert np.array_equal(np.isinf(out), np.isinf(sci)), cfg.short()
    assert np.array_equal(~np.isfinite(sci), uses)  # the rows that use them, and only those
    fin = np.isfinite(sci)
    assert rel_inf(out[fin], sci[fin]) <= TOL, cfg.short()

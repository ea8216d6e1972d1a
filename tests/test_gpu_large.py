"""64-bit addressing at sizes past 2^31 elements.

Every offset on the path is int64 (the reference ABI's ``int64_t`` indptr /
indices and dims).  These tests place nonzeros in columns past 2^31 (SpMV's x)
and rows of the dense operand whose element offset ``j * K`` passes 2^31
(SpMM's B, SDDMM's V), so a 32-bit product anywhere in the address arithmetic
would read the wrong element.  Each dense operand is about 17 GB of device
memory (MI355X has 288 GB), freed after the test.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from tests.util import rel_2, rel_inf
from tilegen_amd.codegen import Config
from tilegen_amd.variant import Variant

pytestmark = pytest.mark.gpu

TOL = 1e-10
BIG = (1 << 31) + 64


def _far_columns(M: int, N: int, per_row: int, seed: int) -> sp.csr_matrix:
    """Rows whose columns sit at both ends of [0, N), most of them past 2^31
    when N is that large."""
    rng = np.random.default_rng(seed)
    rows, cols = [], []
    for r in range(M):
        far = N - 1 - rng.choice(4096, size=per_row // 2, replace=False)
        near = rng.choice(4096, size=per_row - per_row // 2, replace=False)
        c = np.sort(np.concatenate([near, far]))
        rows.append(np.full(c.size, r))
        cols.append(c)
    rows, cols = np.concatenate(rows), np.concatenate(cols).astype(np.int64)
    data = rng.uniform(-1, 1, rows.size)
    return sp.csr_matrix((data, (rows, cols)), shape=(M, N))


def test_spmv_columns_past_2_31(hip_ready):
    A = _far_columns(300, BIG, 16, seed=1)
    assert A.indices.max() > (1 << 31)
    x = np.zeros(BIG)
    used = np.unique(A.indices)
    x[used] = np.random.default_rng(2).uniform(-1, 1, used.size)
    for cfg in (Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128),
                Config(tile_size=32, threads_per_row=1, unroll=1, block_size=64)):
        out = Variant("spmv", cfg).run(A, x=x)
        want = oracle.spmv(A, x)
        assert rel_inf(out, want) <= TOL and rel_2(out, want) <= TOL, cfg.short()


@pytest.mark.parametrize("kernel", ["spmm", "sddmm"])
def test_dense_row_offsets_past_2_31(kernel, hip_ready):
    K = 64
    N = (1 << 25) + 8  # j * K passes 2^31 for the last rows
    A = _far_columns(256, N, 16, seed=3)
    assert int(A.indices.max()) * K > (1 << 31)
    D = np.zeros((N, K))
    used = np.unique(A.indices)
    D[used] = np.random.default_rng(4).uniform(-1, 1, (used.size, K))
    cfg = Config(tile_size=16, threads_per_row=8, unroll=4, vector_width=2, block_size=128)
    if kernel == "spmm":
        out = Variant("spmm", cfg).run(A, B=D)
        want = oracle.spmm(A, D)
    else:
        U = np.random.default_rng(5).uniform(-1, 1, (A.shape[0], K))
        out = Variant("sddmm", cfg).run(A, U=U, V=D)
        want = oracle.sddmm(A, U, D)
    assert rel_inf(out, want) <= TOL and rel_2(out, want) <= TOL

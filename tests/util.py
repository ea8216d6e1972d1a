"""Shared helpers for the parity tests (matrices and error norms)."""

from __future__ import annotations

import numpy as np
import scipy.sparse as sp


def csr(rows, cols, indptr, indices, data) -> sp.csr_matrix:
    return sp.csr_matrix((np.asarray(data, dtype=np.float64), np.asarray(indices, dtype=np.int64),
                          np.asarray(indptr, dtype=np.int64)), shape=(rows, cols))


def mixed_257() -> sp.csr_matrix:
    """257 x 257, every 37th row empty, 1..24 sorted distinct columns per row,
    N(0,1) values from default_rng(2024) -- the construction of the reference's
    GPU test matrix (tests/test_cuda_gpu.py:53-76).  257 exceeds every tile
    and block size, so an undersized grid leaves rows unwritten."""
    rng = np.random.default_rng(2024)
    n = 257
    indptr, indices, data = [0], [], []
    for r in range(n):
        k = 0 if r % 37 == 0 else int(rng.integers(1, 25))
        if k:
            indices.extend(int(c) for c in np.sort(rng.choice(n, size=k, replace=False)))
            data.extend(float(v) for v in rng.standard_normal(k))
        indptr.append(len(indices))
    return csr(n, n, indptr, indices, data)


def ragged(seed: int, rows: int, cols: int, max_len: int, empty_every: int = 0,
           long_rows=()) -> sp.csr_matrix:
    """Random CSR with row lengths 0..max_len plus a few very long rows."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(0, max_len + 1, size=rows)
    if empty_every:
        lengths[::empty_every] = 0
    for r, L in long_rows:
        lengths[r] = min(L, cols)
    indptr = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(lengths, out=indptr[1:])
    indices = np.empty(int(indptr[-1]), dtype=np.int64)
    for r in range(rows):
        L = int(lengths[r])
        if L:
            indices[indptr[r]:indptr[r + 1]] = np.sort(rng.choice(cols, size=L, replace=False))
    data = rng.uniform(-1, 1, size=indices.size)
    return sp.csr_matrix((data, indices, indptr), shape=(rows, cols))


def range_edge_matrix(CH: int, seed: int = 0):
    """Rows at the edges of the hybrid range logic for ranges of CH nonzeros
    (long rows: over LH = CH / 2): lengths LH (not long), LH + 1, three LH + 1
    rows in a row (the most that can meet one range), CH and CH + 1, a row of
    several ranges, rows starting and ending exactly on range boundaries (short
    filler rows align them), with short and empty rows between."""
    rng = np.random.default_rng(seed)
    LH = CH // 2
    lens = []

    def pos():
        return int(sum(lens))

    def align_to(mult, off=0):
        # short filler rows (at most 3 nonzeros each) up to the next position
        # congruent to off modulo mult
        gap = (off - pos()) % mult
        while gap > 0:
            k = min(3, gap)
            lens.append(k)
            gap -= k

    for L in (LH, LH + 1, 0, 2, LH + 1, LH + 1, LH + 1, 1, 2 * LH - 1, CH, 0, CH + 1):
        lens.append(L)
        lens.extend(int(v) for v in rng.integers(0, 4, size=3))
    align_to(CH)
    lens.append(LH + 1)           # starts on a range boundary
    align_to(CH, off=CH - (LH + 1))
    lens.append(LH + 1)           # ends on a range boundary
    align_to(CH, off=CH // 4)
    lens.append(3 * CH + 7)       # four pieces
    lens.append(LH + 2)
    align_to(CH, off=CH - 1)
    lens.append(CH + 2)           # two pieces, one nonzero in the first range
    lens.extend(int(v) for v in rng.integers(0, 4, size=5))
    lens.append(LH + 1)           # the last row reaches nnz
    rows = len(lens)
    cols = 4 * CH + 16
    indptr = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(lens, out=indptr[1:])
    indices = np.empty(int(indptr[-1]), dtype=np.int64)
    for r, L in enumerate(lens):
        if L:
            indices[indptr[r]:indptr[r + 1]] = np.sort(rng.choice(cols, size=L, replace=False))
    return csr(rows, cols, indptr, indices, rng.uniform(-1, 1, size=indices.size))


def rel_inf(out, ref) -> float:
    out = np.asarray(out, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    if ref.size == 0:
        return 0.0
    n = float(np.abs(ref).max())
    e = float(np.abs(out - ref).max())
    return e / n if n > 0 else e


def rel_2(out, ref) -> float:
    out = np.asarray(out, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    if ref.size == 0:
        return 0.0
    n = float(np.linalg.norm(ref))
    e = float(np.linalg.norm(out - ref))
    return e / n if n > 0 else e

"""Deterministic CSR inputs: the reference corpus and the BASELINE configs.

Two families live here.

* The reference corpus (``make_matrix``/``build_corpus``), restating reference
  ``tilegen/matrices.py:49-279``: six classes, each drawn from
  ``numpy.random.default_rng(1234 + fold(name))`` with the same sequence of
  generator calls, so ``nnz``/max/mean/stddev reproduce the reference's
  ``data/matrices/manifest.json`` exactly.  Files: ``.npz`` (indptr, indices,
  data, shape, class_name) and the little-endian TGM1 ``.bin`` the reference's
  C++ harness reads.
* The five BASELINE configs (``make_baseline``): the graded inputs, which differ
  from the corpus (distinct columns per row, U(-1,1) values, K=64, 4x4 blocks).

All CSR matrices are canonical: int64 ``indptr``/``indices``, columns sorted
and unique within each row, float64 ``data``.
"""

from __future__ import annotations

import argparse
import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np
import scipy.sparse as sp

__all__ = [
    "SEED", "build_corpus", "make_matrix", "matrix_stats", "corpus_classes",
    "save_csr_npz", "load_csr_npz", "export_matrix_bin", "load_matrix_bin",
    "BaselineCase", "baseline_ids", "make_baseline", "baseline_operands",
    "compulsory_bytes", "flops", "main",
]

SEED = 1234

# TGM1 binary layout (little-endian), shared with the reference C++ harness
# (reference matrices.py:38-46, cpp/src/harness.cpp:36-55):
#   uint32 magic 0x54474D31 | int64 rows | int64 cols | int64 nnz |
#   int64 indptr[rows+1] | int64 indices[nnz] | float64 data[nnz]
_BIN_MAGIC = 0x54474D31


def _rng(name: str) -> np.random.Generator:
    """Per-class generator: the class name is folded into the seed so each
    matrix is reproducible independent of build order (reference
    ``matrices.py:49-54``)."""
    fold = sum((pos + 1) * ord(ch) for pos, ch in enumerate(name))
    return np.random.default_rng(SEED + fold)


def _canonical(rows: np.ndarray, cols: np.ndarray, vals: np.ndarray,
               shape: Tuple[int, int]) -> sp.csr_matrix:
    """COO triplets -> CSR with duplicates summed and columns sorted."""
    m = sp.coo_matrix((vals, (rows, cols)), shape=shape).tocsr()
    m.sum_duplicates()
    m.sort_indices()
    return _as_int64(m)


def _as_int64(m: sp.csr_matrix) -> sp.csr_matrix:
    m.indptr = m.indptr.astype(np.int64, copy=False)
    m.indices = m.indices.astype(np.int64, copy=False)
    m.data = m.data.astype(np.float64, copy=False)
    return m


# --------------------------------------------------------------------------- #
# reference corpus (the generator call sequence must match for the manifest pin)
# --------------------------------------------------------------------------- #
def _corpus_banded(n: int, width: int, name: str) -> sp.csr_matrix:
    """``width`` diagonals centred on the main one; the diagonal gets +10."""
    rng = _rng(name)
    half = width // 2
    rows, cols, vals = [], [], []
    for off in range(-half, half + 1):
        length = n - abs(off)
        v = rng.standard_normal(length)
        if off == 0:
            v = v + 10.0
        t = np.arange(length, dtype=np.int64)
        # element t of diagonal `off` sits at (t, t+off) above the diagonal and
        # at (t-off, t) below it
        rows.append(t if off >= 0 else t - off)
        cols.append(t + off if off >= 0 else t)
        vals.append(v)
    return _canonical(np.concatenate(rows), np.concatenate(cols), np.concatenate(vals),
                      (n, n))


def _corpus_from_counts(rng: np.random.Generator, counts: np.ndarray, ncols: int
                        ) -> sp.csr_matrix:
    """Columns drawn with replacement, values N(0,1), duplicates summed."""
    rows = np.repeat(np.arange(counts.size, dtype=np.int64), counts)
    cols = rng.integers(0, ncols, size=rows.size, dtype=np.int64)
    vals = rng.standard_normal(rows.size)
    return _canonical(rows, cols, vals, (counts.size, ncols))


def _corpus_uniform(n: int, ncols: int, per_row: int, name: str) -> sp.csr_matrix:
    rng = _rng(name)
    return _corpus_from_counts(rng, np.full(n, per_row, dtype=np.int64), ncols)


def _corpus_power_law(n: int, ncols: int, alpha: float, cap: int, name: str
                      ) -> sp.csr_matrix:
    """Row lengths by inverse-transform sampling of P(k) ~ k^-alpha."""
    rng = _rng(name)
    u = np.clip(rng.random(n), 1e-12, 1.0 - 1e-9)
    if abs(alpha - 2.0) <= 1e-9:
        counts = np.floor(1.0 / u).astype(np.int64)
    else:
        counts = np.floor(np.power(u, -1.0 / (alpha - 1.0))).astype(np.int64)
    counts = np.minimum(np.clip(counts, 1, cap), ncols)
    return _corpus_from_counts(rng, counts, ncols)


def _corpus_dense_rows(n: int, ncols: int, frac: float, big: int, small: int,
                       name: str) -> sp.csr_matrix:
    rng = _rng(name)
    counts = np.full(n, small, dtype=np.int64)
    heavy = rng.choice(n, size=max(1, int(round(frac * n))), replace=False)
    counts[heavy] = big
    return _corpus_from_counts(rng, np.minimum(counts, ncols), ncols)


def _corpus_blocked(n: int, bs: int, per_row: int, name: str) -> sp.csr_matrix:
    """Dense bs x bs blocks: the diagonal block plus random distinct others."""
    if n % bs:
        raise ValueError("blocked matrix requires n divisible by block size")
    rng = _rng(name)
    nb = n // bs
    local = np.arange(bs, dtype=np.int64)
    rr_local = np.repeat(local, bs)
    cc_local = np.tile(local, bs)
    rows, cols, vals = [], [], []
    for br in range(nb):
        chosen = {br}
        while len(chosen) < per_row:
            chosen.add(int(rng.integers(0, nb)))
        # set iteration order decides which values land in which block; it is
        # the same CPython int-set order the reference iterates
        for bc in chosen:
            rows.append(br * bs + rr_local)
            cols.append(bc * bs + cc_local)
            vals.append(rng.standard_normal(bs * bs))
    return _canonical(np.concatenate(rows), np.concatenate(cols), np.concatenate(vals),
                      (n, n))


def make_matrix(class_name: str) -> sp.csr_matrix:
    """One reference-corpus class (reference ``matrices.py:164-178``)."""
    if class_name == "banded":
        return _corpus_banded(200000, 7, "banded")
    if class_name == "uniform_random":
        return _corpus_uniform(100000, 100000, 16, "uniform_random")
    if class_name == "power_law":
        return _corpus_power_law(100000, 100000, 2.0, 2000, "power_law")
    if class_name == "diagonal_heavy":
        return _corpus_banded(200000, 3, "diagonal_heavy")
    if class_name == "dense_rows":
        return _corpus_dense_rows(20000, 20000, 0.01, 2000, 4, "dense_rows")
    if class_name == "blocked":
        return _corpus_blocked(100000, 8, 2, "blocked")
    raise ValueError("unknown matrix class: %s" % class_name)


def corpus_classes() -> List[str]:
    return ["banded", "uniform_random", "power_law", "diagonal_heavy", "dense_rows",
            "blocked"]


def matrix_stats(class_name: str, m: sp.csr_matrix) -> Dict[str, object]:
    """Manifest statistics; ``imbalance_ratio`` = max row nnz / mean row nnz."""
    rows, cols = m.shape
    lengths = np.diff(m.indptr).astype(np.float64)
    has = lengths.size > 0
    mean = float(lengths.mean()) if has else 0.0
    peak = float(lengths.max()) if has else 0.0
    return {
        "class_name": class_name,
        "rows": int(rows),
        "cols": int(cols),
        "nnz": int(m.nnz),
        "nnz_per_row_mean": mean,
        "nnz_per_row_median": float(np.median(lengths)) if has else 0.0,
        "nnz_per_row_max": peak,
        "nnz_per_row_stddev": float(lengths.std()) if has else 0.0,
        "imbalance_ratio": float(peak / mean) if mean > 0 else 0.0,
    }


def save_csr_npz(path: str, class_name: str, m: sp.csr_matrix) -> None:
    m = m.tocsr()
    m.sum_duplicates()
    m.sort_indices()
    np.savez(path, indptr=m.indptr.astype(np.int64), indices=m.indices.astype(np.int64),
             data=m.data.astype(np.float64), shape=np.array(m.shape, dtype=np.int64),
             class_name=np.array(class_name))


def load_csr_npz(path: str) -> sp.csr_matrix:
    with np.load(path, allow_pickle=False) as z:
        m = sp.csr_matrix((z["data"].astype(np.float64), z["indices"].astype(np.int64),
                           z["indptr"].astype(np.int64)),
                          shape=tuple(int(s) for s in z["shape"]))
    return _as_int64(m)


def export_matrix_bin(path: str, m: sp.csr_matrix) -> None:
    """Write the TGM1 binary read by the C++ harnesses."""
    m = m.tocsr()
    m.sum_duplicates()
    m.sort_indices()
    rows, cols = m.shape
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Iqqq", _BIN_MAGIC, rows, cols, int(m.nnz)))
        for arr, dt in ((m.indptr, "<i8"), (m.indices, "<i8"), (m.data, "<f8")):
            fh.write(np.ascontiguousarray(arr, dtype=dt).tobytes())


def load_matrix_bin(path: str) -> sp.csr_matrix:
    """Read a TGM1 file; raises ValueError on a bad magic or a short file."""
    with open(path, "rb") as fh:
        head = fh.read(28)
        if len(head) != 28:
            raise ValueError("%s: truncated TGM1 header" % path)
        magic, rows, cols, nnz = struct.unpack("<Iqqq", head)
        if magic != _BIN_MAGIC:
            raise ValueError("%s: bad magic 0x%08x (want 0x%08x)" % (path, magic, _BIN_MAGIC))
        indptr = np.fromfile(fh, dtype="<i8", count=rows + 1)
        indices = np.fromfile(fh, dtype="<i8", count=nnz)
        data = np.fromfile(fh, dtype="<f8", count=nnz)
    if indptr.size != rows + 1 or indices.size != nnz or data.size != nnz:
        raise ValueError("%s: truncated TGM1 payload" % path)
    return _as_int64(sp.csr_matrix((data, indices, indptr), shape=(rows, cols)))


def build_corpus(outdir: str) -> Dict[str, object]:
    """Write every corpus class (.npz + .bin) and ``manifest.json``."""
    os.makedirs(outdir, exist_ok=True)
    manifest: Dict[str, object] = {"seed": SEED, "matrices": []}
    for name in corpus_classes():
        m = make_matrix(name)
        stats = matrix_stats(name, m)
        save_csr_npz(os.path.join(outdir, "%s.npz" % name), name, m)
        export_matrix_bin(os.path.join(outdir, "%s.bin" % name), m)
        stats["file"] = "%s.npz" % name
        manifest["matrices"].append(stats)
        print("[matrices] %-16s rows=%-8d nnz=%-10d max/row=%-8.0f imbalance=%.2f"
              % (name, stats["rows"], stats["nnz"], stats["nnz_per_row_max"],
                 stats["imbalance_ratio"]))
    with open(os.path.join(outdir, "manifest.json"), "w") as fh:
        json.dump(manifest, fh, indent=2)
    return manifest


# --------------------------------------------------------------------------- #
# BASELINE configs (the graded inputs)
# --------------------------------------------------------------------------- #
def _distinct_columns(rng: np.random.Generator, counts: np.ndarray, ncols: int
                      ) -> np.ndarray:
    """Sorted distinct columns per row, uniform without replacement.

    Rows of equal length are drawn together: sample, sort, and redraw whole
    rows that came out with a repeat until none remain.  Rows longer than 64
    use ``Generator.choice(replace=False)`` one at a time.
    """
    indptr = np.zeros(counts.size + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    out = np.empty(int(indptr[-1]), dtype=np.int64)
    for c in np.unique(counts):
        c = int(c)
        if c == 0:
            continue
        rows = np.nonzero(counts == c)[0]
        if c > 64:
            for r in rows:
                out[indptr[r]:indptr[r + 1]] = np.sort(rng.choice(ncols, size=c,
                                                                  replace=False))
            continue
        block = np.sort(rng.integers(0, ncols, size=(rows.size, c), dtype=np.int64), axis=1)
        while True:
            bad = np.nonzero((np.diff(block, axis=1) == 0).any(axis=1))[0]
            if bad.size == 0:
                break
            block[bad] = np.sort(rng.integers(0, ncols, size=(bad.size, c),
                                              dtype=np.int64), axis=1)
        starts = indptr[rows]
        out[(starts[:, None] + np.arange(c)).ravel()] = block.ravel()
    return out


def _csr_from_counts(rng: np.random.Generator, counts: np.ndarray, ncols: int
                     ) -> sp.csr_matrix:
    indptr = np.zeros(counts.size + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    indices = _distinct_columns(rng, counts, ncols)
    data = rng.uniform(-1.0, 1.0, size=indices.size)
    return _as_int64(sp.csr_matrix((data, indices, indptr), shape=(counts.size, ncols)))


@dataclass(frozen=True)
class BaselineCase:
    """One BASELINE.json config: which kernel, which matrix, dense width K."""

    case_id: str
    kernel: str
    matrix: str
    K: int = 1
    description: str = ""


_CASES = [
    BaselineCase("c1", "spmv", "uniform_random", 1,
                 "SpMV, M=N=100000, 16 distinct uniform columns per row"),
    BaselineCase("c2", "spmv", "banded", 1,
                 "SpMV, M=N=200000, offsets -3..+3 clipped at the edges"),
    BaselineCase("c3a", "spmv", "power_law", 1,
                 "SpMV, M=N=100000, row length min(5000, floor(u^(-1/1.03)))"),
    BaselineCase("c3b", "spmv", "dense_rows", 1,
                 "SpMV, M=N=20000, 200 rows of 2000 nnz, the rest 4"),
    BaselineCase("c4", "spmm", "uniform_random", 64,
                 "SpMM C=A*B, A = c1 pattern, B N x 64"),
    BaselineCase("c5", "sddmm", "blocked4x4", 64,
                 "SDDMM on 4x4 blocks, 4 distinct block columns per block row"),
    BaselineCase("c5x25", "sddmm", "blocked4x4_25", 64,
                 "SDDMM on 4x4 blocks, 25 block columns per block row (10M nnz)"),
]


def baseline_ids() -> List[str]:
    return [c.case_id for c in _CASES]


def baseline_case(case_id: str) -> BaselineCase:
    for c in _CASES:
        if c.case_id == case_id:
            return c
    raise ValueError("unknown baseline case %r (have %s)" % (case_id, baseline_ids()))


def _baseline_matrix(name: str, scale: float = 1.0) -> sp.csr_matrix:
    rng = _rng(name)
    if name == "uniform_random":
        n = int(100000 * scale)
        return _csr_from_counts(rng, np.full(n, 16, dtype=np.int64), n)
    if name == "banded":
        n = int(200000 * scale)
        offsets = np.arange(-3, 4, dtype=np.int64)
        rows = np.repeat(np.arange(n, dtype=np.int64), offsets.size)
        cols = rows + np.tile(offsets, n)
        keep = (cols >= 0) & (cols < n)
        rows, cols = rows[keep], cols[keep]
        counts = np.bincount(rows, minlength=n).astype(np.int64)
        indptr = np.zeros(n + 1, dtype=np.int64)
        np.cumsum(counts, out=indptr[1:])
        data = rng.uniform(-1.0, 1.0, size=cols.size)
        return _as_int64(sp.csr_matrix((data, cols, indptr), shape=(n, n)))
    if name == "power_law":
        n = int(100000 * scale)
        alpha, cap = 2.03, 5000
        u = np.clip(rng.random(n), 1e-12, 1.0 - 1e-9)
        counts = np.floor(np.power(u, -1.0 / (alpha - 1.0))).astype(np.int64)
        counts = np.minimum(np.clip(counts, 1, cap), n)
        return _csr_from_counts(rng, counts, n)
    if name == "dense_rows":
        n = int(20000 * scale)
        counts = np.full(n, 4, dtype=np.int64)
        heavy = rng.choice(n, size=max(1, n // 100), replace=False)
        counts[heavy] = min(2000, n)
        return _csr_from_counts(rng, counts, n)
    if name.startswith("blocked4x4"):
        per_row = 25 if name.endswith("_25") else 4
        bs = 4
        n = int(100000 * scale) // bs * bs
        nb = n // bs
        # distinct block columns per block row, sorted
        bcols = _distinct_columns(rng, np.full(nb, per_row, dtype=np.int64), nb)
        bcols = bcols.reshape(nb, per_row)
        # row r = br*4 + a holds columns bc*4 + b for each chosen bc, b in 0..3
        cols_of_block_row = (bcols[:, :, None] * bs + np.arange(bs)).reshape(nb, per_row * bs)
        indices = np.repeat(cols_of_block_row, bs, axis=0).ravel()
        indptr = np.arange(n + 1, dtype=np.int64) * (per_row * bs)
        data = rng.uniform(-1.0, 1.0, size=indices.size)
        return _as_int64(sp.csr_matrix((data, indices, indptr), shape=(n, n)))
    raise ValueError("unknown baseline matrix %r" % name)


def make_baseline(case_id: str, scale: float = 1.0) -> sp.csr_matrix:
    """The CSR matrix of a BASELINE case; ``scale`` < 1 shrinks the row count
    (same generator, for quick tests)."""
    return _baseline_matrix(baseline_case(case_id).matrix, scale)


def baseline_operands(kernel: str, M: int, N: int, K: int, seed: int = 7
                      ) -> Dict[str, np.ndarray]:
    """Dense operands of a BASELINE case, U(-1,1) from ``default_rng(seed)``.

    Draw order is fixed (x, then B, then U, then V) and only the operands the
    kernel uses are drawn.
    """
    rng = np.random.default_rng(seed)
    if kernel == "spmv":
        return {"x": rng.uniform(-1.0, 1.0, size=N)}
    if kernel == "spmm":
        return {"B": rng.uniform(-1.0, 1.0, size=(N, K))}
    if kernel == "sddmm":
        U = rng.uniform(-1.0, 1.0, size=(M, K))
        V = rng.uniform(-1.0, 1.0, size=(N, K))
        return {"U": U, "V": V}
    raise ValueError("unknown kernel %r" % kernel)


def compulsory_bytes(kernel: str, M: int, N: int, nnz: int, K: int = 1) -> int:
    """Bytes every correct implementation must move at least once: indptr,
    indices and values once, each dense operand once, each output once."""
    base = 8 * (M + 1) + 16 * nnz
    if kernel == "spmv":
        return base + 8 * N + 8 * M
    if kernel == "spmm":
        return base + 8 * N * K + 8 * M * K
    if kernel == "sddmm":
        return base + 8 * M * K + 8 * N * K + 8 * nnz
    if kernel == "fused_spmv_axpy":
        return base + 8 * N + 16 * M
    raise ValueError(kernel)


def flops(kernel: str, nnz: int, K: int = 1, M: int = 0) -> float:
    if kernel in ("spmv", "fused_spmv_axpy"):
        return 2.0 * nnz
    if kernel in ("spmm", "sddmm"):
        return 2.0 * nnz * K
    if kernel == "axpy":
        return 2.0 * M
    raise ValueError(kernel)


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description="Generate the TileGen reference corpus.")
    ap.add_argument("--out", default="data/matrices")
    args = ap.parse_args(argv)
    build_corpus(args.out)
    return 0


if __name__ == "__main__":  # pragma: no cover
    raise SystemExit(main())

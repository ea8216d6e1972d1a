"""Pins the CPU oracle before anything is checked against it.

* the reference's known-answer tests (tests/golden/ref_kats.json, from
  cpp/tests/test_ref.cpp:25-116), exactly;
* brute force on tiny inputs: the CSR kernels equal dense numpy products of
  the densified matrix (a dropped term, a wrong index or a transposed operand
  changes these results);
* float64 SciPy on seeded ragged inputs, within 1e-13 normwise;
* the reference's own ref.cpp (oracle/_ref), bit for bit, when it is built;
* planted mistakes: copies of the oracle's algorithm with one deliberate bug
  each must fail the checks above.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from tests.util import csr, mixed_257, ragged, rel_inf

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _kats():
    with open(os.path.join(GOLDEN, "ref_kats.json")) as fh:
        return json.load(fh)


@pytest.mark.parametrize("kat", _kats(), ids=lambda k: k["case"])
def test_reference_known_answers(kat):
    k = kat["kernel"]
    if k == "dense_spmv":
        Ad = np.array(kat["dense"]).reshape(kat["rows"], kat["cols"])
        got = oracle.dense_spmv(Ad, np.array(kat["x"]))
    else:
        A = csr(kat["rows"], kat["cols"], kat["indptr"], kat["indices"], kat["data"])
        if k == "spmv":
            got = oracle.spmv(A, np.array(kat["x"]))
        elif k == "spmm":
            B = np.array(kat["B"]).reshape(kat["cols"], kat["K"])
            got = oracle.spmm(A, B).ravel()
        elif k == "sddmm":
            U = np.array(kat["U"]).reshape(kat["rows"], kat["K"])
            V = np.array(kat["V"]).reshape(kat["cols"], kat["K"])
            got = oracle.sddmm(A, U, V)
        elif k == "fused_spmv_axpy":
            got = oracle.fused_spmv_axpy(A, np.array(kat["x"]), np.array(kat["w"]),
                                         kat["alpha"], kat["beta"])
        else:  # pragma: no cover
            raise AssertionError(k)
    assert np.array_equal(got, np.array(kat["expected"])), (kat["case"], got)


def _dense(A: sp.csr_matrix) -> np.ndarray:
    """Densify by walking the CSR triplets (independent of scipy's toarray)."""
    D = np.zeros(A.shape)
    for i in range(A.shape[0]):
        for p in range(A.indptr[i], A.indptr[i + 1]):
            D[i, A.indices[p]] += A.data[p]
    return D


TINY = [
    csr(3, 4, [0, 2, 2, 4], [0, 3, 1, 2], [1.5, -2.0, 3.0, 0.25]),
    csr(1, 1, [0, 1], [0], [2.0]),
    csr(4, 2, [0, 0, 0, 0, 0], [], []),
    ragged(11, 7, 9, 5, empty_every=3),
]


@pytest.mark.parametrize("A", TINY, ids=["rect", "1x1", "empty", "ragged"])
def test_brute_force_dense(A):
    # integer-valued data and operands: every product and sum is exact, so the
    # comparison can be bitwise whatever order numpy sums in
    A = A.copy()
    A.data = np.round(A.data * 8.0)
    rng = np.random.default_rng(5)
    M, N = A.shape
    D = _dense(A)
    x = rng.integers(-4, 5, N).astype(float)
    assert np.array_equal(oracle.spmv(A, x), D @ x)
    B = rng.integers(-4, 5, (N, 3)).astype(float)
    assert np.array_equal(oracle.spmm(A, B), D @ B)
    U = rng.integers(-4, 5, (M, 3)).astype(float)
    V = rng.integers(-4, 5, (N, 3)).astype(float)
    want = np.array([A.data[p] * float(U[i] @ V[A.indices[p]])
                     for i in range(M) for p in range(A.indptr[i], A.indptr[i + 1])])
    assert np.array_equal(oracle.sddmm(A, U, V), want.reshape(-1))
    # sampled product = the dense product masked by the pattern, read off by position
    S = (U @ V.T)
    pat = [(i, A.indices[p], A.data[p]) for i in range(M)
           for p in range(A.indptr[i], A.indptr[i + 1])]
    assert np.array_equal(oracle.sddmm(A, U, V), np.array([d * S[i, j] for i, j, d in pat]))
    w = rng.integers(-4, 5, M).astype(float)
    assert np.array_equal(oracle.fused_spmv_axpy(A, x, w, 2.0, -3.0), 2.0 * (D @ x) - 3.0 * w)
    assert np.array_equal(oracle.axpy(x[:1].repeat(M), w, 0.5, 4.0), 0.5 * x[0] + 4.0 * w)
    Dd = rng.integers(-4, 5, (M, N)).astype(float)
    assert np.array_equal(oracle.dense_spmv(Dd, x), Dd @ x)


def test_matches_scipy_float64():
    A = ragged(3, 800, 600, 40, empty_every=7, long_rows=[(5, 600)])
    rng = np.random.default_rng(0)
    x = rng.standard_normal(600)
    B = rng.standard_normal((600, 9))
    U = rng.standard_normal((800, 9))
    V = rng.standard_normal((600, 9))
    assert rel_inf(oracle.spmv(A, x), A @ x) < 1e-13
    assert rel_inf(oracle.spmm(A, B), A @ B) < 1e-13
    coo = A.tocoo()
    want = np.einsum("ik,ik->i", U[coo.row], V[coo.col]) * coo.data
    assert rel_inf(oracle.sddmm(A, U, V), want) < 1e-13


@pytest.mark.skipif(not oracle.reference_available(),
                    reason="oracle/_ref not built (needs /root/reference at build time)")
def test_bit_identical_to_reference_ref_cpp():
    for A in (mixed_257(), ragged(2, 3000, 2500, 30, empty_every=11, long_rows=[(1, 2400)])):
        M, N = A.shape
        rng = np.random.default_rng(1)
        x = rng.uniform(-1, 1, N)
        B = rng.uniform(-1, 1, (N, 13))
        U = rng.uniform(-1, 1, (M, 13))
        V = rng.uniform(-1, 1, (N, 13))
        w = rng.uniform(-1, 1, M)
        rm = oracle.RefMatrix(A)
        rm.set_operands(K=13, x=x, B=B, U=U, V=V)
        y_ref, _ = rm.run("spmv", 1, (M,))
        C_ref, _ = rm.run("spmm", 1, (M, 13))
        s_ref, _ = rm.run("sddmm", 1, (A.nnz,))
        z_ref = np.empty(M)
        rm.L.ref_fused_spmv_axpy(rm.h, w.ctypes.data_as(oracle._F64P), 0.7, -1.3,
                                 z_ref.ctypes.data_as(oracle._F64P))
        rm.close()
        assert oracle.spmv(A, x).tobytes() == y_ref.tobytes()
        assert oracle.spmm(A, B).tobytes() == C_ref.tobytes()
        assert oracle.sddmm(A, U, V).tobytes() == s_ref.tobytes()
        assert oracle.fused_spmv_axpy(A, x, w, 0.7, -1.3).tobytes() == z_ref.tobytes()


# --------------------------------------------------------------------------- #
# planted mistakes: each buggy restatement must be caught by the checks above
# --------------------------------------------------------------------------- #
def _spmv_variant(A, x, bug):
    y = np.zeros(A.shape[0])
    for i in range(A.shape[0]):
        lo, hi = A.indptr[i], A.indptr[i + 1]
        if bug == "drop_last":
            hi = max(lo, hi - 1)
        acc = 0.0
        for p in range(lo, hi):
            j = A.indices[p]
            if bug == "col_off_by_one":
                j = min(j + 1, A.shape[1] - 1)
            acc += A.data[p] * x[j]
        y[i] = acc
    return y


def _sddmm_variant(A, U, V, bug):
    out = []
    for i in range(A.shape[0]):
        for p in range(A.indptr[i], A.indptr[i + 1]):
            j = A.indices[p]
            if bug == "transposed":  # U[j] . V[i] instead of U[i] . V[j]
                out.append(A.data[p] * float(U[j] @ V[i]))
            else:
                out.append(A.data[p] * float(U[i] @ V[j]))
    return np.array(out)


@pytest.mark.parametrize("bug", ["drop_last", "col_off_by_one"])
def test_planted_spmv_mistake_is_caught(bug):
    kats = [k for k in _kats() if k["kernel"] == "spmv"]
    caught_kat = False
    for kat in kats:
        A = csr(kat["rows"], kat["cols"], kat["indptr"], kat["indices"], kat["data"])
        if not np.array_equal(_spmv_variant(A, np.array(kat["x"]), bug),
                              np.array(kat["expected"])):
            caught_kat = True
    A = TINY[0]
    x = np.array([1.0, 2.0, 3.0, 4.0])
    caught_dense = not np.array_equal(_spmv_variant(A, x, bug), _dense(A) @ x)
    assert caught_kat or caught_dense
    # and the real oracle passes the very same checks
    assert np.array_equal(oracle.spmv(A, x), _dense(A) @ x)


def test_planted_sddmm_transpose_is_caught():
    kat = [k for k in _kats() if k["kernel"] == "sddmm"][0]
    A = csr(kat["rows"], kat["cols"], kat["indptr"], kat["indices"], kat["data"])
    U = np.array(kat["U"]).reshape(2, 2)
    V = np.array(kat["V"]).reshape(2, 2)
    assert np.array_equal(_sddmm_variant(A, U, V, "none"), kat["expected"])
    # the KAT's diagonal pattern is symmetric; the ragged brute force is not
    B = ragged(4, 6, 6, 4)
    rng = np.random.default_rng(2)
    U6, V6 = rng.standard_normal((6, 3)), rng.standard_normal((6, 3))
    assert not np.allclose(_sddmm_variant(B, U6, V6, "transposed"), oracle.sddmm(B, U6, V6))

"""DSL / IR behaviour, restating the reference's tests/test_dsl.py:32-143 and
tests/test_pretty.py:10-32 against this package."""

from __future__ import annotations

import pytest

from tilegen_amd.dsl import (
    CSR, DENSE1, Access, Index, Kernel, Mul, Reduce, Schedule, Stmt, TensorDecl, Tile,
    Unroll, Vectorize, assign, dense_tensor, kernel, reduce_sum, scalar_tensor,
    sparse_tensor, standard_kernel_names, standard_kernels,
)
from tilegen_amd.ir import Format, Parallelize, ThreadsPerRow


def test_build_all_standard_kernels():
    ks = standard_kernels()
    assert list(ks) == standard_kernel_names() == ["spmv", "spmm", "sddmm", "fused_spmv_axpy",
                                                   "axpy"]
    for k in ks.values():
        assert k.validate() is True


def test_spmv_ir_shape():
    k = standard_kernels()["spmv"]
    assert isinstance(k.stmt, Stmt) and isinstance(k.stmt.rhs, Reduce)
    assert k.stmt.rhs.index.name == "j"
    assert isinstance(k.stmt.rhs.body, Mul)
    assert [i.name for i in k.free_indices()] == ["i"]
    assert [i.name for i in k.reduce_indices()] == ["j"]
    assert k.sparse_tensor().format.name == "csr"
    assert [t.name for t in k.tensors()] == ["A", "x", "y"]


def test_sddmm_ir_shape():
    k = standard_kernels()["sddmm"]
    inner = k.stmt.rhs
    assert isinstance(inner, Mul) and isinstance(inner.right, Reduce)
    assert inner.right.index.name == "k"
    assert sorted(i.name for i in k.free_indices()) == ["i", "j"]
    assert [t.name for t in k.tensors()] == ["A", "U", "V", "C"]


def test_fused_has_two_statements():
    k = standard_kernels()["fused_spmv_axpy"]
    assert [s.lhs.tensor.name for s in k.stmts] == ["t", "z"]


def test_eq_sugar_builds_assignment():
    i, j = Index("i"), Index("j")
    A = sparse_tensor("A", CSR, shape=("M", "N"))
    x = dense_tensor("x", shape=("N",))
    y = dense_tensor("y", shape=("M",))
    stmt = y[i] == reduce_sum(j, A[i, j] * x[j])
    assert isinstance(stmt, Stmt)
    assert kernel("spmv_sugar", [stmt]).validate() is True


def test_pretty_is_readable():
    for k in standard_kernels().values():
        text = k.pretty()
        assert "kernel" in text and "for" in text
        if k.reduce_node() is not None:
            assert "sum(" in text


def test_roundtrip_to_from_dict():
    for k in standard_kernels().values():
        d = k.to_dict()
        assert Kernel.from_dict(d).to_dict() == d


def test_roundtrip_with_schedule():
    k = standard_kernels()["spmm"]
    k.schedule = Schedule([Tile(Index("i"), 32), Parallelize(Index("i"), "thread", 256),
                           ThreadsPerRow(8), Unroll(Index("j"), 4), Vectorize(2)])
    assert k.validate()
    assert Kernel.from_dict(k.to_dict()).to_dict() == k.to_dict()


def test_reject_unbound_lhs_index():
    i, j, kk = Index("i"), Index("j"), Index("kk")
    A = sparse_tensor("A", CSR, shape=("M", "N"))
    x = dense_tensor("x", shape=("N",))
    y = dense_tensor("y", shape=("M",))
    with pytest.raises(ValueError):
        kernel("bad_unbound", [assign(y[kk], reduce_sum(j, A[i, j] * x[j]))])


def test_reject_format_order_mismatch():
    A = sparse_tensor("A", CSR, shape=("M", "N"))
    x = dense_tensor("x", shape=("N",))
    i = Index("i")
    with pytest.raises(ValueError):
        kernel("bad_rank", [Stmt(lhs=x[i], rhs=Access(A.decl, [i]))])
    broken = TensorDecl(name="Q", order=2, format=DENSE1, dtype="f64", shape=("M", "N"))
    b = dense_tensor("b", shape=("M", "N"))
    with pytest.raises(ValueError):
        kernel("bad_fmt_order", [Stmt(lhs=b[i, i], rhs=Access(broken, [i, i]))])


def test_reject_bad_format_level():
    i = Index("i")
    weird = TensorDecl(name="W", order=1, format=Format("weird", ("sparse",)), shape=("M",))
    y = dense_tensor("y", shape=("M",))
    with pytest.raises(ValueError):
        kernel("bad_level", [Stmt(lhs=y[i], rhs=Access(weird, [i]))])


def test_reject_unknown_schedule_index():
    k = standard_kernels()["spmv"]
    k.schedule = Schedule([Tile(Index("zz"), 32)])
    with pytest.raises(ValueError):
        k.validate()


def test_reject_bad_factors():
    k = standard_kernels()["spmv"]
    for bad in ([Unroll(Index("i"), 0)], [Vectorize(0)], [ThreadsPerRow(0)],
                [Tile(Index("i"), 0)], [Parallelize(Index("i"), "grid")],
                [Parallelize(Index("i"), "thread", -1)]):
        k.schedule = Schedule(bad)
        with pytest.raises(ValueError):
            k.validate()


def test_reduce_index_must_appear_in_body():
    i, j = Index("i"), Index("j")
    x = dense_tensor("x", shape=("M",))
    y = dense_tensor("y", shape=("M",))
    with pytest.raises(ValueError):
        kernel("bad_reduce", [assign(y[i], reduce_sum(j, x[i]))])


def test_scalar_arithmetic_and_sub():
    i = Index("i")
    x = dense_tensor("x", shape=("M",))
    z = dense_tensor("z", shape=("M",))
    a = scalar_tensor("a")
    k = kernel("sub", [assign(z[i], 2.0 * x[i] - a * x[i])])
    assert k.validate()
    assert "z[i] = 2.0 * x[i] + -1.0 * a * x[i]" in k.pretty()


# reference tests/test_pretty.py:10-27
SNAPSHOTS = {
    "spmv": """kernel spmv {
  assign y[i] = sum(j, A[i, j] * x[j])
  // loop nest
  for i:
    for j in reduce(A row):
      assign y[i] += A[i, j] * x[j]
}""",
    "fused_spmv_axpy": """kernel fused_spmv_axpy {
  assign t[i] = sum(j, A[i, j] * x[j])
  assign z[i] = alpha * t[i] + beta * w[i]
  // loop nest
  for i:
    for j in reduce(A row):
      assign t[i] += A[i, j] * x[j]
    assign z[i] = alpha * t[i] + beta * w[i]
}""",
}


@pytest.mark.parametrize("name", sorted(SNAPSHOTS))
def test_pretty_loop_nest_snapshot(name):
    assert standard_kernels()[name].pretty() == SNAPSHOTS[name]


def test_pretty_sddmm_and_schedule_lines():
    k = standard_kernels()["sddmm"]
    k.schedule = Schedule([Tile(Index("i"), 4), Parallelize(Index("i"), "thread", 256)])
    text = k.pretty()
    assert "  for i, j:" in text
    assert "    for k in reduce(dense):" in text
    assert "      assign C[i, j] += A[i, j] * U[i, k] * V[j, k]" in text
    assert "  //   Tile(i, 4)" in text
    assert "  //   Parallelize(i, thread, block=256)" in text

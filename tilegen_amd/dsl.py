"""Index-notation frontend (same API as reference ``tilegen/dsl.py:85-271``).

::

    i, j = Index("i"), Index("j")
    A = sparse_tensor("A", CSR, shape=("M", "N"))
    x = dense_tensor("x", shape=("N",))
    y = dense_tensor("y", shape=("M",))
    spmv = kernel("spmv", [assign(y[i], reduce_sum(j, A[i, j] * x[j]))])

``y[i] == reduce_sum(...)`` is the same assignment as ``assign(y[i], ...)``.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence, Tuple, Union

from .ir import (  # noqa: F401  (re-exported API)
    Access, Add, Assign, BSR, COO, CSC, CSR, Const, DENSE1, DENSE2, ELL, Format,
    Fuse, Index, Kernel, Mul, Parallelize, Reduce, SCALAR, Schedule, Split, Stmt,
    TensorDecl, ThreadsPerRow, Tile, Transform, Unroll, Vectorize,
)

__all__ = [
    "Index", "Tensor", "sparse_tensor", "dense_tensor", "scalar_tensor", "tensor",
    "reduce_sum", "assign", "kernel", "standard_kernels", "standard_kernel_names",
    "CSR", "CSC", "COO", "ELL", "BSR", "DENSE1", "DENSE2", "SCALAR", "Schedule",
    "Tile", "Split", "Parallelize", "Unroll", "Fuse", "ThreadsPerRow", "Vectorize",
    "i", "j", "k",
]


class Tensor:
    """User-facing handle: ``T[i, j]`` builds an Access; order-0 tensors also
    take part in scalar arithmetic directly (``alpha * t[i]``)."""

    def __init__(self, decl: TensorDecl):
        self.decl = decl

    def __getitem__(self, idx: Union[Index, Tuple[Index, ...]]) -> Access:
        return Access(self.decl, list(idx) if isinstance(idx, tuple) else [idx])

    def _scalar(self) -> Access:
        return Access(self.decl, [])

    def __mul__(self, other: Any):
        return self._scalar() * other

    def __rmul__(self, other: Any):
        return other * self._scalar()

    def __add__(self, other: Any):
        return self._scalar() + other

    def __radd__(self, other: Any):
        return other + self._scalar()

    @property
    def name(self) -> str:
        return self.decl.name

    @property
    def shape(self) -> Tuple[Any, ...]:
        return self.decl.shape

    def __repr__(self) -> str:
        d = self.decl
        return "<%s: %s %s%s>" % (d.name, d.dtype, d.format.name,
                                  "" if not d.shape else " " + "x".join(map(str, d.shape)))


def tensor(name: str, fmt: Format, shape: Sequence[Any] = (), dtype: str = "f64") -> Tensor:
    return Tensor(TensorDecl(name=name, order=len(fmt.levels), format=fmt, dtype=dtype,
                             shape=tuple(shape)))


def sparse_tensor(name: str, fmt: Format, shape: Sequence[Any] = (),
                  dtype: str = "f64") -> Tensor:
    if not fmt.is_sparse():
        raise ValueError("sparse_tensor(%r): format %s stores every level dense; pass a "
                         "format with a compressed level such as CSR, or use dense_tensor"
                         % (name, fmt.name))
    return tensor(name, fmt, shape, dtype)


def dense_tensor(name: str, shape: Sequence[Any] = (), dtype: str = "f64") -> Tensor:
    # orders 0-2 take the IR's named format objects, so the kernels' IR compares and
    # serialises like the reference's; higher orders get an all-dense format of their own
    order = len(shape)
    fmt = {0: SCALAR, 1: DENSE1, 2: DENSE2}.get(order) or \
        Format("dense%d" % order, ("dense",) * order)
    return tensor(name, fmt, shape, dtype)


def scalar_tensor(name: str, dtype: str = "f64") -> Tensor:
    return tensor(name, SCALAR, (), dtype)


def _expr(value: Any):
    if isinstance(value, Stmt):
        return value.rhs
    if isinstance(value, Tensor):
        return Access(value.decl, [])
    if isinstance(value, (int, float)):
        return Const(float(value))
    return value


def reduce_sum(index: Index, body: Any) -> Reduce:
    """``sum`` over ``index``; not called ``sum`` so the builtin stays usable."""
    return Reduce(index=index, body=_expr(body))


def assign(lhs: Access, rhs: Any) -> Stmt:
    return Stmt(lhs=lhs, rhs=_expr(rhs))


def kernel(name: str, stmts: Union[Stmt, Sequence[Stmt]],
           schedule: Optional[Schedule] = None) -> Kernel:
    """Build and validate a kernel; formats/dtypes are recorded per distinct
    tensor in discovery order."""
    stmt_list = [stmts] if isinstance(stmts, Stmt) else list(stmts)
    k = Kernel(name=name, stmts=stmt_list,
               schedule=schedule if schedule is not None else Schedule())
    for t in k.tensors():
        k.formats.append(t.format)
        k.dtypes.append(t.dtype)
    k.validate()
    return k


# --------------------------------------------------------------------------- #
# the standard kernels (reference dsl.py:214-271)
# --------------------------------------------------------------------------- #
i = Index("i")
j = Index("j")
k = Index("k")
M, N, K = "M", "N", "K"


def _spmv() -> Kernel:
    A = sparse_tensor("A", CSR, shape=(M, N))
    x = dense_tensor("x", shape=(N,))
    y = dense_tensor("y", shape=(M,))
    return kernel("spmv", [assign(y[i], reduce_sum(j, A[i, j] * x[j]))])


def _spmm() -> Kernel:
    A = sparse_tensor("A", CSR, shape=(M, N))
    B = dense_tensor("B", shape=(N, K))
    C = dense_tensor("C", shape=(M, K))
    return kernel("spmm", [assign(C[i, k], reduce_sum(j, A[i, j] * B[j, k]))])


def _sddmm() -> Kernel:
    A = sparse_tensor("A", CSR, shape=(M, N))
    U = dense_tensor("U", shape=(M, K))
    V = dense_tensor("V", shape=(N, K))
    C = sparse_tensor("C", CSR, shape=(M, N))
    return kernel("sddmm", [assign(C[i, j], A[i, j] * reduce_sum(k, U[i, k] * V[j, k]))])


def _fused_spmv_axpy() -> Kernel:
    A = sparse_tensor("A", CSR, shape=(M, N))
    x = dense_tensor("x", shape=(N,))
    w = dense_tensor("w", shape=(M,))
    z = dense_tensor("z", shape=(M,))
    alpha = scalar_tensor("alpha")
    beta = scalar_tensor("beta")
    t = dense_tensor("t", shape=(M,))
    return kernel("fused_spmv_axpy", [
        assign(t[i], reduce_sum(j, A[i, j] * x[j])),
        assign(z[i], alpha * t[i] + beta * w[i]),
    ])


def _axpy() -> Kernel:
    x = dense_tensor("x", shape=(M,))
    w = dense_tensor("w", shape=(M,))
    z = dense_tensor("z", shape=(M,))
    alpha = scalar_tensor("alpha")
    beta = scalar_tensor("beta")
    return kernel("axpy", [assign(z[i], alpha * x[i] + beta * w[i])])


_BUILDERS = {
    "spmv": _spmv,
    "spmm": _spmm,
    "sddmm": _sddmm,
    "fused_spmv_axpy": _fused_spmv_axpy,
    "axpy": _axpy,
}


def standard_kernel_names() -> List[str]:
    return list(_BUILDERS)


def standard_kernels() -> Dict[str, Kernel]:
    """Fresh instances of the five kernels the DSL must express."""
    return {name: build() for name, build in _BUILDERS.items()}

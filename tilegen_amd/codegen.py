"""Code generation: the HIP (gfx950) emitter and the OpenMP CPU emitter.

``generate(kernel, config, backend)`` runs the pass pipeline and renders one
translation unit per variant; every variant exposes the reference ABI
``extern "C" void launch_<name>(...)`` (reference ``codegen.py:226-280``).

backend "hip"
    ``GeneratedKernel.source`` is device code only (one ``extern "C"
    __global__`` kernel plus small wave64 helpers), compiled at run time by
    hipRTC for gfx950.  ``GeneratedKernel.host_source`` is a C launcher that
    embeds the compiled code object and exports ``launch_<name>`` with the
    reference argument list, plus ``tgv_geometry``/``tgv_function`` for timing
    harnesses.  The device code is written for CDNA4, not translated:

    scalar_reduce (spmv, fused_spmv_axpy)
        ThreadsPerRow(k) lanes per row with a segmented DPP butterfly over k
        lanes of a 64-lane wave; Unroll(u) = each lane owns u consecutive
        nonzeros per step, loaded as 128-bit pairs from a 16-byte aligned base
        (row starts are rounded down, the extra lanes masked; bases that are
        only 8-byte aligned take per-element loads); Tile(T) = a
        workgroup owns T rows whose row pointers are staged once in LDS and
        whose first step is issued for every row before any gather, so each
        wave keeps several rows of loads in flight.  Config.balance picks what
        a tile holds: T rows ("rows"), an equal merge-path window of rows plus
        nonzeros ("nnz"), T rows with the rows longer than B*U nonzeros
        left to workgroups over equal nonzero ranges ("hybrid"), or an equal
        range of B*U nonzeros whose products are staged in LDS and summed
        there for the rows that end in the range ("stream"); rows cut across
        workgroups are combined in a fixed order through module scratch.
    row_dense_out (spmm)
        ThreadsPerRow(k) lanes per output row spread over the K columns,
        Vectorize(2) = 128-bit loads of B rows and stores of C, Unroll(u) =
        u nonzeros' B rows in flight.  With k = 64 the row is wave-uniform and
        (column, value) pairs arrive through the scalar unit.  C is written
        exactly once per element (no read-modify-write), with nontemporal
        stores since the kernel never reads it back.
    sparse_out (sddmm)
        ThreadsPerRow(k) lanes split the K-long dot product of one nonzero,
        Vectorize(2) = 128-bit loads of U and V rows, Unroll(u) = u K-chunks
        per lane.  When k*V*u covers K: one lane group per row (64/k adjacent
        rows per wave, so rows of a dense block gather the same V rows in one
        instruction), U[row, :] held in registers, column indices loaded k at
        a time and broadcast across the group, V gathers batched ahead of the
        FMAs, one coalesced nontemporal store per k outputs (U rows, read once,
        are nontemporal loads too).  Otherwise one wave per row.
    elementwise (axpy)
        one lane per element.

backend "cpu"
    OpenMP C++ restating reference ``_cpu_emit`` (``codegen.py:354-558``): the
    CPU baseline.  One deliberate change: the ``#pragma omp simd`` of spmm
    with vector_width > 1 is placed directly on the loop it vectorizes (the
    reference puts it before a declaration, which fails under -fopenmp and
    makes its compile retry silently without OpenMP).

``inject_bug=True`` makes every emitter stop one row short (the last row is
never written), so the differential tester can show it catches wrong kernels.
"""

from __future__ import annotations

import hashlib
import os
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

from . import passes as _passes
from .ir import (
    Access, Add, Const, Expr, Fuse, Index, Kernel, Mul, Parallelize, Reduce, Split,
    ThreadsPerRow, Tile, Unroll, Vectorize,
)

__all__ = [
    "Config", "GeneratedKernel", "Lowering", "Plan", "LaunchGeometry", "generate",
    "emit_hip", "emit_hip_host", "emit_cpu", "launch_geometry", "abi_of",
    "HIP_ARCH", "WAVE", "LDS_LIMIT",
]

HIP_ARCH = os.environ.get("TILEGEN_HIP_ARCH", "gfx950")
WAVE = 64
LDS_LIMIT = 160 * 1024  # LDS per CU on gfx950, all of which one workgroup may take

_CTYPE = {"f64": "double", "f32": "float", "double": "double", "float": "float"}


def ctype(dtype: str) -> str:
    return _CTYPE.get(dtype, "double")


# --------------------------------------------------------------------------- #
# Config / Lowering
# --------------------------------------------------------------------------- #
@dataclass
class Config:
    """Flat schedule request; the passes lower it into the schedule IR.

    tile_size T (rows per workgroup), threads_per_row TPR, unroll U,
    vector_width V, block_size B (lanes per workgroup).  ``balance`` is what
    a tile holds on the HIP backend: ``"rows"`` (T consecutive rows),
    ``"nnz"`` (an equal share of rows plus nonzeros, about T rows' worth),
    ``"hybrid"`` (T rows, with rows past a length threshold left to extra
    workgroups that each take an equal range of nonzeros) or ``"stream"`` (an
    equal range of B*U nonzeros and the rows that end in it; T is not used);
    the last three are for SpMV-shaped kernels (see ``_hip_scalar_reduce`` and
    ``_hip_stream_reduce``).  ``gather`` is the order of a row tile's
    first-step gathers: ``"direct"`` or ``"sorted"`` (made in the order of the
    gathered operand, sorted in LDS, so that the lanes of one gather
    instruction share cache lines; SpMV-shaped row tiles, see
    ``_sorted_first_step``).  Neither has a counterpart in the reference; both
    are left out of ``to_dict``/``hash`` at their defaults, so every reference
    schedule keeps its name.
    """

    tile_size: int = 32
    threads_per_row: int = 1
    unroll: int = 1
    vector_width: int = 1
    block_size: int = 256
    dtype: str = "f64"
    inject_bug: bool = False
    balance: str = "rows"
    gather: str = "direct"

    def to_dict(self) -> Dict[str, Any]:
        d = {"tile_size": self.tile_size, "threads_per_row": self.threads_per_row,
             "unroll": self.unroll, "vector_width": self.vector_width,
             "block_size": self.block_size, "dtype": self.dtype,
             "inject_bug": self.inject_bug}
        if self.balance != "rows":
            d["balance"] = self.balance
        if self.gather != "direct":
            d["gather"] = self.gather
        return d

    def hash(self) -> str:
        """sha1 of ``T|TPR|U|V|B|dtype|bug``, 10 hex digits (the reference's
        closed form, ``codegen.py:82-87``, so cache names line up); a
        non-default ``balance`` is appended as ``|<balance>``, a non-default
        ``gather`` as ``|gather=<gather>``."""
        key = "%d|%d|%d|%d|%d|%s|%d" % (self.tile_size, self.threads_per_row, self.unroll,
                                        self.vector_width, self.block_size, self.dtype,
                                        int(self.inject_bug))
        if self.balance != "rows":
            key += "|" + self.balance
        if self.gather != "direct":
            key += "|gather=" + self.gather
        return hashlib.sha1(key.encode()).hexdigest()[:10]

    def short(self) -> str:
        return "T%d/TPR%d/U%d/V%d/B%d%s%s" % (self.tile_size, self.threads_per_row,
                                              self.unroll, self.vector_width, self.block_size,
                                              {"rows": ""}.get(self.balance, "/" + self.balance),
                                              "" if self.gather == "direct" else "/" + self.gather)


@dataclass
class Lowering:
    """What the emitters read: the schedule transforms folded into numbers.

    ``tiled`` records whether a Tile transform is present (untiled HIP kernels
    read row pointers straight from global memory; tiled ones stage them).
    """

    tile: int = 1
    threads_per_row: int = 1
    unroll: int = 1
    vector_width: int = 1
    block_size: int = 256
    parallel: bool = False
    tiled: bool = False
    balance: str = "rows"
    gather: str = "direct"

    def to_dict(self) -> Dict[str, Any]:
        d = {"tile": self.tile, "threads_per_row": self.threads_per_row,
             "unroll": self.unroll, "vector_width": self.vector_width,
             "block_size": self.block_size, "parallel": self.parallel}
        if self.balance != "rows":
            d["balance"] = self.balance
        if self.gather != "direct":
            d["gather"] = self.gather
        return d


def _lowering(kernel: Kernel) -> Lowering:
    low = Lowering()
    for t in kernel.schedule:
        if isinstance(t, Tile):
            low.tile, low.tiled, low.balance, low.gather = t.size, True, t.by, t.gather
        elif isinstance(t, ThreadsPerRow):
            low.threads_per_row = t.k
        elif isinstance(t, Unroll):
            low.unroll = t.factor
        elif isinstance(t, Vectorize):
            low.vector_width = t.width
        elif isinstance(t, Parallelize):
            low.parallel = True
            if t.block_size:
                low.block_size = t.block_size
    return low


@dataclass
class LaunchGeometry:
    """Grid rule of a HIP variant: ``grid = ceil(rows / rows_per_block)``,
    plus ``floor(nnz / nnz_chunk) + 1`` workgroups ahead of those when
    ``nnz_chunk`` is set (hybrid tiles' long-row workgroups).  With
    ``stream`` the grid is ``floor(nnz / nnz_chunk) + 1`` alone when there
    are rows (they are written even without nonzeros).  Ranges are counted
    from the even position at or below indptr[0], so nnz nonzeros meet at most
    floor(nnz / nnz_chunk) + 1 of them."""

    rows_per_block: int
    block: int
    lds_bytes: int
    rows_symbol: str = "M"
    nnz_chunk: int = 0
    stream: bool = False

    def grid(self, rows: int, nnz: int = 0) -> int:
        if rows <= 0:
            return 0
        if self.stream:
            return max(0, int(nnz)) // self.nnz_chunk + 1
        g = (int(rows) + self.rows_per_block - 1) // self.rows_per_block
        if self.nnz_chunk:
            g += max(0, int(nnz)) // self.nnz_chunk + 1
        return g

    def to_dict(self) -> Dict[str, Any]:
        d = {"rows_per_block": self.rows_per_block, "block": self.block,
             "lds_bytes": self.lds_bytes, "rows_symbol": self.rows_symbol}
        if self.nnz_chunk:
            d["nnz_chunk"] = self.nnz_chunk
        if self.stream:
            d["stream"] = True
        return d


@dataclass
class GeneratedKernel:
    source: str
    filename: str
    abi_signature: str
    pass_log: List[Dict[str, Any]] = field(default_factory=list)
    backend: str = "cpu"
    kernel_name: str = ""
    config: Optional[Config] = None
    #: HIP only: the C launcher text (a ``{CODE_OBJECT}`` placeholder stands
    #: where the compiled bytes are embedded), the device symbol and geometry.
    host_source: str = ""
    device_symbol: str = ""
    geometry: Optional[LaunchGeometry] = None
    abi_args: List[Tuple[str, str]] = field(default_factory=list)

    def write(self, outdir: str = "build/generated") -> str:
        os.makedirs(outdir, exist_ok=True)
        path = os.path.join(outdir, self.filename)
        with open(path, "w") as fh:
            fh.write(self.source)
        return path


# --------------------------------------------------------------------------- #
# plan: what shape of loop nest the statement needs (reference codegen.py:158-220)
# --------------------------------------------------------------------------- #
@dataclass
class Plan:
    kind: str  # scalar_reduce | row_dense_out | sparse_out | elementwise
    out: Access
    out_tensor: Any
    A: Optional[Any] = None
    row_idx: Optional[Index] = None
    col_idx: Optional[Index] = None
    reduce: Optional[Reduce] = None
    reduce_is_compressed: bool = False
    inner_out: List[Index] = field(default_factory=list)
    value_expr: Optional[Expr] = None
    final_expr: Optional[Expr] = None
    row_extent: str = "M"


def _plan(kernel: Kernel) -> Plan:
    stmt = kernel.stmts[0]
    out = stmt.lhs
    A = kernel.sparse_tensor()
    red = kernel.reduce_node()
    if A is None:
        return Plan(kind="elementwise", out=out, out_tensor=out.tensor,
                    value_expr=stmt.rhs, final_expr=stmt.rhs,
                    row_extent=str(out.tensor.shape[0]) if out.tensor.shape else "M")
    a_acc = next(n for n in stmt.rhs.walk()
                 if isinstance(n, Access) and n.tensor.name == A.name)
    row_idx, col_idx = a_acc.indices[0], a_acc.indices[1]
    over_nnz = red is not None and red.index.name == col_idx.name
    inner = [ix for ix in out.indices if ix.name not in (row_idx.name, col_idx.name)]
    if out.tensor.format.is_sparse():
        kind = "sparse_out"
    elif over_nnz and inner:
        kind = "row_dense_out"
    else:
        kind = "scalar_reduce"
    return Plan(kind=kind, out=out, out_tensor=out.tensor, A=A, row_idx=row_idx,
                col_idx=col_idx, reduce=red, reduce_is_compressed=over_nnz,
                inner_out=inner, value_expr=red.body if red is not None else stmt.rhs,
                final_expr=stmt.rhs, row_extent=str(A.shape[0]) if A.shape else "M")


# --------------------------------------------------------------------------- #
# ABI (reference codegen.py:226-280): arrays in tensor discovery order (a sparse
# input expands to indptr, indices, data), then scalars, then every symbolic
# dimension in first-seen order, then nnz when a sparse tensor is present.
# --------------------------------------------------------------------------- #
def abi_of(kernel: Kernel) -> Tuple[str, List[Tuple[str, str]], Dict[str, Any]]:
    """Return (signature, [(c_type, name)...], info)."""
    out_name = kernel.stmts[0].lhs.tensor.name
    dt = ctype(kernel.dtypes[0] if kernel.dtypes else "f64")
    arrays: List[Tuple[str, Any]] = []
    scalars, dims = [], []
    n_sparse_in = 0
    for t in kernel.tensors():
        if t.order == 0:
            scalars.append(t)
            continue
        if t.format.is_sparse():
            if t.name == out_name:
                arrays.append(("out_sparse", t))
            else:
                n_sparse_in += 1
                arrays.append(("sparse", t))
        else:
            arrays.append(("dense", t))
        for s in t.shape:
            if str(s) not in dims:
                dims.append(str(s))
    if n_sparse_in > 1:
        raise NotImplementedError("codegen supports at most one sparse input")
    args: List[Tuple[str, str]] = []
    for kind, t in arrays:
        if kind == "sparse":
            args += [("const int64_t*", "indptr"), ("const int64_t*", "indices"),
                     ("const %s*" % dt, "data")]
        elif kind == "out_sparse" or t.name == out_name:
            args.append(("%s*" % dt, t.name))
        else:
            args.append(("const %s*" % dt, t.name))
    args += [(dt, t.name) for t in scalars]
    args += [("int64_t", d) for d in dims]
    has_sparse = any(kind != "dense" for kind, _ in arrays)
    if has_sparse:
        args.append(("int64_t", "nnz"))
    sig = "void launch_%s(%s)" % (kernel.name, ", ".join("%s %s" % a for a in args))
    info = {"arrays": arrays, "scalars": [t.name for t in scalars], "dims": dims,
            "dtype": kernel.dtypes[0] if kernel.dtypes else "f64",
            "has_sparse": has_sparse, "decls": ["%s %s" % a for a in args]}
    return sig, args, info


def _abi(kernel: Kernel):
    sig, _args, info = abi_of(kernel)
    return sig, info, info["has_sparse"]


# --------------------------------------------------------------------------- #
# expressions -> C text
# --------------------------------------------------------------------------- #
def _fmt_const(v: float) -> str:
    return "%.1f" % v if v == int(v) else repr(v)


def _row_major_strides(shape) -> List[str]:
    strides, acc = [], "1"
    for s in reversed(shape):
        strides.append(acc)
        acc = str(s) if acc == "1" else "%s*%s" % (acc, s)
    return list(reversed(strides))


class _Env:
    """Variable bindings for expression emission.

    ``bind`` maps index names to C expressions, ``p`` is the current nonzero
    position (None outside a compressed loop), ``acc`` the accumulator text
    that stands for a Reduce node, ``data`` the text of the sparse value load.
    """

    def __init__(self, bind: Dict[str, str], p: Optional[str] = None,
                 acc: Optional[str] = None, data: Optional[str] = None):
        self.bind = dict(bind)
        self.p = p
        self.acc = acc
        self.data = data

    def with_(self, **kw) -> "_Env":
        e = _Env(self.bind, self.p, self.acc, self.data)
        for key, val in kw.items():
            if key == "bind":
                e.bind.update(val)
            else:
                setattr(e, key, val)
        return e


def _offset(t, indices: Sequence[Index], env: _Env) -> str:
    terms = []
    for ix, stride in zip(indices, _row_major_strides(t.shape)):
        c = env.bind.get(ix.name, ix.name)
        terms.append(c if stride == "1" else "(%s)*%s" % (c, stride))
    return " + ".join(terms) if terms else "0"


def _cexpr(e: Expr, env: _Env) -> str:
    if isinstance(e, Access):
        t = e.tensor
        if t.order == 0:
            return t.name
        if t.format.is_sparse():
            if env.p is None:
                raise ValueError("sparse access %s outside a compressed loop" % t.name)
            return env.data if env.data is not None else "data[%s]" % env.p
        return "%s[%s]" % (t.name, _offset(t, e.indices, env))
    if isinstance(e, Const):
        return _fmt_const(e.value)
    if isinstance(e, Mul):
        return "(%s * %s)" % (_cexpr(e.left, env), _cexpr(e.right, env))
    if isinstance(e, Add):
        return "(%s + %s)" % (_cexpr(e.left, env), _cexpr(e.right, env))
    if isinstance(e, Reduce):
        if env.acc is None:
            raise ValueError("Reduce encountered without an accumulator")
        return env.acc
    raise TypeError("cannot emit %r" % (e,))


def _extent_for(plan: Plan, index_name: str) -> str:
    """Extent of a dense index, read off any dense access that carries it."""
    accesses: List[Access] = [plan.out]
    for ex in (plan.value_expr, plan.final_expr):
        if ex is not None:
            accesses += [n for n in ex.walk() if isinstance(n, Access)]
    for acc in accesses:
        if acc.tensor.format.is_sparse():
            continue
        for pos, ix in enumerate(acc.indices):
            if ix.name == index_name and pos < len(acc.tensor.shape):
                return str(acc.tensor.shape[pos])
    return "K"


class _W:
    """Indented line writer."""

    def __init__(self):
        self.lines: List[str] = []
        self.depth = 0

    def __call__(self, text: str = "") -> "_W":
        self.lines.append(("  " * self.depth + text) if text else "")
        return self

    def open(self, text: str) -> "_W":
        self(text + " {" if text else "{")
        self.depth += 1
        return self

    def close(self, tail: str = "") -> "_W":
        self.depth -= 1
        self("}" + tail)
        return self

    def text(self) -> str:
        return "\n".join(self.lines)


# --------------------------------------------------------------------------- #
# CPU (OpenMP) emitter -- the CPU baseline
# --------------------------------------------------------------------------- #
def _cpu_compressed_loop(w: _W, plan: Plan, env: _Env, unroll: int,
                         body: Callable[[_W, _Env], None]) -> None:
    """Loop over the row's nonzeros; unrolled by ``unroll`` with a scalar tail."""
    row = env.bind[plan.row_idx.name]
    w("int64_t p = indptr[%s];" % row)
    w("int64_t pend = indptr[%s + 1];" % row)

    def at(pos: str) -> _Env:
        return env.with_(p=pos, bind={plan.col_idx.name: "indices[%s]" % pos})

    if unroll > 1:
        w("int64_t q = p;")
        w.open("for (; q + %d <= pend; q += %d)" % (unroll, unroll))
        for o in range(unroll):
            w.open("")
            body(w, at("q + %d" % o if o else "q"))
            w.close()
        w.close()
        w.open("for (; q < pend; ++q)")
        body(w, at("q"))
        w.close()
    else:
        w.open("for (int64_t q = p; q < pend; ++q)")
        body(w, at("q"))
        w.close()


def _cpu_dense_reduce(w: _W, extent: str, unroll: int, value: Callable[[str], str]) -> None:
    if unroll > 1:
        w("int64_t rq = 0;")
        w.open("for (; rq + %d <= %s; rq += %d)" % (unroll, extent, unroll))
        for o in range(unroll):
            w("acc += %s;" % value("rq + %d" % o))
        w.close()
        w.open("for (; rq < %s; ++rq)" % extent)
        w("acc += %s;" % value("rq"))
        w.close()
    else:
        w.open("for (int64_t kr = 0; kr < %s; ++kr)" % extent)
        w("acc += %s;" % value("kr"))
        w.close()


def _cpu_body(kernel: Kernel, config: Config, plan: Plan, low: Lowering) -> str:
    dt = ctype(config.dtype)
    tile = low.tile if low.tile > 1 else 1
    unroll = low.unroll
    bound = "(%s - 1)" % plan.row_extent if config.inject_bug else plan.row_extent
    w = _W()

    def rows(body: Callable[[_W, _Env], None]) -> None:
        if low.parallel:
            w("#pragma omp parallel for schedule(dynamic, 256)")
        if tile > 1:
            w.open("for (int64_t i_o = 0; i_o < %s; i_o += %d)" % (bound, tile))
            w("int64_t i_hi = (i_o + %d < %s) ? i_o + %d : %s;" % (tile, bound, tile, bound))
            w.open("for (int64_t i_i = i_o; i_i < i_hi; ++i_i)")
            body(w, _Env({plan.row_idx.name: "i_i"}, acc="acc"))
            w.close()
            w.close()
        else:
            w.open("for (int64_t i = 0; i < %s; ++i)" % bound)
            body(w, _Env({plan.row_idx.name: "i"}, acc="acc"))
            w.close()

    if plan.kind == "elementwise":
        ix = plan.out.indices[0]
        if low.parallel:
            w("#pragma omp parallel for schedule(dynamic, 256)")
        w.open("for (int64_t i = 0; i < %s; ++i)" % bound)
        env = _Env({ix.name: "i"})
        w("%s[%s] = %s;" % (plan.out_tensor.name, _offset(plan.out_tensor, plan.out.indices, env),
                            _cexpr(plan.value_expr, env)))
        w.close()

    elif plan.kind == "scalar_reduce":
        def row_body(w: _W, env: _Env) -> None:
            w("%s acc = 0.0;" % dt)
            if plan.reduce_is_compressed:
                _cpu_compressed_loop(w, plan, env, unroll,
                                     lambda w2, e2: w2("acc += %s;" % _cexpr(plan.value_expr, e2)))
            else:
                ext = _extent_for(plan, plan.reduce.index.name)

                def per_nnz(w2: _W, e2: _Env) -> None:
                    _cpu_dense_reduce(w2, ext, unroll, lambda kx: _cexpr(
                        plan.value_expr, e2.with_(bind={plan.reduce.index.name: kx})))
                _cpu_compressed_loop(w, plan, env, 1, per_nnz)
            w("%s[%s] = %s;" % (plan.out_tensor.name,
                                _offset(plan.out_tensor, plan.out.indices, env),
                                _cexpr(plan.final_expr, env)))
        rows(row_body)

    elif plan.kind == "row_dense_out":
        inner = plan.inner_out[0]
        ext = _extent_for(plan, inner.name)

        def write(w2: _W, e2: _Env, kx: str) -> None:
            e3 = e2.with_(bind={inner.name: kx}, acc=None)
            w2("%s[%s] += %s;" % (plan.out_tensor.name,
                                  _offset(plan.out_tensor, plan.out.indices, e3),
                                  _cexpr(plan.value_expr, e3)))

        def per_nnz(w2: _W, e2: _Env) -> None:
            simd = "#pragma omp simd" if low.vector_width > 1 else None
            if unroll > 1:
                # canonical loop forms, so `omp simd` applies to the main loop
                w2("const int64_t ku_end = %s - %s %% %d;" % (ext, ext, unroll))
                if simd:
                    w2(simd)
                w2.open("for (int64_t ku = 0; ku < ku_end; ku += %d)" % unroll)
                for o in range(unroll):
                    write(w2, e2, "ku + %d" % o)
                w2.close()
                w2.open("for (int64_t ku = ku_end; ku < %s; ++ku)" % ext)
                write(w2, e2, "ku")
                w2.close()
            else:
                if simd:
                    w2(simd)
                w2.open("for (int64_t k = 0; k < %s; ++k)" % ext)
                write(w2, e2, "k")
                w2.close()

        rows(lambda w2, e2: _cpu_compressed_loop(w2, plan, e2, unroll, per_nnz))

    elif plan.kind == "sparse_out":
        ext = _extent_for(plan, plan.reduce.index.name)

        def per_nnz(w2: _W, e2: _Env) -> None:
            w2("%s acc = 0.0;" % dt)
            _cpu_dense_reduce(w2, ext, unroll, lambda kx: _cexpr(
                plan.value_expr, e2.with_(bind={plan.reduce.index.name: kx})))
            w2("%s[%s] = %s;" % (plan.out_tensor.name, e2.p, _cexpr(plan.final_expr, e2)))

        rows(lambda w2, e2: _cpu_compressed_loop(w2, plan, e2, 1, per_nnz))
    else:  # pragma: no cover
        raise NotImplementedError(plan.kind)
    return w.text()


# --------------------------------------------------------------------------- #
# shared header
# --------------------------------------------------------------------------- #
def _transform_text(t) -> str:
    if isinstance(t, Tile):
        extra = ("," + t.by if t.by != "rows" else "") + \
            (",gather=" + t.gather if t.gather != "direct" else "")
        return "Tile(%s,%d%s)" % (t.index.name, t.size, extra)
    if isinstance(t, Split):
        return "Split(%s,%d)" % (t.index.name, t.factor)
    if isinstance(t, Parallelize):
        return ("Parallelize(%s,%s,B%d)" % (t.index.name, t.unit, t.block_size)
                if t.block_size else "Parallelize(%s,%s)" % (t.index.name, t.unit))
    if isinstance(t, Unroll):
        return "Unroll(%s,%d)" % (t.index.name, t.factor)
    if isinstance(t, Fuse):
        return "Fuse(%s,%s)" % (t.index_a.name, t.index_b.name)
    if isinstance(t, ThreadsPerRow):
        return "ThreadsPerRow(%d)" % t.k
    if isinstance(t, Vectorize):
        return "Vectorize(%d)" % t.width
    return t.kind


def _header(kernel: Kernel, config: Config, backend: str, low: Lowering,
            extra: Sequence[str] = ()) -> str:
    lines = [
        "// TileGen generated kernel -- DO NOT EDIT BY HAND.",
        "// kernel      : %s" % kernel.name,
        "// backend     : %s" % backend,
        "// config      : %s" % config.to_dict(),
        "// lowering    : %s" % low.to_dict(),
        "// schedule    : %s" % (", ".join(_transform_text(t) for t in kernel.schedule)
                                 if len(kernel.schedule) else "(default)"),
    ]
    lines += ["// %s" % e for e in extra]
    lines.append("// pass log    :")
    lines += ["//   [%s] %s" % (e.get("pass"), e.get("action")) for e in kernel.pass_log] \
        or ["//   (none)"]
    return "\n".join(lines)


def emit_cpu(kernel: Kernel, config: Config) -> str:
    plan, low = _plan(kernel), _lowering(kernel)
    sig, _args, _info = abi_of(kernel)
    body = _cpu_body(kernel, config, plan, low)
    return "\n".join([_header(kernel, config, "cpu", low), "#include <cstdint>",
                      "#include <cstddef>", "", 'extern "C" %s {' % sig, body, "}", ""])


# --------------------------------------------------------------------------- #
# HIP emitter (gfx950, wave64)
# --------------------------------------------------------------------------- #
# Device helpers emitted into every HIP translation unit.  hipRTC provides the
# HIP device builtins without any #include.
_HIP_PRELUDE = r"""
typedef long long tg_i64;
typedef long long tg_i64x2 __attribute__((ext_vector_type(2)));
typedef double tg_f64x2 __attribute__((ext_vector_type(2)));

// Move a double between lanes with a DPP pattern (within a 16-lane row).
template <int CTRL>
__device__ __forceinline__ double tg_dpp(double v) {
  const tg_i64 b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double(((tg_i64)hi << 32) | (tg_i64)(unsigned)lo);
}

// Sum over each aligned group of W consecutive lanes (W divides 64); every lane
// of a group ends with the group's sum.  Butterfly: quad_perm [1,0,3,2] and
// [2,3,0,1], then row_half_mirror and row_mirror (lane i <-> 7-i, 15-i pair the
// two halves once the halves are uniform), then swizzles across 16 and 32.
template <int W>
__device__ __forceinline__ double tg_segsum(double v) {
  if (W >= 2) v += tg_dpp<0xB1>(v);
  if (W >= 4) v += tg_dpp<0x4E>(v);
  if (W >= 8) v += tg_dpp<0x141>(v);
  if (W >= 16) v += tg_dpp<0x140>(v);
  if (W >= 32) v += __shfl_xor(v, 16);
  if (W >= 64) v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ tg_i64 tg_uniform(tg_i64 v) {
  const int lo = __builtin_amdgcn_readfirstlane((int)v);
  const int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
  return ((tg_i64)hi << 32) | (tg_i64)(unsigned)lo;
}

// Value of v held by lane src of the wave (ds_bpermute; every lane active).
__device__ __forceinline__ tg_i64 tg_lane_bcast(tg_i64 v, int src) {
  const int lo = __shfl((int)v, src);
  const int hi = __shfl((int)(v >> 32), src);
  return ((tg_i64)hi << 32) | (tg_i64)(unsigned)lo;
}
"""


def _hip_decls(args: List[Tuple[str, str]]) -> str:
    """Kernel parameter list: the ABI with restrict-qualified pointers."""
    out = []
    for ct, name in args:
        ct = ct.replace("int64_t", "tg_i64")
        if ct.endswith("*"):
            out.append("%s __restrict__ %s" % (ct, name))
        else:
            out.append("const %s %s" % (ct, name))
    return ", ".join(out)


def _lds_total(arrays: Sequence[Tuple[int, int]]) -> int:
    """Bytes of LDS a kernel's ``__shared__`` arrays take, given as (element
    bytes, elements): their sum rounded up to 16 bytes.  The compiler packs a
    kernel's LDS variables by alignment and rounds the block up to the largest
    alignment (8, or 16 where it widens an array for 128-bit accesses), so this
    is the group segment size it reports, or at most 8 bytes more."""
    total = sum(size * count for size, count in arrays)
    return (total + 15) // 16 * 16


def launch_geometry(plan: Plan, low: Lowering) -> LaunchGeometry:
    """Rows per workgroup and LDS bytes of the HIP variant for this schedule.

    The LDS figure adds up every ``__shared__`` array the emitters declare for
    the form (``_lds_total``); the kernels hold all of it statically."""
    B = min(low.block_size, 1024)
    tpr = max(1, low.threads_per_row)
    if plan.kind == "elementwise":
        return LaunchGeometry(B, B, 0, plan.row_extent)
    slots = max(1, B // tpr)
    waves = max(1, B // WAVE)
    rows = low.tile if low.tiled else slots
    if plan.kind == "sparse_out":
        # the chunked and the wave-per-row paths each list their tile's long rows
        lists = [(4, rows), (4, 1), (8, 1)] if low.tiled else []
        return LaunchGeometry(rows, B, _lds_total(lists + lists), plan.row_extent)
    if plan.kind == "row_dense_out":
        V = 2 if low.vector_width >= 2 else 1
        arrays = [(4, rows), (4, 1), (8, B * V), (8, 1)] if low.tiled else []
        return LaunchGeometry(rows, B, _lds_total(arrays), plan.row_extent)
    if plan.kind != "scalar_reduce" or not low.tiled:
        return LaunchGeometry(rows, B, 0, plan.row_extent)
    if low.balance == "stream":
        CH, RB = stream_chunk(low), stream_batch(low)
        lds = _lds_total([(8, CH), (8, RB + 1), (8, 8), (4, RB), (4, 1), (8, waves)])
        return LaunchGeometry(1, B, lds, plan.row_extent, CH, stream=True)
    # a merge-path batch is at least one row per lane group
    tr = max(rows, slots) if low.balance == "nnz" else rows
    arrays = [(8, tr + 1), (4, tr), (4, 1), (8, waves)]   # pointers, long rows, sums
    if tpr <= 16:
        arrays += [(4, tr), (4, 1)]                          # rows left to one wave each
    if low.balance == "hybrid":
        arrays += [(8, 9), (8, 3 * waves), (8, waves), (8, 2)]
    if low.balance == "nnz":
        arrays += [(8, 6)]                                   # the window's rows and bounds
    if low.gather == "sorted":
        # the sort's bucket counts, sorted entries, operands and wave totals
        items = ((tr + slots - 1) // slots) * max(1, low.unroll) * B
        nb = sort_buckets(B)
        arrays += [(4, nb), (8, items), (8, items), (4, nb // 64)]
    chunk = hybrid_chunk(low) if low.balance == "hybrid" else 0
    return LaunchGeometry(rows, B, _lds_total(arrays), plan.row_extent, chunk)


def module_scratch(plan: Plan, low: Lowering) -> bool:
    """Whether the variant's module keeps row-piece partials in its scratch
    (merge-path windows, hybrid tiles and stream ranges), so that launches of it
    must not overlap on one device."""
    return (plan.kind == "scalar_reduce" and low.tiled
            and low.balance in ("nnz", "hybrid", "stream"))


# Stream ranges: at most this many nonzeros per workgroup (their products are
# staged in LDS, 8 bytes each)
STREAM_MAX_CHUNK = 8192


def stream_chunk(low: Lowering) -> int:
    """Nonzeros per workgroup of the stream form: one pass of the whole
    workgroup, U nonzeros per lane."""
    return min(low.block_size, 1024) * max(1, low.unroll)


def stream_batch(low: Lowering) -> int:
    """Row pointers a stream workgroup stages at a time: a range of CH
    nonzeros ends at most CH non-empty rows, so one batch holds all of them
    unless empty rows pile up."""
    return min(1024, max(64, stream_chunk(low)))


def hybrid_chunk(low: Lowering) -> int:
    """Nonzeros per long-row workgroup of hybrid tiles: two passes of the whole
    workgroup; rows longer than half of it are summed by those workgroups."""
    return 2 * min(low.block_size, 1024) * max(1, low.unroll)


def hybrid_long(low: Lowering) -> int:
    """Rows longer than this are summed by the long-row workgroups of hybrid
    tiles: half a range, so at most 3 of them meet one range."""
    return hybrid_chunk(low) // 2


def _check_hip_schedule(plan: Plan, low: Lowering) -> None:
    B, tpr = low.block_size, low.threads_per_row
    if B % WAVE or B <= 0 or B > 1024:
        raise ValueError("HIP block_size must be a multiple of 64 in [64, 1024], got %d" % B)
    if plan.kind != "elementwise":
        if tpr < 1 or tpr > WAVE or WAVE % tpr:
            raise ValueError("HIP threads_per_row must divide 64, got %d" % tpr)
    if low.vector_width not in (1, 2, 4):
        raise ValueError("vector_width %d not supported" % low.vector_width)
    if low.unroll < 1 or low.unroll > 16:
        raise ValueError("unroll must be in 1..16, got %d" % low.unroll)
    if low.tiled and low.tile > 4096:
        raise ValueError("tile_size %d exceeds 4096 rows per workgroup" % low.tile)
    if low.balance != "rows" and not (low.tiled and plan.kind == "scalar_reduce"):
        raise ValueError("balance '%s' needs a tiled kernel that reduces over each row "
                         "(SpMV-shaped); %s %s" % (low.balance, plan.kind,
                                                   "untiled" if not low.tiled else ""))
    if low.gather != "direct" and not (plan.kind == "scalar_reduce" and low.tiled
                                       and low.balance == "rows"):
        raise ValueError("gather '%s' needs an SpMV-shaped kernel with row tiles" % low.gather)
    if low.balance == "stream" and stream_chunk(low) > STREAM_MAX_CHUNK:
        raise ValueError("stream ranges hold at most %d nonzeros (block_size x unroll), got %d"
                         % (STREAM_MAX_CHUNK, stream_chunk(low)))
    lds = launch_geometry(plan, low).lds_bytes
    if lds > LDS_LIMIT:
        form = "sorted row tile" if low.gather == "sorted" else "%s variant" % low.balance
        raise ValueError("this %s (tile %d, block %d) declares %d B of LDS; a gfx950 "
                         "workgroup holds at most %d" % (form, low.tile, B, lds, LDS_LIMIT))


def _long_row_test(length: str, long_: int, huge: int) -> str:
    """Whether a row leaves its lane group for the whole workgroup: longer than
    ``long_`` and either more than 2x the tile's average row or longer than
    ``huge``.  Rows that are uniformly long stay with their lane groups, which
    keep every group equally busy; a row that dwarfs its tile, or one so long
    that one lane group would walk it for too many steps, is shared."""
    n = "(%s)" % length
    return "(%s > %d && (%s * t_rows > 2 * t_nnz || %s > %d))" % (n, long_, n, n, huge)


def _tile_stats(w: _W, TR: int) -> None:
    """t_rows / t_nnz of this workgroup's tile (rows and nonzeros), and a
    zeroed long-row count; ends with a barrier."""
    w("__shared__ tg_i64 s_tnnz;")
    w.open("if (threadIdx.x == 0)")
    w("s_nlong = 0;")
    w("const tg_i64 t_end = row0 + %d < row_end ? row0 + %d : row_end;" % (TR, TR))
    w("s_tnnz = t_end > row0 ? indptr[t_end] - indptr[row0] : 0;")
    w.close()
    w("__syncthreads();")
    w("const tg_i64 t_rows = row_end - row0 < %d ? row_end - row0 : %d;" % (TR, TR))
    w("const tg_i64 t_nnz = s_tnnz;")


# Merge-path windows (balance "nnz"): windows up to MERGE_CAP have scratch slots
# for the pieces of rows longer than a window; rows reaching past them are summed
# whole by the window they begin in.
MERGE_CAP = 65536


def _merge_decls(pre: _W, scratch_arg: bool = False) -> None:
    """File-scope search, scratch and combine of the merge-path SpMV.  With
    ``scratch_arg`` the kernel takes its scratch as a parameter instead of the
    module-scope array."""
    pre(r"""// Merge path: row r occupies items r + indptr[r] .. r + indptr[r + 1] (its
// nonzeros, then one item that ends it); the launch's items are cut into one
// window per workgroup.
//
// Value of v held by lane src (uniform) of the wave.
__device__ __forceinline__ tg_i64 tg_lane_read(tg_i64 v, int src) {
  const int lo = __builtin_amdgcn_readlane((int)v, src);
  const int hi = __builtin_amdgcn_readlane((int)(v >> 32), src);
  return ((tg_i64)hi << 32) | (tg_i64)(unsigned)lo;
}

// First-round probe of lane l around the guess g, ascending with l: 8 rows at
// growing distances below g, 48 consecutive rows around it, 8 at growing
// distances above.  Every round's probes ascend with the lane, so the lanes
// whose row passes a monotone test are the ones from the first such lane on.
__device__ __forceinline__ tg_i64 tg_mp_probe(tg_i64 g, int l) {
  if (l < 8) return g - 24 - ((tg_i64)32 << (2 * (7 - l)));
  if (l < 56) return g - 32 + l;
  return g + 24 + ((tg_i64)32 << (2 * (l - 56)));
}

// Smallest r in [0, R] with r + indptr[r] - base >= t (R when there is none);
// base = indptr[0], X = R + indptr[R] - base, the launch's items.  Run by all
// 64 lanes of one wave, one row pointer per lane per round; the ballot of the
// test gives the bracket's new ends (the first lane that passes and the lane
// before it), read from those lanes.  Each later round probes 64 evenly spaced
// rows of the bracket left, so the bracket shrinks at least 63-fold per round.
__device__ tg_i64 tg_mp_search(const tg_i64* __restrict__ indptr, tg_i64 R, tg_i64 t, tg_i64 X,
                               tg_i64 base) {
  const int l = threadIdx.x & 63;
  const tg_i64 g = X > 0 ? (tg_i64)((double)t * ((double)R / (double)X)) : 0;
  tg_i64 q = tg_mp_probe(g, l);
  tg_i64 lo = 0, hi = R;
  #pragma unroll 1
  for (;;) {
    q = q < lo ? lo : (q > hi ? hi : q);
    const unsigned long long m = __ballot(q + indptr[q] - base >= t);
    const int f = m ? (int)__builtin_ctzll(m) : 64;   // first lane that passes
    const tg_i64 b = f < 64 ? tg_lane_read(q, f) : hi;
    const tg_i64 a = f > 0 ? tg_lane_read(q, f - 1) : lo - 1;   // rows before t
    lo = a + 1;
    hi = b;
    if (lo >= hi) return hi;
    q = lo + (tg_i64)l * ((hi - lo + 62) / 63);
  }
}

// The row holding nonzero position P, pb <= P < pe, where pb = indptr[0] and
// pe = indptr[R]: the one row r with indptr[r] <= P < indptr[r + 1], returned
// with those two bounds in *rs and *re.  Run by all 64 lanes of one wave, with
// the probes of tg_mp_search; the bracket [lo, hi] keeps indptr[lo] <= P <
// indptr[hi] and carries both values, so the bounds cost no load of their own.
__device__ tg_i64 tg_mp_row(const tg_i64* __restrict__ indptr, tg_i64 R, tg_i64 P, tg_i64 pb,
                            tg_i64 pe, tg_i64* rs, tg_i64* re) {
  const int l = threadIdx.x & 63;
  tg_i64 q = tg_mp_probe((tg_i64)((double)(P - pb) * ((double)R / (double)(pe - pb))), l);
  tg_i64 lo = 0, hi = R, vlo = pb, vhi = pe;   // indptr[0] = pb, indptr[R] = pe
  #pragma unroll 1
  for (;;) {
    q = q < lo ? lo : (q > hi ? hi : q);
    const tg_i64 v = indptr[q];
    const unsigned long long m = __ballot(v > P);
    const int f = m ? (int)__builtin_ctzll(m) : 64;   // first lane past P
    if (f < 64) { hi = tg_lane_read(q, f); vhi = tg_lane_read(v, f); }
    if (f > 0) { lo = tg_lane_read(q, f - 1); vlo = tg_lane_read(v, f - 1); }
    if (hi - lo <= 1) {
      *rs = vlo;
      *re = vhi;
      return lo;
    }
    q = lo + 1 + (tg_i64)l * ((hi - lo + 61) / 63);   // rows strictly inside the bracket
  }
}

// Partial sums of the pieces of rows cut at window edges, two per window w: the
// piece of the row that begins in w (slot 2w + 1) and of the row that began
// before it (slot 2w).  A slot holds 0 when empty and bits(partial) ^ TG_MP_KEY
// when full; TG_MP_KEY is a signalling-NaN pattern, which no floating-point
// sum produces, so a full slot is never 0.  Only device-scope atomics touch the
// slots.  Two launches that share the slots must not overlap on one device.
#define TG_MP_KEY 0x7FF4A5A5A5A5A5A5ull
%(DECL)s

// The value must be in a register (so the atomic that produced it has returned)
// before any later memory operation is issued.
__device__ __forceinline__ void tg_mp_wait(unsigned long long v) {
  asm volatile("" :: "v"(v) : "memory");
}

// Wave: record window w's piece t of the row whose pieces lie in windows
// wf..wl.
//
// Two pieces (wl = wf + 1): lane 0 swaps the partial into the first piece's
// slot.  The piece whose swap is performed first finds the slot empty and
// returns false; the other finds its partner's partial, sums the two in window
// order, empties the slot and returns true with the sum in *tot.  One atomic
// round trip.
//
// More pieces: lane 0 swaps the partial into its own slot; once that swap has
// returned, the lanes read every slot of the row (compare-and-swaps that never
// match, so they change nothing).  The piece whose swap is performed last finds every slot
// full (any other piece's read of its slot came later); it may not be the only
// one.  A piece that finds them all sums them in window order with a fixed
// reduction tree, empties them and returns true with the sum in *tot; pieces
// that find an empty slot return false.
//
// Either way every combiner computes the same bits, every slot is empty again
// when the launch ends, and no wave waits for another.
__device__ bool tg_mp_commit(unsigned long long* __restrict__ part, tg_i64 w, tg_i64 wf,
                             tg_i64 wl, double t, double* tot) {
  const int l = threadIdx.x & 63;
  if (wl == wf + 1) {
    unsigned long long other = 0;
    if (l == 0)
      other = __hip_atomic_exchange(part + 2 * wf + 1,
                                    (unsigned long long)__double_as_longlong(t) ^ TG_MP_KEY,
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    other = (unsigned long long)__shfl((long long)other, 0);
    if (other == 0) return false;
    const double o = __longlong_as_double((long long)(other ^ TG_MP_KEY));
    *tot = w == wf ? t + o : o + t;
    if (l == 0)
      (void)__hip_atomic_exchange(part + 2 * wf + 1, 0ull, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  unsigned long long mine = 0;
  if (l == 0)
    mine = __hip_atomic_exchange(part + 2 * w + (w == wf ? 1 : 0),
                                 (unsigned long long)__double_as_longlong(t) ^ TG_MP_KEY,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  tg_mp_wait(__shfl((long long)mine, 0));
  double sum = 0.0;
  #pragma unroll 1
  for (tg_i64 base = wf; base <= wl; base += 64) {
    const tg_i64 v = base + l;
    unsigned long long b = TG_MP_KEY;   // lanes past wl count as full, adding 0.0
    if (v <= wl) {
      // a compare-and-swap that never matches (no slot holds 1) reads the slot where
      // the swaps are performed; an idempotent add or or may be turned into a load
      b = 1ull;
      __hip_atomic_compare_exchange_strong(part + 2 * v + (v == wf ? 1 : 0), &b, 1ull,
                                           __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (__ballot(b == 0) != 0) return false;
    sum += tg_segsum<64>(__longlong_as_double((long long)(b ^ TG_MP_KEY)));
  }
  #pragma unroll 1
  for (tg_i64 base = wf; base <= wl; base += 64) {
    const tg_i64 v = base + l;
    if (v <= wl)
      (void)__hip_atomic_exchange(part + 2 * v + (v == wf ? 1 : 0), 0ull,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  *tot = sum;
  return true;
}
""" % {"DECL": ("// the slots arrive as the kernel's last parameter, tg_part (%d of them)"
                  % (2 * MERGE_CAP)) if scratch_arg else
          ("// module scratch: the host launcher orders each launch after the previous one\n"
           "// on any stream (tg_launch_ordered)\n"
           "__device__ unsigned long long tg_mp_part[%d];" % (2 * MERGE_CAP))})


def _merge_window(w: _W, TR: int, WAVES: int, plan: Plan) -> None:
    """This workgroup's merge-path window, its rows and its row pieces
    (defines pbase, pend, r0, r1, r_own, pc_in, pc_out, s_win, wdx, D, t0, t1).
    The window searches first run on the launch's own numbers, as if
    indptr[0] = 0 and indptr[M] = nnz, so that they wait for no other load;
    once the row pointers have arrived (after the barrier) a workgroup whose
    guess was wrong searches again."""
    w("// merge-path window of this workgroup: items [t0, t1) of the launch's row_lim +")
    w("// pend - pbase (row r is items r + indptr[r] - pbase ... r + indptr[r + 1] - pbase)")
    w("__shared__ tg_i64 s_win[6];  // r0, r1, indptr[r0 - 1], indptr[r0], indptr[r1 - 1], indptr[r1]")
    w("const tg_i64 G = gridDim.x, wdx = blockIdx.x;")
    sel = "threadIdx.x >= 64 && threadIdx.x < 128" if WAVES > 1 else "threadIdx.x < 64"

    def searches(base: str) -> None:
        w("// first and last rows: the first row beginning at or after t0 (t1)")
        w.open("if (threadIdx.x < 64)")
        w("const tg_i64 a = wdx == 0 ? 0 : tg_mp_search(indptr, row_lim, t0, X, %s);" % base)
        w("if (threadIdx.x == 0) s_win[0] = a;")
        w("if (threadIdx.x < 2) s_win[2 + threadIdx.x] = a - 1 + (tg_i64)threadIdx.x >= 0 ? "
          "indptr[a - 1 + threadIdx.x] : 0;")
        w.close()
        w.open("if (%s)" % sel)
        w("const tg_i64 b = wdx == G - 1 ? row_lim : tg_mp_search(indptr, row_lim, t1, X, %s);"
          % base)
        w("const int l = threadIdx.x & 63;")
        w("if (l == 0) s_win[1] = b;")
        w("if (l < 2) s_win[4 + l] = b - 1 + l >= 0 ? indptr[b - 1 + l] : 0;")
        w.close()

    def window(nz: str) -> None:
        w("const tg_i64 X = row_lim + %s;" % nz)
        w("const tg_i64 D = X > G ? (X + G - 1) / G : 1;  // items per window")
        w("const tg_i64 t0 = wdx * D < X ? wdx * D : X;")
        w("const tg_i64 t1 = t0 + D < X ? t0 + D : X;")

    w("tg_i64 vpb, vpe;")
    _positions(w, plan, declare=False)
    w.open("")
    window("(nnz > 0 ? nnz : 0)")
    searches("0")
    w.close()
    w("__syncthreads();")
    w("const tg_i64 pbase = tg_uniform(vpb), pend = tg_uniform(vpe);")
    window("(pend - pbase)")
    w.open("if (pbase != 0 || pend != nnz)")
    w("// the guess was wrong (a block of rows of a larger matrix, or nnz other than the")
    w("// rows' count): the searches again, on the row pointers' numbers")
    searches("pbase")
    w("__syncthreads();")
    w.close()
    w("const tg_i64 r0 = s_win[0], r1 = s_win[1];")
    w("// a row longer than a window is cut at the window edges when every window it")
    w("// reaches has scratch slots (below %d); this window holds a piece of the row that" % MERGE_CAP)
    w("// began before it, if that row reaches into it, and of its own last row")
    w("const bool pc_in = r0 > 0 && s_win[3] - s_win[2] > D && "
      "(r0 - 1 + s_win[3] - pbase - 1) / D < %d && r0 - 1 + s_win[3] - pbase > t0;" % MERGE_CAP)
    w("const bool pc_out = r1 > r0 && s_win[5] - s_win[4] > D && "
      "(r1 - 1 + s_win[5] - pbase - 1) / D < %d;" % MERGE_CAP)
    w("const tg_i64 r_own = pc_out ? r1 - 1 : r1;  // rows summed whole, %d at a time" % TR)


def _value_row_free(plan: Plan) -> bool:
    """Whether the per-nonzero value reads only the sparse value and the
    gathered operand (so it can be formed before the row is known)."""
    g = _gather_operand(plan)
    for n in plan.value_expr.walk():
        if isinstance(n, Access) and n is not g and not n.tensor.format.is_sparse() \
                and n.tensor.order > 0:
            return False
    return True


def _hybrid_ranges(w: _W, plan: Plan, step, out_name: str, B: int, U: int, ALIGN: int,
                   WAVES: int, CH: int, LH: int) -> None:
    """The long-row workgroups of hybrid tiles (defines GL; those workgroups
    return).  Range e holds the positions [pa, pa + CH), pa = (pbase & ~1) + e CH,
    clipped to [p0, p1) inside [pbase, pend); the GL range workgroups take every
    GL-th range, GL from the launch's nnz, so the ranges (and the result) come
    from the row pointers alone.

    A row longer than LH = CH / 2 that meets the range holds p0, p0 + LH or
    p1 - 1, so three waves (one each) find the rows holding those positions
    with ``tg_mp_row``, which returns each row's bounds with it: no scan of
    the rows in between.  The distinct ones longer than LH are the listed
    rows.  All of their nonzeros in the range are then loaded and gathered
    together, each lane holding a fixed set of positions (every load and
    gather issued before any is used), and each lane adds its products into
    the listed rows in a fixed order.  The workgroup reduces each row's
    partial; wave k writes row k directly when the row lies within one range,
    or combines it with the row's other pieces by ``tg_mp_commit`` (in range
    order).  A row whose last range has no scratch slot is summed whole by its
    first range.  The row tiles own every other row."""
    row = plan.row_idx.name
    NS = CH // (B * U)
    if NS * B * U != CH:
        raise ValueError("hybrid range of %d nonzeros is not a whole number of workgroup "
                         "steps (%d)" % (CH, B * U))
    if not _value_row_free(plan):
        raise ValueError("hybrid tiles need a per-nonzero value that reads only the sparse "
                         "value and the gathered operand")
    gathered = _gather_operand(plan)
    col = plan.col_idx.name
    w("// workgroups below GL sum the rows longer than %d nonzeros, over ranges of %d;" % (LH, CH))
    w("// the rest are row tiles, which leave those rows alone.  GL comes from the")
    w("// launch's nnz (it sized the grid), the ranges from the row pointers: range e")
    w("// holds the positions [pa, pa + %d) from the even anchor pal = pbase & ~1 (so" % CH)
    w("// 128-bit pairs stay aligned), clipped to [p0, p1) inside [pbase, pend).  Only the")
    w("// first NL = min(NR, GL) ranges exist: the last of them also sums what the row")
    w("// holding its last position has past it, and a long row beginning past it stays")
    w("// with its row tile (nothing of either when nnz covers the rows' nonzeros)")
    w("const tg_i64 GL = (nnz > 0 ? nnz : 0) / %d + 1;" % CH)
    w.open("if ((tg_i64)blockIdx.x < GL)")
    w("__shared__ tg_i64 s_lr[9];  // the rows holding p0, p0 + LH, p1 - 1: row, start, end")
    w("__shared__ double s_hred[%d];  // [wave][listed row]" % (3 * WAVES))
    w("__shared__ double s_kred[%d];" % WAVES)
    w("const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);")
    w("const tg_i64 e = blockIdx.x;")

    def searches(sb: str, se: str) -> None:
        """Waves 0-2 find the rows holding the range's three probe positions
        among the nonzeros [sb, se) and stage them in s_lr."""
        w("// a row longer than %d that meets [p0, p1) holds p0, p0 + %d or p1 - 1 (one lying"
          % (LH, LH))
        w("// strictly inside the range is longer than half of it, so it holds the middle):")
        w("// wave k finds the row holding the k-th of those positions, with its bounds")
        w("#pragma unroll 1")
        w.open("for (int k = wv; k < 3 && p0 < p1; k += %d)" % WAVES)
        w("const tg_i64 P = k == 0 ? p0 : (k == 1 && p0 + %d < p1 ? p0 + %d : p1 - 1);" % (LH, LH))
        w("tg_i64 rs, re;")
        w("const tg_i64 r = tg_mp_row(indptr, row_end, P, %s, %s, &rs, &re);" % (sb, se))
        w("if ((threadIdx.x & 63) == 0) { s_lr[3 * k] = r; s_lr[3 * k + 1] = rs; "
          "s_lr[3 * k + 2] = re; }")
        w.close()

    w("// The searches first run on the launch's own numbers, as if indptr[0] = 0 and")
    w("// indptr[M] = nnz (the common case), so that they wait for no other load; the")
    w("// guess is checked once the row pointers have arrived, after the barrier.")
    w("tg_i64 vpb, vpe;")
    _positions(w, plan, declare=False)
    w.open("")
    w("const tg_i64 p0 = e * %d, p1 = p0 + %d < nnz ? p0 + %d : (nnz > p0 ? nnz : p0);"
      % (CH, CH, CH))
    searches("0", "nnz")
    w.close()
    w("__syncthreads();")
    w("const tg_i64 pbase = tg_uniform(vpb), pend = tg_uniform(vpe);")
    w("const tg_i64 pal = pbase & ~(tg_i64)1;")
    w("const tg_i64 NR = pend > pbase ? (pend - pal + %d) / %d : 0;" % (CH - 1, CH))
    w("const tg_i64 NL = NR < GL ? NR : GL;")
    w("if (e >= NL) return;")
    w("const bool last = e == NL - 1;")
    w("const tg_i64 pa = pal + e * %d;" % CH)
    w("const tg_i64 p0 = pa > pbase ? pa : pbase, p1 = pa + %d < pend ? pa + %d : pend;"
      % (CH, CH))
    w.open("if (pbase != 0 || pend != nnz)")
    w("// the guess was wrong (a block of rows of a larger matrix, or nnz other than the")
    w("// rows' count): the searches again, on the row pointers' numbers")
    searches("pbase", "pend")
    w("__syncthreads();")
    w.close()
    def load_range(sel: Callable[[int, str], str]) -> None:
        """Indices and values of lane l's positions pa + s B U + l U + u in hi_/hv_,
        with every load issued unconditionally (a load under a lane-varying branch
        is waited for before the branch joins).  ``sel(s, q)`` is the lane's
        condition to load its own positions; other lanes load the range's first
        ones, which the wave shares.  Positions are masked when used."""
        w("tg_i64 hi_[%d]; double hv_[%d];" % (NS * U, NS * U))
        for s_ in range(NS):
            q = "qs%d" % s_
            w("const tg_i64 %s = pa + %d + (tg_i64)threadIdx.x * %d;" % (q, s_ * B * U, U))
            w("const tg_i64 qe%d = %s ? %s : p0;" % (s_, sel(s_, q), q))
        if U % 2 == 0:
            w("// whole range (so p0 = pa, even), 16-byte aligned bases: 128-bit pairs")
            w.open("if (pair_ok && p1 - p0 == %d)" % CH)
            for s_ in range(NS):
                for u in range(0, U, 2):
                    o = s_ * U + u
                    w("{ const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(indices + qe%d + %d));"
                      " hi_[%d] = a.x; hi_[%d] = a.y; }" % (s_, u, o, o + 1))
                    w("{ const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(data + qe%d + %d));"
                      " hv_[%d] = b.x; hv_[%d] = b.y; }" % (s_, u, o, o + 1))
            w.close()
            w.open("else")
        else:
            w.open("")
        w("// a clipped range, or bases only 8-byte aligned: per element, clamped into [p0, p1)")
        for s_ in range(NS):
            for u in range(U):
                o = s_ * U + u
                w("{ const tg_i64 c = qe%d + %d < p1 ? (qe%d + %d >= p0 ? qe%d + %d : p0) : p1 - 1;"
                  " hi_[%d] = __builtin_nontemporal_load(indices + c);"
                  " hv_[%d] = __builtin_nontemporal_load(data + c); }"
                  % (s_, u, s_, u, s_, u, o, o))
        w.close()

    w("// the distinct long rows among them (the positions ascend, so a row found twice is")
    w("// found by neighbouring waves)")
    w("tg_i64 kr[3], ks[3], ke[3];")
    w("bool kl[3];")
    w("#pragma unroll")
    w.open("for (int k = 0; k < 3; ++k)")
    w("kr[k] = tg_uniform(s_lr[3 * k]); ks[k] = tg_uniform(s_lr[3 * k + 1]); "
      "ke[k] = tg_uniform(s_lr[3 * k + 2]);")
    w("kl[k] = ke[k] - ks[k] > %d && (k == 0 || kr[k] != s_lr[3 * k - 3]);" % LH)
    w.close()
    w("if (!kl[0] && !kl[1] && !kl[2]) return;  // no long row meets this range")
    w("// the listed rows' nonzeros in this range: lane l holds p0 + s * %d + l * %d + u" % (
        B * U, U))
    load_range(lambda s_, q: "((%s < p1) & ((kl[0] & (%s + %d > ks[0]) & (%s < ke[0])) | "
               "(kl[1] & (%s + %d > ks[1]) & (%s < ke[1])) | (kl[2] & (%s + %d > ks[2]) & "
               "(%s < ke[2]))))" % (q, q, U, q, q, U, q, q, U, q))
    w("// the products of the listed rows' nonzeros in this range: every gather is issued")
    w("// (other positions gather element 0) before any is used, then the products are")
    w("// selected, so a non-finite x[0] cannot leak in")
    w("double xg_[%d]; bool mk_[%d];" % (NS * U, NS * U))
    for s_ in range(NS):
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w("const tg_i64 pu = qs%d + u;" % s_)
        w("mk_[%d + u] = (pu < p1) & ((kl[0] & (pu >= ks[0]) & (pu < ke[0])) | "
          "(kl[1] & (pu >= ks[1]) & (pu < ke[1])) | (kl[2] & (pu >= ks[2]) & (pu < ke[2])));"
          % (s_ * U))
        w("const tg_i64 cu = mk_[%d + u] ? hi_[%d + u] : 0;" % (s_ * U, s_ * U))
        w("xg_[%d + u] = %s;" % (s_ * U, _cexpr(gathered, _Env({row: "0", col: "cu"}, p="pu"))))
        w.close()
    w("// each lane's products, into the listed rows they belong to, in a fixed order")
    w("double part[3] = {0.0, 0.0, 0.0};")
    w("#pragma unroll")
    w.open("for (int i = 0; i < %d; ++i)" % (NS * U))
    w("const tg_i64 pu = pa + (i / %d) * %d + (tg_i64)threadIdx.x * %d + i %% %d;"
      % (U, B * U, U, U))
    w("const double pv = mk_[i] ? %s : 0.0;" % _value_with(plan, "hv_[i]", "xg_[i]", "0", "hi_[i]"))
    w("#pragma unroll")
    w("for (int k = 0; k < 3; ++k) part[k] += (kl[k] & (pu >= ks[k]) & (pu < ke[k])) ? pv : 0.0;")
    w.close()
    w("// then the workgroup's, per listed row")
    w("#pragma unroll")
    w.open("for (int k = 0; k < 3; ++k)")
    w.open("if (kl[k])")
    w("const double t = tg_segsum<64>(part[k]);")
    w("if ((threadIdx.x & 63) == 0) s_hred[3 * wv + k] = t;")
    w.close()
    w.close()
    w("__syncthreads();")
    w("// wave k writes or combines listed row k")
    w("#pragma unroll 1")
    w.open("for (int k = wv; k < 3; k += %d)" % WAVES)
    w("const tg_i64 r = s_lr[3 * k], rs = s_lr[3 * k + 1], re = s_lr[3 * k + 2];")
    w("if (!(re - rs > %d && (k == 0 || r != s_lr[3 * k - 3]))) continue;" % LH)
    w("// the ranges it spans (ranges past the grid's last do not exist)")
    w("const tg_i64 ef = (rs - pal) / %d, el0 = (re - 1 - pal) / %d;" % (CH, CH))
    w("const tg_i64 el = el0 < NL - 1 ? el0 : NL - 1;")
    w("const bool cut = el > ef && el < %d;" % MERGE_CAP)
    w("if (!cut && el != ef) continue;  // kept whole: summed by its first range below")
    w("double t = 0.0;")
    w("#pragma unroll")
    w("for (int v = 0; v < %d; ++v) t += s_hred[3 * v + k];" % WAVES)
    w.open("if (last && re > p1)")
    w("// the grid's last range: this row's positions past the range, with its own loads")
    w("double tt = 0.0;")
    w("#pragma unroll 1")
    w.open("for (tg_i64 pq = p1 + (threadIdx.x & 63); pq < re; pq += 64)")
    w("const tg_i64 cq = indices[pq];")
    w("tt += %s;" % _value_with(plan, "data[pq]", _cexpr(gathered, _Env({row: "r", col: "cq"},
                                                                       p="pq")), "r", "cq"))
    w.close()
    w("t += tg_segsum<64>(tt);")
    w.close()
    w("double tot = t;")
    w("const bool done = !cut || tg_mp_commit(tg_part, e, ef, el, t, &tot);")
    w.open("if (done && (threadIdx.x & 63) == 0)")
    w("const tg_i64 row = r;")
    env = _Env({row: "row"}, acc="tot")
    w("__builtin_nontemporal_store(%s, %s + %s);" % (
        _cexpr(plan.final_expr, env), out_name, _offset(plan.out_tensor, plan.out.indices, env)))
    w.close()
    w.close()
    w("// rows reaching past the scratch's last range are summed whole by their first range")
    w("#pragma unroll 1")
    w.open("for (int k = 0; k < 3; ++k)")
    w("const tg_i64 row = s_lr[3 * k], rs = s_lr[3 * k + 1], re = s_lr[3 * k + 2];")
    w("if (!(re - rs > %d && (k == 0 || row != s_lr[3 * k - 3]))) continue;" % LH)
    w("if ((rs - pal) / %d != e || ((re - 1 - pal) / %d < NL - 1 ? (re - 1 - pal) / %d : NL - 1) "
      "< %d) continue;" % (CH, CH, CH, MERGE_CAP))
    w("double cacc = 0.0;")
    w("#pragma unroll 1")
    w.open("for (tg_i64 q = (rs & ~(tg_i64)%d) + (tg_i64)threadIdx.x * %d; q < re; q += %d)"
           % (ALIGN - 1, U, B * U))
    step("q", "rs", "re", "cacc", "rs", "re")
    w.close()
    w("cacc = tg_segsum<64>(cacc);")
    w("if ((threadIdx.x & 63) == 0) s_kred[wv] = cacc;")
    w("__syncthreads();")
    w.open("if (threadIdx.x == 0)")
    w("double t = 0.0;")
    w("#pragma unroll")
    w("for (int v = 0; v < %d; ++v) t += s_kred[v];" % WAVES)
    env = _Env({row: "row"}, acc="t")
    w("__builtin_nontemporal_store(%s, %s + %s);" % (
        _cexpr(plan.final_expr, env), out_name, _offset(plan.out_tensor, plan.out.indices, env)))
    w.close()
    w("__syncthreads();")
    w.close()
    w("return;")
    w.close()


def _positions(w: _W, plan: Plan, declare: bool = True) -> None:
    """vpb / vpe: indptr[0] and indptr[M], the first and one-past-last nonzero
    positions of the rows (pbase, pend once read with tg_uniform).  indptr[0]
    may be nonzero: a block of rows of a larger matrix whose indices/data are
    passed whole, as the reference's kernels allow (they walk rows by indptr
    alone and never read nnz).

    They are vector loads, made relaxed atomic so that the compiler neither
    moves them down to their first use nor waits right after them.  Vector
    loads return in order, so a caller issues them just after the loads its
    next wait is for: that wait then covers them at no cost, and no earlier
    wait includes them."""
    w("// indptr[0] and indptr[M] as vector loads (relaxed atomic: issued here, not moved")
    w("// down to their first use, and not waited for at once)")
    if declare:
        w("tg_i64 vpb, vpe;")
    w.open("")
    w("// a global (not flat) pointer: flat loads also count as LDS accesses, so any wait")
    w("// for an LDS access or a scalar load would wait for them too")
    w("typedef const __attribute__((address_space(1))) tg_i64 tg_gi64;")
    w("tg_gi64* ip_ = (tg_gi64*)indptr;")
    w('asm volatile("" : "+v"(ip_));')
    w("vpb = __hip_atomic_load(ip_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);")
    w("vpe = __hip_atomic_load(ip_ + %s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);"
      % plan.row_extent)
    w.close()


def _hip_stream_reduce(w: _W, plan: Plan, low: Lowering, bound: str, geo: LaunchGeometry,
                       out_name: str, pre: _W, scratch_arg: bool = False) -> None:
    """y[row] = final(sum over the row's nonzeros of value_expr), one equal range of
    nonzeros per workgroup (``balance == "stream"``).

    Range e takes the nonzero positions [p0, p1): the CH = B U positions from
    pa = (pbase & ~1) + e CH, clipped to [pbase, pend) = [indptr[0], indptr[M])
    (the even anchor keeps 128-bit pairs aligned when indptr[0] is odd), and
    owns the rows [ra, rb): ra is the row holding p0 (0 for e = 0, so the first
    range also owns the empty rows ahead of the first nonzero) and rb the row
    holding p1 (M for the last range).  Every row belongs to exactly one range:
    the one its last nonzero lies in (for an empty row, the one its position
    lies in).  The ranges come from the row pointers; workgroup g takes ranges
    g, g + G, ... (G = the grid, sized from nnz), so the launch's nnz changes
    the grid and never the result.

    1. Every lane loads its U nonzeros (128-bit (index, value) pairs, coalesced
       over the workgroup), then waves 0 and 1 find ra and rb with
       ``tg_st_row`` (the merge path's row search with a first round spread
       over 2048 rows either side of the proportional guess) while those
       loads are in flight.  The operands are
       gathered and the products staged in LDS.  Nothing here depends on row
       lengths, so the matrix streams at full width however skewed it is.
    2. After one barrier, the row pieces cut at range edges are committed
       first, so that their atomic round trips overlap the row sums: wave 0
       the last piece of row ra when it began in an earlier range, wave 1 this
       range's piece of row rb.  ``tg_mp_commit`` adds the pieces in range
       order.
    3. The owned rows' pointers are staged RB at a time, and each row is summed
       from the staged products by a lane group of TPR lanes (DPP); rows over
       64 nonzeros are listed and summed by one wave each.
    4. A row with a piece in a range past the scratch's MERGE_CAP ranges is
       summed whole, with its own loads, by the whole workgroup of the range it
       begins in, the waves' sums added in wave order.
    """
    if not _value_row_free(plan):
        raise ValueError("stream ranges need a per-nonzero value that reads only the sparse "
                         "value and the gathered operand")
    B = geo.block
    TPR = max(1, low.threads_per_row)
    U = max(1, low.unroll)
    CH, RB = stream_chunk(low), stream_batch(low)
    WAVES = B // WAVE
    SLOTS = B // TPR
    row = plan.row_idx.name
    col = plan.col_idx.name
    gathered = _gather_operand(plan)

    def pos(u: int) -> str:
        """Position in the range of lane threadIdx.x's u-th nonzero."""
        if U % 2 == 0:
            return "2 * (%d + (int)threadIdx.x)%s" % ((u // 2) * B, " + 1" if u % 2 else "")
        return "%d + (int)threadIdx.x" % (u * B)

    def gather(col_text: str) -> str:
        return _cexpr(gathered, _Env({row: "row", col: col_text}, p="pq"))

    def store(acc: str, row_text: str) -> None:
        w("const tg_i64 row = %s;" % row_text)
        env = _Env({row: "row"}, acc=acc)
        w("__builtin_nontemporal_store(%s, %s + %s);" % (
            _cexpr(plan.final_expr, env), out_name, _offset(plan.out_tensor, plan.out.indices, env)))

    def tail(lo: str, hi: str, acc: str) -> None:
        """One wave adds the row's positions [lo, hi) past the staged ones, with its
        own loads (only the grid's last range, when nnz undercounts the rows'
        nonzeros, has any)."""
        w.open("if (ps < p1)")  # uniform: false unless nnz undercounts
        w("#pragma unroll 1")
        w.open("for (tg_i64 pq = (%s) + l; pq < (%s); pq += 64)" % (lo, hi))
        w("const tg_i64 cq = indices[pq];")
        w("%s += %s;" % (acc, _value_with(plan, "data[pq]", gather("cq"), row, "cq")))
        w.close()
        w.close()

    _merge_decls(pre, scratch_arg)
    pre(r"""// The row holding nonzero position P, pb <= P < pe (pb = indptr[0], pe = indptr[R]),
// with its bounds in *rs and *re: tg_mp_row's contract and later rounds, with a first
// round for skewed rows.  It probes every 64th row across 2048 rows either side of the
// proportional guess, so a row that close is found in two rounds (the second probes its
// bracket row by row); the rows of a power-law or dense-row matrix lie within that
// distance of the guess.
__device__ tg_i64 tg_st_row(const tg_i64* __restrict__ indptr, tg_i64 R, tg_i64 P, tg_i64 pb,
                            tg_i64 pe, tg_i64* rs, tg_i64* re) {
  const int l = threadIdx.x & 63;
  tg_i64 q = (tg_i64)((double)(P - pb) * ((double)R / (double)(pe - pb))) + (tg_i64)(l - 32) * 64;
  tg_i64 lo = 0, hi = R, vlo = pb, vhi = pe;   // indptr[0] = pb, indptr[R] = pe
  #pragma unroll 1
  for (;;) {
    q = q < lo ? lo : (q > hi ? hi : q);
    const tg_i64 v = indptr[q];
    const unsigned long long m = __ballot(v > P);
    const int f = m ? (int)__builtin_ctzll(m) : 64;   // first lane past P
    if (f < 64) { hi = tg_lane_read(q, f); vhi = tg_lane_read(v, f); }
    if (f > 0) { lo = tg_lane_read(q, f - 1); vlo = tg_lane_read(v, f - 1); }
    if (hi - lo <= 1) {
      *rs = vlo;
      *re = vhi;
      return lo;
    }
    q = lo + 1 + (tg_i64)l * ((hi - lo + 61) / 63);   // rows strictly inside the bracket
  }
}
""")
    if not scratch_arg:
        w("unsigned long long* const tg_part = tg_mp_part;")
    w("const tg_i64 row_end = %s;  // rows written" % bound)
    w("const tg_i64 n_rows = %s;  // rows of the matrix" % plan.row_extent)
    w("__shared__ double s_prod[%d];  // this range's products" % CH)
    w("__shared__ tg_i64 s_ptr[%d];  // owned rows' pointers, %d rows at a time" % (RB + 1, RB))
    w("__shared__ tg_i64 s_b[8];  // the rows holding p0 and p1: row, start, end; indptr[0], indptr[M]")
    w("__shared__ int s_long[%d];  // staged rows over 64 nonzeros" % RB)
    w("__shared__ int s_nlong;")
    w("__shared__ double s_wsum[%d];  // the waves' sums of a row past the scratch" % WAVES)
    w("const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);")
    w("const int l = threadIdx.x & 63;")
    w("tg_i64 vpb, vpe;  // indptr[0] and indptr[M], loaded during phase 1")
    if U % 2 == 0:
        w("// 128-bit (index, value) pair loads need 16-byte aligned bases; a caller's")
        w("// sub-buffer may be only 8-byte aligned, which takes the per-element loads")
        w("const bool pair_ok = ((((unsigned long long)indices) | "
          "((unsigned long long)data)) & 15) == 0;")
    w("const tg_i64 e = blockIdx.x;")

    def phase1(positions: bool) -> None:
        """Stage the range's products and find its bounding rows, for positions
        pa + q, q in [qlo, qhi), and the rows holding P0 and P1 among the
        nonzeros [sb, se); with ``positions`` (the first run, whose qlo is 0),
        also load indptr[0] and indptr[M] once the range's own loads are issued."""
        def inr(q: str) -> str:
            # staged position q; the first run's qlo is 0, which q never falls below
            return "(%s < qhi)" % q if positions else "((%s >= qlo) & (%s < qhi))" % (q, q)

        w("// 1. this range's indices and values, every load issued before any is used")
        w("tg_i64 ci[%d]; double cv[%d];" % (U, U))
        if U % 2 == 0:
            for u in range(0, U, 2):
                w.open("")
                w("const int q = %s;" % pos(u))
                w.open("if (pair_ok && %sq + 1 < qhi)" % ("" if positions else "q >= qlo && "))
                w("const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(indices + pa + q));")
                w("const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(data + pa + q));")
                w("ci[%d] = a.x; ci[%d] = a.y; cv[%d] = b.x; cv[%d] = b.y;" % (u, u + 1, u, u + 1))
                w.close()
                w.open("else")
                for d in (0, 1):
                    w("ci[%d] = %s ? __builtin_nontemporal_load(indices + pa + q + %d) : 0;"
                      % (u + d, inr("q + %d" % d), d))
                    w("cv[%d] = %s ? __builtin_nontemporal_load(data + pa + q + %d) : 0.0;"
                      % (u + d, inr("q + %d" % d), d))
                w.close()
                w.close()
        else:
            for u in range(U):
                w.open("")
                w("const int q = %s;" % pos(u))
                w("ci[%d] = %s ? __builtin_nontemporal_load(indices + pa + q) : 0;" % (u, inr("q")))
                w("cv[%d] = %s ? __builtin_nontemporal_load(data + pa + q) : 0.0;" % (u, inr("q")))
                w.close()
        if positions:
            w("// wave 0 alone loads indptr[0] and indptr[M] (for the check after the barrier)")
            w.open("if (wv == 0)")
            _positions(w, plan, declare=False)
            w.close()
        w("if (threadIdx.x == 0) s_nlong = 0;")
        w("// the rows holding P0 (wave 0) and P1 (wave 1), searched while the loads are in")
        w("// flight; the first range owns the rows from 0, the last the rows up to M")
        w("#pragma unroll 1")
        w.open("for (int k = wv; k < 2; k += %d)" % WAVES)
        w("const tg_i64 P = k == 0 ? P0 : P1;")
        w("tg_i64 r = n_rows, rs = se, re = se;")
        w("if (k == 0 && e == 0) { r = 0; rs = sb; re = sb; }")
        w("else if (P < se) r = tg_st_row(indptr, n_rows, P, sb, se, &rs, &re);")
        w("if (l == 0) { s_b[3 * k] = r; s_b[3 * k + 1] = rs; s_b[3 * k + 2] = re; }")
        w.close()
        if positions:
            w("if (threadIdx.x == 0) { s_b[6] = vpb; s_b[7] = vpe; }")
        w("// the operands (positions past the range gather nothing) and the products, in LDS")
        w("double xv[%d];" % U)
        for u in range(U):
            w("{ const int q = %s; xv[%d] = %s ? %s : 0.0; }"
              % (pos(u), u, inr("q"), gather("ci[%d]" % u)))
        for u in range(U):
            w("{ const int q = %s; if %s s_prod[q] = %s; }"
              % (pos(u), inr("q") if not positions else "(q < qhi)",
                 _value_with(plan, "cv[%d]" % u, "xv[%d]" % u, row, "ci[%d]" % u)))

    w("// Phase 1 first runs on the launch's own numbers, as if indptr[0] = 0 and")
    w("// indptr[M] = nnz (the common case), so that its loads wait for nothing: range e")
    w("// stages the positions [e %d, (e + 1) %d) below nnz.  Once the row pointers have" % (CH, CH))
    w("// arrived (after the barrier) the guess is checked, and a workgroup whose guess")
    w("// was wrong runs phase 1 again on the row pointers' numbers (below).")
    w.open("")
    w("const tg_i64 pa = e * %d, sb = 0, se = nnz;" % CH)
    w("const int qlo = 0, qhi = (int)(nnz > pa ? (nnz - pa < %d ? nnz - pa : %d) : 0);" % (CH, CH))
    w("const tg_i64 P0 = pa, P1 = pa + qhi;")
    phase1(True)
    w.close()
    w("__syncthreads();")
    w("const tg_i64 pbase = tg_uniform(s_b[6]), pend = tg_uniform(s_b[7]);")
    w("// range e stages the positions [pa, pa + %d), pa = pal + e * %d from the even"
      % (CH, CH))
    w("// anchor pal = pbase & ~1 (so 128-bit pairs stay aligned), clipped to [p0, ps) inside")
    w("// [pbase, pend); a matrix without nonzeros still has one range, which writes its")
    w("// empty rows.  The ranges come from the row pointers and the grid from nnz: only")
    w("// the first NL = min(NR, grid) ranges exist, and the last of them owns every row up")
    w("// to M, summing what lies past its staged positions with its own loads (nothing")
    w("// when nnz covers the rows' nonzeros), so nnz never changes the product")
    w("const tg_i64 pal = pbase & ~(tg_i64)1;")
    w("const tg_i64 NR = pend > pbase ? (pend - pal + %d) / %d : 1;" % (CH - 1, CH))
    w("const tg_i64 NL = NR < (tg_i64)gridDim.x ? NR : (tg_i64)gridDim.x;")
    w("if (e >= NL) return;")
    w("const bool last = e == NL - 1;")
    w("const tg_i64 pa = pal + e * %d;" % CH)
    w("const tg_i64 p0 = pa > pbase ? pa : pbase;")
    w("const tg_i64 ps = pa + %d < pend ? pa + %d : pend;  // end of the staged positions"
      % (CH, CH))
    w("const tg_i64 p1 = last ? pend : ps;  // end of the positions this range owns")
    w("// staged positions pa + q, q in [qlo, qhi)")
    w("const int qlo = (int)(p0 - pa), qhi = (int)(ps - pa);")
    w.open("if (pbase != 0 || pend != nnz)")
    w("// the guess was wrong (a block of rows of a larger matrix, or nnz other than the")
    w("// rows' count): phase 1 again, on the row pointers' numbers")
    w("const tg_i64 sb = pbase, se = pend, P0 = p0, P1 = p1;")
    phase1(False)
    w("__syncthreads();")
    w.close()
    def phases(general: bool) -> None:
        """Phases 2-4 after the barrier.  Without ``general`` (indptr[0] = 0 and
        indptr[M] = nnz: every range's staged positions end where its owned ones do)
        there are no tail loads, no ranges past the grid and no partly staged rows."""
        w("const tg_i64 ra = s_b[0], ra_s = s_b[1], ra_e = s_b[2];")
        w("const tg_i64 rb = s_b[3], rb_s = s_b[4], rb_e = s_b[5];")
        w("// row ra began in an earlier range, so this range holds its last piece")
        w("const bool ra_cut = e > 0 && ra < rb && ra_s < p0;")
        w("// 2. the pieces cut at range edges first, so that their atomics overlap the row sums")
        w.open("if (wv == 0 && ra_cut)")
        w("// the ranges it spans (ra ends in this range: it holds p0 and ends before rb)")
        w("const tg_i64 ef = (ra_s - pal) / %d, el = e;" % CH)
        w.open("if (el < %d)" % MERGE_CAP)
        w("const int en = (int)(ra_e - pa);")
        w("double t = 0.0;")
        w("#pragma unroll 4")
        w("for (int q = qlo + l; q < (en < qhi ? en : qhi); q += 64) t += s_prod[q];")
        if general:
            tail("ps > ra_s ? ps : ra_s", "ra_e", "t")
        w("t = tg_segsum<64>(t);")
        w("double tot = t;")
        w.open("if (tg_mp_commit(tg_part, e, ef, el, t, &tot) && l == 0 && ra < row_end)")
        store("tot", "ra")
        w.close()
        w.close()
        w("// otherwise the range it begins in sums it whole (below)")
        w.close()
        w.open("if (wv == %d && rb < n_rows && rb_s < p1)" % (1 if WAVES > 1 else 0))
        w("const tg_i64 ef = (rb_s - pal) / %d, el0 = (rb_e - 1 - pal) / %d;" % (CH, CH))
        if general:
            w("const tg_i64 el = el0 < NL - 1 ? el0 : NL - 1;  // ranges past the grid's last do not exist")
        else:
            w("const tg_i64 el = el0;")
        w.open("if (el < %d)" % MERGE_CAP)
        w("const int st = (int)((rb_s > p0 ? rb_s : p0) - pa);")
        w("double t = 0.0;")
        w("#pragma unroll 4")
        w("for (int q = st + l; q < qhi; q += 64) t += s_prod[q];")
        w("t = tg_segsum<64>(t);")
        w("double tot = t;")
        w.open("if (tg_mp_commit(tg_part, e, ef, el, t, &tot) && l == 0 && rb < row_end)")
        store("tot", "rb")
        w.close()
        w.close()
        w("// otherwise, when it begins here, this workgroup sums it whole (below)")
        w.close()
        w("// 3. the owned rows [ra, rb), %d row pointers at a time" % RB)
        w("const int lane = threadIdx.x %% %d;" % TPR)
        w("const int slot = threadIdx.x / %d;" % TPR)
        w("#pragma unroll 1")
        w.open("for (tg_i64 b0 = ra; b0 < rb; b0 += %d)" % RB)
        w("const int nb = (int)(rb - b0 < %d ? rb - b0 : %d);" % (RB, RB))
        w("for (int i = threadIdx.x; i <= nb; i += %d) s_ptr[i] = indptr[b0 + i];" % B)
        w("__syncthreads();")
        w("// rows of up to 64 nonzeros: one lane group each")
        w("#pragma unroll 1")
        w.open("for (int i = slot; i < nb; i += %d)" % SLOTS)
        w("const tg_i64 rs = s_ptr[i], re = s_ptr[i + 1];")
        w("const int st = (int)((rs > p0 ? rs : p0) - pa), en = (int)(re - pa);")
        w("const bool mine = !(b0 + i == ra && ra_cut);  // a cut ra was committed above")
        w("const bool own = mine && en - st <= 64%s;%s" % (
            (" && en <= qhi", "  // staged whole") if general else ("", "")))
        w("double acc = 0.0;")
        w.open("if (own)")
        w("#pragma unroll 4")
        w("for (int q = st + lane; q < en; q += %d) acc += s_prod[q];" % TPR)
        w.close()
        w("if (mine && !own && lane == 0) s_long[atomicAdd(&s_nlong, 1)] = i;")
        w("acc = tg_segsum<%d>(acc);" % TPR)
        w.open("if (own && lane == 0 && b0 + i < row_end)")
        store("acc", "b0 + i")
        w.close()
        w.close()
        w("__syncthreads();")
        w("// longer rows: one wave each")
        w("const int nl = s_nlong;")
        w("#pragma unroll 1")
        w.open("for (int k = wv; k < nl; k += %d)" % WAVES)
        w("const int i = s_long[k];")
        w("const tg_i64 rs = s_ptr[i], re = s_ptr[i + 1];")
        w("const int st = (int)((rs > p0 ? rs : p0) - pa), en = (int)(re - pa);")
        w("double acc = 0.0;")
        w("#pragma unroll 4")
        w("for (int q = st + l; q < (en < qhi ? en : qhi); q += 64) acc += s_prod[q];")
        if general:
            tail("ps > rs ? ps : rs", "re", "acc")
        w("acc = tg_segsum<64>(acc);")
        w.open("if (l == 0 && b0 + i < row_end)")
        store("acc", "b0 + i")
        w.close()
        w.close()
        w("__syncthreads();  // every wave has read s_nlong, s_long and s_ptr")
        w("if (threadIdx.x == 0) s_nlong = 0;")
        w.close()
        w("// 4. row rb, when it begins in this range and reaches past the scratch's last range:")
        w("// summed whole by the whole workgroup with its own loads, the waves' sums added in")
        w("// wave order (the condition is the same for every wave)")
        last_range = ("((rb_e - 1 - pal) / %d < NL - 1 ? (rb_e - 1 - pal) / %d : NL - 1)" % (CH, CH)
                      if general else "(rb_e - 1 - pal) / %d" % CH)
        w.open("if (rb < n_rows && rb_s < p1 && (rb_s - pal) / %d == e && %s >= %d)"
               % (CH, last_range, MERGE_CAP))
        w("double t = 0.0;")
        w("#pragma unroll 4")
        w.open("for (tg_i64 pq = rb_s + (tg_i64)threadIdx.x; pq < rb_e; pq += %d)" % B)
        w("const tg_i64 cq = indices[pq];")
        w("t += %s;" % _value_with(plan, "data[pq]", gather("cq"), row, "cq"))
        w.close()
        w("t = tg_segsum<64>(t);")
        w("if (l == 0) s_wsum[wv] = t;")
        w("__syncthreads();")
        w.open("if (threadIdx.x == 0 && rb < row_end)")
        w("double tot = 0.0;")
        w("#pragma unroll")
        w("for (int v = 0; v < %d; ++v) tot += s_wsum[v];" % WAVES)
        store("tot", "rb")
        w.close()
        w.close()

    w("// 2-4 twice: the common case (indptr[0] = 0, indptr[M] = nnz), where every range's")
    w("// staged positions end where its owned ones do, without the code for other cases")
    w.open("if (pbase == 0 && pend == nnz)")
    phases(False)
    w.close()
    w.open("else")
    phases(True)
    w.close()


SORT_MAX_ITEMS = 8192   # slots of a sorted tile's first step (13 bits in an LDS entry)
SORT_ZPAD = 1024        # zeros read by a sorted tile's guessed loads without a guess (>= 64 x 8 + 2)


def sort_buckets(block: int) -> int:
    """Buckets of a sorted tile: the largest power of two <= the workgroup
    (at least one wave)."""
    nb = 64
    while nb * 2 <= block:
        nb *= 2
    return nb


def _sorted_first_step(w: _W, plan: Plan, R: int, U: int, B: int, SLOTS: int,
                       fpos: Callable[[str, int], str], row: str) -> None:
    """The tile's first-step gathers in operand order (``gather == "sorted"``).

    Every lane holds R x U first-step nonzeros (fci/fcv), slot
    (r U + u) B + threadIdx.x of the tile.  Their columns are counting-sorted
    in LDS by bucket col >> sshift (NB buckets): an atomic add per item gives
    its rank in its bucket, an exclusive scan gives the buckets' offsets, and
    each item writes (col << 13 | slot) to its sorted place.  Lane t then takes
    the sorted items k B + t, so the 64 lanes of a gather instruction take 64
    consecutive sorted items and share lines of the operand, and stores each
    operand in s_x at the item's slot.  Each lane reads its own items' operands
    back and sums them in the order of the direct gathers, so the result bits
    are the same.  Positions outside their row take part in nothing."""
    gathered = _gather_operand(plan)
    NB = sort_buckets(B)
    w("// this tile's first-step nonzeros, sorted by operand bucket (col >> sshift)")
    w("bool fok[%d][%d]; int fky[%d][%d]; unsigned frk[%d][%d];" % (R, U, R, U, R, U))
    w("#pragma unroll")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    for u in range(U):
        w.open("")
        w("const tg_i64 pu = %s;" % fpos("rs[r]", u))
        w("fok[r][%d] = (pu >= rs[r]) & (pu < re[r]);" % u)
        w.close()
    w("#pragma unroll")
    w.open("for (int u = 0; u < %d; ++u)" % U)
    w("fky[r][u] = fok[r][u] ? (int)(fci[r][u] >> sshift) : 0;")
    w("frk[r][u] = fok[r][u] ? atomicAdd(&s_hist[fky[r][u]], 1u) : 0u;  // rank in its bucket")
    w.close()
    w.close()
    w("__syncthreads();")
    w("// exclusive scan of the %d buckets: each wave's, then the waves' totals" % NB)
    w("unsigned sh_ = 0u, sv_ = 0u;")
    w.open("if (threadIdx.x < %d)" % NB)
    w("sh_ = s_hist[threadIdx.x];")
    w("sv_ = sh_;")
    w("#pragma unroll")
    w.open("for (int d = 1; d < 64; d <<= 1)")
    w("const unsigned o = __shfl_up(sv_, d);")
    w("if ((threadIdx.x & 63) >= d) sv_ += o;")
    w.close()
    w("if ((threadIdx.x & 63) == 63) s_swsum[threadIdx.x >> 6] = sv_;")
    w.close()
    w("__syncthreads();")
    w("unsigned nsort = 0u, sbase = 0u;")
    w("#pragma unroll")
    w.open("for (int v = 0; v < %d; ++v)" % (NB // 64))
    w("if (v < (int)(threadIdx.x >> 6)) sbase += s_swsum[v];")
    w("nsort += s_swsum[v];")
    w.close()
    w("if (threadIdx.x < %d) s_hist[threadIdx.x] = sbase + sv_ - sh_;" % NB)
    w("__syncthreads();")
    w("#pragma unroll")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    w("#pragma unroll")
    w.open("for (int u = 0; u < %d; ++u)" % U)
    w("if (fok[r][u]) s_ent[s_hist[fky[r][u]] + frk[r][u]] = "
      "((unsigned long long)fci[r][u] << 13) | (unsigned)((r * %d + u) * %d + threadIdx.x);"
      % (U, B))
    w.close()
    w.close()
    w("__syncthreads();")
    w("// the gathers, 64 consecutive sorted items per instruction")
    w("#pragma unroll")
    w.open("for (int k = 0; k < %d; ++k)" % (R * U))
    w("const unsigned sk = (unsigned)(k * %d) + threadIdx.x;" % B)
    w.open("if (sk < nsort)")
    w("const unsigned long long e = s_ent[sk];")
    w("const tg_i64 cu = (tg_i64)(e >> 13);")
    w("s_x[e & 8191u] = %s;" % _cexpr(gathered, _Env({row: "0", plan.col_idx.name: "cu"},
                                                         p="0")))
    w.close()
    w.close()
    w("__syncthreads();")
    w("#pragma unroll")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    w("const tg_i64 row = row0 + slot + r * %d;" % SLOTS)
    w("(void)row;")
    w("#pragma unroll")
    w.open("for (int u = 0; u < %d; ++u)" % U)
    w("const double xs_ = fok[r][u] ? s_x[(r * %d + u) * %d + threadIdx.x] : 0.0;" % (U, B))
    w("acc[r] = fok[r][u] ? acc[r] + %s : acc[r];"
      % _value_with(plan, "fcv[r][u]", "xs_", row, "fci[r][u]"))
    w.close()
    w.close()


def _hip_scalar_reduce(w: _W, plan: Plan, low: Lowering, bound: str, geo: LaunchGeometry,
                       out_name: str, pre: Optional[_W] = None,
                       scratch_arg: bool = False) -> None:
    """y[row] = final(sum over the row's nonzeros of value_expr).

    Tiled variants also balance skewed rows without any preprocessing: a row
    longer than LONG nonzeros (8 lane-group steps) is not walked by its lane
    group; the group appends it to an LDS list, and after the lane-group phase
    the whole workgroup takes each listed row in turn with coalesced loads and
    a wave + LDS reduction.  Lane groups of 16 lanes or fewer add a middle
    tier: rows over 2 group steps and up to 4 wave steps go to a second list
    whose rows the waves share out, one row per wave at a time, reduced within
    the wave (no barrier); only rows past that go to the workgroup.

    With ``balance == "nnz"`` the workgroups split the merge path (every row
    counts one item plus one per nonzero) into equal windows, one per T rows
    of extent, instead of taking T rows each.  Workgroup w finds its window's
    first and last rows with a 64-wide search of the row pointers, then runs
    the body above over the rows whose first nonzero lies in its window, T
    rows at a time.  A row longer than a window is cut at the window edges;
    each window sums its piece with the whole workgroup and the piece that
    finishes last adds the pieces up in window order (``_merge_decls``).
    """
    if low.tiled and low.balance == "stream":
        if pre is None:
            raise ValueError("stream ranges need file-scope declarations")
        _hip_stream_reduce(w, plan, low, bound, geo, out_name, pre, scratch_arg)
        return
    B, TPR = geo.block, max(1, low.threads_per_row)
    U = max(1, low.unroll)
    SLOTS = B // TPR
    TR = geo.rows_per_block
    R = (TR + SLOTS - 1) // SLOTS
    ALIGN = 2 if U % 2 == 0 else 1
    STEP = TPR * U
    LONG = 8 * STEP    # longer rows leave their lane group
    WAVES = B // WAVE
    coop = low.tiled
    # narrow lane groups also hand a row over 2 steps that is more than twice
    # its tile's average to a whole wave (rows over 8 steps always leave), and
    # rows over 4 wave steps go to the workgroup
    wave_tier = coop and TPR <= 16
    if wave_tier:
        MED = 2 * STEP
        WLONG = 4 * WAVE * U
    row = plan.row_idx.name
    col = plan.col_idx.name
    gathered = _gather_operand(plan)

    def step(q: str, lo: str, hi: str, acc: str, glo: str = "glo", ghi: str = "ghi") -> None:
        """Load U consecutive nonzeros at q (masked to [lo, hi)), gather, FMA.
        Loads touch only positions in [glo, ghi) (the tile's nonzeros, or the
        row's where no tile is staged), which hold [lo, hi)."""
        w("tg_i64 ci[%d]; double cv[%d];" % (U, U))
        if U % 2 == 0:
            w.open("if (pair_ok && %s >= %s && %s + %d <= %s)" % (q, glo, q, U, ghi))
            for u in range(0, U, 2):
                w("{ const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(indices + %s + %d));"
                  " ci[%d] = a.x; ci[%d] = a.y; }" % (q, u, u, u + 1))
                w("{ const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(data + %s + %d));"
                  " cv[%d] = b.x; cv[%d] = b.y; }" % (q, u, u, u + 1))
            w.close()
            w.open("else")
        else:
            w.open("")
        for u in range(U):
            w("ci[%d] = ((%s + %d >= %s) & (%s + %d < %s)) ? "
              "__builtin_nontemporal_load(indices + %s + %d) : 0;" % (u, q, u, glo, q, u, ghi, q, u))
            w("cv[%d] = ((%s + %d >= %s) & (%s + %d < %s)) ? "
              "__builtin_nontemporal_load(data + %s + %d) : 0.0;" % (u, q, u, glo, q, u, ghi, q, u))
        w.close()
        w("double xv[%d]; bool ok[%d];" % (U, U))
        w("// positions outside the row gather element 0 (every gather of the step is issued")
        w("// before any is used) and leave the sum as it was, so a non-finite x[0] cannot")
        w("// leak in")
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w("const tg_i64 pu = %s + u;" % q)
        w("ok[u] = (pu >= %s) & (pu < %s);" % (lo, hi))
        w("ci[u] = ok[u] ? ci[u] : 0;")
        w("xv[u] = %s;" % _cexpr(gathered, _Env({row: "row", col: "ci[u]"}, p="pu")))
        w.close()
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w("%s = ok[u] ? %s + %s : %s;" % (acc, acc, _value_with(plan, "cv[u]", "xv[u]", row,
                                                                   "ci[u]"), acc))
        w.close()

    # positions of a lane's first-step nonzeros: U consecutive ones, or, where a lane
    # group holds several rows' first steps at once (R > 1, U >= 4 even), its U / 2
    # pairs interleaved with the other lanes of its group (pair k at 2 lane + 2 TPR k),
    # so that a pair-load instruction covers whole lines
    IL = U % 2 == 0 and U >= 4 and R > 1

    def fpos(base: str, u: int) -> str:
        if IL:
            return "((%s) & ~(tg_i64)1) + 2 * (tg_i64)lane + %d" % (base, (u // 2) * 2 * TPR
                                                                     + u % 2)
        return "((%s) & ~(tg_i64)%d) + (tg_i64)lane * %d + %d" % (base, ALIGN - 1, U, u)

    def first_loads(rs_: str, re_: str, lo: str, hi: str) -> None:
        """Row r's first-step nonzeros into fci[r]/fcv[r] (zero outside the row),
        loading no position outside [lo, hi)."""
        if IL:
            for k in range(U // 2):
                w.open("")
                w("const tg_i64 q = %s;" % fpos(rs_, 2 * k))
                w("fci[r][%d] = 0; fcv[r][%d] = 0.0; fci[r][%d] = 0; fcv[r][%d] = 0.0;"
                  % (2 * k, 2 * k, 2 * k + 1, 2 * k + 1))
                w.open("if (q < %s && %s < %s)" % (re_, rs_, re_))
                w.open("if (pair_ok && q >= %s && q + 2 <= %s)" % (lo, hi))
                w("{ const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(indices + q));"
                  " fci[r][%d] = a.x; fci[r][%d] = a.y; }" % (2 * k, 2 * k + 1))
                w("{ const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(data + q));"
                  " fcv[r][%d] = b.x; fcv[r][%d] = b.y; }" % (2 * k, 2 * k + 1))
                w.close()
                w.open("else")
                for d in (0, 1):
                    w("fci[r][%d] = ((q + %d >= %s) & (q + %d < %s)) ? "
                      "__builtin_nontemporal_load(indices + q + %d) : 0;"
                      % (2 * k + d, d, lo, d, hi, d))
                    w("fcv[r][%d] = ((q + %d >= %s) & (q + %d < %s)) ? "
                      "__builtin_nontemporal_load(data + q + %d) : 0.0;"
                      % (2 * k + d, d, lo, d, hi, d))
                w.close()
                w.close()
                w.close()
            return
        w("const tg_i64 q = (%s & ~(tg_i64)%d) + (tg_i64)lane * %d;" % (rs_, ALIGN - 1, U))
        w("#pragma unroll")
        w("for (int u = 0; u < %d; ++u) { fci[r][u] = 0; fcv[r][u] = 0.0; }" % U)
        w.open("if (q < %s && %s < %s)" % (re_, rs_, re_))
        if U % 2 == 0:
            w.open("if (pair_ok && q >= %s && q + %d <= %s)" % (lo, U, hi))
            for u in range(0, U, 2):
                w("{ const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(indices + q + %d));"
                  " fci[r][%d] = a.x; fci[r][%d] = a.y; }" % (u, u, u + 1))
                w("{ const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(data + q + %d));"
                  " fcv[r][%d] = b.x; fcv[r][%d] = b.y; }" % (u, u, u + 1))
            w.close()
            w.open("else")
        else:
            w.open("")
        for u in range(U):
            w("fci[r][%d] = ((q + %d >= %s) & (q + %d < %s)) ? "
              "__builtin_nontemporal_load(indices + q + %d) : 0;" % (u, u, lo, u, hi, u))
            w("fcv[r][%d] = ((q + %d >= %s) & (q + %d < %s)) ? "
              "__builtin_nontemporal_load(data + q + %d) : 0.0;" % (u, u, lo, u, hi, u))
        w.close()
        w.close()

    merge = coop and low.balance == "nnz"
    hybrid = coop and low.balance == "hybrid"
    sorted_ = low.gather == "sorted"
    if sorted_:
        if not (coop and low.balance == "rows"):
            raise ValueError("gather 'sorted' needs row tiles (a tile and balance 'rows')")
        if R * U > 8 or R * U * B > SORT_MAX_ITEMS:
            raise ValueError("gather 'sorted' holds a tile's first step in registers: rows "
                             "per lane group x unroll (%d x %d) must be <= 8" % (R, U))
        if not _value_row_free(plan):
            raise ValueError("gather 'sorted' needs a per-nonzero value that reads only the "
                             "sparse value and the gathered operand")
    if merge or hybrid:
        if pre is None:
            raise ValueError("merge-path and hybrid tiles need file-scope declarations")
        _merge_decls(pre, scratch_arg)
        if not scratch_arg:
            w("unsigned long long* const tg_part = tg_mp_part;")
    if merge:
        # a window holds about T rows' worth of items but may hold several times
        # T short rows; a batch is at least one row per lane group
        TR = max(TR, SLOTS)
        R = (TR + SLOTS - 1) // SLOTS
    if hybrid:
        CH = hybrid_chunk(low)
        LH = hybrid_long(low)

    if merge:
        w("const tg_i64 row_lim = %s;  // rows this launch writes" % bound)
    elif hybrid:
        w("const tg_i64 row_end = %s;" % bound)
    else:
        w("const tg_i64 row_end = %s;" % bound)
        w("const tg_i64 row0 = (tg_i64)blockIdx.x * %d;" % TR)
    w("const int lane = threadIdx.x %% %d;" % TPR)
    w("const int slot = threadIdx.x / %d;" % TPR)
    if U % 2 == 0:
        w("// 128-bit (index, value) pair loads need 16-byte aligned bases; a caller's")
        w("// sub-buffer may be only 8-byte aligned, which takes the per-element loads")
        w("const bool pair_ok = ((((unsigned long long)indices) | "
          "((unsigned long long)data)) & 15) == 0;")
    if hybrid:
        _hybrid_ranges(w, plan, step, out_name, B, U, ALIGN, WAVES, CH, LH)
        w("const tg_i64 row0 = ((tg_i64)blockIdx.x - GL) * %d;" % TR)
    if low.tiled:
        w("// row pointers of this tile, staged once in LDS")
        w("__shared__ tg_i64 s_ptr[%d];" % (TR + 1))
        w("__shared__ int s_long[%d];   // rows left to the whole workgroup" % TR)
        w("__shared__ int s_nlong;")
        if wave_tier:
            w("__shared__ int s_med[%d];    // rows left to one wave each" % TR)
            w("__shared__ int s_nmed;")
        w("__shared__ double s_red[%d];" % WAVES)
        if merge:
            _merge_window(w, TR, WAVES, plan)
            w.open("for (tg_i64 row0 = r0; row0 < r_own; row0 += %d)" % TR)
            w("const tg_i64 row_end = row0 + %d < r_own ? row0 + %d : r_own;" % (TR, TR))
        if sorted_:
            NB = sort_buckets(B)
            w("// the first step's gathers, sorted: bucket counts, sorted entries, operands")
            w("__shared__ unsigned s_hist[%d];" % NB)
            w("__shared__ unsigned long long s_ent[%d];" % (R * U * B))
            w("__shared__ double s_x[%d];" % (R * U * B))
            w("__shared__ unsigned s_swsum[%d];" % (NB // 64))
            w("// buckets of 2^sshift columns of the operand: fewer than %d of them" % NB)
            w("const tg_i64 ncol_ = %s;" % _extent_for(plan, plan.col_idx.name))
            w("const int sshift = ncol_ > %d ? 64 - __clzll((unsigned long long)(ncol_ - 1)) - %d"
              " : 0;" % (NB, NB.bit_length() - 1))
            w("if (threadIdx.x < %d) s_hist[threadIdx.x] = 0u;" % NB)
        if sorted_:
            # the row pointers' first pass goes out first: vector loads return in order, so
            # issued after the guessed loads, their staging would wait for all of those too
            w("// the first %d row pointers, loaded before anything else (a relaxed atomic load," % min(TR + 1, B))
            w("// which the compiler issues here rather than at its use below)")
            w("tg_i64 ptr0_ = 0;")
            w.open("if (threadIdx.x <= %d)" % TR)
            w("const tg_i64 r = row0 + threadIdx.x;")
            w("typedef const __attribute__((address_space(1))) tg_i64 tg_gi64;")
            w("ptr0_ = __hip_atomic_load((tg_gi64*)indptr + (r < row_end ? r : row_end), "
              "__ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);")
            w.close()
        if sorted_:
            w("// Before the row pointers, each row's first step is loaded where rows of Ls =")
            w("// nnz / M nonzeros each from position 0 would put it, when nnz is such a multiple")
            w("// of M that every lane's 128-bit pairs lie inside its row (positions below nnz,")
            w("// with no per-lane condition, so they issue back to back).  Rows whose bounds")
            w("// turn out otherwise load again once the row pointers have arrived.")
            w("tg_i64 Ls = nnz > 0 && %s > 0 && nnz %% %s == 0 ? nnz / %s : 0;"
              % (plan.row_extent, plan.row_extent, plan.row_extent))
            w("tg_i64 fci[%d][%d]; double fcv[%d][%d]; tg_i64 gs[%d];" % (R, U, R, U, R))
            if U % 2 == 0:
                w("if (!(pair_ok && Ls >= %d && (Ls & 1) == 0)) Ls = 0;" % (TPR * U))
            else:
                w("Ls = 0;  // odd unroll: no 128-bit pairs to guess with")
            w("#pragma unroll")
            w.open("for (int r = 0; r < %d; ++r)" % R)
            w("const int lr = slot + r * %d;" % SLOTS)
            w("const tg_i64 grow = row0 + lr;")
            w("gs[r] = lr < %d && grow < row_end ? grow * Ls : -1;" % TR)
            w.close()
            if U % 2 == 0:
                if pre is None:
                    raise ValueError("gather 'sorted' needs file-scope declarations")
                pre("// zeros that a sorted tile's guessed loads read when there is no guess, so\n"
                    "// that those loads are issued unconditionally (never written)\n"
                    "__device__ __attribute__((aligned(16))) tg_i64 tg_zpad[%d];" % SORT_ZPAD)
                w("// without a guess the same loads read zeros, so that no branch separates them")
                w("// from the row pointers' load: their staging then waits for that load alone")
                w("const tg_i64* const sidx_ = Ls > 0 ? indices : (const tg_i64*)tg_zpad;")
                w("const double* const sdat_ = Ls > 0 ? data : (const double*)tg_zpad;")
                w("#pragma unroll")
                w.open("for (int r = 0; r < %d; ++r)" % R)
                w("const tg_i64 gb = Ls > 0 && gs[r] >= 0 ? gs[r] : 0;")
                for u in range(0, U, 2):
                    w("{ const tg_i64 q = %s;" % fpos("gb", u))
                    w("  const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(sidx_ + q));"
                      " fci[r][%d] = a.x; fci[r][%d] = a.y;" % (u, u + 1))
                    w("  const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(sdat_ + q));"
                      " fcv[r][%d] = b.x; fcv[r][%d] = b.y; }" % (u, u + 1))
                w.close()
        w("if (threadIdx.x == 0) { s_nlong = 0;%s }" % (" s_nmed = 0;" if wave_tier else ""))
        if sorted_:
            w("if (threadIdx.x <= %d) s_ptr[threadIdx.x] = ptr0_;" % TR)
        if not sorted_ or TR + 1 > B:
            w.open("for (int t = threadIdx.x%s; t <= %d; t += %d)" % (" + %d" % B if sorted_ else "",
                                                                      TR, B))
            w("const tg_i64 r = row0 + t;")
            w("s_ptr[t] = indptr[r < row_end ? r : row_end];")
            w.close()
        if hybrid:
            w("// indptr[0] and indptr[M] with the row pointers: which long rows have ranges")
            w("__shared__ tg_i64 s_lim[2];")
            w("if (threadIdx.x == %d) s_lim[0] = indptr[0];" % (B - 1))
            w("if (threadIdx.x == %d) s_lim[1] = indptr[%s];" % (B - 2 if B > 64 else B - 1,
                                                                plan.row_extent))
        w("__syncthreads();")
        w("// this tile's nonzeros: its loads touch no position outside them")
        w("const tg_i64 glo = tg_uniform(s_ptr[0]), ghi = tg_uniform(s_ptr[%d]);" % TR)
        if hybrid:
            w("const tg_i64 pbase = tg_uniform(s_lim[0]), pend = tg_uniform(s_lim[1]);")
            w("const tg_i64 pal = pbase & ~(tg_i64)1;")
            w("const tg_i64 NR = pend > pbase ? (pend - pal + %d) / %d : 0;" % (CH - 1, CH))
            w("const tg_i64 NL = NR < GL ? NR : GL;  // the ranges that exist")
        if wave_tier:
            w("// rows and nonzeros of this tile (s_ptr[%d] is clamped to the last row)" % TR)
            w("const tg_i64 t_rows = row_end - row0 < %d ? row_end - row0 : %d;" % (TR, TR))
            w("const tg_i64 t_nnz = s_ptr[%d] - s_ptr[0];" % TR)
    w("tg_i64 rs[%d], re[%d];" % (R, R))
    w("double acc[%d];" % R)
    if coop:
        w("bool coop[%d];" % R)
    else:
        w("bool lv[%d];  // the lane's row exists" % R)
    w("#pragma unroll")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    w("const int lr = slot + r * %d;" % SLOTS)
    w("const bool live = lr < %d && row0 + lr < row_end;" % TR)
    if low.tiled:
        w("const int li = lr < %d ? lr : 0;" % TR)
        w("rs[r] = live ? s_ptr[li] : 0;")
        w("re[r] = live ? s_ptr[li + 1] : 0;")
    else:
        w("const tg_i64 ri = live ? row0 + lr : 0;")
        w("rs[r] = live ? indptr[ri] : 0;")
        w("re[r] = live ? indptr[ri + 1] : 0;")
        w("lv[r] = live;")
    if coop:
        skip = ""
        if hybrid:
            w("// summed by the long-row workgroups, when its first range exists")
            w("const bool lw = re[r] - rs[r] > %d && (rs[r] - pal) / %d < NL;" % (LH, CH))
            skip = "lw || "
        if wave_tier:
            w("const tg_i64 len = re[r] - rs[r];")
            w("coop[r] = %slen > %d && (len * t_rows > 2 * t_nnz || len > %d);"
              % (skip, MED, LONG) if not hybrid else
              "coop[r] = lw || (len > %d && (len * t_rows > 2 * t_nnz || len > %d));"
              % (MED, LONG))
        else:
            w("coop[r] = %sre[r] - rs[r] > %d;" % (skip, LONG))
        w.open("if (coop[r])")
        listed = "lane == 0 && !lw" if hybrid else "lane == 0"
        if wave_tier:
            w.open("if (%s)" % listed)
            w("if (re[r] - rs[r] > %d) s_long[atomicAdd(&s_nlong, 1)] = lr;" % WLONG)
            w("else s_med[atomicAdd(&s_nmed, 1)] = lr;")
            w.close()
        else:
            w("if (%s) s_long[atomicAdd(&s_nlong, 1)] = lr;" % listed)
        w("re[r] = rs[r];  // the lane group skips it")
        w.close()
    w("acc[r] = 0.0;")
    w.close()
    if not low.tiled:
        w("// the positions of the wave's rows of each pass, [wlo, whi): the rows ascend with")
        w("// the lane, so these are the first live row's start and the last one's end; a load")
        w("// anywhere in them stays inside the launch's positions")
        w("tg_i64 wlo[%d], whi[%d];" % (R, R))
        w("#pragma unroll")
        w.open("for (int r = 0; r < %d; ++r)" % R)
        w("const unsigned long long m = __ballot(lv[r]);")
        w("const int f = m ? (int)__builtin_ctzll(m) : 0, g = m ? 63 - (int)__builtin_clzll(m) : 0;")
        w("wlo[r] = m ? __shfl(rs[r], f) : 0;")
        w("whi[r] = m ? __shfl(re[r], g) : 0;")
        w.close()

    # every row's first step held at once costs about 6 R U registers per lane: past
    # R U = 8 that spills, so such schedules keep one guarded step per row
    if (R == 1 and not sorted_) or R * U > 8:
        w("// first step of every row in flight before any accumulation")
        w("#pragma unroll")
        w.open("for (int r = 0; r < %d; ++r)" % R)
        w("const tg_i64 row = row0 + slot + r * %d;" % SLOTS)
        w("(void)row;")
        w("const tg_i64 q = (rs[r] & ~(tg_i64)%d) + (tg_i64)lane * %d;" % (ALIGN - 1, U))
        w.open("if (q < re[r] && rs[r] < re[r])")
        step("q", "rs[r]", "re[r]", "acc[r]", *(() if low.tiled else ("wlo[r]", "whi[r]")))
        w.close()
        w.close()
    else:
        w("// first step of every row: every row's loads, then every row's gathers (none")
        w("// behind a per-lane condition, so they issue back to back), then the sums")
        if sorted_:
            w("// rows whose bounds are not the guessed ones load their first step now")
            w("#pragma unroll")
            w.open("for (int r = 0; r < %d; ++r)" % R)
            w.open("if (!(Ls > 0 && rs[r] == gs[r] && re[r] == gs[r] + Ls))")
            first_loads("rs[r]", "re[r]", "glo", "ghi")
            w.close()
            w.close()
        else:
            w("tg_i64 fci[%d][%d]; double fcv[%d][%d];" % (R, U, R, U))
            w("#pragma unroll")
            w.open("for (int r = 0; r < %d; ++r)" % R)
            first_loads("rs[r]", "re[r]", "glo", "ghi")
            w.close()
        w.open("if (ghi > glo)")
        if sorted_:
            _sorted_first_step(w, plan, R, U, B, SLOTS, fpos, row)
        else:
            w("double fxv[%d][%d]; bool fok[%d][%d];" % (R, U, R, U))
            w("#pragma unroll")
            w.open("for (int r = 0; r < %d; ++r)" % R)
            w("const tg_i64 row = row0 + slot + r * %d;" % SLOTS)
            w("(void)row;")
            if IL:
                for u in range(U):
                    w.open("")
                    w("const tg_i64 pu = %s;" % fpos("rs[r]", u))
                    w("fok[r][%d] = (pu >= rs[r]) & (pu < re[r]);" % u)
                    w("const tg_i64 cu = fok[r][%d] ? fci[r][%d] : 0;" % (u, u))
                    w("fxv[r][%d] = %s;" % (u, _cexpr(gathered, _Env({row: "row", col: "cu"},
                                                                     p="pu"))))
                    w.close()
            else:
                w("const tg_i64 q = (rs[r] & ~(tg_i64)%d) + (tg_i64)lane * %d;" % (ALIGN - 1, U))
                w("#pragma unroll")
                w.open("for (int u = 0; u < %d; ++u)" % U)
                w("const tg_i64 pu = q + u;")
                w("fok[r][u] = (pu >= rs[r]) & (pu < re[r]);")
                w("const tg_i64 cu = fok[r][u] ? fci[r][u] : 0;")
                w("fxv[r][u] = %s;" % _cexpr(gathered, _Env({row: "row", col: "cu"}, p="pu")))
                w.close()
            w.close()
            w("#pragma unroll")
            w.open("for (int r = 0; r < %d; ++r)" % R)
            w("const tg_i64 row = row0 + slot + r * %d;" % SLOTS)
            w("(void)row;")
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("acc[r] = fok[r][u] ? acc[r] + %s : acc[r];"
              % _value_with(plan, "fcv[r][u]", "fxv[r][u]", row, "fci[r][u]"))
            w.close()
            w.close()
        w.close()
    w("// remaining steps (rows longer than %d nonzeros)" % (STEP - ALIGN + 1))
    w("#pragma unroll")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    w("const tg_i64 row = row0 + slot + r * %d;" % SLOTS)
    w("(void)row;")
    w("#pragma unroll 1")
    w.open("for (tg_i64 q = (rs[r] & ~(tg_i64)%d) + (tg_i64)lane * %d + %d; q < re[r]; q += %d)"
           % (ALIGN - 1, U, STEP, STEP))
    step("q", "rs[r]", "re[r]", "acc[r]", *(() if low.tiled else ("wlo[r]", "whi[r]")))
    w.close()
    w.close()
    w("#pragma unroll")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    if TPR > 1:
        w("acc[r] = tg_segsum<%d>(acc[r]);" % TPR)
    w("const int lr = slot + r * %d;" % SLOTS)
    w("const tg_i64 row = row0 + lr;")
    w.open("if (%slr < %d && row < row_end%s)" % ("lane == 0 && " if TPR > 1 else "", TR,
                                                   " && !coop[r]" if coop else ""))
    env = _Env({row: "row"}, acc="acc[r]")
    w("__builtin_nontemporal_store(%s, %s + %s);" % (
        _cexpr(plan.final_expr, env), out_name, _offset(plan.out_tensor, plan.out.indices, env)))
    w.close()
    w.close()
    if not coop:
        return
    w("__syncthreads();")
    if wave_tier:
        w("// medium rows: one wave each, no barriers")
        w("const int n_med = s_nmed;")
        w("const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / %d);" % WAVE)
        w("const int wl = threadIdx.x %% %d;" % WAVE)
        w("#pragma unroll 1")
        w.open("for (int k = wv; k < n_med; k += %d)" % WAVES)
        w("const int lr = s_med[k];")
        w("const tg_i64 row = row0 + lr;")
        w("const tg_i64 mrs = s_ptr[lr], mre = s_ptr[lr + 1];")
        w("double macc = 0.0;")
        w("#pragma unroll 1")
        w.open("for (tg_i64 q = (mrs & ~(tg_i64)%d) + (tg_i64)wl * %d; q < mre; q += %d)"
               % (ALIGN - 1, U, WAVE * U))
        step("q", "mrs", "mre", "macc")
        w.close()
        w("macc = tg_segsum<%d>(macc);" % WAVE)
        w.open("if (wl == 0)")
        env = _Env({row: "row"}, acc="macc")
        w("__builtin_nontemporal_store(%s, %s + %s);" % (
            _cexpr(plan.final_expr, env), out_name, _offset(plan.out_tensor, plan.out.indices, env)))
        w.close()
        w.close()
    w("// long rows: the whole workgroup, one row at a time")
    w("const int n_long = s_nlong;")
    w("#pragma unroll 1")
    w.open("for (int k = 0; k < n_long; ++k)")
    w("const int lr = s_long[k];")
    w("const tg_i64 row = row0 + lr;")
    w("const tg_i64 crs = s_ptr[lr], cre = s_ptr[lr + 1];")
    w("double cacc = 0.0;")
    w("#pragma unroll 1")
    w.open("for (tg_i64 q = (crs & ~(tg_i64)%d) + (tg_i64)threadIdx.x * %d; q < cre; q += %d)"
           % (ALIGN - 1, U, B * U))
    step("q", "crs", "cre", "cacc")
    w.close()
    w("cacc = tg_segsum<64>(cacc);")
    w("if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = cacc;")
    w("__syncthreads();")
    w.open("if (threadIdx.x == 0)")
    w("double t = 0.0;")
    w("#pragma unroll")
    w("for (int v = 0; v < %d; ++v) t += s_red[v];" % WAVES)
    env = _Env({row: "row"}, acc="t")
    w("__builtin_nontemporal_store(%s, %s + %s);" % (
        _cexpr(plan.final_expr, env), out_name, _offset(plan.out_tensor, plan.out.indices, env)))
    w.close()
    w("__syncthreads();")
    w.close()
    if not merge:
        return
    w("__syncthreads();  // the next batch rewrites s_ptr and the row lists")
    w.close()
    w("// pieces of rows longer than a window: the one that began before this")
    w("// window (k = 0) and the one that begins in it and runs past its end (k = 1)")
    w("#pragma unroll 1")
    w.open("for (int k = 0; k < 2; ++k)")
    w("if (!(k == 0 ? pc_in : pc_out)) continue;")
    w("const tg_i64 row = k == 0 ? r0 - 1 : r1 - 1;")
    w("const tg_i64 pb = k == 0 ? s_win[2] : s_win[4], pe = k == 0 ? s_win[3] : s_win[5];")
    w("// item t of the row is its position t - row + pbase")
    w("const tg_i64 c0 = k == 0 && t0 - row + pbase > pb ? t0 - row + pbase : pb;")
    w("const tg_i64 c1 = t1 - row + pbase < pe ? t1 - row + pbase : pe;")
    w("double cacc = 0.0;")
    w("#pragma unroll 1")
    w.open("for (tg_i64 q = (c0 & ~(tg_i64)%d) + (tg_i64)threadIdx.x * %d; q < c1; q += %d)"
           % (ALIGN - 1, U, B * U))
    step("q", "c0", "c1", "cacc", "pb", "pe")
    w.close()
    w("cacc = tg_segsum<64>(cacc);")
    w("if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = cacc;")
    w("__syncthreads();")
    w.open("if (threadIdx.x < 64)")
    w("double t = 0.0;")
    w("#pragma unroll")
    w("for (int v = 0; v < %d; ++v) t += s_red[v];" % WAVES)
    w("const tg_i64 wf = (row + pb - pbase) / D, wl = (row + pe - 1 - pbase) / D;  "
      "// its first/last window")
    w("double tot;")
    w.open("if (tg_mp_commit(tg_part, wdx, wf, wl, t, &tot) && threadIdx.x == 0)")
    env = _Env({row: "row"}, acc="tot")
    w("__builtin_nontemporal_store(%s, %s + %s);" % (
        _cexpr(plan.final_expr, env), out_name, _offset(plan.out_tensor, plan.out.indices, env)))
    w.close()
    w.close()
    w("__syncthreads();")
    w.close()


def _gather_operand(plan: Plan) -> Expr:
    """The dense factor of the per-nonzero product (``x[j]`` for spmv)."""
    for n in plan.value_expr.walk():
        if isinstance(n, Access) and not n.tensor.format.is_sparse() and n.tensor.order > 0:
            return n
    raise NotImplementedError("scalar_reduce without a dense gathered operand")


def _value_with(plan: Plan, data_text: str, gathered_text: str, row: str, col_text: str) -> str:
    """value_expr with the sparse value and the gathered operand substituted."""
    g = _gather_operand(plan)

    def rec(e: Expr) -> str:
        if e is g:
            return gathered_text
        if isinstance(e, Access):
            if e.tensor.format.is_sparse():
                return data_text
            return _cexpr(e, _Env({row: "row", plan.col_idx.name: col_text}, p="pu"))
        if isinstance(e, Const):
            return _fmt_const(e.value)
        if isinstance(e, Mul):
            return "(%s * %s)" % (rec(e.left), rec(e.right))
        if isinstance(e, Add):
            return "(%s + %s)" % (rec(e.left), rec(e.right))
        raise TypeError("cannot emit %r" % (e,))
    return rec(plan.value_expr)


def _hip_row_dense_out(w: _W, plan: Plan, low: Lowering, bound: str, geo: LaunchGeometry,
                       out_name: str, b_name: str, kext: str) -> None:
    """C[row, :] = sum over nonzeros data[p] * B[col, :]; written once.

    Tiled variants balance long rows like SpMV does: a row longer than LONG
    nonzeros is skipped by its lane group and listed in LDS; after the lane
    groups' rows, every lane group of the workgroup takes a strided share of
    each listed row's nonzeros for one K-slice at a time, and the partial
    C-row slices are summed by a fixed LDS tree, so the result does not depend
    on timing."""
    B, TPR = geo.block, max(1, low.threads_per_row)
    U = max(1, low.unroll)
    V = 2 if low.vector_width >= 2 else 1
    SLOTS = B // TPR
    TR = geo.rows_per_block
    R = (TR + SLOTS - 1) // SLOTS
    LONG = 16 * U     # longer rows may leave their lane group ...
    HUGE = 64 * U     # ... and always do past this length
    coop = low.tiled
    uniform = TPR == WAVE
    w("const tg_i64 row_end = %s;" % bound)
    w("const tg_i64 row0 = (tg_i64)blockIdx.x * %d;" % TR)
    w("const int lane = threadIdx.x %% %d;" % TPR)
    if uniform:
        w("// a whole wave per row: row bounds and (column, value) pairs are wave-uniform")
        w("const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x / %d);" % TPR)
    else:
        w("const int slot = threadIdx.x / %d;" % TPR)
    if V == 2:
        w("const bool vec_ok = ((%s & 1) == 0) && ((((unsigned long long)%s) | "
          "((unsigned long long)%s)) & 15) == 0;" % (kext, b_name, out_name))
    if coop:
        w("__shared__ int s_long[%d];   // rows left to the whole workgroup" % TR)
        w("__shared__ int s_nlong;")
        w("__shared__ double s_part[%d];  // partial C-row slices, one per lane group" % (B * V))
        _tile_stats(w, TR)
    w("#pragma unroll 1")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    w("const int lr = slot + r * %d;" % SLOTS)
    w("const tg_i64 row = row0 + lr;")
    w("if (lr >= %d || row >= row_end) break;" % TR)
    if uniform:
        w("const tg_i64 rs = tg_uniform(indptr[row]);")
        w("const tg_i64 re = tg_uniform(indptr[row + 1]);")
    else:
        w("const tg_i64 rs = indptr[row];")
        w("const tg_i64 re = indptr[row + 1];")
    if coop:
        w.open("if (%s)" % _long_row_test("re - rs", LONG, HUGE))
        w("if (lane == 0) s_long[atomicAdd(&s_nlong, 1)] = lr;")
        w("continue;")
        w.close()

    def kloop(vec: bool) -> None:
        width = 2 if vec else 1
        w("#pragma unroll 1")
        w.open("for (tg_i64 k0 = (tg_i64)lane * %d; k0 < %s; k0 += %d)" % (width, kext, TPR * width))
        w("double a0 = 0.0%s;" % (", a1 = 0.0" if vec else ""))
        w("tg_i64 p = rs;")
        w("#pragma unroll 1")
        w.open("for (; p + %d <= re; p += %d)" % (U, U))
        w("tg_i64 j[%d]; double v[%d];" % (U, U))
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w("j[u] = indices[p + u]; v[u] = data[p + u];")
        w.close()
        if vec:
            w("tg_f64x2 b[%d];" % U)
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("b[u] = *(const tg_f64x2*)(%s + j[u] * %s + k0);" % (b_name, kext))
            w.close()
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("a0 += v[u] * b[u].x; a1 += v[u] * b[u].y;")
            w.close()
        else:
            w("double b[%d];" % U)
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("b[u] = %s[j[u] * %s + k0];" % (b_name, kext))
            w.close()
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("a0 += v[u] * b[u];")
            w.close()
        w.close()
        w.open("for (; p < re; ++p)")
        w("const tg_i64 jj = indices[p]; const double vv = data[p];")
        if vec:
            w("const tg_f64x2 bb = *(const tg_f64x2*)(%s + jj * %s + k0);" % (b_name, kext))
            w("a0 += vv * bb.x; a1 += vv * bb.y;")
        else:
            w("a0 += vv * %s[jj * %s + k0];" % (b_name, kext))
        w.close()
        if vec:
            w("tg_f64x2 c; c.x = a0; c.y = a1;")
            w("__builtin_nontemporal_store(c, (tg_f64x2*)(%s + row * %s + k0));"
              % (out_name, kext))
        else:
            w("__builtin_nontemporal_store(a0, %s + row * %s + k0);" % (out_name, kext))
        w.close()

    def both(emit) -> None:
        if V == 2:
            w.open("if (vec_ok)")
            emit(True)
            w.close()
            w.open("else")
            emit(False)
            w.close()
        else:
            emit(False)

    both(kloop)
    w.close()
    if not coop:
        return

    def wg_long(vec: bool) -> None:
        width = 2 if vec else 1
        cols = TPR * width
        w("#pragma unroll 1")
        w.open("for (tg_i64 kc = 0; kc < %s; kc += %d)" % (kext, cols))
        w("const tg_i64 k0 = kc + (tg_i64)lane * %d;" % width)
        w("const bool in_k = k0 < %s;" % kext)
        w("double a0 = 0.0%s;" % (", a1 = 0.0" if vec else ""))
        w("#pragma unroll 1")
        w.open("for (tg_i64 p = crs + slot; p < cre; p += %d)" % (SLOTS * U))
        w("tg_i64 j[%d]; double v[%d];" % (U, U))
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w("const tg_i64 pu = p + u * %d;" % SLOTS)
        w("j[u] = pu < cre ? indices[pu] : 0; v[u] = pu < cre ? data[pu] : 0.0;")
        w.close()
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w.open("if (in_k && p + u * %d < cre)" % SLOTS)
        if vec:
            w("const tg_f64x2 b = *(const tg_f64x2*)(%s + j[u] * %s + k0);" % (b_name, kext))
            w("a0 += v[u] * b.x; a1 += v[u] * b.y;")
        else:
            w("a0 += v[u] * %s[j[u] * %s + k0];" % (b_name, kext))
        w.close()
        w.close()
        w.close()
        w("s_part[slot * %d + lane * %d] = a0;" % (cols, width))
        if vec:
            w("s_part[slot * %d + lane * 2 + 1] = a1;" % cols)
        w("__syncthreads();")
        w("// fixed-order tree over the lane groups' partial slices")
        # n slices left: the upper ceil(n/2) fold onto the lower floor(n/2), so an odd
        # count (a block of 3, 5, 6, 7 ... waves) keeps its middle slice for the next level
        n_ = SLOTS
        while n_ > 1:
            h_ = (n_ + 1) // 2
            w("for (int e = threadIdx.x; e < %d; e += %d) s_part[e] += s_part[e + %d];"
              % ((n_ - h_) * cols, B, h_ * cols))
            w("__syncthreads();")
            n_ = h_
        w.open("for (int t = threadIdx.x; t < %d; t += %d)" % (cols, B))
        w("if (kc + t < %s) __builtin_nontemporal_store(s_part[t], %s + row * %s + kc + t);"
          % (kext, out_name, kext))
        w.close()
        w("__syncthreads();")
        w.close()

    w("// long rows: every lane group takes a strided share of the row's nonzeros")
    w("__syncthreads();")
    w("const int n_long = s_nlong;")
    w("#pragma unroll 1")
    w.open("for (int kk = 0; kk < n_long; ++kk)")
    w("const tg_i64 row = row0 + s_long[kk];")
    w("const tg_i64 crs = indptr[row], cre = indptr[row + 1];")
    both(wg_long)
    w.close()


def _hip_sparse_out(w: _W, plan: Plan, low: Lowering, bound: str, geo: LaunchGeometry,
                    out_name: str, u_name: str, v_name: str, kext: str) -> None:
    """out[p] = data[p] * dot(U[row, :], V[col, :]) over the row's nonzeros.

    Two paths in one kernel, chosen by K at run time: the chunked path of
    ``_hip_sparse_out_fast`` when one lane group covers K with registers
    (K <= TPR*V*U), else one wave per row with the lane groups spread over the
    row's nonzeros and each group looping over K."""
    B, TPR = geo.block, max(1, low.threads_per_row)
    U = max(1, low.unroll)
    V = 2 if low.vector_width >= 2 else 1
    WAVES = B // WAVE
    SLOTS = WAVE // TPR
    TR = geo.rows_per_block
    R = (TR + WAVES - 1) // WAVES
    w("const tg_i64 row_end = %s;" % bound)
    w("const tg_i64 row0 = (tg_i64)blockIdx.x * %d;" % TR)
    w("const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / %d);" % WAVE)
    w("const int wl = threadIdx.x %% %d;" % WAVE)
    w("const int kq = wl %% %d;      // lane within the group" % TPR)
    w("const int slot = wl / %d;     // lane group within the wave" % TPR)
    if V == 2:
        w("const bool vec_ok = ((%s & 1) == 0) && ((((unsigned long long)%s) | "
          "((unsigned long long)%s)) & 15) == 0;" % (kext, u_name, v_name))
    _hip_sparse_out_fast(w, plan, TPR, U, V, SLOTS, WAVES, TR, out_name, u_name, v_name, kext,
                         coop=low.tiled)
    w.open("else")
    coop = low.tiled
    LONG = 8 * SLOTS   # 8 wave steps ...
    HUGE = 16 * SLOTS

    def kloop(vec: bool) -> None:
        width = 2 if vec else 1
        chunk = TPR * width
        w("tg_i64 k = (tg_i64)kq * %d;" % width)
        w("#pragma unroll 1")
        w.open("for (; k + %d <= %s; k += %d)" % (chunk * (U - 1) + width, kext, chunk * U))
        if vec:
            w("tg_f64x2 a[%d], b[%d];" % (U, U))
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("a[u] = *(const tg_f64x2*)(urow + k + u * %d);" % chunk)
            w("b[u] = *(const tg_f64x2*)(vrow + k + u * %d);" % chunk)
            w.close()
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("acc += a[u].x * b[u].x; acc += a[u].y * b[u].y;")
            w.close()
        else:
            w("double a[%d], b[%d];" % (U, U))
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("a[u] = urow[k + u * %d]; b[u] = vrow[k + u * %d];" % (chunk, chunk))
            w.close()
            w("#pragma unroll")
            w.open("for (int u = 0; u < %d; ++u)" % U)
            w("acc += a[u] * b[u];")
            w.close()
        w.close()
        w("#pragma unroll 1")
        w.open("for (; k < %s; k += %d)" % (kext, chunk))
        if vec:
            w("const tg_f64x2 a = *(const tg_f64x2*)(urow + k);")
            w("const tg_f64x2 b = *(const tg_f64x2*)(vrow + k);")
            w("acc += a.x * b.x; acc += a.y * b.y;")
        else:
            w("acc += urow[k] * vrow[k];")
        w.close()

    def row_body(p_start: str, p_step: int) -> None:
        """The row's nonzeros from p_start every p_step, SLOTS at a time, each
        lane group looping over K."""
        w("const double* __restrict__ urow = %s + row * %s;" % (u_name, kext))
        w("#pragma unroll 1")
        w.open("for (tg_i64 p0 = %s; p0 < re; p0 += %d)" % (p_start, p_step))
        w("const tg_i64 p = p0 + slot;")
        w("const bool valid = p < re;")
        w("double acc = 0.0;")
        w.open("if (valid)")
        w("const double* __restrict__ vrow = %s + indices[p] * %s;" % (v_name, kext))
        if V == 2:
            w.open("if (vec_ok)")
            kloop(True)
            w.close()
            w.open("else")
            kloop(False)
            w.close()
        else:
            kloop(False)
        w.close()
        if TPR > 1:
            w("acc = tg_segsum<%d>(acc);" % TPR)
        env = _Env({plan.row_idx.name: "row"}, p="p", acc="acc")
        w.open("if (valid%s)" % (" && kq == 0" if TPR > 1 else ""))
        w("%s[p] = %s;" % (out_name, _cexpr(plan.final_expr, env)))
        w.close()
        w.close()

    if coop:
        w("__shared__ int s_long[%d];   // rows left to every wave of the workgroup" % TR)
        w("__shared__ int s_nlong;")
        _tile_stats(w, TR)
    w("#pragma unroll 1")
    w.open("for (int r = 0; r < %d; ++r)" % R)
    w("const int lr = wave + r * %d;" % WAVES)
    w("const tg_i64 row = row0 + lr;")
    w("if (lr >= %d || row >= row_end) break;" % TR)
    w("const tg_i64 rs = tg_uniform(indptr[row]);")
    w("const tg_i64 re = tg_uniform(indptr[row + 1]);")
    if coop:
        w.open("if (%s)" % _long_row_test("re - rs", LONG, HUGE))
        w("if (wl == 0) s_long[atomicAdd(&s_nlong, 1)] = lr;")
        w("continue;")
        w.close()
    row_body("rs", SLOTS)
    w.close()  # for r
    if coop:
        w("// long rows: every wave of the workgroup takes every %d-th step" % WAVES)
        w("__syncthreads();")
        w("const int n_long = s_nlong;")
        w("#pragma unroll 1")
        w.open("for (int kk = 0; kk < n_long; ++kk)")
        w("const tg_i64 row = row0 + s_long[kk];")
        w("const tg_i64 rs = tg_uniform(indptr[row]);")
        w("const tg_i64 re = tg_uniform(indptr[row + 1]);")
        row_body("rs + (tg_i64)wave * %d" % SLOTS, WAVES * SLOTS)
        w.close()
    w.close()  # else (general path)


def _sddmm_batch(TPR: int, E: int) -> int:
    """V-row slices gathered per batch on the chunked SDDMM path: a power of
    two, at most the chunk (TPR nonzeros) and at most 32 doubles of staging
    per lane."""
    nb = 1
    while nb * 2 <= TPR and nb * 2 * E <= 32:
        nb *= 2
    return nb


def _hip_sparse_out_fast(w: _W, plan: Plan, TPR: int, U: int, V: int, SLOTS: int, WAVES: int,
                         TR: int, out_name: str, u_name: str, v_name: str, kext: str,
                         coop: bool = False) -> None:
    """SDDMM path for K <= TPR*V*U.  One lane group per row, SLOTS rows per
    wave, consecutive rows side by side, so rows that share columns (dense
    blocks) gather the same V rows in the same instruction.  Each lane keeps
    its slice of U[row, :] in registers.  The row is walked in chunks of TPR
    nonzeros: lane kq loads index and value of nonzero q+kq (one coalesced
    load each), the column indices are broadcast across the group with lane
    shuffles, the V-row slices of a batch are all in flight before any FMA,
    lane kq keeps the dot product of nonzero q+kq, and the chunk ends with one
    coalesced store.  With ``coop`` (tiled variants) a row longer than 8
    chunks is listed in LDS instead, and after the tile's other rows every
    lane group of the workgroup takes a strided share of its chunks (SDDMM
    outputs need no reduction across nonzeros).  Opens an ``if``; the caller
    emits the general path in the matching ``else``."""
    W = V
    KCAP = TPR * V * U
    E = U * W
    NB = _sddmm_batch(TPR, E)
    B = WAVES * SLOTS * TPR
    LONG = 8 * TPR     # longer rows may leave their lane group ...
    HUGE = 16 * TPR    # ... and always do past this length
    cond = "%s <= %d" % (kext, KCAP) + (" && vec_ok" if V == 2 else "")

    def load_u(live: str) -> None:
        w("const double* __restrict__ urow = %s + (%s ? row : 0) * %s;" % (u_name, live, kext))
        w("double ur[%d];" % E)
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w("const tg_i64 k = (tg_i64)kq * %d + u * %d;" % (W, TPR * W))
        if W == 2:
            w.open("if (%s && k < %s)" % (live, kext))
            w("const tg_f64x2 t = __builtin_nontemporal_load((const tg_f64x2*)(urow + k));")
            w("ur[2 * u] = t.x; ur[2 * u + 1] = t.y;")
            w.close()
            w("else { ur[2 * u] = 0.0; ur[2 * u + 1] = 0.0; }")
        else:
            w("ur[u] = (%s && k < %s) ? __builtin_nontemporal_load(urow + k) : 0.0;"
              % (live, kext))
        w.close()

    def chunks(q0: str, step: int) -> None:
        """Chunks of TPR nonzeros of [rs, rs + len) starting at q0, every step."""
        w("#pragma unroll 1")
        w.open("for (tg_i64 q = %s; __builtin_amdgcn_ballot_w64(q < len) != 0; q += %d)"
               % (q0, step))
        w("const bool mine = q + kq < len;")
        w("const tg_i64 jl = mine ? indices[rs + q + kq] : 0;")
        w("const double dl = mine ? data[rs + q + kq] : 0.0;")
        w("double res = 0.0;")
        w("#pragma unroll")
        w.open("for (int n0 = 0; n0 < %d; n0 += %d)" % (TPR, NB))
        w("double x[%d][%d];" % (NB, E))
        w("#pragma unroll")
        w.open("for (int n = 0; n < %d; ++n)" % NB)
        if TPR > 1:
            w("const tg_i64 j = tg_lane_bcast(jl, slot * %d + n0 + n);" % TPR)
        else:
            w("const tg_i64 j = jl;")
        w("const bool v = q + n0 + n < len;")
        w("const double* __restrict__ vr = %s + j * %s;" % (v_name, kext))
        w("#pragma unroll")
        w.open("for (int u = 0; u < %d; ++u)" % U)
        w("const tg_i64 k = (tg_i64)kq * %d + u * %d;" % (W, TPR * W))
        if W == 2:
            w.open("if (v && k < %s)" % kext)
            w("const tg_f64x2 t = *(const tg_f64x2*)(vr + k);")
            w("x[n][2 * u] = t.x; x[n][2 * u + 1] = t.y;")
            w.close()
            w("else { x[n][2 * u] = 0.0; x[n][2 * u + 1] = 0.0; }")
        else:
            w("x[n][u] = (v && k < %s) ? vr[k] : 0.0;" % kext)
        w.close()
        w.close()
        w("#pragma unroll")
        w.open("for (int n = 0; n < %d; ++n)" % NB)
        w("double acc = 0.0;")
        w("#pragma unroll")
        w("for (int e = 0; e < %d; ++e) acc += ur[e] * x[n][e];" % E)
        if TPR > 1:
            w("acc = tg_segsum<%d>(acc);" % TPR)
        w("if (kq == n0 + n) res = acc;")
        w.close()
        w.close()
        env = _Env({plan.row_idx.name: "row"}, p="(rs + q + kq)", acc="res", data="dl")
        w("if (mine) __builtin_nontemporal_store(%s, %s + rs + q + kq);"
          % (_cexpr(plan.final_expr, env), out_name))
        w.close()

    w.open("if (%s)" % cond)
    w("// one lane group per row; chunks of %d nonzeros, V slices gathered %d at a time"
      % (TPR, NB))
    if coop:
        w("__shared__ int s_long[%d];   // rows left to the whole workgroup" % TR)
        w("__shared__ int s_nlong;")
        _tile_stats(w, TR)
    w("#pragma unroll 1")
    w.open("for (int c = wave; c * %d < %d; c += %d)" % (SLOTS, TR, WAVES))
    w("const int lr = c * %d + slot;" % SLOTS)
    w("const tg_i64 row = row0 + lr;")
    w("const bool live = lr < %d && row < row_end;" % TR)
    w("const tg_i64 rs = live ? indptr[row] : 0;")
    if coop:
        w("tg_i64 len = live ? indptr[row + 1] - rs : 0;")
        w.open("if (%s)" % _long_row_test("len", LONG, HUGE))
        w("if (kq == 0) s_long[atomicAdd(&s_nlong, 1)] = lr;")
        w("len = 0;  // the lane group skips it")
        w.close()
    else:
        w("const tg_i64 len = live ? indptr[row + 1] - rs : 0;")
    load_u("live")
    chunks("0", TPR)
    w.close()  # for c
    if coop:
        w("// long rows: every lane group of the workgroup takes a strided share of the chunks")
        w("__syncthreads();")
        w("const int n_long = s_nlong;")
        w("#pragma unroll 1")
        w.open("for (int kk = 0; kk < n_long; ++kk)")
        w("const tg_i64 row = row0 + s_long[kk];")
        w("const tg_i64 rs = indptr[row];")
        w("const tg_i64 len = indptr[row + 1] - rs;")
        load_u("true")
        chunks("(tg_i64)(wave * %d + slot) * %d" % (SLOTS, TPR), B)
        w.close()
    w.close()  # if fast


def _hip_elementwise(w: _W, plan: Plan, bound: str, geo: LaunchGeometry, out_name: str) -> None:
    ix = plan.out.indices[0]
    w("const tg_i64 i = (tg_i64)blockIdx.x * %d + threadIdx.x;" % geo.block)
    w("if (i >= %s) return;" % bound)
    env = _Env({ix.name: "i"})
    w("%s[%s] = %s;" % (out_name, _offset(plan.out_tensor, plan.out.indices, env),
                        _cexpr(plan.value_expr, env)))


def _dense_name(plan: Plan, which: int) -> str:
    dense = []
    for n in plan.value_expr.walk():
        if (isinstance(n, Access) and not n.tensor.format.is_sparse() and n.tensor.order > 0
                and n.tensor.name not in dense):
            dense.append(n.tensor.name)
    return dense[which]


def _hip_kernel_text(kernel: Kernel, config: Config, plan: Plan, low: Lowering,
                     args: List[Tuple[str, str]], geo: LaunchGeometry,
                     scratch_arg: bool = False) -> str:
    bound = "(%s - 1)" % plan.row_extent if config.inject_bug else plan.row_extent
    out_name = plan.out_tensor.name
    pre = _W()  # file-scope declarations the kernel needs
    w = _W()
    w("extern \"C\" __global__ __launch_bounds__(%d)" % geo.block)
    params = _hip_decls(args)
    if scratch_arg:
        params += ", unsigned long long* __restrict__ tg_part"
    w.open("void %s_kernel(%s)" % (kernel.name, params))
    if plan.kind == "scalar_reduce":
        if not plan.reduce_is_compressed:
            raise NotImplementedError("HIP scalar_reduce needs the reduction over the "
                                      "compressed index")
        _hip_scalar_reduce(w, plan, low, bound, geo, out_name, pre=pre,
                           scratch_arg=scratch_arg)
    elif plan.kind == "row_dense_out":
        kext = _extent_for(plan, plan.inner_out[0].name)
        _hip_row_dense_out(w, plan, low, bound, geo, out_name, _dense_name(plan, 0), kext)
    elif plan.kind == "sparse_out":
        kext = _extent_for(plan, plan.reduce.index.name)
        _hip_sparse_out(w, plan, low, bound, geo, out_name, _dense_name(plan, 0),
                        _dense_name(plan, 1), kext)
    elif plan.kind == "elementwise":
        _hip_elementwise(w, plan, bound, geo, out_name)
    else:  # pragma: no cover
        raise NotImplementedError(plan.kind)
    w.close()
    return pre.text() + ("\n" if pre.lines else "") + w.text()


def _check_hip_dtype(config: Config) -> None:
    """The HIP kernels accumulate in float64 only.  The reference declares its
    accumulator in ``Config.dtype`` (reference ``codegen.py:416``, ``:565``); a
    request for another type is refused rather than silently given float64."""
    if config.dtype not in ("f64", "double"):
        raise ValueError("the HIP backend accumulates in float64 only; Config.dtype=%r is "
                         "not supported (use the cpu backend for a %s accumulator)"
                         % (config.dtype, config.dtype))


def _grid_text(geo: LaunchGeometry) -> str:
    if geo.stream:
        return "floor(nnz / %d) + 1 (0 without rows)" % geo.nnz_chunk
    return "ceil(%s / %d)%s" % (geo.rows_symbol, geo.rows_per_block,
                                " + floor(nnz / %d) + 1" % geo.nnz_chunk if geo.nnz_chunk
                                else "")


def emit_hip(kernel: Kernel, config: Config, scratch_arg: bool = False) -> str:
    """Device translation unit of a lowered kernel (hipRTC input).

    ``scratch_arg`` (merge-path, hybrid and stream variants only): the kernel takes the
    slots it combines row pieces through as a last parameter,
    ``unsigned long long* tg_part`` (2 * MERGE_CAP of them, all zero between
    launches), instead of declaring them as module scratch."""
    _check_hip_dtype(config)
    plan, low = _plan(kernel), _lowering(kernel)
    if scratch_arg and not module_scratch(plan, low):
        raise ValueError("scratch_arg applies to merge-path, hybrid and stream variants "
                         "only; %s combines nothing across workgroups" % config.short())
    if config.balance != "rows" and config.tile_size <= 1:
        raise ValueError("balance '%s' needs a tile (tile_size > 1); %s is untiled"
                         % (config.balance, config.short()))
    _check_hip_schedule(plan, low)
    _sig, args, _info = abi_of(kernel)
    geo = launch_geometry(plan, low)
    extra = ["target      : %s (wave%d)" % (HIP_ARCH, WAVE),
             "launch      : grid = %s, block = %d, static lds = %d B, dynamic lds = 0"
             % (_grid_text(geo), geo.block, geo.lds_bytes)]
    return "\n".join([_header(kernel, config, "hip", low, extra), _HIP_PRELUDE.strip(), "",
                      _hip_kernel_text(kernel, config, plan, low, args, geo, scratch_arg), ""])


def emit_hip_host(kernel: Kernel, config: Config) -> str:
    """C launcher for a HIP variant.

    ``{CODE_OBJECT}`` and ``{CODE_SIZE}`` are replaced by the compiled bytes
    when the variant is built.  The launcher exports the reference ABI
    (synchronous, device pointers, errors reported through ``tg_last_error``)
    plus ``tgv_geometry``, ``tgv_function`` and ``tgv_launch_async`` for
    harnesses that time the kernel on their own stream.  Variants that combine
    row pieces through module scratch (``module_scratch``) launch through
    ``tg_launch_ordered`` keyed by their code object, so calls on different
    streams never overlap on the scratch.
    """
    _check_hip_dtype(config)
    plan, low = _plan(kernel), _lowering(kernel)
    sig, args, _info = abi_of(kernel)
    geo = launch_geometry(plan, low)
    sym = "%s_kernel" % kernel.name
    names = [n for _t, n in args]
    dims = {n for t, n in args if t == "int64_t"}
    rows = geo.rows_symbol
    pack = []
    for ct, n in args:
        if ct.endswith("*"):
            pack.append("  a[%d] = (uint64_t)(uintptr_t)%s;" % (len(pack), n))
        elif ct in ("double", "float"):
            pack.append("  memcpy(&a[%d], &%s, sizeof(double));" % (len(pack), n))
        else:
            pack.append("  a[%d] = (uint64_t)%s;" % (len(pack), n))
    uses_scratch = module_scratch(plan, low)
    kdim = "K" if "K" in dims else "0"
    ndim = "N" if "N" in dims else "0"
    nnz = "nnz" if "nnz" in dims else "0"
    params = ", ".join("%s %s" % a for a in args)
    text = """/* TileGen HIP launcher for %(sym)s -- generated, DO NOT EDIT.
 * schedule %(sched)s; grid = %(grid_text)s, block = %(block)d, static lds = %(lds)d B */
#include <stdint.h>
#include <string.h>
#include "tgrt.h"

static const unsigned char tg_code[{CODE_SIZE}] = {{CODE_OBJECT}};

/* the runtime caches the loaded module by tg_code's address: drop that entry
   when this library is unloaded, before another can be mapped there */
__attribute__((destructor)) static void tgv_unload(void) {
  tg_code_release(tg_code, sizeof(tg_code));
}

void* tgv_function(void) {
  tg_function fn = 0;
  if (tg_code_function(tg_code, sizeof(tg_code), "%(sym)s", &fn) != 0) return 0;
  return fn;
}

const char* tgv_kernel_name(void) { return "%(name)s"; }

int tgv_geometry(int64_t M, int64_t N, int64_t K, int64_t nnz,
                 int64_t* grid, int32_t* block, int32_t* lds) {
  (void)N; (void)K; (void)nnz;
  const int64_t rows = %(rows_expr)s;
  *grid = %(grid_expr)s;%(extra)s
  *block = %(block)d;
  /* dynamic LDS: none, the kernel declares its %(lds)d bytes of LDS statically (a
     launch that passed them again would reserve them twice per workgroup) */
  *lds = 0;
  return 0;
}

static int tgv_pack(uint64_t* a, %(params)s) {
%(pack)s
  return %(nargs)d;
}

int tgv_launch_async(void* stream, %(params)s) {
  tg_function fn = (tg_function)tgv_function();
  if (!fn) return tg_last_status();
  int64_t grid; int32_t block, lds;
  tgv_geometry(%(M)s, %(N)s, %(K)s, %(nnz)s, &grid, &block, &lds);
  if (grid == 0) return 0;
  uint64_t a[%(nargs)d];
  int n = tgv_pack(a, %(names)s);%(launch)s
}

%(sig)s {
  tg_clear_error();
  if (tgv_launch_async(0, %(names)s) == 0) tg_synchronize();
}
""" % {
        "sym": sym, "name": kernel.name, "sched": config.short(), "rows": rows,
        "rpb": geo.rows_per_block, "block": geo.block, "lds": geo.lds_bytes,
        "rows_expr": rows if rows in dims else "M", "params": params,
        "pack": "\n".join(pack), "nargs": len(args), "names": ", ".join(names),
        "sig": sig, "M": "M" if "M" in dims else "0", "N": ndim, "K": kdim, "nnz": nnz,
        "grid_text": _grid_text(geo),
        "grid_expr": ("rows > 0 ? (nnz > 0 ? nnz : 0) / %d + 1 : 0"
                      % geo.nnz_chunk if geo.stream else
                      "rows > 0 ? (rows + %d - 1) / %d : 0" % (geo.rows_per_block,
                                                             geo.rows_per_block)),
        "launch": ("\n  /* row pieces are combined through this module's scratch, which one launch"
                   "\n     at a time may use: order after its previous launch on any stream */"
                   "\n  return tg_launch_ordered(tg_code, fn, grid, block, lds, a, n, stream, 0);"
                   if uses_scratch else
                   "\n  return tg_launch(fn, grid, block, lds, a, n, stream, 0);"),
        "extra": ("\n  /* long-row workgroups of hybrid tiles, ahead of the row tiles: one per"
                  "\n     range that nnz nonzeros can meet (ranges start at an even position) */"
                  "\n  if (*grid > 0) *grid += (nnz > 0 ? nnz : 0) / %d + 1;"
                  % geo.nnz_chunk) if geo.nnz_chunk and not geo.stream else "",
    }
    return text


# --------------------------------------------------------------------------- #
# public entry point
# --------------------------------------------------------------------------- #
def generate(kernel: Kernel, config: Config, backend: str = "cpu",
             outdir: Optional[str] = "build/generated", write: bool = True,
             skip_passes: Sequence[str] = ()) -> GeneratedKernel:
    """Run the pass pipeline and emit source for ``backend`` ("hip" or "cpu")."""
    if backend not in ("hip", "cpu"):
        raise ValueError("backend must be 'hip' or 'cpu', got %r" % backend)
    optimized = _passes.run_pipeline(kernel, config, backend=backend, skip=skip_passes)
    sig, args, _info = abi_of(optimized)
    if backend == "hip":
        source, ext = emit_hip(optimized, config), "hip"
        host = emit_hip_host(optimized, config)
        plan, low = _plan(optimized), _lowering(optimized)
        geo = launch_geometry(plan, low)
        sym = "%s_kernel" % optimized.name
    else:
        source, ext, host, geo, sym = emit_cpu(optimized, config), "cpp", "", None, ""
    digest = hashlib.sha1((source + host).encode()).hexdigest()[:8]
    gen = GeneratedKernel(
        source=source, filename="%s_%s_%s.%s" % (optimized.name, config.hash(), digest, ext),
        abi_signature=sig, pass_log=optimized.pass_log, backend=backend,
        kernel_name=optimized.name, config=config, host_source=host, device_symbol=sym,
        geometry=geo, abi_args=args)
    if write and outdir:
        gen.write(outdir)
    return gen

"""The seven-pass schedule pipeline (same passes, order and effects as
reference ``tilegen/passes.py:157-474``).

Each pass is ``pass(kernel) -> kernel``, rewrites ``kernel`` in place and
appends one ``{"pass", "action", "before", "after"}`` record to
``kernel.pass_log``.  Lowering passes turn the flat ``Config`` (read from the
transient ``kernel._config``) into typed transforms in ``kernel.schedule``; the
emitters read only those transforms.  Running the pipeline on its own output is
a no-op on the IR.

    canonicalize   constant folding, unit elimination, left-leaning reassociation
    loop_fusion    inline a producer statement into its consumer when the
                   temporary is read at exactly the indices it is written at
    tiling         Tile(outer free index, tile_size) when tile_size > 1
    thread_mapping Parallelize(outer, "thread", block_size); ThreadsPerRow(k>1)
    unroll         Unroll(reduction index, factor) when factor > 1
    vectorize      Vectorize(width) when a dense operand of order >= 2 exists
    dead_code_elim drop statements whose result nobody reads and is not an output
"""

from __future__ import annotations

import copy
from typing import Any, Callable, List, Optional, Sequence

from .ir import (
    Access, Add, Const, Expr, Index, Kernel, Mul, Parallelize, Reduce, Stmt,
    ThreadsPerRow, Tile, Unroll, Vectorize, _fmt_expr,
)

__all__ = [
    "PASSES", "PASS_NAMES", "run_pipeline", "optimize", "canonicalize",
    "loop_fusion", "tiling", "thread_mapping", "unroll", "vectorize",
    "dead_code_elim",
]


def _log(kernel: Kernel, name: str, action: str, before: Any = "", after: Any = "") -> None:
    kernel.pass_log.append({"pass": name, "action": action, "before": before,
                            "after": after})


def _set_transform(kernel: Kernel, cls, pred: Callable[[Any], bool], new) -> None:
    """Replace the first matching transform where it stands, else append.

    Editing in place keeps the schedule order stable, so re-running the
    pipeline reproduces the same schedule instead of reordering it.
    """
    ts = kernel.schedule.transforms
    for pos, t in enumerate(ts):
        if isinstance(t, cls) and pred(t):
            ts[pos] = new
            return
    ts.append(new)


def _remove_transforms(kernel: Kernel, cls, pred: Callable[[Any], bool] = lambda t: True) -> None:
    kernel.schedule.transforms = [t for t in kernel.schedule.transforms
                                  if not (isinstance(t, cls) and pred(t))]


def _cfg(kernel: Kernel, attr: str, default: int) -> int:
    value = getattr(getattr(kernel, "_config", None), attr, default)
    return value or default


def _outer_index(kernel: Kernel) -> Optional[Index]:
    free = kernel.free_indices()
    return free[0] if free else None


# --------------------------------------------------------------------------- #
# 1. canonicalize
# --------------------------------------------------------------------------- #
def _fold(e: Expr) -> Expr:
    if isinstance(e, Reduce):
        return Reduce(e.index, _fold(e.body))
    if not isinstance(e, (Add, Mul)):
        return e
    a, b = _fold(e.left), _fold(e.right)
    is_add = isinstance(e, Add)
    unit = 0.0 if is_add else 1.0
    if isinstance(a, Const) and isinstance(b, Const):
        return Const(a.value + b.value if is_add else a.value * b.value)
    if isinstance(a, Const) and a.value == unit:
        return b
    if isinstance(b, Const) and b.value == unit:
        return a
    cls = Add if is_add else Mul
    if isinstance(b, cls):
        # x op (y op z)  ->  (x op y) op z
        return cls(cls(a, b.left), b.right)
    return cls(a, b)


def canonicalize(kernel: Kernel) -> Kernel:
    first_before = _fmt_expr(kernel.stmts[0].rhs) if kernel.stmts else ""
    changed = False
    rewritten = []
    for st in kernel.stmts:
        rhs = _fold(st.rhs)
        changed = changed or _fmt_expr(rhs) != _fmt_expr(st.rhs)
        rewritten.append(Stmt(lhs=st.lhs, rhs=rhs))
    kernel.stmts = rewritten
    first_after = _fmt_expr(kernel.stmts[0].rhs) if kernel.stmts else ""
    action = ("folded constants, dropped unit operands, reassociated left"
              if changed else "no change (already canonical)")
    _log(kernel, "canonicalize", action, first_before, first_after)
    return kernel


# --------------------------------------------------------------------------- #
# 2. loop_fusion
# --------------------------------------------------------------------------- #
def _substitute(e: Expr, name: str, replacement: Expr) -> Expr:
    if isinstance(e, Access):
        return copy.deepcopy(replacement) if e.tensor.name == name else e
    if isinstance(e, (Add, Mul)):
        return type(e)(_substitute(e.left, name, replacement),
                       _substitute(e.right, name, replacement))
    if isinstance(e, Reduce):
        return Reduce(e.index, _substitute(e.body, name, replacement))
    return e


def _reads(e: Expr) -> List[str]:
    return [n.tensor.name for n in e.walk() if isinstance(n, Access)]


def loop_fusion(kernel: Kernel) -> Kernel:
    if len(kernel.stmts) < 2:
        _log(kernel, "loop_fusion", "single statement; nothing to fuse")
        return kernel
    for w, producer in enumerate(kernel.stmts):
        temp = producer.lhs.tensor.name
        written_at = [ix.name for ix in producer.lhs.indices]
        for r, consumer in enumerate(kernel.stmts):
            if r == w or temp not in _reads(consumer.rhs):
                continue
            read_at = [[ix.name for ix in n.indices] for n in consumer.rhs.walk()
                       if isinstance(n, Access) and n.tensor.name == temp]
            if any(idx != written_at for idx in read_at):
                # reading the temporary anywhere but where it was written is a
                # loop-carried (true) dependency: fusing would be wrong
                _log(kernel, "loop_fusion",
                     "refused: true dependency on '%s' (read at %s, written at %s)"
                     % (temp, read_at, written_at),
                     _fmt_expr(consumer.rhs), _fmt_expr(producer.rhs))
                return kernel
            before = " | ".join(_fmt_expr(s.rhs) for s in kernel.stmts)
            fused = Stmt(lhs=consumer.lhs, rhs=_substitute(consumer.rhs, temp, producer.rhs))
            rest = [s for pos, s in enumerate(kernel.stmts) if pos not in (w, r)]
            kernel.stmts = [fused] + rest
            _log(kernel, "loop_fusion",
                 "fused statements over index %s; temporary '%s' eliminated "
                 "(read index == write index, no carried dependency)"
                 % (written_at[0] if written_at else "?", temp),
                 before, _fmt_expr(fused.rhs))
            return kernel
    _log(kernel, "loop_fusion", "no fusable producer/consumer pair found")
    return kernel


# --------------------------------------------------------------------------- #
# 3. tiling
# --------------------------------------------------------------------------- #
def tiling(kernel: Kernel) -> Kernel:
    size = _cfg(kernel, "tile_size", 1)
    outer = _outer_index(kernel)
    if outer is None:
        _log(kernel, "tiling", "no free indices; skipped")
        return kernel
    same = lambda t: t.index.name == outer.name  # noqa: E731
    if size <= 1:
        _remove_transforms(kernel, Tile, same)
        _log(kernel, "tiling", "tile_size <= 1; no tiling applied")
        return kernel
    balance = getattr(getattr(kernel, "_config", None), "balance", "rows") or "rows"
    gather = getattr(getattr(kernel, "_config", None), "gather", "direct") or "direct"
    _set_transform(kernel, Tile, same, Tile(outer, size, balance, gather))
    if balance == "hybrid":
        _log(kernel, "tiling",
             "strip-mined '%s' into tiles of %d rows; rows longer than a long-row "
             "workgroup's half share are summed by workgroups that each take an equal range "
             "of nonzeros" % (outer.name, size),
             "for %s in 0..extent" % outer.name,
             "for nonzero range: long rows' pieces; for %s_o step %d: short %s_i: ..."
             % (outer.name, size, outer.name))
        return kernel
    if balance == "stream":
        _log(kernel, "tiling",
             "split '%s' by nonzeros: each workgroup takes an equal range of nonzeros and "
             "sums the rows that end in it; rows cut at range edges are shared by the ranges "
             "they span" % outer.name,
             "for %s in 0..extent" % outer.name,
             "for nonzero range: products; for %s ending in the range: sum" % outer.name)
        return kernel
    if balance == "nnz":
        _log(kernel, "tiling",
             "split '%s' into windows of equal rows-plus-nonzeros (merge path), one per %d "
             "rows of extent; rows longer than a window are shared by the windows they span"
             % (outer.name, size),
             "for %s in 0..extent" % outer.name,
             "for window w: for %s whose first nonzero is in w: ..." % outer.name)
        return kernel
    if gather == "sorted":
        _log(kernel, "tiling",
             "strip-mined '%s' into tiles of %d rows ('%s_o' over tiles, '%s_i' within); "
             "each tile makes its first-step gathers in the order of the gathered operand, "
             "sorted in LDS" % (outer.name, size, outer.name, outer.name),
             "for %s in 0..extent" % outer.name,
             "for %s_o step %d: sort gathers; for %s_i: ..." % (outer.name, size, outer.name))
        return kernel
    _log(kernel, "tiling",
         "strip-mined '%s' into tiles of %d rows ('%s_o' over tiles, '%s_i' within)"
         % (outer.name, size, outer.name, outer.name),
         "for %s in 0..extent" % outer.name,
         "for %s_o step %d: for %s_i: ..." % (outer.name, size, outer.name))
    return kernel


# --------------------------------------------------------------------------- #
# 4. thread_mapping
# --------------------------------------------------------------------------- #
def thread_mapping(kernel: Kernel) -> Kernel:
    tpr = _cfg(kernel, "threads_per_row", 1)
    block = _cfg(kernel, "block_size", 256)
    backend = getattr(kernel, "_backend", "cpu")
    outer = _outer_index(kernel) or Index("?")
    _set_transform(kernel, Parallelize, lambda t: t.index.name == outer.name,
                   Parallelize(outer, "thread", block_size=block))
    if tpr > 1:
        _set_transform(kernel, ThreadsPerRow, lambda t: True, ThreadsPerRow(tpr))
    else:
        _remove_transforms(kernel, ThreadsPerRow)
    if backend == "hip":
        how = ("%d lanes per row, segmented wave64 DPP reduction" % tpr if tpr > 1
               else "one lane per row")
        action = ("map index '%s' to HIP workgroups of %d lanes (wave64); %s"
                  % (outer.name, block, how))
    else:
        action = ("map index '%s' to OpenMP parallel for schedule(dynamic, 256); "
                  "threads_per_row=%d has no CPU meaning" % (outer.name, tpr))
    _log(kernel, "thread_mapping", action, None, None)
    return kernel


# --------------------------------------------------------------------------- #
# 5. unroll
# --------------------------------------------------------------------------- #
def unroll(kernel: Kernel) -> Kernel:
    factor = _cfg(kernel, "unroll", 1)
    if factor <= 1:
        _remove_transforms(kernel, Unroll)
        _log(kernel, "unroll", "unroll factor <= 1; no unrolling")
        return kernel
    red = kernel.reduce_node()
    target = red.index if red is not None else (_outer_index(kernel) or Index("?"))
    _set_transform(kernel, Unroll, lambda t: True, Unroll(target, factor))
    _log(kernel, "unroll",
         "unroll innermost loop over '%s' by %d with a remainder tail" % (target.name, factor),
         "for %s: step 1" % target.name,
         "for %s: step %d { unrolled body } ; tail remainder" % (target.name, factor))
    return kernel


# --------------------------------------------------------------------------- #
# 6. vectorize
# --------------------------------------------------------------------------- #
def _unit_stride_dense(kernel: Kernel) -> Optional[Access]:
    """First dense rhs access of order >= 2 (its last index is unit-stride)."""
    for st in kernel.stmts:
        for n in st.rhs.walk():
            if (isinstance(n, Access) and not n.tensor.format.is_sparse()
                    and n.tensor.order >= 2 and len(n.tensor.shape) >= 2):
                return n
    return None


def vectorize(kernel: Kernel) -> Kernel:
    width = _cfg(kernel, "vector_width", 1)
    if width <= 1:
        _remove_transforms(kernel, Vectorize)
        _log(kernel, "vectorize", "vector_width <= 1; skipped")
        return kernel
    acc = _unit_stride_dense(kernel)
    if acc is None:
        _remove_transforms(kernel, Vectorize)
        _log(kernel, "vectorize",
             "skipped: no unit-stride dense access to widen (the spmv gather of x "
             "is not vectorizable)")
        return kernel
    extent = acc.tensor.shape[-1]
    if isinstance(extent, int) and extent % width:
        _remove_transforms(kernel, Vectorize)
        _log(kernel, "vectorize",
             "skipped: extent %d not divisible by vector_width %d" % (extent, width))
        return kernel
    _set_transform(kernel, Vectorize, lambda t: True, Vectorize(width))
    _log(kernel, "vectorize",
         "widened unit-stride dense access %s along its last axis by %d "
         "(%d x f64 = %d-bit loads)" % (acc.tensor.name, width, width, 64 * width),
         "%s[j*K + k]" % acc.tensor.name, "%s vectorized loads" % acc.tensor.name)
    return kernel


# --------------------------------------------------------------------------- #
# 7. dead_code_elim
# --------------------------------------------------------------------------- #
def dead_code_elim(kernel: Kernel) -> Kernel:
    read = {name for st in kernel.stmts for name in _reads(st.rhs)}
    outputs = {st.lhs.tensor.name for st in kernel.stmts} - read
    keep = [st for st in kernel.stmts
            if st.lhs.tensor.name in read or st.lhs.tensor.name in outputs]
    dropped = [st.lhs.tensor.name for st in kernel.stmts if st not in keep]
    kernel.stmts = keep
    _log(kernel, "dead_code_elim", "removed %d unused temporary(ies)%s"
         % (len(dropped), (": " + ", ".join(dropped)) if dropped else ""))
    return kernel


# --------------------------------------------------------------------------- #
# pipeline
# --------------------------------------------------------------------------- #
PASSES = [canonicalize, loop_fusion, tiling, thread_mapping, unroll, vectorize,
          dead_code_elim]
PASS_NAMES = [p.__name__ for p in PASSES]


def run_pipeline(kernel: Kernel, config: Any = None, backend: str = "cpu",
                 fresh: bool = True, skip: Sequence[str] = ()) -> Kernel:
    """Apply every pass in order except those named in ``skip``."""
    k = copy.deepcopy(kernel) if fresh else kernel
    k._config = config
    k._backend = backend
    k.pass_log = []
    skipped = set(skip)
    for p in PASSES:
        if p.__name__ not in skipped:
            p(k)
    try:
        k.validate()
    except ValueError as exc:  # pragma: no cover - defensive
        raise ValueError("pass pipeline produced an invalid kernel: %s" % exc)
    return k


optimize = run_pipeline

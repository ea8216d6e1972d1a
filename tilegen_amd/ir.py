"""Index-notation IR for the CSR kernels (TACO-style tree of dataclasses).

Same public surface as the reference IR (``tilegen/ir.py:1-556``): the class
names, their fields, ``Kernel.validate/pretty/to_dict/from_dict`` and the
dictionary schema are kept so kernels, schedules and serialized IR move between
the two unchanged.  The implementation here is written from scratch.

    Format      per-level storage kinds, "dense" or "compressed"
    TensorDecl  named tensor: order, format, dtype, symbolic shape
    Expr        Access | Mul | Add | Const | Reduce
    Stmt        lhs Access = rhs Expr
    Transform   Tile | Split | Parallelize | Unroll | Fuse | ThreadsPerRow | Vectorize
    Schedule    ordered list of transforms
    Kernel      statements + schedule; the unit every pass rewrites
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, ClassVar, Dict, Iterator, List, Optional, Tuple

__all__ = [
    "Index", "Format", "DENSE1", "DENSE2", "CSR", "CSC", "COO", "ELL", "BSR",
    "SCALAR", "FORMAT_REGISTRY", "TensorDecl", "Expr", "Access", "Mul", "Add",
    "Const", "Reduce", "Stmt", "Assign", "Transform", "Tile", "Split",
    "Parallelize", "Unroll", "Fuse", "ThreadsPerRow", "Vectorize", "Schedule",
    "Kernel",
]

_LEVEL_KINDS = ("dense", "compressed")
_PAR_UNITS = ("block", "warp", "thread")


# --------------------------------------------------------------------------- #
# indices, formats, tensors
# --------------------------------------------------------------------------- #
@dataclass(frozen=True)
class Index:
    """An iteration variable (``i``, ``j``, ``k`` ...)."""

    name: str

    def __repr__(self) -> str:  # pragma: no cover - cosmetic
        return self.name


@dataclass(frozen=True)
class Format:
    """A storage format given by one kind per level (reference ``ir.py:71-93``)."""

    name: str
    levels: Tuple[str, ...]
    ell_width: Optional[int] = None
    block_size: Optional[int] = None

    @property
    def order(self) -> int:
        return len(self.levels)

    def is_sparse(self) -> bool:
        return any(kind == "compressed" for kind in self.levels)

    def compressed_positions(self) -> List[int]:
        return [pos for pos, kind in enumerate(self.levels) if kind == "compressed"]


DENSE1 = Format("dense1", ("dense",))
DENSE2 = Format("dense2", ("dense", "dense"))
CSR = Format("csr", ("dense", "compressed"))
CSC = Format("csc", ("compressed", "dense"))
COO = Format("coo", ("compressed", "compressed"))
ELL = Format("ell", ("dense", "compressed"), ell_width=8)
BSR = Format("bsr", ("dense", "compressed"), block_size=4)
SCALAR = Format("scalar", ())

FORMAT_REGISTRY: Dict[str, Format] = {
    f.name: f for f in (DENSE1, DENSE2, CSR, CSC, COO, ELL, BSR, SCALAR)
}


@dataclass
class TensorDecl:
    """A tensor of a kernel; ``shape`` holds symbolic extents such as ``"M"``."""

    name: str
    order: int
    format: Format
    dtype: str = "f64"
    shape: Tuple[Any, ...] = ()

    def is_scalar(self) -> bool:
        return self.order == 0

    def __hash__(self) -> int:
        return hash((self.name, self.order, self.dtype))


# --------------------------------------------------------------------------- #
# expressions
# --------------------------------------------------------------------------- #
def _to_expr(value: Any) -> "Expr":
    if isinstance(value, Expr):
        return value
    if isinstance(value, TensorDecl):
        return Access(value, [])
    if isinstance(value, (int, float)):
        return Const(float(value))
    raise TypeError("cannot use %r as an index expression" % (value,))


class Expr:
    """Base of index expressions; arithmetic operators build the tree."""

    def __mul__(self, other: Any) -> "Mul":
        return Mul(self, _to_expr(other))

    def __rmul__(self, other: Any) -> "Mul":
        return Mul(_to_expr(other), self)

    def __add__(self, other: Any) -> "Add":
        return Add(self, _to_expr(other))

    def __radd__(self, other: Any) -> "Add":
        return Add(_to_expr(other), self)

    def __sub__(self, other: Any) -> "Add":
        return Add(self, Mul(Const(-1.0), _to_expr(other)))

    def children(self) -> List["Expr"]:
        return []

    def walk(self) -> Iterator["Expr"]:
        """Pre-order traversal: this node, then each child subtree."""
        stack: List[Expr] = [self]
        while stack:
            node = stack.pop()
            yield node
            stack.extend(reversed(node.children()))


@dataclass(eq=False)
class Access(Expr):
    tensor: TensorDecl
    indices: List[Index]

    def bound_indices(self) -> List[Index]:
        return list(self.indices)

    def __repr__(self) -> str:  # pragma: no cover - cosmetic
        return "%s[%s]" % (self.tensor.name, ", ".join(i.name for i in self.indices))


@dataclass(eq=False)
class Mul(Expr):
    left: Expr
    right: Expr

    def children(self) -> List[Expr]:
        return [self.left, self.right]


@dataclass(eq=False)
class Add(Expr):
    left: Expr
    right: Expr

    def children(self) -> List[Expr]:
        return [self.left, self.right]


@dataclass(eq=False)
class Const(Expr):
    value: float


@dataclass(eq=False)
class Reduce(Expr):
    index: Index
    body: Expr

    def children(self) -> List[Expr]:
        return [self.body]


@dataclass(eq=False)
class Stmt:
    lhs: Access
    rhs: Expr


def Assign(lhs: Access, rhs: Expr) -> Stmt:
    """Assignment statement; ``lhs == rhs`` on an Access builds the same thing."""
    return Stmt(lhs=lhs, rhs=rhs)


def _access_assign(self: Access, other: Any) -> Stmt:
    return Stmt(lhs=self, rhs=_to_expr(other))


# ``y[i] == expr`` is assignment sugar (reference ``ir.py:256-262``).
Access.__eq__ = _access_assign  # type: ignore[assignment]


# --------------------------------------------------------------------------- #
# schedule transforms
# --------------------------------------------------------------------------- #
@dataclass
class Transform:
    kind: ClassVar[str] = "transform"


@dataclass
class Tile(Transform):
    index: Index = None  # type: ignore[assignment]
    size: int = 0
    #: what a tile holds: ``rows`` (``size`` consecutive rows), ``nnz`` (an equal
    #: share of rows plus nonzeros, about ``size`` rows' worth: merge-path windows)
    #: ``hybrid`` (``size`` rows, rows past a length threshold left to
    #: workgroups that each take an equal range of nonzeros) or ``stream`` (an
    #: equal range of nonzeros per workgroup and the rows that end in it; ``size``
    #: is not used)
    by: str = "rows"
    #: the order of a tile's gathers: ``direct`` (each lane gathers its own
    #: nonzeros' operands) or ``sorted`` (the tile's first-step gathers are made in
    #: operand order, sorted in LDS, so that one gather instruction's lanes share
    #: cache lines)
    gather: str = "direct"
    kind: ClassVar[str] = "tile"


@dataclass
class Split(Transform):
    index: Index = None  # type: ignore[assignment]
    factor: int = 0
    kind: ClassVar[str] = "split"


@dataclass
class Parallelize(Transform):
    index: Index = None  # type: ignore[assignment]
    unit: str = "thread"
    #: workgroup size chosen by thread_mapping; 0 leaves the backend default.
    block_size: int = 0
    kind: ClassVar[str] = "parallelize"


@dataclass
class Unroll(Transform):
    index: Index = None  # type: ignore[assignment]
    factor: int = 0
    kind: ClassVar[str] = "unroll"


@dataclass
class Fuse(Transform):
    index_a: Index = None  # type: ignore[assignment]
    index_b: Index = None  # type: ignore[assignment]
    kind: ClassVar[str] = "fuse"


@dataclass
class ThreadsPerRow(Transform):
    k: int = 1
    kind: ClassVar[str] = "threads_per_row"


@dataclass
class Vectorize(Transform):
    width: int = 1
    kind: ClassVar[str] = "vectorize"


@dataclass
class Schedule:
    transforms: List[Transform] = field(default_factory=list)

    def append(self, t: Transform) -> "Schedule":
        self.transforms.append(t)
        return self

    def __iter__(self):
        return iter(self.transforms)

    def __len__(self) -> int:
        return len(self.transforms)


# --------------------------------------------------------------------------- #
# kernel
# --------------------------------------------------------------------------- #
def _accesses(stmt: Stmt) -> List[Access]:
    """Accesses of a statement: rhs in pre-order, then the lhs."""
    found = [n for n in stmt.rhs.walk() if isinstance(n, Access)]
    found.append(stmt.lhs)
    return found


def _free_of(expr: Expr, bound: frozenset) -> List[Index]:
    """Indices of ``expr`` not bound by an enclosing Reduce, in leaf order."""
    if isinstance(expr, Reduce):
        return _free_of(expr.body, bound | {expr.index.name})
    if isinstance(expr, Access):
        return [ix for ix in expr.indices if ix.name not in bound]
    out: List[Index] = []
    for child in expr.children():
        out.extend(_free_of(child, bound))
    return out


def _first_unique(indices: List[Index]) -> List[Index]:
    seen, out = set(), []
    for ix in indices:
        if ix.name not in seen:
            seen.add(ix.name)
            out.append(ix)
    return out


@dataclass(eq=False)
class Kernel:
    name: str
    stmts: List[Stmt]
    schedule: Schedule = field(default_factory=Schedule)
    formats: List[Format] = field(default_factory=list)
    dtypes: List[str] = field(default_factory=list)
    pass_log: List[Dict[str, Any]] = field(default_factory=list)

    @property
    def stmt(self) -> Stmt:
        return self.stmts[0]

    def tensors(self) -> List[TensorDecl]:
        """Distinct tensors in discovery order (each rhs pre-order, then lhs)."""
        out: List[TensorDecl] = []
        names = set()
        for st in self.stmts:
            for acc in _accesses(st):
                if acc.tensor.name not in names:
                    names.add(acc.tensor.name)
                    out.append(acc.tensor)
        return out

    def free_indices(self) -> List[Index]:
        """Iteration-space indices: every lhs index first, then free rhs ones."""
        collected: List[Index] = []
        for st in self.stmts:
            collected.extend(st.lhs.indices)
        for st in self.stmts:
            collected.extend(_free_of(st.rhs, frozenset()))
        return _first_unique(collected)

    def _free_of(self, expr: Expr, bound: set) -> List[Index]:
        return _free_of(expr, frozenset(bound))

    def reduce_indices(self) -> List[Index]:
        return [n.index for st in self.stmts for n in st.rhs.walk()
                if isinstance(n, Reduce)]

    def all_indices(self) -> List[Index]:
        return _first_unique(self.free_indices() + self.reduce_indices())

    def reduce_node(self) -> Optional[Reduce]:
        for st in self.stmts:
            for n in st.rhs.walk():
                if isinstance(n, Reduce):
                    return n
        return None

    def sparse_tensor(self) -> Optional[TensorDecl]:
        return next((t for t in self.tensors() if t.format.is_sparse()), None)

    # -- validation ------------------------------------------------------ #
    def validate(self) -> bool:
        """Raise ValueError on the first structural problem; True otherwise.

        Checks mirror reference ``ir.py:431-518``: format levels, access rank
        versus tensor order, lhs indices bound by the rhs, reduce indices used in
        their body, schedule transforms naming known indices with sane sizes.
        """
        if not self.stmts:
            raise ValueError("kernel %r has no statements" % self.name)
        for fmt in self.formats:
            _check_format(fmt)
        for st in self.stmts:
            for acc in _accesses(st):
                t = acc.tensor
                if len(acc.indices) != t.order:
                    raise ValueError("access %s has %d indices but order is %d"
                                     % (t.name, len(acc.indices), t.order))
                if t.format.order != t.order:
                    raise ValueError("tensor %s: format %r order %d != declared order %d"
                                     % (t.name, t.format.name, t.format.order, t.order))
            rhs_free = {ix.name for ix in _free_of(st.rhs, frozenset())}
            for ix in st.lhs.indices:
                if ix.name not in rhs_free:
                    raise ValueError("index %r appears in the lhs but is not bound by "
                                     "the rhs" % ix.name)
            for node in st.rhs.walk():
                if isinstance(node, Reduce):
                    used = {ix.name for n in node.body.walk() if isinstance(n, Access)
                            for ix in n.indices}
                    if node.index.name not in used:
                        raise ValueError("reduce index %r does not appear in its body"
                                         % node.index.name)
        known = {ix.name for ix in self.all_indices()}
        for t in self.schedule:
            _check_transform(t, known)
        return True

    # -- rendering --------------------------------------------------------- #
    def pretty(self) -> str:
        """Readable loop-nest rendering (format pinned by the reference's
        ``tests/test_pretty.py:10-27`` snapshots)."""
        out = ["kernel %s {" % self.name]
        for st in self.stmts:
            out.append("  assign %s = %s" % (_lhs_text(st.lhs), _math(st.rhs)))
        out.append("  // loop nest")
        out.extend(_loop_nest_lines(self))
        if len(self.schedule):
            out.append("  // schedule")
            out.extend("  //   " + _transform_text(t) for t in self.schedule)
        out.append("}")
        return "\n".join(out)

    # -- serialization ------------------------------------------------------ #
    def to_dict(self) -> Dict[str, Any]:
        return {
            "name": self.name,
            "stmts": [{"lhs": _expr_dump(s.lhs), "rhs": _expr_dump(s.rhs)}
                      for s in self.stmts],
            "schedule": [_transform_dump(t) for t in self.schedule],
            "formats": [_format_dump(f) for f in self.formats],
            "dtypes": list(self.dtypes),
            "pass_log": list(self.pass_log),
        }

    @staticmethod
    def from_dict(d: Dict[str, Any]) -> "Kernel":
        return Kernel(
            name=d["name"],
            stmts=[Stmt(lhs=_expr_load(s["lhs"]), rhs=_expr_load(s["rhs"]))
                   for s in d["stmts"]],
            schedule=Schedule([_transform_load(t) for t in d["schedule"]]),
            formats=[_format_load(f) for f in d["formats"]],
            dtypes=list(d.get("dtypes", [])),
            pass_log=list(d.get("pass_log", [])),
        )


def _check_format(fmt: Format) -> None:
    if len(fmt.levels) != fmt.order:
        raise ValueError("format %r: %d levels for order %d"
                         % (fmt.name, len(fmt.levels), fmt.order))
    bad = [kind for kind in fmt.levels if kind not in _LEVEL_KINDS]
    if bad:
        raise ValueError("format %r has invalid level %r" % (fmt.name, bad[0]))


def _check_transform(t: Transform, known: set) -> None:
    named = []
    if isinstance(t, (Tile, Split, Parallelize, Unroll)):
        named = [t.index]
    elif isinstance(t, Fuse):
        named = [t.index_a, t.index_b]
    for ix in named:
        if ix is not None and ix.name not in known:
            raise ValueError("schedule transform %r refers to unknown index %r"
                             % (t.kind, ix.name))
    if isinstance(t, Tile) and t.size <= 0:
        raise ValueError("transform %r factor/size must be > 0" % t.kind)
    if isinstance(t, Tile) and t.by not in ("rows", "nnz", "hybrid", "stream"):
        raise ValueError("tile 'by' must be 'rows', 'nnz', 'hybrid' or 'stream', got %r" % t.by)
    if isinstance(t, Tile) and t.gather not in ("direct", "sorted"):
        raise ValueError("tile 'gather' must be 'direct' or 'sorted', got %r" % t.gather)
    if isinstance(t, Split) and t.factor <= 0:
        raise ValueError("transform %r factor/size must be > 0" % t.kind)
    if isinstance(t, Unroll) and t.factor <= 0:
        raise ValueError("Unroll factor must be > 0 (got %d)" % t.factor)
    if isinstance(t, ThreadsPerRow) and t.k <= 0:
        raise ValueError("ThreadsPerRow must be > 0 (got %d)" % t.k)
    if isinstance(t, Vectorize) and t.width <= 0:
        raise ValueError("Vectorize width must be > 0 (got %d)" % t.width)
    if isinstance(t, Parallelize):
        if t.unit not in _PAR_UNITS:
            raise ValueError("Parallelize unit must be block|warp|thread")
        if t.block_size < 0:
            raise ValueError("Parallelize block_size must be >= 0")


# --------------------------------------------------------------------------- #
# text rendering helpers
# --------------------------------------------------------------------------- #
def _access_text(a: Access) -> str:
    return "%s[%s]" % (a.tensor.name, ", ".join(ix.name for ix in a.indices))


def _fmt_expr(e: Expr) -> str:
    """Fully parenthesised rendering; used as a structural key by the passes."""
    if isinstance(e, Access):
        return _access_text(e)
    if isinstance(e, Const):
        return repr(e.value)
    if isinstance(e, Mul):
        return "(%s * %s)" % (_fmt_expr(e.left), _fmt_expr(e.right))
    if isinstance(e, Add):
        return "(%s + %s)" % (_fmt_expr(e.left), _fmt_expr(e.right))
    if isinstance(e, Reduce):
        return "sum(%s, %s)" % (e.index.name, _fmt_expr(e.body))
    return repr(e)  # pragma: no cover


def _lhs_text(a: Access) -> str:
    return a.tensor.name if a.tensor.order == 0 else _access_text(a)


# binding strength: products bind tighter than sums
_PREC = {Add: 1, Mul: 2}


def _math(e: Expr, outer: int = 0) -> str:
    """Math rendering with only the parentheses precedence needs."""
    if isinstance(e, Access):
        return _lhs_text(e)
    if isinstance(e, Const):
        return repr(e.value)
    if isinstance(e, Reduce):
        return "sum(%s, %s)" % (e.index.name, _math(e.body))
    prec = _PREC.get(type(e))
    if prec is None:  # pragma: no cover
        return repr(e)
    op = " * " if isinstance(e, Mul) else " + "
    text = _math(e.left, prec) + op + _math(e.right, prec)
    return "(%s)" % text if outer > prec else text


def _without_reduces(e: Expr) -> Expr:
    """The per-trip body of every reduction (Reduce nodes replaced by bodies)."""
    if isinstance(e, Reduce):
        return _without_reduces(e.body)
    if isinstance(e, Mul):
        return Mul(_without_reduces(e.left), _without_reduces(e.right))
    if isinstance(e, Add):
        return Add(_without_reduces(e.left), _without_reduces(e.right))
    return e


def _reductions_in(e: Expr) -> List[Reduce]:
    if isinstance(e, Reduce):
        return [e] + _reductions_in(e.body)
    if isinstance(e, (Mul, Add)):
        return _reductions_in(e.left) + _reductions_in(e.right)
    return []


def _loop_nest_lines(kernel: Kernel) -> List[str]:
    sparse = kernel.sparse_tensor()
    compressed_names = set()
    if sparse is not None:
        for st in kernel.stmts:
            hit = next((n for n in st.rhs.walk()
                        if isinstance(n, Access) and n.tensor.name == sparse.name), None)
            if hit is not None:
                for pos in sparse.format.compressed_positions():
                    if pos < len(hit.indices):
                        compressed_names.add(hit.indices[pos].name)
                break

    def source(ix: Index) -> str:
        return "%s row" % sparse.name if ix.name in compressed_names else "dense"

    lines: List[str] = []
    free = kernel.free_indices()
    depth = 1
    if free:
        lines.append("  for %s:" % ", ".join(ix.name for ix in free))
        depth = 2
    for st in kernel.stmts:
        level = depth
        reds = _reductions_in(st.rhs)
        for red in reds:
            lines.append("%sfor %s in reduce(%s):" % ("  " * level, red.index.name,
                                                       source(red.index)))
            level += 1
        body = _without_reduces(st.rhs) if reds else st.rhs
        lines.append("%sassign %s %s %s" % ("  " * level, _lhs_text(st.lhs),
                                            "+=" if reds else "=", _math(body)))
    return lines


def _transform_text(t: Transform) -> str:
    if isinstance(t, Tile):
        extra = (", by=%s" % t.by if t.by != "rows" else "") + \
            (", gather=%s" % t.gather if t.gather != "direct" else "")
        return "Tile(%s, %d%s)" % (t.index.name, t.size, extra)
    if isinstance(t, Split):
        return "Split(%s, %d)" % (t.index.name, t.factor)
    if isinstance(t, Parallelize):
        if t.block_size:
            return "Parallelize(%s, %s, block=%d)" % (t.index.name, t.unit, t.block_size)
        return "Parallelize(%s, %s)" % (t.index.name, t.unit)
    if isinstance(t, Unroll):
        return "Unroll(%s, %d)" % (t.index.name, t.factor)
    if isinstance(t, Fuse):
        return "Fuse(%s, %s)" % (t.index_a.name, t.index_b.name)
    if isinstance(t, ThreadsPerRow):
        return "ThreadsPerRow(%d)" % t.k
    if isinstance(t, Vectorize):
        return "Vectorize(%d)" % t.width
    return t.kind  # pragma: no cover


# --------------------------------------------------------------------------- #
# (de)serialization -- the dict schema of reference ir.py:705-822
# --------------------------------------------------------------------------- #
def _format_dump(f: Format) -> Dict[str, Any]:
    return {"name": f.name, "levels": list(f.levels), "ell_width": f.ell_width,
            "block_size": f.block_size}


def _format_load(d: Dict[str, Any]) -> Format:
    return Format(d["name"], tuple(d["levels"]), d.get("ell_width"), d.get("block_size"))


def _tensor_dump(t: TensorDecl) -> Dict[str, Any]:
    return {"name": t.name, "order": t.order, "format": _format_dump(t.format),
            "dtype": t.dtype, "shape": list(t.shape)}


def _tensor_load(d: Dict[str, Any]) -> TensorDecl:
    return TensorDecl(name=d["name"], order=d["order"], format=_format_load(d["format"]),
                      dtype=d["dtype"], shape=tuple(d["shape"]))


def _expr_dump(e: Expr) -> Dict[str, Any]:
    if isinstance(e, Access):
        return {"op": "access", "tensor": _tensor_dump(e.tensor),
                "indices": [{"name": ix.name} for ix in e.indices]}
    if isinstance(e, Const):
        return {"op": "const", "value": e.value}
    if isinstance(e, (Mul, Add)):
        return {"op": "mul" if isinstance(e, Mul) else "add",
                "left": _expr_dump(e.left), "right": _expr_dump(e.right)}
    if isinstance(e, Reduce):
        return {"op": "reduce", "index": {"name": e.index.name},
                "body": _expr_dump(e.body)}
    raise TypeError("unknown expr %r" % (e,))


def _expr_load(d: Dict[str, Any]) -> Expr:
    op = d["op"]
    if op == "access":
        return Access(_tensor_load(d["tensor"]), [Index(ix["name"]) for ix in d["indices"]])
    if op == "const":
        return Const(d["value"])
    if op in ("mul", "add"):
        cls = Mul if op == "mul" else Add
        return cls(_expr_load(d["left"]), _expr_load(d["right"]))
    if op == "reduce":
        return Reduce(Index(d["index"]["name"]), _expr_load(d["body"]))
    raise TypeError("unknown expr op %r" % op)


def _transform_dump(t: Transform) -> Dict[str, Any]:
    out: Dict[str, Any] = {"kind": t.kind}
    if isinstance(t, Tile):
        out.update(index={"name": t.index.name}, size=t.size)
        if t.by != "rows":
            out.update(by=t.by)
        if t.gather != "direct":
            out.update(gather=t.gather)
    elif isinstance(t, (Split, Unroll)):
        out.update(index={"name": t.index.name}, factor=t.factor)
    elif isinstance(t, Parallelize):
        out.update(index={"name": t.index.name}, unit=t.unit, block_size=t.block_size)
    elif isinstance(t, Fuse):
        out.update(index_a={"name": t.index_a.name}, index_b={"name": t.index_b.name})
    elif isinstance(t, ThreadsPerRow):
        out.update(k=t.k)
    elif isinstance(t, Vectorize):
        out.update(width=t.width)
    return out


def _transform_load(d: Dict[str, Any]) -> Transform:
    kind = d["kind"]
    ix = Index(d["index"]["name"]) if "index" in d else None
    if kind == "tile":
        return Tile(ix, d["size"], d.get("by", "rows"), d.get("gather", "direct"))
    if kind == "split":
        return Split(ix, d["factor"])
    if kind == "parallelize":
        return Parallelize(ix, d["unit"], d.get("block_size", 0))
    if kind == "unroll":
        return Unroll(ix, d["factor"])
    if kind == "fuse":
        return Fuse(Index(d["index_a"]["name"]), Index(d["index_b"]["name"]))
    if kind == "threads_per_row":
        return ThreadsPerRow(d["k"])
    if kind == "vectorize":
        return Vectorize(d["width"])
    raise TypeError("unknown transform kind %r" % kind)

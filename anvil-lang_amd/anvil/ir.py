"""Anvil's kernel IR: the data model the HIP backend consumes.

The class and attribute names are those of the reference's IR (anvil/ir.py:62-736), so that
`backend.hip.generate` accepts a program built by the reference's own front end as well as one
loaded from JSON (`irjson.load`). Only what a backend needs is here: the program tree, buffers,
loop variables, affine offsets and scalar expressions, with the same dtype rules.

A program is a tree of blocks. A kernel is a tensor comprehension

    for d in domain:                       # output loops
        acc = op over red.vars of red.body   # optional reduction (sum max min prod argmax argmin)
        let ...; store buf[offset] (=|+=) value ...

Every memory access is `buffer + affine offset` in elements, where an offset is
c0 + sum(ci * var_i) + sum(dj * scalar_j) + sum(ek * gather_k) (ir.py:1-12).
"""
from __future__ import annotations

import itertools
import math
from dataclasses import dataclass, field

F32 = "f32"
I32 = "i32"
EXTERN_KINDS = ("input", "output")          # the caller's arrays in library mode (ir.py:26)

_next_id = itertools.count(1)


def fresh_id() -> int:
    return next(_next_id)


def bump_ids(at_least: int) -> None:
    """Make later fresh ids larger than `at_least` (after loading a program with its own ids)."""
    global _next_id
    cur = next(_next_id)
    _next_id = itertools.count(max(cur, at_least + 1))


def prod(xs) -> int:
    out = 1
    for x in xs:
        out *= int(x)
    return out


def row_major_strides(shape) -> list[int]:
    out, s = [], 1
    for d in reversed(list(shape)):
        out.append(s)
        s *= int(d)
    return out[::-1]


# ----------------------------------------------------------------------------- buffers and vars

class Buffer:
    """A statically shaped f32/i32 array. `kind` is one of param state data temp var const grad
    scalar input output. `storage` points at the buffer whose memory this one reuses."""

    def __init__(self, name, shape, dtype=F32, kind="temp", init=None, span=None):
        self.id = fresh_id()
        self.name = name
        self.shape = tuple(int(d) for d in shape)
        self.dims = tuple(shape)
        self.dtype = dtype
        self.kind = kind
        self.init = init
        self.span = span
        self.storage = self

    @property
    def numel(self) -> int:
        return prod(self.shape)

    @property
    def nbytes(self) -> int:
        return 4 * self.numel

    @property
    def strides(self) -> list[int]:
        return row_major_strides(self.shape)

    @property
    def root(self) -> "Buffer":
        b = self
        while b.storage is not b:
            b = b.storage
        return b

    def __repr__(self):
        return f"{self.name}#{self.id}"


class Var:
    """A loop variable with a static extent."""

    def __init__(self, name, extent=None):
        self.id = fresh_id()
        self.name = name
        self.dim = None
        self.extent = None if extent is None else int(extent)

    @property
    def size(self):
        return self.extent

    def __repr__(self):
        return self.name


# ----------------------------------------------------------------------------- affine offsets

class ScalarRef:
    """The run-time value of an i32 0-d buffer used inside an offset."""

    def __init__(self, buf: Buffer):
        self.buf = buf

    def key(self):
        return ("s", self.buf.id)

    def __eq__(self, o):
        return isinstance(o, ScalarRef) and o.buf is self.buf

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return self.buf.name


class Gather:
    """A data-dependent index: the i32 loaded by `load`, checked against the dimension size
    `bound` (together with `rest`, the affine part added to it) at run time (ir.py:139-170)."""

    def __init__(self, load: "Load", bound: int, where: str = "", rest: "Affine | None" = None):
        self.load = load
        self.bound = int(bound)
        self.where = where
        self.rest = rest

    def key(self):
        return ("g", self.load.key(), self.bound, None if self.rest is None else self.rest.key())

    def check_range(self) -> tuple[int, int]:
        """The gathered value v must satisfy lo <= v < hi."""
        if self.rest is None:
            return 0, self.bound
        lo, hi = self.rest.var_bounds()
        return -lo, self.bound - hi

    def __eq__(self, o):
        return isinstance(o, Gather) and o.key() == self.key()

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return repr(self.load)


def _term_key(t):
    return ("v", t.id) if isinstance(t, Var) else t.key()


class Affine:
    """An immutable integer affine expression: const + sum(coef * term)."""

    __slots__ = ("const", "terms")

    def __init__(self, const: int = 0, terms: dict | None = None):
        self.const = int(const)
        self.terms = {k: int(v) for k, v in (terms or {}).items() if v != 0}

    @staticmethod
    def of(x) -> "Affine":
        if isinstance(x, Affine):
            return x
        if isinstance(x, int):
            return Affine(x)
        return Affine(0, {x: 1})

    def __add__(self, o):
        o = Affine.of(o)
        t = dict(self.terms)
        for k, v in o.terms.items():
            t[k] = t.get(k, 0) + v
        return Affine(self.const + o.const, t)

    __radd__ = __add__

    def __neg__(self):
        return Affine(-self.const, {k: -v for k, v in self.terms.items()})

    def __sub__(self, o):
        return self + (-Affine.of(o))

    def __mul__(self, c: int):
        return Affine(self.const * c, {k: v * c for k, v in self.terms.items()})

    __rmul__ = __mul__

    def is_const(self) -> bool:
        return not self.terms

    def coef(self, v) -> int:
        return self.terms.get(v, 0)

    def direct_vars(self) -> list[Var]:
        return [k for k in self.terms if isinstance(k, Var)]

    def vars(self) -> list[Var]:
        out = []
        for k in self.terms:
            if isinstance(k, Var):
                if k not in out:
                    out.append(k)
            elif isinstance(k, Gather):
                for v in k.load.offset.vars():
                    if v not in out:
                        out.append(v)
        return out

    def scalars(self) -> list[ScalarRef]:
        return [k for k in self.terms if isinstance(k, ScalarRef)]

    def gathers(self) -> list[Gather]:
        return [k for k in self.terms if isinstance(k, Gather)]

    def key(self):
        return (self.const, tuple(sorted(((_term_key(k), c) for k, c in self.terms.items()), key=repr)))

    def __eq__(self, o):
        return isinstance(o, Affine) and self.key() == o.key()

    def __hash__(self):
        return hash(self.key())

    def var_bounds(self) -> tuple[int, int]:
        """Min and max of the loop-variable part (scalars and gathers ignored)."""
        lo = hi = self.const
        for k, c in self.terms.items():
            if isinstance(k, Var):
                span = c * ((k.extent or 1) - 1)
                if span >= 0:
                    hi += span
                else:
                    lo += span
        return lo, hi

    def __repr__(self):
        return fmt_affine(self)


def fmt_affine(a: Affine) -> str:
    parts = []
    for k, c in a.terms.items():
        name = k.name if isinstance(k, Var) else repr(k)
        parts.append(name if c == 1 else f"{c}*{name}")
    if a.const or not parts:
        parts.append(str(a.const))
    return " + ".join(parts).replace("+ -", "- ")


# ----------------------------------------------------------------------------- expressions

UNARY_OPS = {"neg", "abs", "exp", "log", "sqrt", "tanh", "sigmoid", "sin", "cos", "floor", "ceil",
             "round", "sign", "not", "f32", "i32", "detach", "rsqrt", "recip"}
BINARY_OPS = {"add", "sub", "mul", "div", "max", "min", "pow", "idiv", "mod",
              "lt", "le", "gt", "ge", "eq", "ne", "and", "or"}
COMPARISONS = {"lt", "le", "gt", "ge", "eq", "ne"}
FLOAT_UNARY = {"exp", "log", "sqrt", "tanh", "sigmoid", "sin", "cos", "rsqrt", "recip"}


class Expr:
    dtype = F32

    def key(self):
        raise NotImplementedError

    def children(self):
        return []

    def rebuild(self, kids):
        return self

    def __eq__(self, o):
        return isinstance(o, Expr) and self.key() == o.key()

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return fmt_expr(self)


class Const(Expr):
    def __init__(self, value, dtype=F32):
        self.dtype = dtype
        self.value = float(value) if dtype == F32 else int(value)

    def key(self):
        return ("c", self.dtype, self.value)


class Load(Expr):
    def __init__(self, buf: Buffer, offset: Affine):
        self.buf = buf
        self.offset = offset
        self.dtype = buf.dtype

    def key(self):
        return ("ld", self.buf.id, self.offset.key())


class Index(Expr):
    """The i32 value of an affine expression of loop variables."""
    dtype = I32

    def __init__(self, affine: Affine):
        self.affine = affine

    def key(self):
        return ("ix", self.affine.key())


class Unary(Expr):
    def __init__(self, op, a, dtype=None):
        assert op in UNARY_OPS, op
        self.op = op
        self.a = a
        if dtype is None:
            dtype = {"f32": F32, "i32": I32, "not": F32}.get(op, a.dtype)
            if op in FLOAT_UNARY:
                dtype = F32
        self.dtype = dtype

    def key(self):
        return ("u", self.op, self.dtype, self.a.key())

    def children(self):
        return [self.a]

    def rebuild(self, kids):
        return Unary(self.op, kids[0], self.dtype)


class Binary(Expr):
    def __init__(self, op, a, b, dtype=None):
        assert op in BINARY_OPS, op
        self.op = op
        self.a = a
        self.b = b
        if dtype is None:
            both_int = a.dtype == I32 and b.dtype == I32
            if op in COMPARISONS or op in ("and", "or", "div"):
                dtype = F32
            else:
                dtype = I32 if both_int else F32
        self.dtype = dtype

    def key(self):
        return ("b", self.op, self.dtype, self.a.key(), self.b.key())

    def children(self):
        return [self.a, self.b]

    def rebuild(self, kids):
        return Binary(self.op, kids[0], kids[1], self.dtype)


class Select(Expr):
    def __init__(self, c, a, b):
        self.c = c
        self.a = a
        self.b = b
        self.dtype = F32 if F32 in (a.dtype, b.dtype) else I32

    def key(self):
        return ("sel", self.c.key(), self.a.key(), self.b.key())

    def children(self):
        return [self.c, self.a, self.b]

    def rebuild(self, kids):
        return Select(*kids)


class Acc(Expr):
    """The kernel's reduction result (valid in its statements only)."""

    def __init__(self, dtype=F32):
        self.dtype = dtype

    def key(self):
        return ("acc", self.dtype)


class LetRef(Expr):
    def __init__(self, let: "Let"):
        self.let = let
        self.dtype = let.value.dtype

    def key(self):
        return ("let", id(self.let))


class Rand(Expr):
    """A uniform f32 in [0, 1) (or (0, 1] when open_low) from a counter-based hash of
    (seed, stream, flattened domain index, salt)."""
    dtype = F32

    def __init__(self, salt: int, open_low: bool = False):
        self.salt = int(salt)
        self.open_low = bool(open_low)

    def key(self):
        return ("rand", self.salt, self.open_low)


def iter_expr(e):
    """Every node of e, pre-order, including the index loads of gathers in load offsets."""
    yield e
    for k in e.children():
        yield from iter_expr(k)
    if isinstance(e, Load):
        for g in e.offset.gathers():
            yield from iter_expr(g.load)


def loads_in(e) -> list:
    return [x for x in iter_expr(e) if isinstance(x, Load)]


def map_expr(e, fn):
    kids = e.children()
    if kids:
        new = [map_expr(k, fn) for k in kids]
        if any(n is not k for n, k in zip(new, kids)):
            e = e.rebuild(new)
    return fn(e)


def uses_rand(e) -> bool:
    return any(isinstance(x, Rand) for x in iter_expr(e))


# ----------------------------------------------------------------------------- kernels

@dataclass(eq=False)
class Let:
    name: str
    value: Expr


@dataclass
class Store:
    buf: Buffer
    offset: Affine
    value: Expr
    accumulate: bool = False


@dataclass
class Reduction:
    vars: list
    op: str                  # sum | max | min | prod | argmax | argmin
    body: Expr

    @property
    def dtype(self):
        return I32 if self.op in ("argmax", "argmin") else self.body.dtype


@dataclass
class Kernel:
    domain: list
    stmts: list
    red: Reduction | None = None
    name: str = ""
    label: str = ""
    span: object = None
    id: int = field(default_factory=fresh_id)

    @property
    def stores(self) -> list:
        return [s for s in self.stmts if isinstance(s, Store)]

    def exprs(self):
        if self.red is not None:
            yield self.red.body
        for s in self.stmts:
            yield s.value

    def reads(self) -> set:
        out = set()
        for e in self.exprs():
            for ld in loads_in(e):
                out.add(ld.buf.root)
        for s in self.stores:
            if s.accumulate:
                out.add(s.buf.root)
            for g in s.offset.gathers():
                out.add(g.load.buf.root)
        return out

    def writes(self) -> set:
        return {s.buf.root for s in self.stores}

    def all_vars(self) -> list:
        return list(self.domain) + (list(self.red.vars) if self.red is not None else [])

    def iterations(self) -> int:
        return prod(v.extent for v in self.all_vars())

    def uses_rand(self) -> bool:
        return any(uses_rand(e) for e in self.exprs())


# ----------------------------------------------------------------------------- statements

class Stmt:
    pass


@dataclass
class KernelStmt(Stmt):
    kernel: Kernel


@dataclass
class Block:
    stmts: list = field(default_factory=list)
    is_loop: bool = False


@dataclass
class For(Stmt):
    counter: Buffer
    start: object            # int or an i32 0-d Buffer
    stop: object
    step: int
    body: Block
    span: object = None


@dataclass
class While(Stmt):
    cond_block: Block
    cond: Buffer
    body: Block
    span: object = None


@dataclass
class If(Stmt):
    cond: Buffer
    then: Block
    orelse: Block
    span: object = None


@dataclass
class Break(Stmt):
    pass


@dataclass
class Continue(Stmt):
    pass


@dataclass
class PrintItem:
    kind: str                # text | scalar | tensor | pick | chars
    text: str = ""
    buf: Buffer | None = None
    fmt: str = ""
    choices: list | None = None


@dataclass
class Print(Stmt):
    items: list
    end: str = "\n"
    err: bool = False


@dataclass
class Check(Stmt):
    """A run-time assertion lo <= value <= hi, value an affine of run-time scalars."""
    value: Affine
    lo: int
    hi: int
    message: str
    span: object = None


@dataclass
class RTCall(Stmt):
    name: str
    args: dict
    span: object = None


@dataclass
class Program:
    main: Block
    buffers: list
    source: object = None


def walk_blocks(block: Block):
    yield block
    for s in block.stmts:
        if isinstance(s, For):
            yield from walk_blocks(s.body)
        elif isinstance(s, While):
            yield from walk_blocks(s.cond_block)
            yield from walk_blocks(s.body)
        elif isinstance(s, If):
            yield from walk_blocks(s.then)
            yield from walk_blocks(s.orelse)


def all_kernels(prog: Program) -> list:
    return [s.kernel for b in walk_blocks(prog.main) for s in b.stmts if isinstance(s, KernelStmt)]


def ckpt_key(b: Buffer) -> int:
    """The 64-bit checkpoint key of a tensor: its element count in the low 32 bits and an FNV-1a
    hash of `name-inside-model:dtype:shape` in the high 32 bits (ir.py:753-764)."""
    if b.numel >= 1 << 32:
        raise ValueError(f"{b.name} is too large to checkpoint")
    inside = b.name.split(".", 1)[1] if "." in b.name else ""
    h = 0x811C9DC5
    for byte in f"{inside}:{b.dtype}:{','.join(str(d) for d in b.shape)}".encode():
        h = ((h ^ byte) * 0x01000193) & 0xFFFFFFFF
    return ((h or 1) << 32) | b.numel


# ----------------------------------------------------------------------------- printing (comments)

def fmt_expr(e) -> str:
    if isinstance(e, Const):
        if e.dtype == F32 and math.isinf(e.value):
            return "inf" if e.value > 0 else "-inf"
        return repr(e.value)
    if isinstance(e, Load):
        return f"{e.buf.name}{{{fmt_affine(e.offset)}}}"
    if isinstance(e, Index):
        return f"({fmt_affine(e.affine)})"
    if isinstance(e, Acc):
        return "acc"
    if isinstance(e, LetRef):
        return e.let.name
    if isinstance(e, Rand):
        return f"rand{e.salt}{'+' if e.open_low else ''}"
    if isinstance(e, Unary):
        return f"{e.op}({fmt_expr(e.a)})"
    if isinstance(e, Binary):
        return f"{e.op}({fmt_expr(e.a)}, {fmt_expr(e.b)})"
    if isinstance(e, Select):
        return f"({fmt_expr(e.a)} if {fmt_expr(e.c)} else {fmt_expr(e.b)})"
    return f"<{type(e).__name__}>"


def fmt_kernel(k: Kernel) -> str:
    parts = []
    if k.red is not None:
        parts.append(f"acc = {k.red.op}_{','.join(v.name for v in k.red.vars)} {fmt_expr(k.red.body)}")
    for s in k.stmts:
        if isinstance(s, Let):
            parts.append(f"let {s.name} = {fmt_expr(s.value)}")
        else:
            parts.append(f"{s.buf.name}{{{fmt_affine(s.offset)}}} {'+=' if s.accumulate else '='} "
                         f"{fmt_expr(s.value)}")
    return "; ".join(parts)

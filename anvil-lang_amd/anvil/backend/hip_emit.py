"""Scalar C code for IR expressions and statements (one output element's worth of work).

An `Emitter` turns expression trees into C statements that assign temporaries, sharing common
subexpressions; the same emitter writes device code (kernels) and host code (scalar kernels run on
the host). Where things live is the `Scope`'s business: loop variables, buffer pointers, host
scalars, the reduction result, the random stream, and any value the schedule already holds in a
register (a forwarded store or a cached load).

Semantics (those of the reference interpreter, interp.py:540-632, and the CUDA emitter's scalar
rules, cuda.py:78-199): comparisons and logic give 1.0f/0.0f; i32 add/sub/mul wrap; i32 floor
division and modulo follow Python with a zero divisor counted as 1; float `//` is floor(a/b) and
float `%` has the divisor's sign; max/min propagate NaN; `i32()` truncates; `round` is rint
(half to even); rsqrt is 1/sqrt; a gathered index is checked against its dimension, a failure is
latched (device) or reported (host) and the index clamped.
"""
from __future__ import annotations

import math

from .. import ir
from ..ir import F32, I32, Acc, Const, Gather, Index, LetRef, Load, Rand, ScalarRef, Select, Unary, Binary, Var

INT_MIN_LIT = "(-2147483647 - 1)"


def ctype(dtype) -> str:
    return "int" if dtype == I32 else "float"


def flit(v: float) -> str:
    """A C float literal that reads back as the same float32."""
    v = float(v)
    if math.isnan(v):
        return "__builtin_nanf(\"\")"
    if math.isinf(v):
        return "__builtin_inff()" if v > 0 else "(-__builtin_inff())"
    r = repr(v)
    if "e" not in r and "." not in r:
        r += ".0"
    return r + "f"


def ilit(v: int) -> str:
    v = int(v)
    if v == -(1 << 31):
        return INT_MIN_LIT
    return str(v)


def c_string(s: str) -> str:
    out = []
    for ch in s:
        o = ord(ch)
        if ch == "\\":
            out.append("\\\\")
        elif ch == '"':
            out.append('\\"')
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\t":
            out.append("\\t")
        elif ch == "\r":
            out.append("\\r")
        elif o < 32 or o == 127:
            out.append(f"\\{o:03o}")
        elif o > 127:
            out.extend(f"\\{b:03o}" for b in ch.encode("utf-8"))
        else:
            out.append(ch)
    return '"' + "".join(out) + '"'


def sanitize(name: str) -> str:
    s = "".join(c if c.isalnum() else "_" for c in name)
    return s[:40]


class Scope:
    """Where the values an expression needs come from. Subclassed by each schedule."""

    device = True                    # device code: faults are latched, not reported

    def var(self, v: Var) -> str:
        raise NotImplementedError

    def buf(self, b: ir.Buffer) -> str:
        """The C pointer expression of a buffer (device code: a kernel parameter)."""
        raise NotImplementedError

    def host_scalar(self, b: ir.Buffer) -> str | None:
        """The C name of a host scalar's value (a kernel argument or a host variable), or None."""
        return None

    def acc(self) -> str:
        return "acc"

    def rand_index(self) -> str:
        raise NotImplementedError

    def stream(self) -> str:
        return "anvil_rs"

    def seed(self) -> str:
        return "anvil_seed"

    def fault(self, message: str) -> int:
        raise NotImplementedError

    def override_load(self, ld: Load) -> str | None:
        """A register already holding this load's value, or None."""
        return None

    def loaded(self, ld: Load, name: str) -> None:
        """Called once a load's value is held in the C constant `name`."""

    def int_offsets(self, b: ir.Buffer) -> bool:
        """May offsets into b be computed in 32-bit arithmetic?"""
        return b.root.numel < (1 << 30)


class Emitter:
    def __init__(self, scope: Scope, lines: list, ind: str, prefix: str = "t"):
        self.s = scope
        self.lines = lines
        self.ind = ind
        self.prefix = prefix
        self.n = 0
        self.memo: dict = {}
        self.lets: dict[int, str] = {}

    def tmp(self) -> str:
        self.n += 1
        return f"{self.prefix}{self.n}"

    def emit(self, line: str) -> None:
        self.lines.append(self.ind + line)

    # ------------------------------------------------------------------ offsets
    def affine(self, a: ir.Affine, buf: ir.Buffer | None = None) -> str:
        wide = buf is None or not self.s.int_offsets(buf)
        cast = "(long long)" if wide else "(int)"
        parts = []
        if a.const:
            parts.append(f"{a.const}LL" if wide else ilit(a.const))
        for t, c in sorted(a.terms.items(), key=lambda tc: _term_order(tc[0])):
            if isinstance(t, Var):
                x = f"{cast}{self.s.var(t)}"
            elif isinstance(t, ScalarRef):
                x = f"{cast}{self.scalar_ref(t.buf)}"
            elif isinstance(t, Gather):
                x = self.gather(t)
                x = f"{cast}{x}"
            else:
                raise NotImplementedError(type(t).__name__)
            parts.append(x if c == 1 else f"{c}{'LL' if wide else ''} * {x}")
        return " + ".join(parts) if parts else "0"

    def scalar_ref(self, b: ir.Buffer) -> str:
        h = self.s.host_scalar(b)
        if h is not None:
            return h
        return f"{self.s.buf(b)}[0]"

    def gather(self, g: Gather) -> str:
        key = ("gather", g.key())
        if key in self.memo:
            return self.memo[key]
        v = self.ex(g.load)
        name = self.tmp()
        lo, hi = g.check_range()
        code = self.s.fault(f"index out of bounds ({g.where or 'gather'}; dimension size {g.bound})")
        self.emit(f"int {name} = {v};")
        if self.s.device:
            self.emit(f"if ({name} < {ilit(lo)} || {name} >= {ilit(hi)}) {{ anvil_fault({code}, {name}); {name} = {ilit(lo)}; }}")
        else:
            self.emit(f"if ({name} < {ilit(lo)} || {name} >= {ilit(hi)}) anvil_bad_value(anvil_fault_text[{code}], {name});")
        self.memo[key] = name
        return name

    # ------------------------------------------------------------------ expressions
    def ex(self, e) -> str:
        if isinstance(e, Const):
            return flit(e.value) if e.dtype == F32 else ilit(e.value)
        if isinstance(e, Acc):
            return self.s.acc()
        if isinstance(e, LetRef):
            return self.lets[id(e.let)]
        key = e.key()
        if key in self.memo:
            return self.memo[key]
        if isinstance(e, Load):
            got = self.s.override_load(e)
            if got is not None:
                self.memo[key] = got
                return got
            h = self.s.host_scalar(e.buf) if not e.buf.root.shape else None
            if h is not None:
                self.memo[key] = h
                return h
        text = self.build(e)
        name = self.tmp()
        self.emit(f"const {ctype(e.dtype)} {name} = {text};")
        self.memo[key] = name
        if isinstance(e, Load):
            self.s.loaded(e, name)
        return name

    def as_float(self, e) -> str:
        s = self.ex(e)
        return s if e.dtype == F32 else f"(float)({s})"

    def as_type(self, e, dtype) -> str:
        s = self.ex(e)
        if e.dtype == dtype:
            return s
        return f"(float)({s})" if dtype == F32 else f"anvil_trunci({s})"

    def build(self, e) -> str:
        if isinstance(e, Load):
            return f"{self.s.buf(e.buf)}[{self.affine(e.offset, e.buf)}]"
        if isinstance(e, Index):
            return f"(int)({self.affine(e.affine)})"
        if isinstance(e, Rand):
            return (f"anvil_uniform((uint32_t)({self.s.rand_index()}), {self.s.stream()}, {e.salt}u, "
                    f"{self.s.seed()}, {1 if e.open_low else 0})")
        if isinstance(e, Unary):
            return self.unary(e)
        if isinstance(e, Binary):
            return self.binary(e)
        if isinstance(e, Select):
            c = self.ex(e.c)
            a = self.as_type(e.a, e.dtype)
            b = self.as_type(e.b, e.dtype)
            return f"(({c}) != 0 ? {a} : {b})"
        raise NotImplementedError(type(e).__name__)

    def unary(self, e: Unary) -> str:
        op = e.op
        isint = e.a.dtype == I32
        a = self.ex(e.a)
        if op == "detach":
            return a
        if op == "neg":
            return f"(int)(0u - (uint32_t)({a}))" if isint else f"(-({a}))"
        if op == "abs":
            return f"(({a}) < 0 ? (int)(0u - (uint32_t)({a})) : ({a}))" if isint else f"fabsf({a})"
        if op == "not":
            return f"(({a}) == 0 ? 1.0f : 0.0f)"
        if op == "f32":
            return f"(float)({a})"
        if op == "i32":
            return a if isint else f"anvil_trunci({a})"
        if op == "sign":
            return f"anvil_signi({a})" if isint else f"anvil_signf({a})"
        if op in ("floor", "ceil", "round"):
            if isint:
                return a
            return {"floor": "floorf", "ceil": "ceilf", "round": "rintf"}[op] + f"({a})"
        fa = f"(float)({a})" if isint else a
        if op == "rsqrt":
            return f"(1.0f / sqrtf({fa}))"
        if op == "recip":
            return f"(1.0f / ({fa}))"
        if op == "sigmoid":
            return f"anvil_sigmoidf({fa})"
        fn = {"exp": "expf", "log": "logf", "sqrt": "sqrtf", "tanh": "tanhf", "sin": "sinf", "cos": "cosf"}[op]
        return f"{fn}({fa})"

    def binary(self, e: Binary) -> str:
        op = e.op
        if op in ir.COMPARISONS:
            a, b = self.ex(e.a), self.ex(e.b)
            if e.a.dtype != e.b.dtype:            # NumPy compares i32 with f32 in float64: exactly
                a, b = f"(double)({a})", f"(double)({b})"
            sym = {"lt": "<", "le": "<=", "gt": ">", "ge": ">=", "eq": "==", "ne": "!="}[op]
            return f"(({a}) {sym} ({b}) ? 1.0f : 0.0f)"
        if op in ("and", "or"):
            a, b = self.ex(e.a), self.ex(e.b)
            return f"((({a}) != 0 {'&&' if op == 'and' else '||'} ({b}) != 0) ? 1.0f : 0.0f)"
        if e.dtype == I32:
            a, b = self.as_type(e.a, I32), self.as_type(e.b, I32)
            if op in ("add", "sub", "mul"):
                return f"anvil_wrap_{op}({a}, {b})"
            if op == "pow":
                return f"(int)powf((float)({a}), (float)({b}))"
            return {"idiv": "anvil_floordiv", "mod": "anvil_floormod", "max": "anvil_maxi",
                    "min": "anvil_mini"}[op] + f"({a}, {b})"
        a, b = self.as_float(e.a), self.as_float(e.b)
        if op in ("add", "sub", "mul", "div"):
            return f"(({a}) {dict(add='+', sub='-', mul='*', div='/')[op]} ({b}))"
        if op == "max":
            return f"anvil_maxf({a}, {b})"
        if op == "min":
            return f"anvil_minf({a}, {b})"
        if op == "pow":
            return f"powf({a}, {b})"
        if op == "idiv":
            return f"floorf(({a}) / ({b}))"
        if op == "mod":
            return f"anvil_pymodf({a}, {b})"
        raise NotImplementedError(op)

    # ------------------------------------------------------------------ statements
    def let(self, st: ir.Let) -> str:
        v = self.ex(st.value)
        name = self.tmp()
        self.emit(f"const {ctype(st.value.dtype)} {name} = {v};")
        self.lets[id(st)] = name
        return name

    def store_value(self, st: ir.Store) -> str:
        return self.as_type(st.value, st.buf.dtype)

    def reset_memo(self) -> None:
        """After a store, loads read memory again (a later load may see what was stored)."""
        self.memo = {}


def _term_order(t):
    if isinstance(t, Var):
        return (0, t.id)
    if isinstance(t, ScalarRef):
        return (1, t.buf.id)
    return (2, repr(t.key()))

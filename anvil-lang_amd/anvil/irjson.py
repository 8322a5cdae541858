"""Kernel IR <-> JSON.

`dump` reads a program by attribute and class name only (it imports nothing from this package), so
it serializes any object graph with the IR's shape: this package's own `ir` objects, or the
reference front end's (anvil/ir.py:62-736). `load` rebuilds the program as this package's `ir`
objects, keeping buffer, variable and kernel ids, so generated code and checkpoints are the same
for the loaded program as for the original.

Format "anvil-ir/1":
    {"format", "source", "buffers": [buffer], "main": [stmt]}
    buffer = {"id", "name", "shape", "dtype", "kind", "init", "storage", "heap"}
    stmt   = {"t": "kernel"|"for"|"while"|"if"|"break"|"continue"|"print"|"check"|"rt", ...}
    expr   = ["c", dtype, v] | ["ld", buf, aff] | ["ix", aff] | ["u", op, dtype, e]
           | ["b", op, dtype, e, e] | ["sel", e, e, e] | ["acc", dtype] | ["let", i] | ["rand", salt, open]
    aff    = [const, [[term, coef], ...]],  term = ["v", var] | ["s", buf] | ["g", ld, bound, where, aff|null]
"""
from __future__ import annotations

import json
import math

FORMAT = "anvil-ir/1"


# ----------------------------------------------------------------------------- dump (duck-typed)

def _cls(x) -> str:
    return type(x).__name__


def _num(v):
    if isinstance(v, float):
        if math.isnan(v):
            return "nan"
        if math.isinf(v):
            return "inf" if v > 0 else "-inf"
    return v


class _Dumper:
    def __init__(self):
        self.bufs = {}

    def buf(self, b) -> int:
        self.bufs[b.id] = b
        s = b.storage
        if s is not b:
            self.buf(s)
        return b.id

    def aff(self, a, lets):
        terms = []
        for t, c in a.terms.items():
            n = _cls(t)
            if n == "Var":
                terms.append([["v", t.id], c])
            elif n == "ScalarRef":
                terms.append([["s", self.buf(t.buf)], c])
            elif n == "Gather":
                terms.append([["g", self.expr(t.load, lets), t.bound, t.where,
                               None if t.rest is None else self.aff(t.rest, lets)], c])
            else:
                raise TypeError(f"unknown affine term {n}")
        return [a.const, terms]

    def expr(self, e, lets):
        n = _cls(e)
        if n == "Const":
            return ["c", e.dtype, _num(e.value)]
        if n == "Load":
            return ["ld", self.buf(e.buf), self.aff(e.offset, lets)]
        if n == "Index":
            return ["ix", self.aff(e.affine, lets)]
        if n == "Unary":
            return ["u", e.op, e.dtype, self.expr(e.a, lets)]
        if n == "Binary":
            return ["b", e.op, e.dtype, self.expr(e.a, lets), self.expr(e.b, lets)]
        if n == "Select":
            return ["sel", self.expr(e.c, lets), self.expr(e.a, lets), self.expr(e.b, lets)]
        if n == "Acc":
            return ["acc", e.dtype]
        if n == "LetRef":
            return ["let", lets[id(e.let)]]
        if n == "Rand":
            return ["rand", e.salt, bool(e.open_low)]
        raise TypeError(f"unknown expression {n}")

    @staticmethod
    def var(v):
        return {"id": v.id, "name": v.name, "extent": v.extent}

    def kernel(self, k):
        lets = {}
        stmts = []
        red = None
        if k.red is not None:
            red = {"vars": [self.var(v) for v in k.red.vars], "op": k.red.op,
                   "body": self.expr(k.red.body, lets)}
        for i, s in enumerate(k.stmts):
            if _cls(s) == "Let":
                stmts.append({"t": "let", "name": s.name, "value": self.expr(s.value, lets)})
                lets[id(s)] = i
            else:
                stmts.append({"t": "store", "buf": self.buf(s.buf), "offset": self.aff(s.offset, lets),
                              "value": self.expr(s.value, lets), "acc": bool(s.accumulate)})
        line = getattr(k.span, "line", None) if k.span is not None else None
        out = {"id": k.id, "name": k.name, "label": k.label, "line": line,
               "domain": [self.var(v) for v in k.domain], "red": red, "stmts": stmts}
        loc = self.loc(k.span)
        if loc:                                         # where the kernel comes from (--check messages)
            out["loc"] = loc
            try:
                out["src"] = k.span.file.line_text(k.span.line).strip()
            except Exception:
                pass
        return out

    @staticmethod
    def loc(span):
        if span is None:
            return None
        try:
            return span.location()
        except Exception:
            return None

    def bound(self, x):
        return x if isinstance(x, int) else {"buf": self.buf(x)}

    def rt_arg(self, v):
        n = _cls(v)
        if n == "Buffer":
            return {"buf": self.buf(v)}
        if isinstance(v, (bytes, bytearray)):
            return {"bytes": bytes(v).hex()}
        if isinstance(v, (list, tuple)):
            if v and all(_cls(x) == "Buffer" for x in v):
                return {"bufs": [self.buf(x) for x in v]}
            return {"list": [self.rt_arg(x) for x in v]}
        if isinstance(v, (str, int, float, bool)) or v is None:
            return {"v": _num(v)}
        raise TypeError(f"unknown run-time call argument {n}")

    def block(self, blk):
        return [self.stmt(s) for s in blk.stmts]

    def stmt(self, s):
        n = _cls(s)
        if n == "KernelStmt":
            return {"t": "kernel", "kernel": self.kernel(s.kernel)}
        if n == "For":
            return {"t": "for", "counter": self.buf(s.counter), "start": self.bound(s.start),
                    "stop": self.bound(s.stop), "step": s.step, "body": self.block(s.body)}
        if n == "While":
            return {"t": "while", "cond_block": self.block(s.cond_block), "cond": self.buf(s.cond),
                    "body": self.block(s.body)}
        if n == "If":
            return {"t": "if", "cond": self.buf(s.cond), "then": self.block(s.then),
                    "else": self.block(s.orelse)}
        if n == "Break":
            return {"t": "break"}
        if n == "Continue":
            return {"t": "continue"}
        if n == "Print":
            items = []
            for it in s.items:
                items.append({"kind": it.kind, "text": it.text,
                              "buf": None if it.buf is None else self.buf(it.buf),
                              "fmt": it.fmt, "choices": it.choices})
            return {"t": "print", "items": items, "end": s.end, "err": bool(s.err)}
        if n == "Check":
            return {"t": "check", "value": self.aff(s.value, {}), "lo": s.lo, "hi": s.hi,
                    "message": s.message, "loc": self.loc(s.span)}
        if n == "RTCall":
            return {"t": "rt", "name": s.name, "args": {k: self.rt_arg(v) for k, v in s.args.items()},
                    "loc": self.loc(s.span)}
        raise TypeError(f"unknown statement {n}")


def dump(prog) -> dict:
    """The program as a JSON-ready dict."""
    d = _Dumper()
    main = d.block(prog.main)
    for b in prog.buffers:
        d.buf(b)
    bufs = []
    for bid in sorted(d.bufs):
        b = d.bufs[bid]
        init = None
        if b.init is not None:
            init = [_num(float(v)) if b.dtype == "f32" else int(v) for v in b.init]
        bufs.append({"id": b.id, "name": b.name, "shape": list(b.shape), "dtype": b.dtype, "kind": b.kind,
                     "init": init, "storage": b.storage.id, "heap": bool(getattr(b, "heap", False))})
    src = None
    if getattr(prog, "source", None) is not None:
        try:
            src = prog.source.display_path()
        except Exception:
            src = getattr(prog.source, "path", None)
    return {"format": FORMAT, "source": src, "buffers": bufs, "main": main}


def dumps(prog) -> str:
    return json.dumps(dump(prog), separators=(",", ":"))


# ----------------------------------------------------------------------------- load

def _fnum(v):
    if isinstance(v, str):
        return float(v)
    return v


class _Span:
    """A source location that only knows its text (what error messages print) and line."""

    def __init__(self, text, line=None, src=None):
        self.text = text
        self.line = line
        self.src = src                  # the text of the source line, when the program recorded it

    def location(self):
        return self.text


class _Source:
    def __init__(self, path):
        self.path = path

    def display_path(self):
        return self.path


def load(data) -> "ir.Program":
    from . import ir
    if isinstance(data, (str, bytes)):
        data = json.loads(data)
    if data.get("format") != FORMAT:
        raise ValueError(f"not an {FORMAT} program")
    bufs = {}
    for bd in data["buffers"]:
        init = bd["init"]
        if init is not None and bd["dtype"] == "f32":
            init = [_fnum(v) for v in init]
        b = ir.Buffer(bd["name"], bd["shape"], bd["dtype"], bd["kind"], init=init)
        b.id = bd["id"]                                 # the ids the front end gave them
        if bd.get("heap"):
            b.heap = True
        bufs[b.id] = b
    for bd in data["buffers"]:
        bufs[bd["id"]].storage = bufs[bd["storage"]]
    max_id = max([0] + list(bufs))
    vars_ = {}

    def var(vd):
        nonlocal max_id
        v = vars_.get(vd["id"])
        if v is None:
            v = vars_[vd["id"]] = ir.Var(vd["name"], vd["extent"])
            v.id = vd["id"]
            max_id = max(max_id, v.id)
        return v

    def aff(a, lets):
        const, terms = a
        out = {}
        for term, c in terms:
            kind = term[0]
            if kind == "v":
                t = vars_[term[1]]
            elif kind == "s":
                t = ir.ScalarRef(bufs[term[1]])
            else:
                _, ld, bound, where, rest = term
                t = ir.Gather(expr(ld, lets), bound, where, None if rest is None else aff(rest, lets))
            out[t] = out.get(t, 0) + c
        return ir.Affine(const, out)

    def expr(e, lets):
        tag = e[0]
        if tag == "c":
            return ir.Const(_fnum(e[2]), e[1])
        if tag == "ld":
            return ir.Load(bufs[e[1]], aff(e[2], lets))
        if tag == "ix":
            return ir.Index(aff(e[1], lets))
        if tag == "u":
            return ir.Unary(e[1], expr(e[3], lets), e[2])
        if tag == "b":
            return ir.Binary(e[1], expr(e[3], lets), expr(e[4], lets), e[2])
        if tag == "sel":
            return ir.Select(expr(e[1], lets), expr(e[2], lets), expr(e[3], lets))
        if tag == "acc":
            return ir.Acc(e[1])
        if tag == "let":
            return ir.LetRef(lets[e[1]])
        if tag == "rand":
            return ir.Rand(e[1], e[2])
        raise ValueError(f"unknown expression tag {tag}")

    def kernel(kd):
        nonlocal max_id
        domain = [var(v) for v in kd["domain"]]
        red = None
        if kd["red"] is not None:
            rv = [var(v) for v in kd["red"]["vars"]]
            red = ir.Reduction(rv, kd["red"]["op"], None)
        lets = {}
        if red is not None:
            red.body = expr(kd["red"]["body"], lets)
        stmts = []
        for i, sd in enumerate(kd["stmts"]):
            if sd["t"] == "let":
                let = ir.Let(sd["name"], expr(sd["value"], lets))
                lets[i] = let
                stmts.append(let)
            else:
                stmts.append(ir.Store(bufs[sd["buf"]], aff(sd["offset"], lets), expr(sd["value"], lets),
                                      bool(sd["acc"])))
        max_id = max(max_id, kd["id"])
        span = None if kd.get("line") is None else _Span(kd.get("loc"), kd["line"], kd.get("src"))
        k = ir.Kernel(domain, stmts, red, name=kd["name"], label=kd["label"], span=span, id=kd["id"])
        if kd.get("desc"):
            k.desc = kd["desc"]                         # what --check says about it, as recorded
        return k

    def bound(x):
        return x if isinstance(x, int) else bufs[x["buf"]]

    def rt_arg(a):
        if "buf" in a:
            return bufs[a["buf"]]
        if "bufs" in a:
            return [bufs[i] for i in a["bufs"]]
        if "bytes" in a:
            return bytes.fromhex(a["bytes"])
        if "list" in a:
            return [rt_arg(x) for x in a["list"]]
        return a["v"]

    def block(items):
        return ir.Block([stmt(s) for s in items])

    def stmt(s):
        t = s["t"]
        if t == "kernel":
            return ir.KernelStmt(kernel(s["kernel"]))
        if t == "for":
            return ir.For(bufs[s["counter"]], bound(s["start"]), bound(s["stop"]), s["step"], block(s["body"]))
        if t == "while":
            return ir.While(block(s["cond_block"]), bufs[s["cond"]], block(s["body"]))
        if t == "if":
            return ir.If(bufs[s["cond"]], block(s["then"]), block(s["else"]))
        if t == "break":
            return ir.Break()
        if t == "continue":
            return ir.Continue()
        if t == "print":
            items = [ir.PrintItem(it["kind"], it["text"], None if it["buf"] is None else bufs[it["buf"]],
                                  it["fmt"], it["choices"]) for it in s["items"]]
            return ir.Print(items, s["end"], s["err"])
        if t == "check":
            return ir.Check(aff(s["value"], {}), s["lo"], s["hi"], s["message"],
                            None if s["loc"] is None else _Span(s["loc"]))
        if t == "rt":
            return ir.RTCall(s["name"], {k: rt_arg(v) for k, v in s["args"].items()},
                             None if s["loc"] is None else _Span(s["loc"]))
        raise ValueError(f"unknown statement {t}")

    main = block(data["main"])
    prog = ir.Program(main, [bufs[i] for i in sorted(bufs)],
                      None if data.get("source") is None else _Source(data["source"]))
    ir.bump_ids(max_id)                 # ids made later in this process do not collide with these
    return prog


def load_file(path: str):
    with open(path) as f:
        return load(json.load(f))

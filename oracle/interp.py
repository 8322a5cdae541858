"""Oracle: a CPU restatement of Anvil's reference interpreter (anvil/interp.py), in NumPy.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker or the timed CPU baseline. The product (the HIP
backend and its libraries) never imports, links or runs it.

It follows the reference interpreter's semantics and its evaluation strategy, so that its float32
results are the reference's, bit for bit, on the same program:
  - every kernel is evaluated as NumPy broadcasting over a grid of its loop variables, domain
    first then reduction variables (interp.py:425-433, 435-466);
  - a kernel with more than CHUNK = 2^22 grid points is evaluated in chunks of its first domain
    variable, or, with no domain, in chunks of its first reduction variable whose partial results
    are combined in order (interp.py:383-406, 484-519);
  - reductions are NumPy's own (sum and prod in the body's dtype, max, min, argmax/argmin as the
    first extreme index; interp.py:468-482);
  - accumulating stores are np.add.at, plain stores a fancy-index assignment (interp.py:457-466);
  - gathers are bounds-checked and raise (interp.py:521-537);
  - the counter-based RNG, the Fisher-Yates shuffle, the print formats, the checkpoint format and
    the integer rules are restated from interp.py:40-115, 232-381, 561-632.

Pinned by tests/test_oracle.py against the reference interpreter's own output on the committed
fixtures (tests/golden/vectors), and against closed forms (RNG hash, shuffle by brute force,
matmul/softmax/layernorm/Adam in float64).
"""
from __future__ import annotations

import gzip
import re
import struct
import sys
import time

import numpy as np

CHUNK = 1 << 22
_M32 = np.uint64(0xFFFFFFFF)
GOLDEN_GAMMA = 0x9E3779B1
STREAM_MUL = 0x85EBCA77
SALT_MUL = 0xC2B2AE3D
MIX = 0x632BE5AB
SHUFFLE_SALT = 7
CKPT_MAGIC = b"EINW"
CKPT_HEAD = struct.Struct("<4sIQ")
NUMBER = re.compile(r"[-+]?(?:\d+(?:\.\d*)?|\.\d+)(?:[eE][-+]?\d+)?")


class RuntimeFault(Exception):
    """A run-time error of the program (the compiled code prints it and exits with status 1)."""


class ProgramExit(Exception):
    def __init__(self, code: int):
        super().__init__(f"exit status {code}")
        self.code = code


class StopRun(Exception):
    """Raised by a loop hook to end a bounded run early (the CPU baseline's sample)."""


class _Break(Exception):
    pass


class _Continue(Exception):
    pass


class _EndOfInput(Exception):
    pass


# ----------------------------------------------------------------------------- RNG (interp.py:55-71)

def lowbias32(x) -> np.ndarray:
    """Chris Wellons' lowbias32 integer hash (hash-prospector), in uint32 arithmetic."""
    x = np.asarray(x).astype(np.uint32)
    x = x ^ (x >> np.uint32(16))
    x = ((x.astype(np.uint64) * np.uint64(0x7FEB352D)) & _M32).astype(np.uint32)
    x = x ^ (x >> np.uint32(15))
    x = ((x.astype(np.uint64) * np.uint64(0x846CA68B)) & _M32).astype(np.uint32)
    x = x ^ (x >> np.uint32(16))
    return x


def rand_bits(idx, stream: int, salt: int, seed: int) -> np.ndarray:
    k = (stream * STREAM_MUL + salt * SALT_MUL + seed + MIX) & 0xFFFFFFFF
    h = (np.asarray(idx, dtype=np.uint64) * np.uint64(GOLDEN_GAMMA) + np.uint64(k)) & _M32
    return lowbias32(lowbias32(h))


def rand_uniform(bits, open_low: bool, dtype=np.float32) -> np.ndarray:
    hi = (np.asarray(bits) >> np.uint32(8)).astype(np.float64)
    if open_low:
        hi = hi + 1.0
    return (hi * (2.0 ** -24)).astype(dtype)


def shuffle_inplace(p: np.ndarray, n: int, stream: int, seed: int) -> None:
    """Fisher-Yates with the backends' shared draws (interp.py:309-320; anvil_host.h:269-276)."""
    if n <= 1:
        return
    draws = rand_bits(np.arange(n - 1), stream, SHUFFLE_SALT, seed)
    for k in range(n - 1):
        i = n - 1 - k
        j = int(draws[k]) % (i + 1)
        p[i], p[j] = p[j], p[i]


# ----------------------------------------------------------------------------- printing (interp.py:74-115)

def fmt_f32(v) -> str:
    v = float(v)
    a = abs(v)
    if v == 0 or v != v or 1e-4 <= a < 1e6:
        return "%.4f" % v
    return "%.4e" % v


def fmt_elem(v, is_int: bool) -> str:
    return "%d" % int(v) if is_int else fmt_f32(v)


def format_tensor(flat, shape, is_int: bool) -> str:
    rank = len(shape)
    if rank == 0:
        return fmt_elem(flat[0], is_int)
    numel = 1
    for d in shape:
        numel *= d
    if numel == 0:
        return "[]"
    summarize = numel > 1000
    strides = []
    s = 1
    for d in reversed(shape):
        strides.append(s)
        s *= d
    strides.reverse()

    def rec(off, d):
        n = shape[d]
        picks = [0, 1, 2, None, n - 3, n - 2, n - 1] if summarize and n > 6 else list(range(n))
        parts = []
        for i in picks:
            if i is None:
                parts.append("...")
            elif d == rank - 1:
                parts.append(fmt_elem(flat[off + i], is_int))
            else:
                parts.append(rec(off + i * strides[d], d + 1))
        return "[" + (", " if d == rank - 1 else ",\n" + " " * (d + 1)).join(parts) + "]"
    return rec(0, 0)


def ckpt_key(name: str, dtype: str, shape) -> int:
    """FNV-1a of `name-inside-model:dtype:shape` over the element count (ir.py:753-764)."""
    numel = 1
    for d in shape:
        numel *= d
    inside = name.split(".", 1)[1] if "." in name else ""
    h = 0x811C9DC5
    for byte in f"{inside}:{dtype}:{','.join(str(d) for d in shape)}".encode():
        h = ((h ^ byte) * 0x01000193) & 0xFFFFFFFF
    return ((h or 1) << 32) | numel


# ----------------------------------------------------------------------------- the machine

def _prod(xs) -> int:
    p = 1
    for x in xs:
        p *= x
    return p


def _strides(shape):
    out, s = [], 1
    for d in reversed(list(shape)):
        out.append(s)
        s *= d
    return out[::-1]


def check_description(k) -> str:
    """Where a kernel comes from, for --check (aarch64.py:82-89): the description the program
    recorded for it, else its label, source location and line, and its computation."""
    if getattr(k, "desc", None):
        return k.desc
    head = f"  made by `{k.label or 'a computation'}`"
    line = ""
    span = getattr(k, "span", None)
    if span is not None and span.location():
        head += f" at {span.location()}"
        if getattr(span, "src", None):
            line = "\n      " + span.src
    from anvil import ir
    return f"{head}:{line}\n  computing ({k.name}):  {ir.fmt_kernel(k)}"


class Machine:
    """Runs an `ir.Program` (this package's IR, or anything with the same shape) on the CPU.

    float_dtype: np.float32 for the reference semantics (np.float64 for gradient checks).
    sum_order: "numpy" (the reference's: NumPy's own float sums) for every parity check; "reversed"
    (each float sum over its reduction variables taken from the last element to the first) or
    "sequential" (one running float sum, in index order) measure how far the same algorithm moves
    when only the order of its additions changes (tests/golden/make_noise_floor.py).
    loop_hook(counter_name, value): called before each iteration of every `for` loop; it may raise
    StopRun to end the run (the CPU baseline times a bounded sample this way).
    """

    def __init__(self, prog, out=None, seed: int = 0, inp=None, float_dtype=np.float32, loop_hook=None,
                 check=None, sum_order="numpy"):
        if sum_order not in ("numpy", "reversed", "sequential"):
            raise ValueError(f"sum_order {sum_order!r}")
        self.prog = prog
        self.sum_order = sum_order
        self.check = check                # "nan" | "inf": stop at the first nan (or infinity) a kernel makes
        self.out = out if out is not None else sys.stdout
        self.inp = inp if inp is not None else sys.stdin
        self.fdt = float_dtype
        self.seed = seed & 0xFFFFFFFF
        self.stream = 0
        self.loop_hook = loop_hook
        self.t0 = time.perf_counter()
        self.kernels_run = 0
        self.mem = {}
        for b in prog.buffers:
            r = b.root
            if r.id in self.mem:
                continue
            a = np.zeros(max(r.numel, 1), dtype=np.int32 if r.dtype == "i32" else self.fdt)
            if r.init is not None:
                a[:len(r.init)] = np.asarray(r.init, dtype=a.dtype)
            self.mem[r.id] = a

    def arr(self, b) -> np.ndarray:
        return self.mem[b.root.id]

    def run(self):
        try:
            self.block(self.prog.main)
        except _EndOfInput:
            pass
        if hasattr(self.out, "flush"):
            self.out.flush()
        return self

    # ------------------------------------------------------------------ statements
    def block(self, blk):
        for st in blk.stmts:
            self.stmt(st)

    def stmt(self, st):
        kind = type(st).__name__
        if kind == "KernelStmt":
            self.kernel(st.kernel)
        elif kind == "For":
            self.for_loop(st)
        elif kind == "While":
            while True:
                self.block(st.cond_block)
                if self.arr(st.cond)[0] == 0:
                    break
                try:
                    self.block(st.body)
                except _Break:
                    break
                except _Continue:
                    continue
        elif kind == "If":
            self.block(st.then if self.arr(st.cond)[0] != 0 else st.orelse)
        elif kind == "Break":
            raise _Break()
        elif kind == "Continue":
            raise _Continue()
        elif kind == "Print":
            self.print_(st)
        elif kind == "Check":
            v = int(np.asarray(self.affine(st.value, {}, None)).reshape(-1)[0])
            if not st.lo <= v <= st.hi:
                loc = st.span.location() if st.span is not None else "?"
                raise RuntimeFault(f"{loc}: {st.message} (value {v})")
        elif kind == "RTCall":
            self.rtcall(st)
        else:
            raise NotImplementedError(kind)

    def scalar(self, x) -> int:
        return x if isinstance(x, int) else int(self.arr(x)[0])

    def for_loop(self, st):
        c = self.arr(st.counter)
        c[0] = self.scalar(st.start)
        stop = self.scalar(st.stop)
        while c[0] < stop:
            if self.loop_hook is not None:
                self.loop_hook(st.counter.name, int(c[0]))
            try:
                self.block(st.body)
            except _Break:
                break
            except _Continue:
                pass
            c[0] += st.step

    def print_(self, st):
        parts = []
        for it in st.items:
            if it.kind == "text":
                parts.append(it.text)
            elif it.kind == "scalar":
                v = self.arr(it.buf)[0]
                is_int = it.buf.dtype == "i32"
                if not it.fmt:
                    parts.append(fmt_elem(v, is_int))
                elif is_int or it.fmt.endswith("d"):
                    parts.append(it.fmt % int(v))
                else:
                    parts.append(it.fmt % float(v))
            elif it.kind == "chars":
                codes = self.arr(it.buf)[:it.buf.numel].astype(np.int64) & 0xFF
                parts.append(codes.astype(np.uint8).tobytes().decode("utf-8", errors="replace"))
            elif it.kind == "pick":
                k = int(self.arr(it.buf)[0])
                parts.append(it.choices[k] if 0 <= k < len(it.choices) else "?")
            else:
                b = it.buf
                parts.append(format_tensor(self.arr(b)[:b.numel], b.shape, b.dtype == "i32"))
        if st.err:
            if hasattr(self.out, "flush"):
                self.out.flush()
            sys.stderr.write("".join(parts) + st.end)
        else:
            self.out.write("".join(parts) + st.end)

    def rtcall(self, st):
        a, name = st.args, st.name
        if name == "seed":
            self.seed = a["value"] & 0xFFFFFFFF
            self.stream = 0
        elif name == "skip_rand":
            self.stream += 1
        elif name in ("iota", "iota_once"):
            b = a["buf"]
            self.arr(b)[:b.numel] = np.arange(b.numel, dtype=np.int32)
        elif name == "shuffle":
            b = a["buf"]
            stream = self.stream
            self.stream += 1
            shuffle_inplace(self.arr(b), b.numel, stream, self.seed)
        elif name == "exit":
            if hasattr(self.out, "flush"):
                self.out.flush()
            raise ProgramExit(a["value"])
        elif name == "clock":
            self.arr(a["buf"])[0] = time.perf_counter() - self.t0
        elif name == "sleep":
            time.sleep(max(0.0, float(self.arr(a["buf"])[0])))
        elif name == "nonzero":
            src, b = a["src"], a["buf"]
            found = np.flatnonzero(self.arr(src)[:src.numel])[:b.numel]
            o = self.arr(b)
            o[:b.numel] = -1
            o[:len(found)] = found
        elif name == "load_idx":
            b = a["buf"]
            with (gzip.open if a["gz"] else open)(a["path"], "rb") as f:
                f.read(a["header"])
                raw = np.frombuffer(f.read(b.numel), dtype=np.uint8)
            if raw.size != b.numel:
                raise RuntimeFault(f"{a['path']}: file is truncated")
            self.arr(b)[:b.numel] = raw.astype(self.arr(b).dtype)
        elif name == "load_bytes":
            b = a["buf"]
            try:
                raw = open(a["path"], "rb").read()
            except OSError:
                raise RuntimeFault(f"cannot open data file {a['path']}")
            if len(raw) != b.numel:
                raise RuntimeFault(f"data file {a['path']} does not have the shape this program was compiled for")
            self.arr(b)[:b.numel] = np.frombuffer(raw, dtype=np.uint8)
        elif name == "load_csv":
            b = a["buf"]
            try:
                text = open(a["path"], encoding="utf-8", errors="replace").read()
            except OSError:
                raise RuntimeFault(f"cannot open data file {a['path']}")
            pos = 0
            for _ in range(a["skip"]):
                pos = text.index("\n", pos) + 1
            vals = NUMBER.findall(text, pos)
            if len(vals) < b.numel:
                raise RuntimeFault(f"data file {a['path']} does not have the shape this program was compiled for")
            self.arr(b)[:b.numel] = np.array(vals[:b.numel], dtype=np.float32)
        elif name == "input":
            if hasattr(self.out, "flush"):
                self.out.flush()
            line = self.inp.readline()
            if not line:
                self.out.write("\n")
                raise _EndOfInput()
            m = NUMBER.search(line)
            self.arr(a["buf"])[0] = float(m.group(0)) if m else np.nan
        elif name == "show":
            g = a["glyphs"]
            data = self.arr(a["buf"])
            rows = []
            for r in range(a["rows"]):
                row = data[r * a["cols"]:(r + 1) * a["cols"]]
                rows.append("".join(g[v] if 0 <= v < len(g) else "?" for v in row))
            self.out.write("\n".join(rows) + "\n")
        elif name == "save":
            bufs = a["bufs"]
            try:
                with open(a["path"], "wb") as f:
                    f.write(CKPT_HEAD.pack(CKPT_MAGIC, 2, len(bufs)))
                    f.write(struct.pack(f"<{len(bufs)}Q", *[ckpt_key(b.root.name, b.root.dtype, b.root.shape)
                                                          for b in bufs]))
                    for b in bufs:
                        f.write(self.arr(b)[:b.numel].astype(np.int32 if b.dtype == "i32" else np.float32).tobytes())
            except OSError:
                sys.stderr.write(f"anvil: cannot write {a['path']}\n")
        elif name == "load":
            bufs = a["bufs"]
            ok = 0.0
            try:
                raw = open(a["path"], "rb").read()
                sizes = [b.numel for b in bufs]
                head = CKPT_HEAD.size + 8 * len(bufs)
                magic, version, n = CKPT_HEAD.unpack_from(raw) if len(raw) >= CKPT_HEAD.size else (None, 0, 0)
                want = ([ckpt_key(b.root.name, b.root.dtype, b.root.shape) for b in bufs] if version == 2
                        else sizes)
                if (len(raw) == head + 4 * sum(sizes) and magic == CKPT_MAGIC and version in (1, 2)
                        and n == len(bufs)
                        and list(struct.unpack_from(f"<{len(bufs)}Q", raw, CKPT_HEAD.size)) == want):
                    pos = head
                    for b in bufs:
                        self.arr(b)[:b.numel] = np.frombuffer(raw, np.int32 if b.dtype == "i32" else np.float32,
                                                              b.numel, pos)
                        pos += 4 * b.numel
                    ok = 1.0
            except OSError:
                pass
            self.arr(a["buf"])[0] = ok
        elif name == "save_npy":
            b = a["buf"]
            try:
                with open(a["path"], "wb") as f:
                    f.write(a["header"])
                    f.write(self.arr(b)[:b.numel].astype(np.int32 if b.dtype == "i32" else np.float32).tobytes())
            except OSError:
                sys.stderr.write(f"anvil: cannot write {a['path']}\n")
        elif name == "load_npy":
            b = a["buf"]
            try:
                if a["kind"] & 16:
                    dt = {(0, 4): "<f4", (1, 8): "<f8", (2, 2): "<f2", (3, 4): "<i4", (4, 8): "<i8", (5, 1): "u1",
                          (6, 1): "i1", (7, 2): "<u2", (8, 2): "<i2"}[(a["kind"] & 15, a["size"])]
                    data = np.fromfile(a["path"], dtype=dt, count=b.numel, offset=a["offset"])
                else:
                    data = np.load(a["path"], allow_pickle=False)
            except (OSError, ValueError):
                raise RuntimeFault(f"cannot open data file {a['path']}")
            if data.size != b.numel:
                raise RuntimeFault(f"data file {a['path']} does not have the shape this program was compiled for")
            self.arr(b)[:b.numel] = data.reshape(-1).astype(self.arr(b).dtype)
        else:
            raise NotImplementedError(name)

    # ------------------------------------------------------------------ kernels
    def kernel(self, k):
        self.kernels_run += 1
        stream = None
        if k.uses_rand():
            stream = self.stream
            self.stream += 1
        dom = list(k.domain)
        red = list(k.red.vars) if k.red is not None else []
        total = _prod(v.extent for v in dom + red)
        if total == 0:
            return
        if total <= CHUNK or (not dom and not red):
            self.evaluate(k, dom, red, None, stream)
        elif dom:
            v0 = dom[0]
            per = max(1, CHUNK // max(1, total // v0.extent))
            for lo in range(0, v0.extent, per):
                self.evaluate(k, dom, red, (v0, lo, min(v0.extent, lo + per)), stream)
        else:
            self.evaluate(k, dom, red, None, stream, chunk_reduction=True)
        self.check_kernel(k)

    def check_kernel(self, k):
        """--check (interp.py:408-423): the first nan (or infinity) in a tensor k wrote ends the
        program, with a message naming the tensor, the element and where the kernel comes from."""
        if not self.check:
            return
        written = []
        for st in k.stores:
            if st.buf.root.dtype != "i32" and st.buf.root not in written:
                written.append(st.buf.root)
        for b in written:
            a = self.arr(b)[:b.numel]
            bad = np.isnan(a) if self.check == "nan" else ~np.isfinite(a)
            if bad.any():
                i = int(np.flatnonzero(bad)[0])
                where = f" at {[int(v) for v in np.unravel_index(i, b.shape)]}" if b.shape else ""
                raise RuntimeFault(f"--check: {a[i]} in `{b.name}`{where}\n{check_description(k)}")

    @staticmethod
    def grid(vars_, ranges):
        env = {}
        n = len(vars_)
        for axis, v in enumerate(vars_):
            lo, hi = ranges.get(v, (0, v.extent))
            shape = [1] * n
            shape[axis] = hi - lo
            env[v] = np.arange(lo, hi, dtype=np.int64).reshape(shape)
        return env

    def evaluate(self, k, dom, red, chunk, stream, chunk_reduction=False):
        ranges = {}
        if chunk is not None:
            ranges[chunk[0]] = (chunk[1], chunk[2])
        env = self.grid(dom + red, ranges)
        dshape = tuple(ranges.get(v, (0, v.extent))[1] - ranges.get(v, (0, v.extent))[0] for v in dom)
        full = dshape + tuple(v.extent for v in red)
        ctx = {"env": env, "ndim": len(dom) + len(red), "stream": stream, "D": dom, "shape": full, "lets": {}}
        acc = None
        if k.red is not None:
            if chunk_reduction and red:
                acc = self.reduce_in_chunks(k, dom, red, ctx)
            else:
                body = np.broadcast_to(self.eval(k.red.body, ctx), full)
                acc = self.reduce(k.red.op, body, len(dom))
        denv = {v: env[v].reshape(env[v].shape[:len(dom)]) for v in dom}
        sctx = {"env": denv, "ndim": len(dom), "stream": stream, "D": dom, "shape": dshape, "lets": {}, "acc": acc}
        for st in k.stmts:
            if type(st).__name__ == "Let":
                sctx["lets"][id(st)] = self.eval(st.value, sctx)
                continue
            val = np.broadcast_to(self.eval(st.value, sctx), dshape)
            off = np.broadcast_to(self.affine(st.offset, denv, sctx), dshape)
            a = self.arr(st.buf)
            val = val.astype(a.dtype, copy=False)
            if st.accumulate:
                np.add.at(a, off.reshape(-1), val.reshape(-1))
            else:
                a[off.reshape(-1)] = val.reshape(-1)

    def reduce(self, op, body, nd):
        axes = tuple(range(nd, body.ndim))
        if op == "sum":
            if self.sum_order == "numpy" or body.dtype.kind != "f" or not axes:
                return body.sum(axis=axes, dtype=body.dtype)
            flat = body.reshape(body.shape[:nd] + (-1,))
            if self.sum_order == "reversed":
                return flat[..., ::-1].sum(axis=-1, dtype=body.dtype)
            acc = np.zeros(flat.shape[:-1], body.dtype)
            for i in range(flat.shape[-1]):
                acc += flat[..., i]
            return acc
        if op == "prod":
            return body.prod(axis=axes, dtype=body.dtype)
        if op == "max":
            return body.max(axis=axes)
        if op == "min":
            return body.min(axis=axes)
        if op in ("argmax", "argmin"):
            flat = body.reshape(body.shape[:nd] + (-1,))
            return (flat.argmax(axis=-1) if op == "argmax" else flat.argmin(axis=-1)).astype(np.int32)
        raise NotImplementedError(op)

    def reduce_in_chunks(self, k, dom, red, ctx):
        r0 = red[0]
        per = max(1, CHUNK // max(1, _prod(v.extent for v in red) // r0.extent))
        op = k.red.op
        acc = best = None
        for lo in range(0, r0.extent, per):
            hi = min(r0.extent, lo + per)
            env = self.grid(dom + red, {r0: (lo, hi)})
            shape = tuple(v.extent for v in dom) + tuple((hi - lo) if v is r0 else v.extent for v in red)
            body = np.broadcast_to(self.eval(k.red.body, dict(ctx, env=env, shape=shape)), shape)
            if op in ("argmax", "argmin"):
                part = self.reduce("max" if op == "argmax" else "min", body, len(dom))
                where = self.reduce(op, body, len(dom)) + lo
                if acc is None:
                    acc, best = part, where
                else:
                    better = part > acc if op == "argmax" else part < acc
                    acc = np.where(better, part, acc)
                    best = np.where(better, where, best)
                continue
            part = self.reduce(op, body, len(dom))
            if acc is None:
                acc = part
            elif op == "sum":
                acc = acc + part
            elif op == "prod":
                acc = acc * part
            elif op == "max":
                acc = np.maximum(acc, part)
            else:
                acc = np.minimum(acc, part)
        return best.astype(np.int32) if op in ("argmax", "argmin") else acc

    # ------------------------------------------------------------------ expressions
    def affine(self, a, env, ctx):
        v = np.int64(a.const)
        for t, c in a.terms.items():
            kind = type(t).__name__
            if kind == "Var":
                v = v + c * env[t]
            elif kind == "ScalarRef":
                v = v + c * np.int64(self.arr(t.buf)[0])
            else:
                g = self.eval(t.load, ctx if ctx is not None else {"env": env, "lets": {}}).astype(np.int64)
                lo, hi = t.check_range()
                bad = (g < lo) | (g >= hi)
                if np.any(bad):
                    value = int(np.asarray(g)[bad].reshape(-1)[0])
                    raise RuntimeFault(f"index {value} out of bounds for a dimension of size {t.bound} ({t.where})")
                v = v + c * g
        return v

    def eval(self, e, ctx):
        kind = type(e).__name__
        fdt = self.fdt
        if kind == "Const":
            return np.asarray(e.value, dtype=np.int32 if e.dtype == "i32" else fdt)
        if kind == "Load":
            return self.arr(e.buf)[self.affine(e.offset, ctx["env"], ctx)]
        if kind == "Index":
            return np.asarray(self.affine(e.affine, ctx["env"], ctx), dtype=np.int32)
        if kind == "Acc":
            return ctx["acc"]
        if kind == "LetRef":
            return ctx["lets"][id(e.let)]
        if kind == "Rand":
            dom = ctx["D"]
            idx = np.int64(0)
            for v, s in zip(dom, _strides([v.extent for v in dom])):
                ev = ctx["env"][v]
                idx = idx + ev.reshape(ev.shape[:len(dom)] + (1,) * (ctx["ndim"] - len(dom))) * s
            return rand_uniform(rand_bits(idx, ctx["stream"], e.salt, self.seed), e.open_low, fdt)
        if kind == "Unary":
            return self.unary(e.op, self.eval(e.a, ctx))
        if kind == "Binary":
            return self.binary(e.op, self.eval(e.a, ctx), self.eval(e.b, ctx), e.dtype == "i32")
        if kind == "Select":
            c = self.eval(e.c, ctx)
            x = self.eval(e.a, ctx)
            y = self.eval(e.b, ctx)
            return np.where(c != 0, x, y).astype(np.int32 if e.dtype == "i32" else fdt)
        raise NotImplementedError(kind)

    def unary(self, op, a):
        f = self.fdt
        with np.errstate(all="ignore"):
            if op == "neg":
                return -a
            if op == "abs":
                return np.abs(a)
            if op == "exp":
                return np.exp(a.astype(f))
            if op == "log":
                return np.log(a.astype(f))
            if op == "sqrt":
                return np.sqrt(a.astype(f))
            if op == "rsqrt":
                return (1 / np.sqrt(a.astype(f))).astype(f)
            if op == "recip":
                return (1 / a.astype(f)).astype(f)
            if op == "tanh":
                return np.tanh(a.astype(f))
            if op == "sigmoid":
                return (1 / (1 + np.exp(-a.astype(f)))).astype(f)
            if op == "sin":
                return np.sin(a.astype(f))
            if op == "cos":
                return np.cos(a.astype(f))
            if op == "floor":
                return np.floor(a)
            if op == "ceil":
                return np.ceil(a)
            if op == "round":
                return np.round(a)
            if op == "sign":
                return np.sign(a).astype(a.dtype)
            if op == "not":
                return (a == 0).astype(f)
            if op == "f32":
                return a.astype(f)
            if op == "i32":
                return a if a.dtype == np.int32 else np.trunc(a).astype(np.int32)
            if op == "detach":
                return a
        raise NotImplementedError(op)

    def binary(self, op, a, b, is_int):
        f = self.fdt
        with np.errstate(all="ignore"):
            if op == "add":
                r = a + b
            elif op == "sub":
                r = a - b
            elif op == "mul":
                r = a * b
            elif op == "div":
                r = a.astype(f) / b.astype(f)
            elif op == "idiv":
                r = np.floor_divide(a, np.where(b == 0, 1, b)) if is_int else np.floor(a / b)
            elif op == "mod":
                r = np.mod(a, np.where(b == 0, 1, b)) if is_int else np.mod(a, b)
            elif op == "max":
                r = np.maximum(a, b)
            elif op == "min":
                r = np.minimum(a, b)
            elif op == "pow":
                r = np.power(a.astype(f), b.astype(f))
            elif op == "lt":
                r = a < b
            elif op == "le":
                r = a <= b
            elif op == "gt":
                r = a > b
            elif op == "ge":
                r = a >= b
            elif op == "eq":
                r = a == b
            elif op == "ne":
                r = a != b
            elif op == "and":
                r = (a != 0) & (b != 0)
            elif op == "or":
                r = (a != 0) | (b != 0)
            else:
                raise NotImplementedError(op)
        return np.asarray(r).astype(np.int32 if is_int else f)


def run(prog, **kw) -> Machine:
    return Machine(prog, **kw).run()

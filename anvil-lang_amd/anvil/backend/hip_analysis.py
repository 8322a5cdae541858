"""Program analyses the HIP generator relies on.

- read/write sets of statements (what a kernel, a loop or a run-time call touches);
- `parallel_safe`: may every output element of a kernel run in its own thread, in any order? The
  same question the reference's CUDA emitter asks (cuda.py:380-395, 618-633): plain stores must be
  injective over the domain and free of gathers, and a kernel may read a buffer it writes only at the
  element it writes;
- `host_scalars`: the 0-d buffers that only the host computes (loop counters, and results of scalar
  kernels that read only such values and constants), found by iterating to a fixed point, as the
  reference's Metal backend does (metal.py:365-432). Kernels get them by value, so a training loop
  needs no device round trip for its counters, its `if step >= N: break` or Adam's step count;
- `plan_arena`: byte offsets of every device buffer in one allocation; temporaries whose lifetimes
  do not overlap share bytes (the reference's arena.py:1-144 lifetime rule: a lifetime that touches
  a loop covers the whole loop, and only buffers whose first use writes all of them take part);
- `rematerialize`: temporaries that are a cheap elementwise function of another buffer (GELU's
  tanh and 0.044715·x², which the reference's autodiff saves for the backward) recomputed where
  they are read instead of written to and read back from memory.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from .. import ir
from ..ir import Buffer, Gather, Index, KernelStmt, Load, ScalarRef, Var

# Run-time calls: which arguments they read and write (the reference's optimize.py:20-32 tables).
RT_READS = {"shuffle": ("buf",), "show": ("buf",), "sleep": ("buf",), "nonzero": ("src",), "save": ("bufs",),
            "save_npy": ("buf",)}
RT_WRITES = {"load_idx": ("buf",), "load_csv": ("buf",), "load_bytes": ("buf",), "load_npy": ("buf",),
             "iota": ("buf",), "iota_once": ("buf",), "shuffle": ("buf",), "clock": ("buf",), "nonzero": ("buf",),
             "input": ("buf",), "load": ("bufs", "buf")}
RT_FULL_WRITES = ("nonzero", "input", "clock", "iota", "iota_once", "load_idx", "load_csv", "load_bytes",
                  "load_npy")
ARENA_ALIGN = 256
_UNSHARED = set(filter(None, __import__("os").environ.get("ANVIL_HIP_UNSHARED", "").split(",")))
SHARED_KINDS = ("temp", "grad")


# ----------------------------------------------------------------------------- ids of added objects

class IdSource:
    """Ids for the loop variables and scratch buffers the backend adds to a program. Ids name
    variables and buffers in the generated source, so they are counted up from the program's own
    largest id: one program always gives one source (and one library name), whatever else the
    process built, and nothing outside this generation is touched (the IR module's own counter is
    left alone)."""

    def __init__(self, prog: ir.Program):
        self.next = program_max_id(prog) + 1

    def take(self) -> int:
        self.next += 1
        return self.next - 1


def program_max_id(prog: ir.Program) -> int:
    """The largest id of any buffer, kernel or loop variable of the program."""
    top = max([0] + [b.id for b in prog.buffers] + [b.root.id for b in prog.buffers])
    for k in ir.all_kernels(prog):
        top = max(top, k.id, *[v.id for v in k.domain], *([v.id for v in k.red.vars] if k.red else []))
    return top


def _numbered(make, ident: int):
    """make() (an IR constructor call) given the id `ident`, without drawing from the IR module's
    id counter: the constructors take their id from the module's fresh_id, which is replaced by a
    stand-in while they run (generation is single-threaded). Objects the front end numbers later
    in the same process then get the ids they would have got without this generation."""
    saved = ir.fresh_id
    ir.fresh_id = lambda: ident
    try:
        obj = make()
    finally:
        ir.fresh_id = saved
    obj.id = ident
    return obj


def new_var(ident: int, name: str, extent: int) -> Var:
    """A loop variable with a chosen id (built with the IR's own constructor)."""
    return _numbered(lambda: Var(name, extent), ident)


def new_buffer(ident: int, name: str, shape, dtype: str, kind: str) -> Buffer:
    """A buffer of the backend's own (scratch, host-scalar copies) with a fixed id."""
    return _numbered(lambda: Buffer(name, shape, dtype, kind), ident)


def rt_args(st, table) -> list:
    out = []
    for key in table.get(st.name, ()):
        v = st.args.get(key)
        if v is None:
            continue
        out.extend(v if isinstance(v, list) else [v])
    return [b for b in out if isinstance(b, Buffer)]


# ----------------------------------------------------------------------------- loads and offsets

def offset_loads(a: ir.Affine, out: list) -> None:
    for g in a.gathers():
        out.append(g.load)
        offset_loads(g.load.offset, out)


def kernel_loads(k: ir.Kernel) -> list:
    """Every load of k: in its expressions, in their offsets' gathers, and in its stores' offsets."""
    out = []
    for e in k.exprs():
        for x in ir.iter_expr(e):
            if isinstance(x, Load):
                out.append(x)
            elif isinstance(x, Index):
                offset_loads(x.affine, out)
    for st in k.stores:
        offset_loads(st.offset, out)
    return out


def affine_scalars(a: ir.Affine, out: set) -> None:
    for t in a.terms:
        if isinstance(t, ScalarRef):
            out.add(t.buf.root)
        elif isinstance(t, Gather):
            affine_scalars(t.load.offset, out)
            if t.rest is not None:
                affine_scalars(t.rest, out)


def kernel_reads(k: ir.Kernel) -> set:
    out = {ld.buf.root for ld in kernel_loads(k)}
    for e in k.exprs():
        for x in ir.iter_expr(e):
            if isinstance(x, Load):
                affine_scalars(x.offset, out)
            elif isinstance(x, Index):
                affine_scalars(x.affine, out)
    for st in k.stores:
        affine_scalars(st.offset, out)
        if st.accumulate:
            out.add(st.buf.root)
    return out


def kernel_writes(k: ir.Kernel) -> set:
    return {st.buf.root for st in k.stores}


def stmt_reads(st) -> set:
    if isinstance(st, KernelStmt):
        return kernel_reads(st.kernel)
    out: set = set()
    if isinstance(st, ir.For):
        for b in (st.start, st.stop):
            if isinstance(b, Buffer):
                out.add(b.root)
        out |= block_reads(st.body)
    elif isinstance(st, ir.While):
        out |= block_reads(st.cond_block) | block_reads(st.body)
        out.add(st.cond.root)
    elif isinstance(st, ir.If):
        out.add(st.cond.root)
        out |= block_reads(st.then) | block_reads(st.orelse)
    elif isinstance(st, ir.Print):
        out |= {it.buf.root for it in st.items if it.buf is not None}
    elif isinstance(st, ir.Check):
        affine_scalars(st.value, out)
    elif isinstance(st, ir.RTCall):
        out |= {b.root for b in rt_args(st, RT_READS)}
    return out


def stmt_writes(st) -> set:
    if isinstance(st, KernelStmt):
        return kernel_writes(st.kernel)
    out: set = set()
    if isinstance(st, ir.For):
        out.add(st.counter.root)
        out |= block_writes(st.body)
    elif isinstance(st, ir.While):
        out |= block_writes(st.cond_block) | block_writes(st.body)
    elif isinstance(st, ir.If):
        out |= block_writes(st.then) | block_writes(st.orelse)
    elif isinstance(st, ir.RTCall):
        out |= {b.root for b in rt_args(st, RT_WRITES)}
    return out


def block_reads(b: ir.Block) -> set:
    out: set = set()
    for st in b.stmts:
        out |= stmt_reads(st)
    return out


def block_writes(b: ir.Block) -> set:
    out: set = set()
    for st in b.stmts:
        out |= stmt_writes(st)
    return out


# ----------------------------------------------------------------------------- parallel safety

def injective_over(off: ir.Affine, vars_) -> bool:
    """Distinct values of vars_ give distinct offsets: sorted by |coefficient|, each var's step must
    exceed everything the smaller ones reach (a sufficient, exact-for-row-major test)."""
    steps = []
    for v in vars_:
        if v.extent <= 1:
            continue
        c = abs(off.coef(v))
        if c == 0:
            return False
        steps.append((c, v.extent))
    reach = 0
    for c, n in sorted(steps):
        if c <= reach:
            return False
        reach += c * (n - 1)
    return True


def sole_writer(k: ir.Kernel, st) -> bool:
    """Does each element of k's domain own the element that store `st` adds to? Its offset is
    injective over the domain and has no gathers, and every other store of k to that buffer uses
    the same offset. Then `+=` needs no atomic: no other lane of the launch touches the element."""
    if st.offset.gathers() or not injective_over(st.offset, k.domain):
        return False
    return all(o.offset == st.offset for o in k.stores if o.buf.root is st.buf.root)


def parallel_safe(k: ir.Kernel) -> bool:
    """May every point of k's domain run in a lane of its own, in any order (the question of the
    reference's cuda.py:380-395)? Not when two points can write one element with a plain store
    (through an index array with repeated values, or an offset that is not one-to-one over the
    domain: then the last write must win, in domain order), and not when a point reads an element
    of a buffer the kernel writes other than the one it stores itself (or adds into it)."""
    for st in k.stores:
        if not st.accumulate and (st.offset.gathers() or not injective_over(st.offset, k.domain)):
            return False
    by_buffer: dict = {}
    for st in k.stores:
        by_buffer.setdefault(st.buf.root.id, []).append(st)
    return all(not st.accumulate and st.offset == ld.offset
               for ld in kernel_loads(k) for st in by_buffer.get(ld.buf.root.id, ()))


# ----------------------------------------------------------------------------- host scalars

def is_scalar_kernel(k: ir.Kernel) -> bool:
    return (not k.domain and k.red is None and not k.uses_rand()
            and all(not st.buf.shape and not st.accumulate for st in k.stores))


def host_scalars(prog: ir.Program) -> set:
    """Ids of the 0-d buffers the host computes and keeps itself (the decision the reference's Metal
    backend makes, metal.py:365-432, restated): a loop counter that only its loop writes, and a 0-d
    result all of whose writers are scalar kernels (no domain, no reduction, no random draws) that
    read only host buffers and constants, and write only host buffers. A kernel may read a buffer it
    writes (Adam's t = t + 1). Derivation runs upward from the counters (a result joins once one of
    its writers can be computed from host values) and is checked downward (a buffer with a writer
    that cannot run on the host is refused for good), until neither changes the set."""
    buffers = {b.root.id: b.root for b in prog.buffers}
    written_by: dict[int, list] = {}          # 0-d buffer -> "loop", "call" or the kernels storing it
    loop_counters = set()
    for blk in ir.walk_blocks(prog.main):
        for st in blk.stmts:
            if isinstance(st, ir.For):
                loop_counters.add(st.counter.root.id)
                written_by.setdefault(st.counter.root.id, []).append("loop")
            elif isinstance(st, KernelStmt):
                for store in st.kernel.stores:
                    written_by.setdefault(store.buf.root.id, []).append(st.kernel)
            elif isinstance(st, ir.RTCall):
                for b in rt_args(st, RT_WRITES):
                    written_by.setdefault(b.root.id, []).append("call")

    def scalar_candidate(bid) -> bool:
        b = buffers.get(bid)
        return b is not None and not b.shape and b.kind not in ir.EXTERN_KINDS

    scalar_kernels = [k for k in ir.all_kernels(prog) if is_scalar_kernel(k)]
    inputs = {id(k): {b.id for b in kernel_reads(k) if b.kind != "const"} for k in scalar_kernels}
    results = {id(k): {st.buf.root.id for st in k.stores} for k in scalar_kernels}

    def only_scalar_writers(bid) -> bool:
        return all(isinstance(w, ir.Kernel) and is_scalar_kernel(w) for w in written_by.get(bid, []))

    def runs_on_host(k, on_host) -> bool:
        return isinstance(k, ir.Kernel) and is_scalar_kernel(k) and inputs[id(k)] <= on_host \
            and results[id(k)] <= on_host

    on_host = {c for c in loop_counters
               if scalar_candidate(c) and all(w == "loop" for w in written_by.get(c, []))}
    refused: set = set()
    while True:
        state = (len(on_host), len(refused))
        for k in scalar_kernels:                   # upward: computable from host values
            if inputs[id(k)] - on_host - (results[id(k)] - refused):
                continue
            on_host |= {r for r in results[id(k)] - refused
                        if scalar_candidate(r) and only_scalar_writers(r)}
        for bid in sorted(on_host - loop_counters):  # downward: every writer must run on the host
            if not all(runs_on_host(w, on_host) for w in written_by.get(bid, [])):
                on_host.discard(bid)
                refused.add(bid)
        if (len(on_host), len(refused)) == state:
            return on_host


def is_host_kernel(k: ir.Kernel, hosts: set) -> bool:
    if not is_scalar_kernel(k) or not k.stores:
        return False
    if any(st.buf.root.id not in hosts for st in k.stores):
        return False
    return all(b.id in hosts or b.kind == "const" for b in kernel_reads(k))


# ----------------------------------------------------------------------------- reordering

def commutes(a: ir.Kernel, b: ir.Kernel) -> bool:
    """May kernels a and b (a first) run in the other order? No buffer (or scalar) that one writes
    is read or written by the other, and they do not both draw random numbers (each launch that
    does takes the next stream number)."""
    ra, wa = {x.id for x in kernel_reads(a)}, {x.id for x in kernel_writes(a)}
    rb, wb = {x.id for x in kernel_reads(b)}, {x.id for x in kernel_writes(b)}
    if wa & (rb | wb) or ra & wb:
        return False
    return not (a.uses_rand() and b.uses_rand())


def sink_scalar_kernels(prog: ir.Program) -> ir.Program:
    """The program with each kernel that produces one value (a loss, an accuracy: an empty domain)
    moved later in its straight run of kernels, past every kernel it commutes with. A per-row
    chain (logits, log-softmax, their gradient) then stays unbroken, and the moved kernel can share
    a later launch. The caller's program is not changed (blocks are copied)."""
    import dataclasses

    def block(blk: ir.Block) -> ir.Block:
        out = [stmt(st) for st in blk.stmts]
        for idx in range(len(out) - 1, -1, -1):
            st = out[idx]
            if not (isinstance(st, KernelStmt) and not st.kernel.domain and st.kernel.red is not None):
                continue
            j = idx
            while j + 1 < len(out) and isinstance(out[j + 1], KernelStmt) and commutes(st.kernel, out[j + 1].kernel):
                j += 1
            if j > idx:
                out.insert(j, out.pop(idx))
        return dataclasses.replace(blk, stmts=out)

    def stmt(st):
        if isinstance(st, ir.For):
            return dataclasses.replace(st, body=block(st.body))
        if isinstance(st, ir.While):
            return dataclasses.replace(st, cond_block=block(st.cond_block), body=block(st.body))
        if isinstance(st, ir.If):
            return dataclasses.replace(st, then=block(st.then), orelse=block(st.orelse))
        return st
    return dataclasses.replace(prog, main=block(prog.main))


# ----------------------------------------------------------------------------- rematerialization

REMAT_MAX_COST = 24     # recomputed per element read: a transcendental counts 8, any other op 1
TRANSCENDENTAL = {"exp", "log", "sqrt", "tanh", "sigmoid", "sin", "cos", "rsqrt", "recip"}


def _inline_lets(e):
    """e with every Let reference replaced by the Let's (inlined) value."""
    return ir.map_expr(e, lambda x: _inline_lets(x.let.value) if isinstance(x, ir.LetRef) else x)


def _remat_cost(e) -> int:
    n = 0
    for x in ir.iter_expr(e):
        if isinstance(x, ir.Unary):
            n += 8 if x.op in TRANSCENDENTAL else (0 if x.op == "detach" else 1)
        elif isinstance(x, (ir.Binary, ir.Select)):
            n += 1
    return n


def _writers(prog: ir.Program) -> dict:
    """buffer root id -> the statements (kernels, run-time calls, loop counters) that write it."""
    out: dict[int, list] = {}

    def walk(blk):
        for st in blk.stmts:
            if isinstance(st, ir.For):
                out.setdefault(st.counter.root.id, []).append(st)
                walk(st.body)
            elif isinstance(st, ir.While):
                walk(st.cond_block)
                walk(st.body)
            elif isinstance(st, ir.If):
                walk(st.then)
                walk(st.orelse)
            else:
                for b in stmt_writes(st):
                    out.setdefault(b.id, []).append(st)
    walk(prog.main)
    return out


def _blocks(blk):
    yield blk
    for st in blk.stmts:
        if isinstance(st, ir.For):
            yield from _blocks(st.body)
        elif isinstance(st, ir.While):
            yield from _blocks(st.cond_block)
            yield from _blocks(st.body)
        elif isinstance(st, ir.If):
            yield from _blocks(st.then)
            yield from _blocks(st.orelse)


def _remat_candidate(prog: ir.Program, max_cost: int):
    """The first (block, index of the writing kernel, its store, indices of the reading kernels)
    whose temporary may be recomputed where it is read, or None.

    Temporary T qualifies when: one kernel M writes it, with one plain store that covers every
    element, whose value (Let references inlined) is built from constants and loads at the store's
    own offset of buffers Z other than T (no loop index, random draw or reduction result), within
    max_cost; each Z is written by one kernel that comes before M in the same block (so Z holds,
    wherever T is read, the values M computed T from); and every statement that reads T is a kernel
    after M in that block that reads it in values only (not as a gather index). T's element e is
    then g(Z[e]), so a load T[o] can be replaced by g with each Z loaded at o. A T that some kernel
    reads inside its reduction (an operand of a product) stays in memory."""
    readers = all_readers(prog)
    writers = _writers(prog)
    for blk in _blocks(prog.main):
        for i, st in enumerate(blk.stmts):
            if not isinstance(st, KernelStmt):
                continue
            m = st.kernel
            for s in m.stores:
                t = s.buf
                if t.root is not t or t.kind != "temp" or len(writers.get(t.id, ())) != 1:
                    continue
                if sum(1 for x in m.stores if x.buf.root is t) != 1 or not _store_covers(m, s, t):
                    continue
                g = _inline_lets(s.value)
                if _remat_cost(g) > max_cost:
                    continue
                okey, ok, zs = s.offset.key(), True, set()
                for x in ir.iter_expr(g):
                    if isinstance(x, (ir.Index, ir.Rand, ir.Acc, ir.LetRef)):
                        ok = False
                    elif isinstance(x, Load):
                        z = x.buf.root
                        if x.offset.key() != okey or z is t or z in kernel_writes(m):
                            ok = False
                        else:
                            zs.add(z)
                    if not ok:
                        break
                if not ok or not zs:
                    continue
                for z in zs:
                    w = writers.get(z.id, ())
                    if len(w) != 1 or not any(w[0] is x for x in blk.stmts[:i]):
                        ok = False
                if not ok:
                    continue
                users = [j for j in range(i + 1, len(blk.stmts)) if isinstance(blk.stmts[j], KernelStmt)
                         and t in kernel_reads(blk.stmts[j].kernel)]
                if not users or readers.get(t.id, 0) != len(users):
                    continue
                for j in users:
                    k = blk.stmts[j].kernel
                    idx_loads = [ld for e in k.exprs() for ld in ir.loads_in(e)
                                 for gth in ld.offset.gathers() if gth.load.buf.root is t]
                    if idx_loads or any(gth.load.buf.root is t for x in k.stores for gth in x.offset.gathers()):
                        ok = False
                    # read inside a reduction (a product's operand), g would run once per term
                    if k.red is not None and any(ld.buf.root is t for ld in ir.loads_in(k.red.body)):
                        ok = False
                if ok:
                    return blk, i, s, users
    return None


def _substitute(k: ir.Kernel, t: Buffer, g, okey) -> ir.Kernel:
    """Kernel k with each load of t at offset o replaced by g, its loads (at offset okey) moved to o."""
    import dataclasses

    def at(o):
        def fn(x):
            if isinstance(x, Load) and x.offset.key() == okey:
                return Load(x.buf, o)
            return x
        return fn

    lets: dict = {}

    def fn(x):
        if isinstance(x, Load) and x.buf.root is t:
            return ir.map_expr(g, at(x.offset))
        if isinstance(x, ir.LetRef) and x.let in lets:
            return ir.LetRef(lets[x.let])
        return x

    stmts = []
    for st in k.stmts:
        if isinstance(st, ir.Let):
            new = ir.Let(st.name, ir.map_expr(st.value, fn))
            lets[st] = new
            stmts.append(new)
        else:
            stmts.append(dataclasses.replace(st, value=ir.map_expr(st.value, fn)))
    red = k.red
    if red is not None:
        red = dataclasses.replace(red, body=ir.map_expr(red.body, fn))
    return dataclasses.replace(k, stmts=stmts, red=red)


def rematerialize(prog: ir.Program, max_cost: int = REMAT_MAX_COST) -> ir.Program:
    """The program with every temporary that `_remat_candidate` finds recomputed in the kernels that
    read it, and its store dropped from the kernel that wrote it (the kernel itself too, if nothing
    is left for it to store). The values are the same expressions of the same inputs, so with the
    generated code's floating-point contraction off they are bit for bit what was stored before. The
    caller's program is not changed."""
    import dataclasses
    for _ in range(10_000):
        found = _remat_candidate(prog, max_cost)
        if found is None:
            break
        blk, i, s, users = found
        t, g, okey = s.buf, _inline_lets(s.value), s.offset.key()
        stmts = list(blk.stmts)
        for j in users:
            stmts[j] = dataclasses.replace(stmts[j], kernel=_substitute(stmts[j].kernel, t, g, okey))
        m = stmts[i].kernel
        rest = [x for x in m.stmts if x is not s]
        if any(isinstance(x, ir.Store) for x in rest):
            stmts[i] = dataclasses.replace(stmts[i], kernel=dataclasses.replace(m, stmts=rest))
        else:
            del stmts[i]
        prog = dataclasses.replace(prog, main=_replace_block(prog.main, blk, dataclasses.replace(blk, stmts=stmts)))
    return prog


def _replace_block(blk, old, new):
    """blk with the block `old` (found by identity) replaced by `new`, copying the blocks on the way."""
    import dataclasses
    if blk is old:
        return new
    out, changed = [], False
    for st in blk.stmts:
        n = st
        if isinstance(st, ir.For):
            b = _replace_block(st.body, old, new)
            n = st if b is st.body else dataclasses.replace(st, body=b)
        elif isinstance(st, ir.While):
            c, b = _replace_block(st.cond_block, old, new), _replace_block(st.body, old, new)
            n = st if (c is st.cond_block and b is st.body) else dataclasses.replace(st, cond_block=c, body=b)
        elif isinstance(st, ir.If):
            a, b = _replace_block(st.then, old, new), _replace_block(st.orelse, old, new)
            n = st if (a is st.then and b is st.orelse) else dataclasses.replace(st, then=a, orelse=b)
        changed |= n is not st
        out.append(n)
    return dataclasses.replace(blk, stmts=out) if changed else blk


# ----------------------------------------------------------------------------- program-wide reads

def all_readers(prog: ir.Program) -> dict:
    """buffer id -> number of statements (kernels, prints, calls, conditions) that read it."""
    out: dict[int, int] = {}

    def note(bs):
        for b in bs:
            out[b.id] = out.get(b.id, 0) + 1

    def walk(blk):
        for st in blk.stmts:
            if isinstance(st, ir.For):
                note({b.root for b in (st.start, st.stop) if isinstance(b, Buffer)})
                note({st.counter.root})
                walk(st.body)
            elif isinstance(st, ir.While):
                walk(st.cond_block)
                note({st.cond.root})
                walk(st.body)
            elif isinstance(st, ir.If):
                note({st.cond.root})
                walk(st.then)
                walk(st.orelse)
            else:
                note(stmt_reads(st))
    walk(prog.main)
    return out


# ----------------------------------------------------------------------------- the arena

@dataclass
class ArenaPlan:
    offsets: dict = field(default_factory=dict)     # buffer id -> byte offset
    size: int = 0
    shared_bytes: int = 0                            # what the shared buffers would take apart
    placed_bytes: int = 0
    spans: dict = field(default_factory=dict)       # buffer id -> (first, last) program position, if shared


def _full_write(k: ir.Kernel, b: Buffer) -> bool:
    """Does kernel k write every element of b (with plain stores)?"""
    return any(st.buf.root is b and _store_covers(k, st, b) for st in k.stores)


def _store_covers(k: ir.Kernel, st, b: Buffer) -> bool:
    """Does store st of kernel k write every element of b, each once (a plain store)?"""
    if st.accumulate or st.offset.scalars() or st.offset.gathers() or st.offset.const != 0:
        return False
    n = ir.prod(v.extent for v in k.domain)
    if n != b.numel or not injective_over(st.offset, k.domain):
        return False
    lo, hi = st.offset.var_bounds()
    return lo == 0 and hi == b.numel - 1


def plan_arena(prog: ir.Program, device_bufs: list, full_writer, share: bool = True, fused=None,
               extra=None) -> ArenaPlan:
    """Offsets for device_bufs. full_writer(stmt, buf) says whether a statement writes all of buf.
    fused(kernel) -> (group key, buffers the group writes) or None: the kernels of one generated
    kernel run together, so they are one position of the program (reads of what the group itself
    writes are of the lane's own elements and do not start a lifetime early).
    extra(stmt) -> buffers the statement's launch reads beyond its IR kernel (a fused chain that
    reads a buffer the IR's own kernels had finished with): they stay live up to it.
    share=False gives every buffer its own bytes ($ANVIL_HIP_SHARE=0: for inspecting temporaries)."""
    uses: dict[int, list] = {}
    loops: list[tuple[int, int]] = []
    pos = 0
    by_id = {b.id: b for b in device_bufs}

    here = [0]                                          # the position uses are noted at

    def note(b, chain, write=False, full=False):
        if b.id in by_id:
            uses.setdefault(b.id, []).append((here[0], chain, write, full))

    def block(blk, chain):
        for st in blk.stmts:
            stmt(st, chain)

    def stmt(st, chain):
        nonlocal pos
        pos += 1
        here[0] = pos
        if isinstance(st, ir.For):
            start = pos
            for b in (st.start, st.stop):
                if isinstance(b, Buffer):
                    note(b.root, chain)
            note(st.counter.root, chain, write=True)
            block(st.body, chain + (("loop", id(st)),))
            pos += 1
            loops.append((start, pos))
        elif isinstance(st, ir.While):
            start = pos
            inner = chain + (("loop", id(st)),)
            block(st.cond_block, inner)
            pos += 1
            here[0] = pos
            note(st.cond.root, inner)
            block(st.body, inner)
            pos += 1
            loops.append((start, pos))
        elif isinstance(st, ir.If):
            note(st.cond.root, chain)
            block(st.then, chain + (("then", id(st)),))
            block(st.orelse, chain + (("else", id(st)),))
            pos += 1
        elif isinstance(st, (ir.Break, ir.Continue)):
            pass
        else:
            group = fused(st.kernel) if fused is not None and isinstance(st, KernelStmt) else None
            own: set = set()
            if group is not None:
                key, own = group
                here[0] = group_pos.setdefault(key, pos)    # every part of one launch: one position
            for b in stmt_reads(st) | (extra(st) if extra is not None else set()):
                if b not in own:
                    note(b, chain)
            for b in stmt_writes(st):
                note(b, chain, write=True, full=full_writer(st, b))
    group_pos: dict = {}
    block(prog.main, ())

    def lifetime(us):
        us = sorted(us, key=lambda u: u[0])
        first = us[0][0]
        at_first = [u for u in us if u[0] == first]
        if any(not u[2] for u in at_first) or not any(u[3] for u in at_first):
            return None                                 # read before it is all written
        chain = at_first[0][1]
        if any(u[1][:len(chain)] != chain for u in us):
            return None                                 # the first write might not have run
        lo, hi = first, us[-1][0]
        grown = True
        while grown:
            grown = False
            for a, b in loops:
                if lo <= b and a <= hi and (a < lo or b > hi) and not (a <= lo and hi <= b):
                    lo, hi = min(lo, a), max(hi, b)
                    grown = True
        return lo, hi

    def rounded(b):
        return max(ARENA_ALIGN, (b.nbytes + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN)

    plan = ArenaPlan()
    fixed, shared = [], []
    for b in device_bufs:
        span = None
        if share and b.kind in SHARED_KINDS and not getattr(b, "heap", False) and b.id in uses \
                and str(b.id) not in _UNSHARED:
            span = lifetime(uses[b.id])
        if span is None:
            fixed.append(b)
        else:
            shared.append((b, span, rounded(b)))
    off = 0
    for b in sorted(fixed, key=lambda b: b.id):
        plan.offsets[b.id] = off
        off += rounded(b)
    base = off
    shared.sort(key=lambda it: (-it[2], it[1][0], it[0].id))
    placed = []
    top = 0
    for b, (lo, hi), n in shared:
        busy = sorted((o, o + s) for (l2, h2, o, s) in placed if l2 <= hi and lo <= h2)
        o = 0
        for s, e in busy:
            if o + n <= s:
                break
            o = max(o, e)
        placed.append((lo, hi, o, n))
        plan.offsets[b.id] = base + o
        plan.spans[b.id] = (lo, hi)
        top = max(top, o + n)
    plan.shared_bytes = sum(n for _, _, n in shared)
    plan.placed_bytes = top
    plan.size = base + top
    return plan

"""Contractions on the matrix cores: recognising C = Σ_k A·B in an IR kernel and generating an
fp32 MFMA kernel for it (the device side is hip_rt/anvil_mfma.h).

A kernel qualifies when its reduction is a sum of a product of two operands, each an elementwise
function of one load (relu(x), 0.35·k, a plain load), times constants, with loads at affine offsets
of the loop variables alone (the reference's BLAS matcher, blas.py:113-172, finds the same shapes).
Its variables split into
    k: the reduction variables (in both operands), merged into one index when their strides allow;
    m: domain variables only A uses, n: those only B uses (each merged into one row / column index);
    batch: the rest (heads of attention, images of a convolution), one grid slice each.
The product accumulates in the matrix cores; then every output element runs the kernel's own
statements with acc = alpha * (the dot product): a bias add, an activation, the first moment of
Adam, the store of a gradient — whatever the optimizer fused after the reduction. Nothing is
split off into a second kernel.
"""
from __future__ import annotations

import math
import os

from .. import ir
from ..ir import F32, Binary, Const, KernelStmt, Load, Unary, Var
from . import hip_analysis as A
from .hip_emit import Emitter, flit
from .hip_kernels import KernelScope, Plan, canon_key, decode

MIN_WORK = 1 << 16           # M·N·K below which the generic schedules are as good
MIN_SIDE = 32                # a narrower product (10 classes) wastes most of a 32-wide MFMA tile
MIN_K = 16                   # a shorter sum (a 3 x 3 convolution of one input channel: K = 9) is
                             # memory-bound: OuterPlan, or a map where each lane sums its K terms
OUTER_MAX_M = 64             # rows an OuterPlan lane runs in turn against its column
OUTER_MIN_N = 4096           # columns (one lane each) that make an OuterPlan launch worth it
OUTER_ROWS = 8               # rows per OuterPlan lane: more wavefronts in flight, and the row
                             # operand's loads of a group issued together
CUS = 256                    # compute units of an MI355X
CU_WAVES = CUS * 4           # wavefronts that fill it once (one per SIMD)


def _factors(e, out):
    if isinstance(e, Binary) and e.op == "mul" and e.dtype == F32:
        _factors(e.a, out)
        _factors(e.b, out)
    else:
        out.append(e)
    return out


def _const_value(e):
    if isinstance(e, Const) and e.dtype == F32:
        return float(e.value)
    return None


def gathered_row(ld):
    """(gather, its coefficient, the variable it is indexed by) when ld's offset is c·G + (terms in
    other loop variables), G = idx[v + scalars + const] a checked gather: an operand whose rows are
    picked through an index array (a shuffled batch). None otherwise."""
    gs = ld.offset.gathers()
    if len(gs) != 1 or gs[0].rest is not None:
        return None
    g = gs[0]
    c = ld.offset.terms[g]
    inner = g.load.offset
    vs = [t for t in inner.terms if isinstance(t, Var)]
    if c <= 0 or len(vs) != 1 or inner.terms[vs[0]] != 1 or inner.gathers():
        return None
    if any(not isinstance(t, (Var, ir.ScalarRef)) for t in inner.terms):
        return None
    v = vs[0]
    if any(not isinstance(t, Var) for t in ld.offset.terms if t is not g) or ld.offset.coef(v):
        return None
    return g, c, v


def _coef_fn(ld):
    """Coefficient of each loop variable in an operand's offset; a gathered row counts its gather's
    coefficient for the variable that indexes it."""
    gr = gathered_row(ld)
    if gr is None:
        return ld.offset.coef
    _, c, gv = gr
    return lambda v: c if v is gv else ld.offset.coef(v)


def _single_load(e):
    """The one array load of an elementwise operand expression (other leaves constants), or None."""
    loads = []
    for x in ir.iter_expr(e):
        if isinstance(x, Load):
            loads.append(x)
        elif not isinstance(x, (Const, Unary, Binary, Load)):
            return None
    loads = [x for x in loads if not any(x is g.load for y in loads for g in y.offset.gathers())]
    if len(loads) != 1 or not loads[0].buf.root.shape or loads[0].buf.dtype != F32:
        return None
    ld = loads[0]
    if any(not isinstance(t, Var) for t in ld.offset.terms) and gathered_row(ld) is None:
        return None
    return ld


def _merge(vars_, coef, coef2=None):
    """Order vars so that their offsets form one linear index: returns (vars outer->inner, stride)
    or None. coef2: the same vars must merge identically in a second operand."""
    vs = sorted(vars_, key=lambda v: (abs(coef(v)), v.id))
    if not vs:
        return [], 0
    base = coef(vs[0])
    base2 = coef2(vs[0]) if coef2 else None
    span = 1
    for v in vs:
        if coef(v) != base * span:
            return None
        if coef2 is not None and coef2(v) != base2 * span:
            return None
        span *= v.extent
    return list(reversed(vs)), base


class GemmSpec:
    pass


def analyse(k: ir.Kernel):
    red = k.red
    if red is None or red.op != "sum" or red.body.dtype != F32 or not red.vars or not k.domain:
        return None
    fs = _factors(red.body, [])
    alpha = 1.0
    ops = []
    for f in fs:
        c = _const_value(f)
        if c is not None:
            alpha *= c
        else:
            ops.append(f)
    if len(ops) != 2:
        return None
    lds = [_single_load(e) for e in ops]
    if None in lds:
        return None
    dom, rv = list(k.domain), list(red.vars)
    best = None
    for (ea, la), (eb, lb) in (((ops[0], lds[0]), (ops[1], lds[1])), ((ops[1], lds[1]), (ops[0], lds[0]))):
        ca, cb = _coef_fn(la), _coef_fn(lb)
        if any(not ca(v) or not cb(v) for v in rv):
            continue
        mv = [v for v in dom if ca(v) and not cb(v)]
        nv = [v for v in dom if cb(v) and not ca(v)]
        bv = [v for v in dom if v not in mv and v not in nv]
        if any(not ca(v) and not cb(v) for v in bv) or not mv or not nv:
            continue
        km = _merge(rv, ca, cb)
        kmulti = None
        ktab = None
        if km is None:
            # K linear with unit stride in one operand (a convolution's weights over c, u, v) but not
            # in the other (its input: 676c + 26u + v): k in the linear operand's order, and the other
            # operand's offset of each k from a table
            for which, lin_c, tab_c in (("b", ca, cb), ("a", cb, ca)):
                lin = _merge(rv, lin_c)
                K_ = ir.prod(v.extent for v in rv)
                # (K a multiple of 8 for the matrix cores' 8-k chunks; with $ANVIL_GEMM_SHORT_KTAB=1
                # also a sum too short for them, which OuterPlan adds up one k at a time: C5's first
                # convolution, K = 3 x 3, which can then read its input in place of the im2col copy,
                # and so can its weight gradient; measured 197.2 -> 200.7 us per step, so the copy stays)
                if (lin is not None and abs(lin[1]) == 1 and (K_ % 8 == 0 or (K_ < MIN_K and os.environ.get("ANVIL_GEMM_SHORT_KTAB", "0") == "1"))
                        and K_ <= 4096):
                    km = lin
                    steps = [(v.extent, tab_c(v)) for v in lin[0]]
                    ktab = (which, steps)
                    break
        if km is None:
            # K over several variables that are not one linear index of both operands (a weight
            # gradient summed over the batch and a convolution's positions, or a convolution's
            # channels and window): k decomposes over them, outer to inner; the innermost is the
            # most contiguous of those whose extent is a multiple of 4 (the 4 consecutive k a lane
            # loads at once never straddle two of its runs)
            fit = [v for v in rv if v.extent % 4 == 0]
            if not fit:
                continue
            inner = min(fit, key=lambda v: (min(abs(ca(v)), abs(cb(v))), v.id))
            order = sorted([v for v in rv if v is not inner], key=lambda v: (-abs(ca(v)), v.id)) + [inner]
            km = (order, ca(inner))
            kmulti = [(v.extent, ca(v), cb(v)) for v in order]
        rows_multi = {}

        def rows(vs, coef, which):
            """vs as one row index: merged when their offsets form one linear index; else the
            densest one, the rest batched; else, when that one is too narrow for a tile (the
            positions of a convolution's output, a row of 24 in a plane of 26 x 26), all of them,
            the operand's row offset then computed from each one's digit of the row index."""
            mg = _merge(vs, coef)
            if mg is not None:
                return mg
            inner = min(vs, key=lambda v: (abs(coef(v)), v.id))
            if inner.extent >= MIN_SIDE:
                bv.extend(v for v in vs if v is not inner)
                return [inner], coef(inner)
            rows_multi[which] = [(v.extent, coef(v)) for v in vs]
            g = 0
            for v in vs:
                g = math.gcd(g, abs(coef(v)))
            return list(vs), g
        mm = rows(mv, ca, "a")
        nm = rows(nv, cb, "b")
        s = GemmSpec()
        s.k, s.alpha = k, alpha
        s.ea, s.la, s.eb, s.lb = ea, la, eb, lb
        s.m_vars, s.a_rs = mm
        s.n_vars, s.b_rs = nm
        s.k_vars, s.a_ks = km
        s.b_ks = cb(km[0][-1]) if km[0] else 0
        s.batch = [v for v in dom if v in bv]
        s.M = ir.prod(v.extent for v in s.m_vars)
        s.N = ir.prod(v.extent for v in s.n_vars)
        s.K = ir.prod(v.extent for v in s.k_vars)
        s.B = ir.prod(v.extent for v in s.batch)
        s.a_gather, s.b_gather = gathered_row(la), gathered_row(lb)
        s.k_multi = kmulti
        s.a_multi, s.b_multi = rows_multi.get("a"), rows_multi.get("b")
        s.a_ktab = s.b_ktab = None
        if ktab is not None:
            offs = [0] * s.K
            strides = ir.row_major_strides([e for e, _ in ktab[1]])
            for kk in range(s.K):
                offs[kk] = sum(c * ((kk // st) % e) for (e, c), st in zip(ktab[1], strides))
            if ktab[0] == "a":
                s.a_ktab = offs
            else:
                s.b_ktab = offs
            if ktab[0] == "b":
                s.b_ks = 0
            else:
                s.a_ks, s.b_ks = 0, km[1]
        if (s.a_gather and (s.m_vars != [s.a_gather[2]] or s.batch or any(ca(v) for v in nv))) or \
                (s.b_gather and (s.n_vars != [s.b_gather[2]] or s.batch or any(cb(v) for v in mv))):
            continue                                    # rows picked through an index: one plain row variable
        # prefer the assignment whose n is the output's innermost (contiguous) variable
        score = 1 if dom[-1] in s.n_vars else 0
        if best is None or score > best[0]:
            best = (score, s)
    return None if best is None else best[1]


def load_mode(rs, ks, T, K, const, batch_strides):
    aligned = const % 4 == 0 and all(c % 4 == 0 for c in batch_strides)
    if ks == 1 and K % 4 == 0 and rs % 4 == 0 and aligned:
        return "ANVIL_LD_KC"
    if rs == 1 and T % 4 == 0 and ks % 4 == 0 and aligned:
        return "ANVIL_LD_RC"
    return "ANVIL_LD_ANY"


def gathered_ok(s) -> bool:
    """Operands with gathered rows, and K over several variables, are supported by the pipelined K
    split only; gathered rows load 16 bytes along k (so K a multiple of 8, rows on 16 bytes)."""
    pipe = os.environ.get("ANVIL_GEMM_PIPE", "1") != "0"
    for g, rs, ks, T in ((s.a_gather, s.a_rs, s.a_ks, s.M), (s.b_gather, s.b_rs, s.b_ks, s.N)):
        if g is not None and (s.K % 8 or ks != 1 or g[1] % 4 or not pipe):
            return False
    if s.k_multi and (not pipe or s.batch):
        return False
    if (s.a_multi or s.b_multi or s.a_ktab or s.b_ktab) and not pipe:
        return False
    return True


def qualifies(s) -> bool:
    """Is the product worth the matrix cores? Enough work, a sum of at least MIN_K terms, and both
    sides at least a tile wide;
    a narrower one (a convolution's 32 x 9 weight gradient) only when K is long enough to be split
    across workgroups, each reading its slice of both operands once."""
    if s.M * s.N * s.K < MIN_WORK or s.K < MIN_K or not gathered_ok(s):
        return False
    if min(s.M, s.N) >= MIN_SIDE:
        return True
    return min(s.M, s.N) >= 8 and s.K >= 16384 and s.K % 8 == 0 and not s.batch


def match(gen, k: ir.Kernel, name: str):
    """A GemmPlan for a contraction kernel (its stores may add to their buffer, `+=`: a gradient
    that collects several products; the epilogue then adds atomically, as the reference's parallel
    kernels do)."""
    if gen.emulate:
        return None
    s = analyse(k)
    if s is None:
        return None
    if not qualifies(s):
        if outer_ok(s):
            return OuterPlan(gen, k, name, s)
        return None
    return GemmPlan(gen, k, name, s)


def outer_ok(s) -> bool:
    """A product with a sum too short for the matrix cores, few rows and many columns, plainly
    addressed rows of A (what OuterPlan runs)."""
    return (s.K < MIN_K and s.M <= OUTER_MAX_M and s.N >= OUTER_MIN_N and s.B == 1 and not s.k_multi
            and not s.a_gather and not s.a_multi and os.environ.get("ANVIL_GEMM_OUTER", "1") != "0")


def forward_gather_copies(prog: ir.Program, hosts: set) -> ir.Program:
    """A kernel that only copies rows picked through an index array into a batch buffer
    (xb[i, j] = X[perm[s·B + i], j]) and a later product that reads the batch buffer: the product
    reads X through the index instead (its operand rows are gathered as it loads them), so it no
    longer waits for the copy, and the two can run side by side. The copy stays for the batch
    buffer's other readers. Done only where the product then keeps its matrix-core schedule."""
    import dataclasses
    from . import hip_analysis as A

    def copy_kernel(st):
        if not isinstance(st, KernelStmt):
            return None
        k = st.kernel
        if k.red is not None or len(k.stmts) != 1 or not isinstance(k.stmts[0], ir.Store) or not k.domain:
            return None
        store = k.stmts[0]
        if store.accumulate or not isinstance(store.value, Load) or not A.parallel_safe(k):
            return None
        strides = ir.row_major_strides([v.extent for v in k.domain])
        want = ir.Affine(0, {v: st_ for v, st_ in zip(k.domain, strides) if v.extent > 1})
        if store.offset != want or store.buf.root.numel != ir.prod(v.extent for v in k.domain):
            return None
        if not store.value.offset.gathers():
            return None
        return k, store.buf.root, store.value, dict(zip(k.domain, strides))

    def subst(off: ir.Affine, m: dict) -> ir.Affine:
        out = ir.Affine(off.const)
        for t, c in off.terms.items():
            if isinstance(t, Var):
                out = out + m.get(t, ir.Affine(0)) * c
            elif isinstance(t, ir.Gather):
                g = ir.Gather(Load(t.load.buf, subst(t.load.offset, m)), t.bound, t.where, None)
                out = out + ir.Affine(0, {g: c})
            else:
                out = out + ir.Affine(0, {t: c})
        return out

    def rewrite(c: ir.Kernel, cp):
        pk, dst, src, strides = cp
        by_stride = {st_: v for v, st_ in strides.items() if v.extent > 1}
        ok = [True]

        def fn(e):
            if not isinstance(e, Load) or e.buf.root is not dst:
                return e
            off = e.offset
            if off.const or off.gathers() or off.scalars():
                ok[0] = False
                return e
            m, used = {}, set()
            for t, coef in off.terms.items():
                v = by_stride.get(coef)
                if v is None or v in used or t.extent > v.extent:
                    ok[0] = False
                    return e
                used.add(v)
                m[v] = ir.Affine(0, {t: 1})
            return Load(src.buf, subst(src.offset, m))
        if c.red is None:
            return None
        body = ir.map_expr(c.red.body, fn)
        lets: dict = {}                                   # old Let -> its copy (LetRefs follow)

        def fn2(e):
            if isinstance(e, ir.LetRef) and id(e.let) in lets:
                return ir.LetRef(lets[id(e.let)])
            return fn(e)
        stmts = []
        for st in c.stmts:
            new = dataclasses.replace(st, value=ir.map_expr(st.value, fn2))
            if isinstance(st, ir.Let):
                lets[id(st)] = new
            stmts.append(new)
        if not ok[0] or any(st.buf.root is dst for st in c.stores):
            return None
        k2 = dataclasses.replace(c, red=dataclasses.replace(c.red, body=body), stmts=stmts)
        if any(ld.buf.root is dst for ld in A.kernel_loads(k2)):
            return None                                   # still reads the batch buffer elsewhere
        s = analyse(k2)
        if s is None or not (s.a_gather or s.b_gather) or not qualifies(s):
            return None
        return k2

    def block(blk: ir.Block) -> ir.Block:
        out = [stmt(st) for st in blk.stmts]
        for i, st in enumerate(out):
            cp = copy_kernel(st)
            if cp is None:
                continue
            pk, dst, src, _ = cp
            guard = {dst.id} | {x.id for x in A.kernel_reads(pk)}
            for j in range(i + 1, len(out)):
                s2 = out[j]
                if (isinstance(s2, ir.If) and not s2.orelse.stmts and len(s2.then.stmts) == 1
                        and isinstance(s2.then.stmts[0], (ir.Break, ir.Continue))):
                    continue                              # leaves the loop; writes nothing
                if not isinstance(s2, KernelStmt):
                    break
                c = s2.kernel
                if dst.id in {x.id for x in A.kernel_reads(c)}:
                    k2 = rewrite(c, cp)
                    if k2 is not None:
                        out[j] = dataclasses.replace(s2, kernel=k2)
                if guard & {x.id for x in A.kernel_writes(out[j].kernel)}:
                    break
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


def subst_affine(a: ir.Affine, m: dict):
    """a with its loop variables replaced by affine expressions (None if a has gathers)."""
    out = ir.Affine(a.const)
    for t, c in a.terms.items():
        if isinstance(t, Var):
            if t not in m:
                return None
            out = out + m[t] * c
        elif isinstance(t, ir.ScalarRef):
            out = out + ir.Affine(0, {t: c})
        else:
            return None
    return out


def follower_map(k: ir.Kernel, e: ir.Kernel):
    """e's domain variables as affine functions of k's, when e walks k's output elements in the same
    row-major order (the same shape, or one flattened variable)."""
    ke, ee = [v.extent for v in k.domain], [v.extent for v in e.domain]
    if ir.prod(ke) != ir.prod(ee) or not ee:
        return None
    if ke == ee:
        return {ev: ir.Affine.of(kv) for ev, kv in zip(e.domain, k.domain)}
    # each of e's variables spans a run of k's (one flattened variable; or a product whose merged
    # variables were split back out, an implicit convolution)
    m, i = {}, 0
    for ev in e.domain:
        run, span = [], 1
        while span < ev.extent and i < len(k.domain):
            run.append(k.domain[i])
            span *= k.domain[i].extent
            i += 1
        if span != ev.extent:
            return None
        aff = ir.Affine(0)
        for kv, st in zip(run, ir.row_major_strides([v.extent for v in run])):
            aff = aff + ir.Affine(0, {kv: st})
        m[ev] = aff
    if any(v.extent != 1 for v in k.domain[i:]):
        return None
    return m


def follower(k: ir.Kernel, e: ir.Kernel, hosts: set, prior=()):
    """(var map, forwarded loads) if elementwise kernel e can run in k's epilogue, element by element,
    after the followers already taken (prior: (kernel, its var map) pairs): every load e makes of
    what k or a prior follower writes is of the element written there in the same lane (a value of
    k's comes from a register), and neither k nor a prior follower reads anything that e writes."""
    if (e.red is not None or e.uses_rand() or A.is_host_kernel(e, hosts) or not A.parallel_safe(e)
            or any(st.accumulate for st in e.stores)):
        return None
    m = follower_map(k, e)
    if m is None:
        return None
    stored = {}
    for st in k.stores:
        if st.buf.root.id in stored:
            return None
        stored[st.buf.root.id] = st.offset
    added = {st.buf.root.id for st in k.stores if st.accumulate}   # k adds to them: no value to forward
    later = {}                          # buffers prior followers store to: the element, in k's variables
    for f, mf in prior:
        for st in f.stores:
            off = subst_affine(st.offset, mf)
            if off is None or later.get(st.buf.root.id, off) != off:
                return None
            later[st.buf.root.id] = off
    fwd = []
    for ld in A.kernel_loads(e):
        bid = ld.buf.root.id
        if bid in added:
            return None
        if bid in stored or bid in later:
            sub = subst_affine(ld.offset, m)
            if sub is None or sub != later.get(bid, stored.get(bid)):
                return None
            if bid not in later:
                fwd.append(ld)
    readers = {b.id for f in [k] + [f for f, _ in prior] for b in A.kernel_reads(f)}
    if {b.id for b in A.kernel_writes(e)} & readers:
        return None
    return m, fwd


class GemmPlan(Plan):
    """Schedules: "tile" (a 64 x 64 or 128 x 128 tile per workgroup, 2 x 2 wavefronts) when there are
    enough tiles to fill the chip; else "ksplit" (a 32 x 32 tile per workgroup, K split over its four
    wavefronts)."""

    kind = "gemm"

    def __init__(self, gen, k, name, spec: GemmSpec):
        super().__init__(gen, [k], name)
        self.k = k
        self.s = s = spec
        tiles = lambda bm, bn: -(-s.M // bm) * -(-s.N // bn) * s.B
        if tiles(128, 128) >= 2 * CUS:
            self.sched, self.BM, self.BN = "tile", 128, 128
        elif tiles(64, 64) >= 4 * CUS:
            self.sched, self.BM, self.BN = "tile", 64, 64
        else:
            self.sched, self.BM, self.BN = "ksplit", 32, 32
        # the K split. With K in 8-k chunks (anvil_mm_tile_kpipe), four wavefronts with two or four
        # chunks in flight each measured best for batch-256 layers (fewer requests in flight than
        # 8 or 16 wavefronts, and a shorter reduction through LDS); otherwise the older loop wants
        # enough wavefronts that each one's share is in flight at once.
        self.pipe = s.K % 8 == 0 and os.environ.get("ANVIL_GEMM_PIPE", "1") != "0"
        if self.pipe:
            self.waves = 4
        else:
            self.waves = 16 if s.K >= 512 else (8 if s.K >= 128 else 4)
        self.unroll = 4
        ca, cb = s.la.offset.coef, s.lb.offset.coef
        self.amode = load_mode(s.a_rs, s.a_ks, s.M, s.K, s.la.offset.const, [ca(v) for v in s.batch])
        self.bmode = load_mode(s.b_rs, s.b_ks, s.N, s.K, s.lb.offset.const, [cb(v) for v in s.batch])
        if s.a_ktab:
            self.amode = "ANVIL_LD_KT"
        if s.b_ktab:
            self.bmode = "ANVIL_LD_KT"
        self.slab = 0
        self.ptm = self.ptn = 1             # 32 x 32 MFMA tiles per wavefront in the pipelined split
        # tuning: $ANVIL_GEMM_FORCE = comma-separated "tile64" | "tile128" | "ksplit:W:U" | "slab:KC" |
        # "kpipe:W:TM:TN", each optionally "@NN" / "@NT" / "@TN" (only products whose operands load
        # that way) or "@MxNxK" (only products of that shape)
        layout = {("ANVIL_LD_KC", "ANVIL_LD_RC"): "NN", ("ANVIL_LD_KC", "ANVIL_LD_KC"): "NT",
                  ("ANVIL_LD_RC", "ANVIL_LD_RC"): "TN"}.get((self.amode, self.bmode), "?")
        shape = f"{s.M}x{s.N}x{s.K}"
        self.forced = False
        for force in os.environ.get("ANVIL_GEMM_FORCE", "").split(","):
            force, _, only = force.partition("@")
            if not force or (only and only not in (layout, shape)):
                continue
            self.forced = True
            parts = force.split(":")
            if parts[0].startswith("tile"):
                self.sched, self.BM = "tile", int(parts[0][4:])
                self.BN = self.BM
            elif parts[0] == "slab":
                self.sched, self.BM, self.BN = "ksplit", 32, 32
                self.slab, self.waves = int(parts[1]), 4
            elif parts[0] == "kpipe":
                self.waves, self.ptm, self.ptn = int(parts[1]), int(parts[2]), int(parts[3])
                self.sched, self.BM, self.BN = "ksplit", 32 * self.ptm, 32 * self.ptn
            else:
                self.sched, self.BM, self.BN = "ksplit", 32, 32
                self.waves, self.unroll = int(parts[1]), int(parts[2])
        if (s.a_gather or s.b_gather or s.k_multi or s.a_multi or s.b_multi or s.a_ktab or s.b_ktab
                or min(s.M, s.N) < MIN_SIDE):                   # the pipelined K split only
            if self.ptm * self.ptn == 1:
                self.sched, self.BM, self.BN, self.slab, self.pipe, self.waves = "ksplit", 32, 32, 0, True, 4
            self.pipe = True
        self.followers = []             # (kernel, var map, forwarded loads) run in the epilogue
        self.layout()

    def layout(self):
        """What follows from the schedule: the K split across workgroups, pipeline depth, workgroup
        size and tile grid."""
        s = self.s
        self.pipe = self.pipe and self.sched == "ksplit" and not self.slab
        if not self.pipe:
            self.ptm = self.ptn = 1
        # K split across workgroups as well, when the output has few tiles and K is long (a
        # convolution's weight gradient: 64 x 288 outputs, K = 73728): each workgroup computes a
        # slice of K into a partial tile, and a second kernel adds the S partials in order and runs
        # the epilogue (see GemmReducePlan)
        tiles = -(-s.M // self.BM) * -(-s.N // self.BN) * s.B if self.pipe else -(-s.M // 32) * -(-s.N // 32) * s.B
        self.kslices, self.kslice = 1, s.K
        if (self.pipe and tiles * self.waves < int(os.environ.get("ANVIL_GEMM_SPLITK_WAVES", str(CU_WAVES // 2)))
                and s.K >= int(os.environ.get("ANVIL_GEMM_SPLITK_MINK", "4096"))
                and os.environ.get("ANVIL_GEMM_SPLITK", "1") != "0"):
            S = int(os.environ.get("ANVIL_GEMM_SPLITK_S", "0")) or max(2, min(1024 // tiles, s.K // 512))
            self.kslice = -(-(-(-s.K // S)) // 8) * 8
            self.kslices = -(-s.K // self.kslice)
        # chunks of 8·G k (anvil_mm_tile_kpipe): two 16-byte loads per lane of an operand contiguous
        # in k (half a cache line of each row) when each wavefront has K ≥ 128 to cover (measured:
        # C2's 256 x 1024 x 1024 products 9.7 -> 8.6 µs, C4's weight gradients with K = 4096 in
        # slices of 512 96 -> 86 µs; with K = 64 per wavefront, fewer and larger chunks were up to
        # 3 µs slower), while the registers in flight stay within 96 per lane ($ANVIL_GEMM_KREGS):
        # C3's one-wavefront 2 x 4 tile takes G = 2 with 96, 129.2 -> 131.7 TFLOP/s (three runs each)
        self.kgroup = 1
        plain = {self.amode, self.bmode} <= {"ANVIL_LD_KC", "ANVIL_LD_RC"}
        for g in (4, 2):
            if (self.pipe and plain and g <= int(os.environ.get("ANVIL_GEMM_KGROUP", "2"))
                    and s.K % (8 * g) == 0 and self.kslice % (8 * g) == 0
                    and self.kslice // self.waves >= 128
                    and 2 * (self.ptm + self.ptn) * 4 * g <= int(os.environ.get("ANVIL_GEMM_KREGS", "96"))):
                self.kgroup = g
                break
        nch = -(-(self.kslice // (8 * self.kgroup)) // self.waves)      # chunks per wave
        self.depth = max(1, min(int(os.environ.get("ANVIL_GEMM_DEPTH", "2" if nch <= 32 else "4")), nch))
        # independent accumulator chains per wavefront when it has one 32 x 32 tile and a long run of
        # chunks ($ANVIL_GEMM_CHAINS_NCH of them at least). Measured (one MI355X, three runs each): C4 at
        # T = 256, whose weight gradients run 64 chunks per wavefront, 1386-1387 -> 1382 µs per step;
        # C5 194.8 -> 194.0-194.1; two chains on the short runs too (C2's batch-256 products) no faster
        one = self.ptm * self.ptn == 1 and nch >= int(os.environ.get("ANVIL_GEMM_CHAINS_NCH", "32"))
        self.chains = int(os.environ.get("ANVIL_GEMM_CHAINS", "2")) if one else 1
        self.threads = 64 * self.waves if self.sched == "ksplit" else 256
        self.tm = -(-s.M // self.BM)
        self.tn = -(-s.N // self.BN)

    def settle(self):
        """Once the epilogue is known (its followers absorbed): a product whose epilogue is light (a
        bias, a plain store) and whose operands load plainly takes the larger per-wavefront tiles; a
        heavy epilogue (GELU, Adam: each lane of a one-wavefront workgroup would run it for 64
        outputs, serially; C4's GELU products measured 17 µs slower) or per-element operand
        addressing (a convolution's input through its table: 14 µs slower) keeps four wavefronts."""
        from .hip_cost import expr_ops
        s = self.s
        light = not self.followers and sum(expr_ops(st.value) for st in self.k.stmts) <= 2
        plain = not (s.a_gather or s.b_gather or s.k_multi or s.a_multi or s.b_multi or s.a_ktab or s.b_ktab)
        if (light and plain and not self.forced and s.K % 8 == 0 and min(s.M, s.N) >= MIN_SIDE and not self.slab
                and os.environ.get("ANVIL_GEMM_PIPE", "1") != "0"):
            self.choose_pipe_tiles()
            self.layout()

    def choose_pipe_tiles(self):
        """The pipelined K split's shape: W wavefronts per workgroup splitting K, each computing TM x TN
        32 x 32 MFMA tiles. The largest tiles that still give every SIMD a wavefront (CU_WAVES of
        them) win: the loaded operands serve TN (TM) products each and the wavefront carries
        independent accumulator chains. Measured (fp32, one MI355X): 8192 x 4096 x 4096 at 139
        TFLOP/s with one wavefront of 2 x 4 tiles (116 with the LDS-staged 128 x 128 tile); C4's
        4096 x 1024 x 256 at 79-84 with 2 x 2 (68-73); C4's 4096 x 256 x 1024 and 4096 x 256 x 768
        products (forward and input gradients) 21-22 µs with four wavefronts of 2 x 2 against 25-27
        with four of 1 x 2 (hipBLASLt: 18.6-22.1); batch-256 products stay at four wavefronts of
        one tile."""
        s = self.s
        for W, TM, TN, kmin in ((1, 2, 4, 0), (1, 2, 2, 0), (4, 2, 2, 512), (4, 1, 2, 512), (4, 1, 1, 0)):
            if -(-s.M // (32 * TM)) * -(-s.N // (32 * TN)) * s.B * W >= CU_WAVES and s.K >= kmin:
                break
        self.sched, self.slab, self.pipe = "ksplit", 0, True
        self.waves, self.ptm, self.ptn = W, TM, TN
        self.BM, self.BN = 32 * TM, 32 * TN

    def hoistable(self, stages):
        """(stage, load) pairs of the epilogue that may be issued before the K loop: plain loads of
        buffers no earlier epilogue statement stores to (later statements must see those stores)."""
        stored: set = set()
        out, seen = [], set()
        for si, (e, m, fwd) in enumerate(stages):
            fwd_ids = {id(ld) for ld in fwd}
            canon = {v: ("e", v.id) for v in e.domain}
            for st in e.stmts:
                for ld in ir.loads_in(st.value):
                    b = ld.buf.root
                    if id(ld) in fwd_ids or not b.shape or b.id in stored or ld.offset.gathers():
                        continue
                    if any(isinstance(t, ir.ScalarRef) for t in ld.offset.terms):
                        continue
                    key = (si, canon_key(ld.buf, ld.offset, canon))
                    if key not in seen:
                        seen.add(key)
                        out.append((si, ld))
                if isinstance(st, ir.Store):
                    stored.add(st.buf.root.id)
        return out

    def template_lds(self) -> int:
        """LDS of the anvil_mfma.h templates the kernel instantiates."""
        if self.slab:
            return 4 * (2 * 2 * self.slab * 33 + 4 * 16 * 64)
        if self.sched == "tile":
            return 2 * 4 * 16 * ((self.BM + 4) + (self.BN + 4))
        if self.pipe:
            return 0                   # anvil_kp_lds, declared in the kernel's own text
        return self.waves * self.ptm * self.ptn * 16 * 64 * 4

    def absorb(self, e, how):
        m, fwd = how
        self.followers.append((e, m, fwd))
        self.kernels.append(e)
        self.label += " + " + (e.label or e.name)

    def grid(self):
        return (self.tn, self.tm, self.s.B * self.kslices), self.threads

    def row_fn(self, sc, name, gather, rs, multi=None) -> str:
        """A device lambda: where row t of an operand starts (t·rs; c·idx[t + ...] for a gathered
        row, with the gather's bounds check; or, for rows over several variables, the sum of each
        one's coefficient times its digit of t)."""
        if multi:
            parts, rest = [], "(uint32_t)t"
            for depth, (ext, c) in enumerate(reversed(multi)):
                idx = rest if depth == len(multi) - 1 else f"({rest} % {ext}u)"
                if c:
                    parts.append(f"{c}LL * (long long){idx}")
                rest = f"({rest} / {ext}u)"
            return f"    auto {name} = [=](int t) -> long long {{ return {' + '.join(parts) or '0LL'}; }};"
        if gather is None:
            return f"    auto {name} = [=](int t) -> long long {{ return (long long)t * {rs}LL; }};"
        g, c, v = gather
        lines: list[str] = []
        em = Emitter(sc, lines, "        ", prefix=f"{name}_")
        saved = dict(sc.names)
        sc.names[v] = "t"
        val = em.gather(g)
        sc.names = saved
        return "\n".join([f"    auto {name} = [=](int t) -> long long {{"] + lines +
                         [f"        return {c}LL * (long long){val};", "    };"])

    def operand(self, sc, e, ld, name) -> str:
        """A device lambda applying the operand's elementwise function to a loaded value."""
        if e is ld:
            return f"    anvil_identity_op {name};"
        lines: list[str] = []
        em = Emitter(sc, lines, "        ", prefix=f"{name}_")
        saved = sc.fwd, sc.canon
        sc.canon = {v: ("v", v.id) for v in ld.offset.terms}
        sc.fwd = {_key(ld): "x"}
        v = em.ex(e)
        sc.fwd, sc.canon = saved
        return "\n".join([f"    auto {name} = [=](float x) -> float {{"] + lines + [f"        return {v};", "    };"])

    def run_order(self):
        """Which grids give each XCD one contiguous run of tiles (anvil_run_of) instead of every
        eighth: "split", a K split across workgroups, its runs walking slice by slice, so the tiles
        that read one slice's K range of both operands share an L2 (C5's update launch fetched
        250 MB against 89 MB of algorithmic reads in launch order, 83 MB in runs: 58.8 -> 52.3 µs;
        C4's weight gradients measured the same either way). With $ANVIL_GEMM_RUNS=all also
        "wide", a grid of 8 or more tile columns per row (C5's forward convolution: adjacent
        position tiles read overlapping input rows), its runs walking the tile rows of one column
        before the next: the convolution's fetch 64.9 -> 11.7 MB at the same 39 µs, and the step no
        faster, so it is not the default. None for the others."""
        mode = os.environ.get("ANVIL_GEMM_RUNS", "1")
        if mode == "0":
            return None
        if self.kslices > 1:
            return "split"
        if (mode == "all" and self.s.B == 1 and self.tn >= 8 * self.tm and self.tn * self.tm >= 16):
            return "wide"
        return None

    def tile_origin(self, runs=None) -> str:
        """m0, n0 of the workgroup's tile (and, for a K split in runs, zr_: its slice and batch
        index). A tall grid (tile rows ≥ 8 × tile columns: C4's 4096 x 256
        products) takes the XCD-aware order: in launch order, linear id mod 8 would be the tile
        column whenever the columns are a multiple of 8, so every XCD would read all of A (3-5 µs
        of 35 measured). Square grids measured faster in launch order (C2's weight gradients)."""
        tiles = self.tn * self.tm
        if runs == "split":
            return (f"    const int p_ = anvil_run_of(((int)blockIdx.z * {self.tm} + (int)blockIdx.y) * {self.tn} "
                    f"+ (int)blockIdx.x, {tiles * self.s.B * self.kslices});\n"
                    f"    const uint32_t zr_ = (uint32_t)(p_ / {tiles});\n"
                    f"    const int m0 = (p_ % {tiles}) / {self.tn} * {self.BM}, n0 = (p_ % {tiles}) % {self.tn} * {self.BN};")
        if runs == "wide":
            return (f"    const int p_ = anvil_run_of((int)blockIdx.y * {self.tn} + (int)blockIdx.x, {tiles});\n"
                    f"    const int m0 = (p_ % {self.tm}) * {self.BM}, n0 = (p_ / {self.tm}) * {self.BN};")
        mode = os.environ.get("ANVIL_GEMM_SWIZZLE", "1")
        if mode == "0" or self.tn * self.tm < 16 or (self.tm < 8 * self.tn and mode != "all"):
            return f"    const int m0 = blockIdx.y * {self.BM}, n0 = blockIdx.x * {self.BN};"
        G = int(os.environ.get("ANVIL_GEMM_SWIZZLE_ROWS", "8"))
        return (f"    int tx_, ty_;\n"
                f"    anvil_tile_of(blockIdx.y * {self.tn} + blockIdx.x, {self.tn}, {self.tm}, {G}, tx_, ty_);\n"
                f"    const int m0 = ty_ * {self.BM}, n0 = tx_ * {self.BN};")

    def k_table(self, which) -> str:
        """The file-scope table of an operand's k offsets (one int per k), when it has one."""
        tab = self.s.a_ktab if which == "a" else self.s.b_ktab
        if not tab:
            return ""
        body = ", ".join(str(x) for x in tab)
        return (f"static __device__ const int anvil_ktab_{self.name}_{which}[{len(tab)}] __attribute__((aligned(16))) "
                f"= {{{body}}};\n")

    def k_fn(self, name, which) -> str:
        """A device lambda: where k-index k of an operand starts (k·stride, or the offsets of the
        several K variables it decomposes into); for an operand with a table, an object that reads
        the table (one k, or four consecutive ones at once)."""
        s = self.s
        if (s.a_ktab if which == "a" else s.b_ktab):
            t = f"anvil_ktab_{self.name}_{which}"
            return "\n".join([
                "    struct {",
                f"        __device__ long long operator()(int k) const {{ return {t}[k]; }}",
                "        __device__ void quad(int k, long long (&o)[4]) const {",
                f"            const anvil_i32x4 q = *(const anvil_i32x4 *)({t} + k);",
                "            o[0] = q.x; o[1] = q.y; o[2] = q.z; o[3] = q.w;",
                "        }",
                f"    }} {name};"])
        if not s.k_multi:
            ks = s.a_ks if which == "a" else s.b_ks
            return f"    auto {name} = [=](int k) -> long long {{ return (long long)k * {ks}LL; }};"
        parts, rest = [], "k"
        for depth, (ext, sa, sb) in enumerate(reversed(s.k_multi)):
            st = sa if which == "a" else sb
            outer = depth == len(s.k_multi) - 1
            idx = rest if outer else f"({rest} % {ext})"
            if st:
                parts.append(f"{st}LL * (long long){idx}")
            rest = f"({rest} / {ext})"
        return f"    auto {name} = [=](int k) -> long long {{ return {' + '.join(parts) or '0LL'}; }};"

    def second(self):
        """The launch that adds the partial tiles of a K split across workgroups."""
        return GemmReducePlan(self)

    def ws_buffer(self):
        """The partial tiles of a K split across workgroups: [slice][batch][M][N] floats."""
        if not hasattr(self, "_ws"):
            s = self.s
            self._ws = A.new_buffer(800_000_000 + self.k.id, f"{self.name}.partials",
                                    (self.kslices * s.B * s.M * s.N,), F32, "scratch")
        return self._ws

    def epilogue(self, sc, loop, slot, value, hoisted, per):
        """The statements of the product's kernel and its followers for each of the lane's output
        elements (the loop), with acc = alpha · value; hoisted: loads issued before the K loop."""
        s, k = self.s, self.k
        stages = [(k, None, [])] + list(self.followers)

        def element_vars(em):
            for line in decode(s.m_vars, "(uint32_t)mi", "uint32_t"):
                em.emit(line)
            for line in decode(s.n_vars, "(uint32_t)ni", "uint32_t"):
                em.emit(line)
            for e, m, _ in self.followers:
                for ev, aff in m.items():
                    em.emit(f"const int v{ev.id} = (int)({em.affine(aff)});")
        pre = []
        if hoisted:
            pre.append("    " + " ".join(f"float pre{i}[{per}];" for i in range(len(hoisted))))
            pre += loop
            pl: list[str] = []
            pem = Emitter(sc, pl, "        ", prefix="p")
            element_vars(pem)
            for i, (si, ld) in enumerate(hoisted):
                pem.emit(f"pre{i}[{slot}] = {pem.build(ld)};")
            pre += pl + ["    }"]
        body = loop + [f"        const float acc_v = {flit(s.alpha)} * {value};"]
        lines: list[str] = []
        em = Emitter(sc, lines, "        ")
        element_vars(em)
        strides = ir.row_major_strides([v.extent for v in k.domain])
        sc.rand = " + ".join(f"{st}u * (uint32_t)v{v.id}" for v, st in zip(k.domain, strides)) or "0u"
        sc.acc_name = "acc_v"
        stored = {}

        def on_store(st, val):
            if not st.accumulate:                     # an addition leaves no value to forward
                stored[st.buf.root.id] = val
        for si, (e, m, fwd) in enumerate(stages):
            em.reset_memo()
            canon = {v: ("e", v.id) for v in e.domain}
            sc.canon = canon
            sc.fwd = {canon_key(ld.buf, ld.offset, canon): stored[ld.buf.root.id] for ld in fwd}
            for i, (sj, ld) in enumerate(hoisted):
                if sj == si:
                    sc.fwd[canon_key(ld.buf, ld.offset, canon)] = f"pre{i}[{slot}]"
            self.statements(em, e, sc, parallel=True, on_store=on_store)
        sc.canon, sc.fwd = None, {}
        return pre, body + lines + ["    }"]

    def source(self) -> str:
        s, k = self.s, self.k
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        a_ptr = sc.buf(s.la.buf)
        b_ptr = sc.buf(s.lb.buf)
        body = [self.operand(sc, s.ea, s.la, "opa"), self.operand(sc, s.eb, s.lb, "opb"),
                self.tile_origin(self.run_order()),
                "    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;"]
        ca, cb = s.la.offset.coef, s.lb.offset.coef
        a_off = [str(s.la.offset.const)]
        b_off = [str(s.lb.offset.const)]
        zsrc = "blockIdx.z"
        if self.kslices > 1:
            z = "zr_" if self.run_order() == "split" else "blockIdx.z"
            body.append(f"    const uint32_t slice = {z} % {self.kslices}u, bz = {z} / {self.kslices}u;")
            zsrc = "bz"
        if s.batch:
            body += ["    " + line for line in decode(s.batch, zsrc, "uint32_t")]
            for v in s.batch:
                if ca(v):
                    a_off.append(f"{ca(v)}LL * v{v.id}")
                if cb(v):
                    b_off.append(f"{cb(v)}LL * v{v.id}")
        body.append(f"    const float *pa = {a_ptr} + ({' + '.join(a_off)});")
        body.append(f"    const float *pb = {b_ptr} + ({' + '.join(b_off)});")
        args = f"pa, {s.a_rs}LL, {s.a_ks}LL, pb, {s.b_rs}LL, {s.b_ks}LL, {s.M}, {s.N}, m0, n0, 0, {s.K}, opa, opb"
        if self.sched == "tile":
            tm, tn = self.BM // 64, self.BN // 64
            per = tm * tn * 16
            loop = ["#pragma unroll", f"    for (int ti = 0; ti < {tm}; ti++)",
                    "#pragma unroll", f"    for (int tj = 0; tj < {tn}; tj++)",
                    "#pragma unroll", "    for (int vv = 0; vv < 16; vv++) {",
                    "        const int mi = m0 + wm + 32 * ti + 8 * (vv >> 2) + 4 * (lane >> 5) + (vv & 3);",
                    "        const int ni = n0 + wn + 32 * tj + (lane & 31);",
                    f"        if (mi >= {s.M} || ni >= {s.N}) continue;"]
            slot = f"(ti * {tn} + tj) * 16 + vv"
            body.append(f"    const int wm = (wave >> 1) * {self.BM // 2}, wn = (wave & 1) * {self.BN // 2};")
            main = [f"    anvil_mm_acc<{tm}, {tn}> acc;",
                    f"    anvil_mm_tile<{self.BM}, {self.BN}, {self.amode}, {self.bmode}>(acc, {args});"]
            value = "acc.c[ti][tj][vv]"
        else:
            W = self.waves
            TM, TN = self.ptm, self.ptn
            per = 16 // W
            if TM * TN == 1:
                loop = ["#pragma unroll", f"    for (int q = 0; q < {per}; q++) {{",
                        f"        const int vv = {per} * wave + q;",
                        "        const int mi = m0 + 8 * (vv >> 2) + 4 * (lane >> 5) + (vv & 3);",
                        "        const int ni = n0 + (lane & 31);",
                        f"        if (mi >= {s.M} || ni >= {s.N}) continue;"]
                slot = "q"
            else:
                loop = ["#pragma unroll", f"    for (int ijq = 0; ijq < {TM * TN * per}; ijq++) {{",
                        f"        const int ti = ijq / {TN * per}, tj = (ijq / {per}) % {TN}, q = ijq % {per};",
                        f"        const int vv = {per} * wave + q;",
                        "        const int mi = m0 + 32 * ti + 8 * (vv >> 2) + 4 * (lane >> 5) + (vv & 3);",
                        "        const int ni = n0 + 32 * tj + (lane & 31);",
                        f"        if (mi >= {s.M} || ni >= {s.N}) continue;"]
                slot = "ijq"
                per = TM * TN * per
            chk = lambda n, t=32: "true" if n % t else "false"
            if self.slab:
                kargs = (f"pa, {s.a_rs}LL, {s.a_ks}LL, pb, {s.b_rs}LL, {s.b_ks}LL, {s.M}, {s.N}, m0, n0, {s.K}, "
                         "opa, opb")
                main = [f"    float part[1][1][{per}];",
                        f"    anvil_mm_tile_kslab<{self.amode}, {self.bmode}, {self.slab}, {chk(s.M)}, {chk(s.N)}>"
                        f"(part, {kargs});"]
            elif self.pipe:
                body += [self.row_fn(sc, "arow", s.a_gather, s.a_rs, s.a_multi),
                         self.row_fn(sc, "brow", s.b_gather, s.b_rs, s.b_multi),
                         self.k_fn("ak", "a"), self.k_fn("bk", "b")]
                if self.kslices > 1:
                    krange = (f"(int)slice * {self.kslice}, min({self.kslice}, {s.K} - (int)slice * {self.kslice})")
                else:
                    krange = f"0, {s.K}"
                a_ks = s.a_ks if not s.k_multi else s.k_multi[-1][1]
                b_ks = s.b_ks if not s.k_multi else s.k_multi[-1][2]
                kargs = (f"pa, arow, ak, {a_ks}LL, pb, brow, bk, {b_ks}LL, {s.M}, {s.N}, m0, n0, {krange}, "
                         "opa, opb")
                G = self.kgroup
                nch = -(-(self.kslice // (8 * G)) // W)
                main = [f"    __shared__ float anvil_kp_lds[{W * TM * TN * 16 * 64}];",
                        f"    float part[{TM}][{TN}][{16 // W}];"]
                if getattr(self, "rowpro", None) is not None:
                    # A's rows computed here from the row chain's input (hip_rowpro)
                    main += self.rowpro.source(self, sc, W, TM, G, nch, chk(s.M, self.BM))
                    main.append(f"    anvil_mm_tile_kpipe_areg<{W}, {TM}, {TN}, {self.bmode}, {nch}, {min(self.depth, nch)}, "
                                f"{chk(s.N, self.BN)}, {G}, {self.chains}>(anvil_kp_lds, part, xa_, pb, brow, bk, "
                                f"{b_ks}LL, {s.N}, n0, opb);")
                else:
                    main.append(f"    anvil_mm_tile_kpipe<{W}, {TM}, {TN}, {self.amode}, {self.bmode}, {nch}, {min(self.depth, nch)}, "
                                f"{chk(s.M, self.BM)}, {chk(s.N, self.BN)}, {G}, {self.chains}>(anvil_kp_lds, part, {kargs});")
            else:
                main = [f"    float part[1][1][{per}];",
                        f"    anvil_mm_tile_ksplit<{W}, 1, 1, {self.amode}, {self.bmode}, {self.unroll}>(part, {args});"]
            value = "part[0][0][q]" if TM * TN == 1 else "part[ti][tj][q]"
        def head():                                   # after the body: its buffers are the parameters
            return [self.k_table("a") + self.k_table("b") + self.comment() + f" · {s.M}x{s.N}x{s.K}" + (f" x{s.B}" if s.B > 1 else "")
                    + f" · {self.sched} {self.BM}x{self.BN}, A {self.amode[9:]}, "
                    f"B {self.bmode[9:]}"
                    + (f" · K in {self.kslices} slices of {self.kslice}, partial tiles" if self.kslices > 1 else "")
                    + (f" · K over {len(s.k_multi)} variables" if s.k_multi else ""),
                    self.header(self.threads)]
        if self.kslices > 1:
            # partial tiles: GemmReducePlan adds them up and runs the epilogue, or (fixup) the last
            # workgroup of each tile to finish does, here
            ws = sc.buf(self.ws_buffer())
            store = loop + [f"        {ws}[(((long long)slice * {s.B} + bz) * {s.M} + mi) * {s.N} + ni] = {value};",
                            "    }"]
            if not getattr(self, "fixup", False):
                return "\n".join(head() + body + main + store + ["}"])
            S, cnt = self.kslices, f"anvil_cnt_{self.name}"
            fix = ["    // the tile's last workgroup to finish (its S partial tiles stored, made visible device-wide",
                   "    // before the count) adds them in slice order and runs the epilogue: the sum of the",
                   "    // partial-tile launch, without that launch; it sets the count back to 0 for the next one",
                   "    __shared__ int anvil_last_;",
                   f"    const int tile_ = ((int)bz * {self.tm} + m0 / {self.BM}) * {self.tn} + n0 / {self.BN};",
                   "    __threadfence();",
                   "    __syncthreads();",
                   f"    if (threadIdx.x == 0) anvil_last_ = atomicAdd(&{cnt}[tile_], 1u) == {S - 1}u;",
                   "    __syncthreads();",
                   "    if (!anvil_last_) return;",
                   "    __threadfence();",
                   "    auto fx_ = [&](int mi, int ni) -> float {",
                   "        float sum = 0.0f;",
                   f"        for (int sl = 0; sl < {S}; sl++) sum += {ws}[(((long long)sl * {s.B} + bz) * {s.M} + mi) * {s.N} + ni];",
                   "        return sum;",
                   "    };"]
            _, post = self.epilogue(sc, loop, slot, "fx_(mi, ni)", [], per)
            tail = [f"    if (threadIdx.x == 0) {cnt}[tile_] = 0u;"]
            decl = f"static __device__ unsigned {cnt}[{self.tn * self.tm * s.B}];   // finished slices per tile\n"
            text = "\n".join(head() + body + main + store + fix + post + tail + ["}"])
            return decl + text
        hoisted = []
        if per * 4 <= 64 and os.environ.get("ANVIL_GEMM_HOIST", "1") != "0":
            hoisted = self.hoistable([(k, None, [])] + list(self.followers))[:max(0, 64 // per)]
        pre, post = self.epilogue(sc, loop, slot, value, hoisted, per)
        return "\n".join(head() + body + pre + main + post + ["}"])


class OuterPlan(GemmPlan):
    """A product whose sum is too short for the matrix cores (K < MIN_K: C5's first convolution,
    one input channel, K = 3 x 3) with few rows (M ≤ OUTER_MAX_M: its 32 output channels) and many
    columns (N: its 128 x 26 x 26 output positions). One lane per column and group of OUTER_ROWS
    rows (the grid's y): it loads the column's K operands of B into registers, then for each row of
    its group sums the K products with that row of A in k order (the same addresses across the
    wavefront: scalar loads, a group's issued together) and runs the epilogue, the followers
    included. The column operand is read once per group and each result written once, a
    wavefront's 64 stores of one row contiguous when the columns are the output's innermost index;
    a row-per-lane map instead reloads the column's K operands for every row. (One lane per column
    and all 32 rows left C5's 86528 columns 1352 wavefronts for 1024 SIMDs: 9.3 µs.)"""

    def __init__(self, gen, k, name, spec: GemmSpec):
        Plan.__init__(self, gen, [k], name)
        self.k = k
        self.s = spec
        self.sched, self.BM, self.BN = "outer", spec.M, 1
        self.kslices, self.kslice = 1, spec.K
        self.waves, self.ptm, self.ptn = 4, 1, 1
        self.threads = 256
        self.forced = False
        self.followers = []
        self.rows = min(spec.M, int(os.environ.get("ANVIL_GEMM_OUTER_ROWS", OUTER_ROWS)))   # rows per lane
        self.tm, self.tn = -(-spec.M // self.rows), -(-spec.N // self.threads)

    def layout(self):
        pass

    def settle(self):
        pass

    def template_lds(self) -> int:
        return 0

    def grid(self):
        return (self.tn, self.tm, 1), self.threads

    def source(self) -> str:
        s, k = self.s, self.k
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        a_ptr = sc.buf(s.la.buf)
        b_ptr = sc.buf(s.lb.buf)
        body = [self.operand(sc, s.ea, s.la, "opa"), self.operand(sc, s.eb, s.lb, "opb"),
                f"    const float *pa = {a_ptr} + ({s.la.offset.const});",
                f"    const float *pb = {b_ptr} + ({s.lb.offset.const});",
                self.row_fn(sc, "arow", None, s.a_rs),
                self.row_fn(sc, "brow", s.b_gather, s.b_rs, s.b_multi),
                self.k_fn("ak", "a"), self.k_fn("bk", "b"),
                f"    const int ni = (int)(blockIdx.x * {self.threads}u + threadIdx.x);",
                f"    if (ni >= {s.N}) return;",
                f"    float bv[{s.K}];",
                "    {",
                "        const long long bo = brow(ni);",
                "#pragma unroll",
                f"        for (int kk = 0; kk < {s.K}; kk++) bv[kk] = opb(pb[bo + bk(kk)]);",
                "    }"]
        loop = ["#pragma unroll", f"    for (int r = 0; r < {self.rows}; r++) {{",
                f"        const int mi = (int)blockIdx.y * {self.rows} + r;"]
        if s.M % self.rows:
            loop.append(f"        if (mi >= {s.M}) continue;")
        loop += ["        const long long ao = arow(mi);",
                "        float acc = 0.0f;",
                "#pragma unroll",
                f"        for (int kk = 0; kk < {s.K}; kk++) acc += opa(pa[ao + ak(kk)]) * bv[kk];"]
        pre, post = self.epilogue(sc, loop, "0", "acc", [], 1)
        head = [self.k_table("a") + self.k_table("b") + self.comment() + f" · {s.M}x{s.N}x{s.K} · outer: one lane "
                f"per column and group of {self.rows} rows",
                self.header(self.threads)]
        return "\n".join(head + body + pre + post + ["}"])


class GemmReducePlan(Plan):
    """The second kernel of a K split across workgroups: for each output element, the S partial
    tiles added in slice order (the result does not depend on timing), then the product kernel's
    statements and its followers' (a weight update)."""

    kind = "gemm-reduce"

    def __init__(self, gemm: "GemmPlan"):
        super().__init__(gemm.gen, [], gemm.name + "r")
        self.gemm = gemm
        self.label = "partial-tile sum + " + gemm.label
        s = gemm.s
        self.total = s.B * s.M * s.N
        self.blocks = max(1, min(-(-self.total // 256), 1 << 16))
        self.streams = list(gemm.streams)

    def grid(self):
        return self.blocks, 256

    def source(self) -> str:
        g, s = self.gemm, self.gemm.s
        self.skip_stores = g.skip_stores
        sc = KernelScope(self)
        sc.stream_name = g.stream_param(g.k)
        ws = sc.buf(g.ws_buffer())
        body = [f"    for (uint32_t e = blockIdx.x * 256u + threadIdx.x; e < {self.total}u; e += gridDim.x * 256u) {{",
                f"        const uint32_t bz = e / {s.M * s.N}u;",
                f"        const int mi = (int)((e / {s.N}u) % {s.M}u), ni = (int)(e % {s.N}u);"]
        body += ["        " + line for line in decode(s.batch, "bz", "uint32_t")]
        body += ["        float sum = 0.0f;",
                 f"        for (int sl = 0; sl < {g.kslices}; sl++) "
                 f"sum += {ws}[(((long long)sl * {s.B} + bz) * {s.M} + mi) * {s.N} + ni];"]
        # the epilogue's statements, for this one element (its buffers become this kernel's)
        _, post = g.epilogue(sc, [], "0", "sum", [], 1)
        head = [f"// gemm-reduce: {g.name}: {g.kslices} partial tiles of {s.M}x{s.N}" + (f" x{s.B}" if s.B > 1 else "")
                + " added in order, then the epilogue", self.header(256)]
        return "\n".join(head + body + post[:-1] + ["    }", "}"])


def _key(ld):
    from .hip_kernels import canon_key
    return canon_key(ld.buf, ld.offset, {v: ("v", v.id) for v in ld.offset.terms})

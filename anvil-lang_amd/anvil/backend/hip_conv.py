"""Convolutions as implicit products: the im2col copy read through by the products that consume it.

The reference lowers a convolution (prelude.anvil's conv2d) to a copy kernel that lays the input's
windows out as rows, patches[n, i, j, c, u, v] = f(x[n, c, i+u, j+v]) (f: an activation of the
layer before, or nothing), and products over it: the forward Σ_cuv W[o, cuv]·patches[n, ij, cuv]
and the weight gradient Σ_{n, ij} dY[n, o, ij]·patches[n, ij, cuv]. The optimizer merges the
window's variables into one (ij, cuv), which the copy's row-major layout makes linear.

Here each such product reads x itself: its merged variables are split back into the copy's own
(ij into i, j; cuv into c, u, v: the same element order, so the same values), after which its
load of patches is exactly the copy's store, and the copy's value f(x[...]) takes its place. The
product then runs on the matrix cores with rows and k over several variables (hip_gemm.py: the
row offset of position (i, j) is 26i + j, not 24i + j), and when no reader of patches is left the
copy is not run at all: the 85 MB patches tensor of the CNN's second convolution is never written.
"""
from __future__ import annotations

import dataclasses
import os

from .. import ir
from ..ir import KernelStmt, Load, Var
from . import hip_analysis as A
from .hip_emit import flit
from .hip_kernels import KernelScope, Plan


def subst_affine(a: ir.Affine, m: dict) -> ir.Affine:
    """a with each variable in m replaced by its affine expression (gathers' index loads too)."""
    out = ir.Affine(a.const)
    for t, c in a.terms.items():
        if isinstance(t, Var) and t in m:
            out = out + m[t] * c
        elif isinstance(t, ir.Gather):
            g = ir.Gather(Load(t.load.buf, subst_affine(t.load.offset, m)), t.bound, t.where,
                          None if t.rest is None else subst_affine(t.rest, m))
            out = out + ir.Affine(0, {g: c})
        else:
            out = out + ir.Affine(0, {t: c})
    return out


def subst_expr(e, m: dict):
    def fn(x):
        if isinstance(x, Load):
            return Load(x.buf, subst_affine(x.offset, m))
        if isinstance(x, ir.Index):
            return ir.Index(subst_affine(x.affine, m))
        return x
    return ir.map_expr(e, fn)


def split_vars(k: ir.Kernel, splits: dict) -> ir.Kernel:
    """k with each variable t in splits replaced by the list of variables splits[t] (outer to inner,
    extents multiplying to t's): t = their row-major index, in the domain or reduction alike."""
    m = {}
    for t, parts in splits.items():
        aff = ir.Affine(0)
        for v, st in zip(parts, ir.row_major_strides([p.extent for p in parts])):
            aff = aff + ir.Affine(0, {v: st})
        m[t] = aff

    def expand(vs):
        out = []
        for v in vs:
            out.extend(splits.get(v, [v]))
        return out
    lets: dict = {}

    def fix(e):
        def fn(x):
            if isinstance(x, ir.LetRef) and id(x.let) in lets:
                return ir.LetRef(lets[id(x.let)])
            return x
        return ir.map_expr(subst_expr(e, m), fn)
    stmts = []
    for st in k.stmts:
        if isinstance(st, ir.Let):
            new = dataclasses.replace(st, value=fix(st.value))
            lets[id(st)] = new
        else:
            new = dataclasses.replace(st, offset=subst_affine(st.offset, m), value=fix(st.value))
        stmts.append(new)
    red = k.red
    if red is not None:
        red = dataclasses.replace(red, vars=expand(red.vars), body=fix(red.body))
    return dataclasses.replace(k, domain=expand(k.domain), red=red, stmts=stmts)


def im2col_copy(st):
    """(kernel, patches buffer, value expression, its one load) for a copy kernel that fills a
    whole buffer row-major over its domain with an elementwise function of one plain load."""
    if not isinstance(st, KernelStmt):
        return None
    k = st.kernel
    if k.red is not None or len(k.stmts) != 1 or not isinstance(k.stmts[0], ir.Store) or not k.domain:
        return None
    store = k.stmts[0]
    if store.accumulate or k.uses_rand() or not A.parallel_safe(k) or store.buf.dtype != ir.F32:
        return None
    strides = ir.row_major_strides([v.extent for v in k.domain])
    want = ir.Affine(0, {v: s for v, s in zip(k.domain, strides) if v.extent > 1})
    # a variable of extent 1 (C5's single input channel) is always 0, whatever its coefficient
    got = ir.Affine(store.offset.const, {t: c for t, c in store.offset.terms.items()
                                         if not (isinstance(t, Var) and t.extent == 1)})
    if got != want or store.buf.root.numel != ir.prod(v.extent for v in k.domain):
        return None
    loads = ir.loads_in(store.value)
    if len(loads) != 1 or any(not isinstance(t, Var) for t in loads[0].offset.terms):
        return None
    if any(not isinstance(x, (ir.Const, ir.Unary, ir.Binary, Load)) for x in ir.iter_expr(store.value)):
        return None
    return k, store.buf.root, store.value, loads[0]


def rewrite(c: ir.Kernel, cp, ids):
    """c reading the copy's source in place of patches, or None (c is left as it is)."""
    from . import hip_gemm
    pk, dst, value, src = cp
    if c.red is None or c.red.op != "sum":
        return None
    if any(ld.buf.root is dst for st in c.stmts for ld in ir.loads_in(st.value)):
        return None
    if any(st.buf.root in (dst, src.buf.root) for st in c.stores):
        return None
    uses = [ld for ld in ir.loads_in(c.red.body) if ld.buf.root is dst]
    if len(uses) != 1:
        return None
    off = uses[0].offset
    if off.const or any(not isinstance(t, Var) for t in off.terms):
        return None
    strides = ir.row_major_strides([v.extent for v in pk.domain])
    pos = {s: i for i, (v, s) in enumerate(zip(pk.domain, strides)) if v.extent > 1}
    splits, pmap, used = {}, {}, set()
    for t, coef in off.terms.items():
        i = pos.get(coef)
        if i is None:
            return None
        run, span = [pk.domain[i]], pk.domain[i].extent
        while span < t.extent and i > 0:                  # a merged variable: the copy's vars it spans
            i -= 1
            run.insert(0, pk.domain[i])
            span *= pk.domain[i].extent
        if (span != t.extent if len(run) > 1 else span < t.extent) or any(id(v) in used for v in run):
            return None
        used.update(id(v) for v in run)
        if len(run) == 1:
            pmap[run[0]] = ir.Affine.of(t)
        else:
            parts = [A.new_var(ids.take(), v.name, v.extent) for v in run]
            splits[t] = parts
            for v, p in zip(run, parts):
                pmap[v] = ir.Affine.of(p)
    for v in pk.domain:
        pmap.setdefault(v, ir.Affine(0))
    c2 = split_vars(c, splits) if splits else c
    new_src = Load(src.buf, subst_affine(src.offset, pmap))
    operand = ir.map_expr(value, lambda x: new_src if x is src else x)

    def fn(x):
        return operand if isinstance(x, Load) and x.buf.root is dst else x
    c3 = dataclasses.replace(c2, red=dataclasses.replace(c2.red, body=ir.map_expr(c2.red.body, fn)))
    s = hip_gemm.analyse(c3)
    # a matrix-core product, or a short sum (K < MIN_K) that each lane adds up itself: either way the
    # window is read in place of the copy
    if s is None or not (hip_gemm.qualifies(s) or s.K < hip_gemm.MIN_K):
        return None
    return c3


def forward_im2col_copies(prog: ir.Program, ids) -> ir.Program:
    """Each product that reads an im2col copy's output reads the copy's source instead (see the
    module docstring), when every reader of the copy's output can, and the copy is dropped. (One
    product left reading patches keeps the copy, and then the products over patches, with one
    linear k, are the better ones.)"""
    rewritten: list = []
    readers = A.all_readers(prog)

    def block(blk: ir.Block) -> ir.Block:
        out = [stmt(st) for st in blk.stmts]
        for i, st in enumerate(out):
            cp = im2col_copy(st)
            if cp is None or cp[1].kind not in A.SHARED_KINDS:
                continue
            pk, dst, _, src = cp
            guard = {dst.id, src.buf.root.id}
            new = {}
            for j in range(i + 1, len(out)):
                s2 = out[j]
                if isinstance(s2, ir.If) and not A.block_writes(s2.then) and not A.block_writes(s2.orelse):
                    if guard & {b.id for b in A.stmt_reads(s2)}:
                        break
                    continue                              # a print, a loop exit: writes nothing
                if not isinstance(s2, KernelStmt):
                    break
                c = s2.kernel
                if dst.id in {x.id for x in A.kernel_reads(c)}:
                    k2 = rewrite(c, cp, ids)
                    if k2 is None:
                        break
                    new[j] = dataclasses.replace(s2, kernel=k2)
                if guard & {x.id for x in A.kernel_writes(c)}:
                    break
            if new and len(new) == readers.get(dst.id, 0):
                for j, s2 in new.items():
                    out[j] = s2
                rewritten.append(dst)
        return dataclasses.replace(blk, stmts=out)

    def stmt(st):
        if isinstance(st, ir.For):
            return dataclasses.replace(st, body=block(st.body))
        if isinstance(st, ir.While):
            return dataclasses.replace(st, cond_block=block(st.cond_block), body=block(st.body))
        if isinstance(st, ir.If):
            return dataclasses.replace(st, then=block(st.then), orelse=block(st.orelse))
        return st
    prog = dataclasses.replace(prog, main=block(prog.main))
    if not rewritten:
        return prog
    readers = A.all_readers(prog)
    dead = {b.id for b in rewritten if not readers.get(b.id) and b.kind in A.SHARED_KINDS}

    def drop(blk: ir.Block) -> ir.Block:
        keep = []
        for st in blk.stmts:
            if isinstance(st, KernelStmt) and im2col_copy(st) is not None and im2col_copy(st)[1].id in dead:
                continue
            keep.append(drop_in(st))
        return dataclasses.replace(blk, stmts=keep)

    def drop_in(st):
        if isinstance(st, ir.For):
            return dataclasses.replace(st, body=drop(st.body))
        if isinstance(st, ir.While):
            return dataclasses.replace(st, cond_block=drop(st.cond_block), body=drop(st.body))
        if isinstance(st, ir.If):
            return dataclasses.replace(st, then=drop(st.then), orelse=drop(st.orelse))
        return st
    return dataclasses.replace(prog, main=drop(prog.main))


# ----------------------------------------------------------------------------- the input gradient

def _acc_store(k: ir.Kernel):
    """k's one statement, a store of its sum (no epilogue), into a buffer it fills row-major."""
    if k.red is None or k.red.op != "sum" or len(k.stmts) != 1 or not isinstance(k.stmts[0], ir.Store):
        return None
    st = k.stmts[0]
    if st.accumulate or not isinstance(st.value, ir.Acc):
        return None
    strides = ir.row_major_strides([v.extent for v in k.domain])
    want = ir.Affine(0, {v: s for v, s in zip(k.domain, strides) if v.extent > 1})
    if st.offset != want or st.buf.root.numel != ir.prod(v.extent for v in k.domain):
        return None
    return st


def _zero_fill(k: ir.Kernel, buf) -> bool:
    """Does k set every element of buf to 0 (and do nothing else)?"""
    if k.red is not None or len(k.stmts) != 1 or not isinstance(k.stmts[0], ir.Store) or not k.domain:
        return False
    st = k.stmts[0]
    if st.buf.root is not buf or st.accumulate or not isinstance(st.value, ir.Const) or float(st.value.value) != 0.0:
        return False
    strides = ir.row_major_strides([v.extent for v in k.domain])
    want = ir.Affine(0, {v: s for v, s in zip(k.domain, strides) if v.extent > 1})
    return st.offset == want and buf.numel == ir.prod(v.extent for v in k.domain)


def _digits(vs, src: str) -> dict:
    """C expressions of each variable's digit of the row-major index src over vs (outer to inner)."""
    out, rest = {}, f"(uint32_t)({src})"
    for depth, v in enumerate(reversed(vs)):
        out[v] = rest if depth == len(vs) - 1 else f"({rest} % {v.extent}u)"
        rest = f"({rest} / {v.extent}u)"
    return out


def _offset_fn(vs, coef, src: str) -> str:
    d = _digits(vs, src)
    parts = [f"{coef(v)}LL * (long long){d[v]}" for v in vs if coef(v)]
    return " + ".join(parts) or "0LL"


# the largest operand copied for an input gradient (floats): a copy of at most 1 MB beside the launch
# before the product
PACK_MAX = 1 << 18


class PackPlan(Plan):
    """The first operand of an input gradient's product copied in the order the product reads it:
    dst[t, k] = W[row(t) + k(k)], t over the product's rows (the input channels), k over (u, v, o)
    in the product's k order. It runs in the launch before the product (side by side with it when
    that launch does not write W, else alone), so it copies W as the product would have read it."""

    kind = "pack"

    def __init__(self, gen, dgrad, src, dst, off2):
        super().__init__(gen, [], f"k{dgrad.G.id}p")
        self.dgrad, self.src, self.dst, self.off2 = dgrad, src, dst, off2
        self.total = dgrad.M * dgrad.K
        self.threads = 256
        self.label = f"operand copy: {dgrad.G.name}'s weights in k order"

    def with_threads(self, threads):
        """The same copy with `threads` lanes per workgroup (to run beside a launch of that size)."""
        q = PackPlan(self.gen, self.dgrad, self.src, self.dst, self.off2)
        q.threads = threads
        return q

    def grid(self):
        from .hip_kernels import MAX_BLOCKS
        return max(1, min(-(-self.total // self.threads), MAX_BLOCKS)), self.threads

    def source(self) -> str:
        d, off2 = self.dgrad, self.off2
        row = _offset_fn(d.rows[0], off2.coef, "t")
        kof = _offset_fn(d.korder, off2.coef, "k")
        t = self.threads
        return "\n".join([
            f"// pack: the weights of {d.G.name} as rows of its {d.K} k · {d.M}x{d.K}",
            self.header(t),
            f"    for (uint32_t w = (uint32_t)blockIdx.x * {t}u + threadIdx.x; w < {self.total}u; "
            f"w += (uint32_t)gridDim.x * {t}u) {{",
            f"        const uint32_t t = w / {d.K}u, k = w % {d.K}u;",
            f"        {self.use_buf(self.dst)}[w] = {self.use_buf(self.src.root)}[{off2.const}LL + {row} + {kof}];",
            "    }",
            "}"])


def match_dgrad(gen, stmts: list, i: int):
    """(DgradPlan, statements it takes) for a product that fills im2col-shaped gradients
    dP[n, i, j, c, u, v] = Σ_o dY[n, o, i, j]·W[o, c, u, v], an optional zero fill of dX, and the
    scatter dX[n, c, i+u, j+v] += dP[...] that is dP's only reader; else None."""
    from . import hip_gemm
    from .hip_kernels import scatter_targets
    if gen.emulate or gen.check or os.environ.get("ANVIL_HIP_DGRAD", "1") == "0":
        return None
    if i + 1 >= len(stmts) or not isinstance(stmts[i], KernelStmt):
        return None
    G = stmts[i].kernel
    gst = _acc_store(G)
    if gst is None:
        return None
    dP = gst.buf.root
    if dP.kind not in A.SHARED_KINDS or gen.readers.get(dP.id, 0) != 1:
        return None
    s = hip_gemm.analyse(G)
    if s is None:
        return None
    zero, j = None, i + 1
    if (j + 1 < len(stmts) and isinstance(stmts[j], KernelStmt) and isinstance(stmts[j + 1], KernelStmt)
            and stmts[j].kernel.stores and not stmts[j].kernel.red):
        zero = stmts[j].kernel
        j += 1
    if not isinstance(stmts[j], KernelStmt):
        return None
    S = stmts[j].kernel
    if (len(S.stmts) != 1 or not isinstance(S.stmts[0], ir.Store) or not isinstance(S.stmts[0].value, Load)
            or S.stmts[0].value.buf.root is not dP):
        return None
    sst = S.stmts[0]
    dX = sst.buf.root
    scat = scatter_targets(S)
    if scat is None or dX.id in {b.id for b in A.kernel_reads(G)}:
        return None
    targets, summed = scat
    if zero is not None and (not _zero_fill(zero, dX) or ir.prod(t[1] for t in targets) != dX.numel):
        return None                                   # the fill is absorbed only if every element is a target
    # dP's element as S reads it, in G's variables: each of G's (merged) variables is a mixed-radix
    # number over S's variables
    loff = sst.value.offset
    if loff.const or any(not isinstance(t, Var) for t in loff.terms):
        return None
    gmap, claimed = {}, set()
    for g, st_g in zip(G.domain, ir.row_major_strides([v.extent for v in G.domain])):
        mine = sorted([v for v in S.domain if v.extent > 1 and st_g <= loff.coef(v) < st_g * g.extent
                       and loff.coef(v) % st_g == 0], key=lambda v: loff.coef(v))
        span, aff = 1, ir.Affine(0)
        for v in mine:
            if loff.coef(v) != st_g * span:
                return None
            aff = aff + ir.Affine(0, {v: span})
            span *= v.extent
        if span != g.extent and g.extent > 1:
            return None
        gmap[g] = aff
        claimed.update(id(v) for v in mine)
    if any(v.extent > 1 and id(v) not in claimed for v in S.domain):
        return None
    # the target coordinates: a solved variable i = y - u (others of its group)
    tvars, rmap, preds = [], {}, []
    for c, ext, members, solved in targets:
        if solved is None:
            tvars.append((members[0], c))
            continue
        y = A.new_var(gen.ids.take(), f"{solved.name}+", ext)
        tvars.append((y, c))
        rmap[solved] = ir.Affine.of(y) - sum((ir.Affine.of(m) for m in members if m is not solved), ir.Affine(0))
        preds.append((solved, y, [m for m in members if m is not solved]))
    ops = []
    for e, ld in ((s.ea, s.la), (s.eb, s.lb)):
        off1 = subst_affine(ld.offset, gmap)
        if off1.gathers() or off1.scalars():
            return None
        off2 = subst_affine(off1, rmap)
        ops.append((e, ld, off1, off2))
    # which operand each coordinate, each k variable and each window check belongs to
    side_pred = {0: [], 1: []}
    for solved, y, others in preds:
        users = [n for n in (0, 1) if ops[n][2].coef(solved)]
        if len(users) != 1:
            return None
        side_pred[users[0]].append((solved, y, others))
    rows = {0: [], 1: []}
    for tv, c in sorted(tvars, key=lambda t: -abs(t[1])):
        users = {n for n in (0, 1) if ops[n][3].coef(tv)} | {n for n in (0, 1) for _, y, _ in side_pred[n] if y is tv}
        if len(users) != 1:
            return None
        rows[users.pop()].append(tv)
    if not rows[0] or not rows[1]:
        return None
    innermost = min(tvars, key=lambda t: abs(t[1]))[0]
    if innermost in rows[0]:                        # lanes step along dX's contiguous coordinate
        ops.reverse()
        rows = {0: rows[1], 1: rows[0]}
        side_pred = {0: side_pred[1], 1: side_pred[0]}
    kv = list(summed) + list(G.red.vars)
    in_pred = {id(m) for n in (0, 1) for _, _, others in side_pred[n] for m in others}
    coefs = lambda v: (ops[0][3].coef(v), ops[1][3].coef(v))
    fit = [v for v in kv if v.extent % 4 == 0 and id(v) not in in_pred and any(coefs(v))]
    if not fit or any(not any(coefs(v)) and id(v) not in in_pred for v in kv):
        return None
    inner = min(fit, key=lambda v: (min(abs(c) for c in coefs(v) if c), v.id))
    korder = sorted([v for v in kv if v is not inner], key=lambda v: (-max(abs(c) for c in coefs(v)), v.id)) + [inner]
    M = ir.prod(v.extent for v in rows[0])
    N = ir.prod(v.extent for v in rows[1])
    K = ir.prod(v.extent for v in kv)
    if K % 8 or M < 8 or N < 32 or M * N * K < hip_gemm.MIN_WORK:
        return None
    plan = DgradPlan(gen, [G] + ([zero] if zero is not None else []) + [S], f"k{G.id}", G, S, zero is not None,
                     s.alpha, ops, rows, korder, side_pred, tvars, sst, M, N, K)
    used = j + 1 - i
    # every element of dX is computed here (so the follower meets each one), at its row-major index
    covered = ((zero is not None or ir.prod(t[1] for t in targets) == dX.numel) and not sst.offset.const)
    if (covered and i + used < len(stmts) and isinstance(stmts[i + used], KernelStmt)
            and os.environ.get("ANVIL_HIP_MAP_FUSE", "1") != "0"):
        fwd = dgrad_follower(gen, plan, stmts[i + used].kernel, dX)
        if fwd is not None:
            plan.follow(stmts[i + used].kernel, fwd)
            used += 1
    return plan, used


def dgrad_follower(gen, plan, e: ir.Kernel, dX):
    """The loads of dX of elementwise kernel e, if e can run in the input gradient's epilogue
    element by element (ReLU's gradient after a convolution's: dZ = dX·(z > 0)): e walks dX's
    elements in row-major order, reads dX only at its own element, and neither writes what the
    product reads or writes nor reads anything else it writes; else None."""
    if (e.red is not None or e.uses_rand() or A.is_host_kernel(e, gen.hosts) or not A.parallel_safe(e)
            or any(st.accumulate for st in e.stores) or ir.prod(v.extent for v in e.domain) != dX.numel):
        return None
    lin = ir.Affine(0)
    for v, st in zip(e.domain, ir.row_major_strides([v.extent for v in e.domain])):
        lin = lin + ir.Affine(0, {v: st})
    fwd = []
    for ld in A.kernel_loads(e):
        if ld.buf.root is dX:
            if ld.offset != lin:
                return None
            fwd.append(ld)
    if not fwd:
        return None
    product_io = {b.id for k in plan.kernels for b in A.kernel_reads(k)} | {dX.id}
    if {b.id for b in A.kernel_writes(e)} & product_io:
        return None
    return fwd


class DgradPlan(Plan):
    """A convolution's input gradient in one pass over the matrix cores, without its im2col-shaped
    intermediate: dX[n, c, y, x] (+)= Σ_{u, v, o} W[o, c, u, v]·dY[n, o, y-u, x-v], K running over the
    window and the output channels; a window position that hangs over dY's edge (y-u outside
    0..23) is not loaded and counts as zero, which is exactly the scatter's missing term. Each output
    element is written once, by the lane that owns it (no atomics); when the zero fill of dX was part
    of the run, the sum is stored over it. The terms add in the matrix cores' order rather than the
    scatter's, as any product's do."""

    kind = "conv-dgrad"

    def __init__(self, gen, kernels, name, G, S, zeroed, alpha, ops, rows, korder, side_pred, tvars, sst, M, N, K):
        super().__init__(gen, kernels, name)
        self.G, self.S, self.zeroed, self.alpha = G, S, zeroed, alpha
        self.ops, self.rows, self.korder, self.side_pred = ops, rows, korder, side_pred
        self.tvars, self.sst, self.M, self.N, self.K = tvars, sst, M, N, K
        self.skip_stores = {(k.id, 0) for k in kernels if k is not S}     # dP is never written; dX once
        # W wavefronts splitting K, each with TM x TN 32 x 32 tiles ($ANVIL_DGRAD_TILES = "W:TM:TN"):
        # four with 1 x 2 measured best on C5 (50.8 µs; 1 x 1: 63.8, 1 x 4: 55.7, two waves of 1 x 2:
        # 58.5), each weight load serving two tiles of positions
        W, TM, TN = (int(x) for x in os.environ.get("ANVIL_DGRAD_TILES", "4:1:2").split(":"))
        if M < 32 * TM or N < 32 * TN:
            W, TM, TN = 4, 1, 1
        self.W, self.TM, self.TN = W, TM, TN
        self.tm, self.tn = -(-M // (32 * TM)), -(-N // (32 * TN))
        # k in chunks of 8·kg per wavefront, `depth` chunks of loads in flight ($ANVIL_DGRAD_KG,
        # $ANVIL_DGRAD_DEPTH)
        kg = int(os.environ.get("ANVIL_DGRAD_KG", "1"))
        if K % (8 * kg * W):
            kg = 1
        nch = -(-(K // (8 * kg)) // W)
        depth = int(os.environ.get("ANVIL_DGRAD_DEPTH", "0")) or (2 if nch <= 32 else 4)
        self.kg, self.nch, self.depth = kg, nch, min(depth, nch)
        self.follower, self.fwd, self.dx_dead = None, [], False
        self.pack = self.make_pack()

    def make_pack(self):
        """A PackPlan for the first operand (the weights, W[o, c, u, v] read as A[c, (u, v, o)]:
        each lane's four consecutive k lie 288 floats apart and the lanes 9 apart) when it is an
        f32 buffer read without a window check and small: the product then reads 4 consecutive k
        with one 16-byte load from the packed copy A[c, k] (a timing copy with the rows read that
        way: C5 192 -> 185 us per step). $ANVIL_DGRAD_PACK=0 reads the weights in place."""
        e, ld, off1, off2 = self.ops[0]
        b = ld.buf.root
        if (os.environ.get("ANVIL_DGRAD_PACK", "1") == "0" or self.side_pred[0] or b.dtype != "f32"
                or self.K % 4 or self.M * self.K > PACK_MAX or off2.gathers() or off2.scalars()):
            return None
        buf = A.new_buffer(self.gen.ids.take(), f"{b.name}.packed", (self.M, self.K), "f32", "scratch")
        return PackPlan(self.gen, self, ld.buf, buf, off2)

    def follow(self, e, fwd):
        """Run elementwise kernel e (which reads dX only at its own element) on each dX element as
        it is computed; dX itself is then not stored unless something else reads it."""
        dX = self.sst.buf.root
        self.follower, self.fwd = e, fwd
        self.kernels.append(e)
        self.label += " + " + (e.label or e.name)
        inside = sum(1 for k in self.kernels if dX.id in {b.id for b in A.kernel_reads(k)})
        self.dx_dead = (dX.kind in A.SHARED_KINDS and not self.gen.is_host(dX) and not getattr(dX, "heap", False)
                        and self.gen.readers.get(dX.id, 0) == inside)

    def hoistable(self):
        """The follower's plain loads of buffers it does not write, other than dX (at most two)."""
        if self.follower is None:
            return []
        e, out, seen = self.follower, [], set()
        fwd = {id(ld) for ld in self.fwd}
        written = {b.id for b in A.kernel_writes(e)}
        for ld in A.kernel_loads(e):
            if (id(ld) in fwd or ld.buf.root.id in written or not ld.buf.root.shape or ld.offset.gathers()
                    or ld.offset.scalars()):
                continue
            key = (ld.buf.root.id, ld.offset.key() if hasattr(ld.offset, "key") else repr(ld.offset))
            if key not in seen:
                seen.add(key)
                out.append(ld)
        return out[:2]

    def grid(self):
        return (self.tn, self.tm, 1), 64 * self.W

    def source(self) -> str:
        from . import hip_gemm
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(self.G)
        body = []
        names = ("a", "b")
        for n in (0, 1):
            e, ld, off1, off2 = self.ops[n]
            body.append(hip_gemm.GemmPlan.operand(self, sc, e, ld, f"op{names[n]}"))
        W, TM, TN = self.W, self.TM, self.TN
        body += [f"    const int m0 = blockIdx.y * {32 * TM}, n0 = blockIdx.x * {32 * TN};"]
        for n in (0, 1):
            e, ld, off1, off2 = self.ops[n]
            if n == 0 and self.pack is not None:                 # row t of the packed copy: K floats
                body += [f"    const float *pa = {sc.buf(self.pack.dst)};",
                         f"    auto arow = [=](int t) -> long long {{ return {self.K}LL * (long long)(uint32_t)(t); }};",
                         "    auto ak = [=](int k) -> long long { return (long long)(uint32_t)(k); };",
                         "    anvil_all_pred apred;"]
                continue
            body.append(f"    const float *p{names[n]} = {sc.buf(ld.buf)} + ({off2.const}LL);")
            body.append(f"    auto {names[n]}row = [=](int t) -> long long {{ return "
                        f"{_offset_fn(self.rows[n], off2.coef, 't')}; }};")
            body.append(f"    auto {names[n]}k = [=](int k) -> long long {{ return "
                        f"{_offset_fn(self.korder, off2.coef, 'k')}; }};")
            checks = []
            if self.side_pred[n]:
                td, kd = _digits(self.rows[n], "t"), _digits(self.korder, "k")
                for solved, y, others in self.side_pred[n]:
                    diff = " - ".join([f"(int){td[y]}"] + [f"(int){kd[m]}" for m in others])
                    checks.append(f"(unsigned)({diff}) < {solved.extent}u")
            if checks:
                body.append(f"    auto {names[n]}pred = [=](int t, int k) -> bool {{ return {' && '.join(checks)}; }};")
            else:
                body.append(f"    anvil_all_pred {names[n]}pred;")
        inner = self.korder[-1]
        a_ks, b_ks = self.ops[0][3].coef(inner), self.ops[1][3].coef(inner)
        amode = "ANVIL_LD_ANY"
        if self.pack is not None:
            a_ks, amode = 1, "ANVIL_LD_KC"
        chk = lambda x, t: "true" if x % t else "false"
        per = 16 // W
        # the follower's other loads (ReLU's z at the element) are issued before the product
        elem = ["#pragma unroll",
                f"    for (int ijq = 0; ijq < {TM * TN * per}; ijq++) {{",
                f"        const int ti = ijq / {TN * per}, tj = (ijq / {per}) % {TN}, q = ijq % {per};",
                f"        const int vv = {per} * wave + q;",
                "        const int mi = m0 + 32 * ti + 8 * (vv >> 2) + 4 * (lane >> 5) + (vv & 3);",
                "        const int ni = n0 + 32 * tj + (lane & 31);",
                f"        if (mi >= {self.M} || ni >= {self.N}) continue;"]
        dm, dn = _digits(self.rows[0], "mi"), _digits(self.rows[1], "ni")
        out = [str(self.sst.offset.const)] if self.sst.offset.const else []
        for tv, c in self.tvars:
            d = dm.get(tv, dn.get(tv))
            out.append(f"{c}LL * (long long){d}")
        hoisted = self.hoistable()
        if hoisted:
            from .hip_kernels import decode
            from .hip_emit import Emitter
            e = self.follower
            body.append("    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;")
            body.append("    " + " ".join(f"float pre{h}[{TM * TN * per}];" for h in range(len(hoisted))))
            body += elem
            body.append(f"        const uint32_t lin_ = (uint32_t)({' + '.join(out) or '0'});")
            pl: list[str] = []
            pem = Emitter(sc, pl, "        ", prefix="p")
            for line in decode(e.domain, "lin_", "uint32_t"):
                pem.emit(line)
            for h, ld in enumerate(hoisted):
                pem.emit(f"pre{h}[ijq] = {pem.build(ld)};")
            body += pl + ["    }"]
        body += [f"    __shared__ float anvil_kp_lds[{W * TM * TN * 16 * 64}];",
                 f"    float part[{TM}][{TN}][{per}];",
                 f"    anvil_mm_tile_kpipe<{W}, {TM}, {TN}, {amode}, ANVIL_LD_ANY, {self.nch}, {self.depth}, "
                 f"{chk(self.M, 32 * TM)}, {chk(self.N, 32 * TN)}, {self.kg}>(anvil_kp_lds, part, pa, arow, ak, {a_ks}LL, pb, brow, bk, "
                 f"{b_ks}LL, {self.M}, {self.N}, m0, n0, 0, {self.K}, opa, opb, apred, bpred);"]
        if not hoisted:
            body.append("    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;")
        body += elem
        target = f"{sc.buf(self.sst.buf)}[{' + '.join(out)}]"
        base = "0.0f" if self.zeroed else target
        if self.follower is None:
            body.append(f"        {target} = {base} + {flit(self.alpha)} * part[ti][tj][q];")
        else:
            from .hip_kernels import canon_key, decode
            from .hip_emit import Emitter
            e = self.follower
            body.append(f"        const float dx_ = {base} + {flit(self.alpha)} * part[ti][tj][q];")
            if not self.dx_dead:
                body.append(f"        {target} = dx_;")
            body.append(f"        const uint32_t lin_ = (uint32_t)({' + '.join(out) or '0'});")
            lines: list[str] = []
            em = Emitter(sc, lines, "        ")
            for line in decode(e.domain, "lin_", "uint32_t"):
                em.emit(line)
            canon = {v: ("e", v.id) for v in e.domain}
            sc.canon = canon
            sc.fwd = {canon_key(ld.buf, ld.offset, canon): "dx_" for ld in self.fwd}
            for h, ld in enumerate(hoisted):
                sc.fwd[canon_key(ld.buf, ld.offset, canon)] = f"pre{h}[ijq]"
            self.statements(em, e, sc, parallel=True)
            sc.canon, sc.fwd = None, {}
            body += lines
        body.append("    }")
        head = [f"// conv-dgrad: {self.G.name} (product into an im2col-shaped gradient) and {self.S.name} (its "
                f"scatter) as one product · {self.M}x{self.N}x{self.K}, window terms over the edge skipped"
                + (f", the weights from their packed copy ({self.pack.name})" if self.pack is not None else ""),
                self.header(64 * W)]
        return "\n".join(head + body + ["}"])

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

from .. import ir
from ..ir import KernelStmt, Load, Var
from . import hip_analysis as A


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
    if store.offset != want or store.buf.root.numel != ir.prod(v.extent for v in k.domain):
        return None
    loads = ir.loads_in(store.value)
    if len(loads) != 1 or any(not isinstance(t, Var) for t in loads[0].offset.terms):
        return None
    if any(not isinstance(x, (ir.Const, ir.Unary, ir.Binary, Load)) for x in ir.iter_expr(store.value)):
        return None
    return k, store.buf.root, store.value, loads[0]


def rewrite(c: ir.Kernel, cp):
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
            parts = [Var(v.name, v.extent) for v in run]
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
    if s is None or not hip_gemm.qualifies(s):
        return None
    return c3


def forward_im2col_copies(prog: ir.Program) -> ir.Program:
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
                    k2 = rewrite(c, cp)
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

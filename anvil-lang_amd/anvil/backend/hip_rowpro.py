"""Row statistics computed in the product that reads them: a layer norm's kernels folded into the
prologue of the matrix product whose A operand is the normalized rows.

The reference's layer norm (prelude `layer_norm`, lowered by the front end) is a chain of kernels
over the R rows of a matrix x of width D: reductions over a row (the mean, then the variance
around it), then an elementwise kernel that writes y[r, j] from x[r, j] and those row values;
the next kernel multiplies y by a weight matrix (C4: y·Wqkv and y·W1 after each layer's norms,
y·Wout after the last). Run as written, the chain is a launch of its own (4096 rows of 256 in
about 5 µs, most of it the launch) whose output the product then reads back.

Here the product's workgroups compute y themselves. A product with K = D reads whole rows of y
as its A operand, so a workgroup that owns rows m0 .. m0 + 32·TM − 1 loads those rows of x
instead (the same bytes), sums each row's reduction terms over its four wavefronts (each holds a
quarter of every row: the K split's own layout), and evaluates the elementwise kernel on the
registers, which then feed the matrix cores with no A loads in the K loop. The workgroups of the
first tile column also store y and the row values, for the kernels that read them later (the
backward); the others only use them. The reductions add their terms in another order than the
chain's row kernel, as any schedule's sums do.

Every tile column's workgroups recompute the rows they read, so the fold pays only for products
with few tile columns: C4's last norm before the 96-wide output product (three tile columns)
8.5 us against 6.5 + 5.1 for the product and the norm's launch; its per-layer norms before y·Wqkv
(24 tile columns) 32.5 us against 23.1 + 5.1 (C4 at T = 256: 1390 -> 1407 us per step with all
five folded). Products with more than $ANVIL_HIP_ROWPRO_COLS (4) tile columns keep the norm's
own launch.

Matched (hip.HipGen.plan_run, before row blocks): one or more sum reductions over the row, each
storing one value per row, then one elementwise kernel over (row, column) storing y, then a
product whose A operand is y itself at [row, k] with unit stride along k and K = D, that takes the
pipelined K split with every wavefront's share of K a whole number of chunks. Every load of the
chain is x at [row, column], a row value an earlier kernel of the chain stored, or an array the
chain does not write indexed by the column alone (a scale or shift per column); nothing after the
chain in the product's epilogue reads what the chain writes.
"""
from __future__ import annotations

import os

from .. import ir
from ..ir import KernelStmt, Load, Var
from . import hip_analysis as A
from .hip_emit import Emitter
from .hip_kernels import canon_key


class RowPrologue:
    def __init__(self, gen, stages, elem, x, xconst, R, D):
        self.gen = gen
        self.stages = stages            # the row reductions, in order
        self.elem = elem                # the elementwise kernel that writes y
        self.x, self.xconst = x, xconst
        self.R, self.D = R, D
        self.y = elem.stores[0].buf.root
        self.kernels = stages + [elem]

    def stored(self, b) -> bool:
        """Is b read outside the chain and its product (so the first tile column stores it)?"""
        inside = sum(1 for k in self.kernels if b.id in {x.id for x in A.kernel_reads(k)})
        if b is self.y:
            inside += 1                                 # the product's A operand
        return self.gen.readers.get(b.id, 0) > inside or b.kind not in A.SHARED_KINDS

    def source(self, plan, sc, W, TM, G, NCH, chkm) -> list[str]:
        """The prologue's lines: the rows loaded, each reduction summed over the workgroup, the
        elementwise kernel applied in place (xa_ then holds the A operand), and the first tile
        column's stores."""
        Q = NCH * 4 * G
        out = [f"    float xa_[{TM}][{Q}];",
               f"    anvil_rowpro_load<{TM}, {NCH}, {G}, {chkm}>(xa_, {sc.buf(self.x)} + ({self.xconst}LL), "
               f"{self.D}LL, m0, {self.R});",
               "    const int rr_ = lane & 31, hh_ = lane >> 5;"]

        def scope_for(k, rvars):
            r, j = rvars
            canon = {r: ("o", 0), j: ("i", 0)}
            fwd = {canon_key(self.x, ir.Affine(self.xconst, {r: self.D, j: 1}), canon): "xa_[i_][q_]"}
            for n, st in enumerate(self.stages):
                b = st.stores[0].buf.root
                fwd[canon_key(b, ir.Affine(st.stores[0].offset.const, {r: 1}), canon)] = f"rv{n}_[i_]"
            sc.canon, sc.fwd = canon, fwd
            sc.names = dict(sc.names)
            sc.names[r] = "row_"
            sc.names[j] = "kq_"

        loop_head = ["#pragma unroll", f"    for (int i_ = 0; i_ < {TM}; i_++) {{",
                     "        const int row_ = m0 + 32 * i_ + rr_;",
                     "#pragma unroll", f"        for (int q_ = 0; q_ < {Q}; q_++) {{",
                     f"            const int kq_ = anvil_rowpro_k<{NCH}, {G}>(q_);", "            (void)kq_;"]
        saved = (sc.canon, sc.fwd, dict(sc.names))
        for n, st in enumerate(self.stages):
            out.append(f"    float rv{n}_[{TM}];")
            out += loop_head[:3] + [f"        float p_ = 0.0f;"] + loop_head[3:]
            scope_for(st, (st.domain[0], st.red.vars[0]))
            lines: list[str] = []
            em = Emitter(sc, lines, "            ", prefix=f"s{n}_")
            val = em.ex(st.red.body)
            out += lines + [f"            p_ = p_ + {val};", "        }", f"        rv{n}_[i_] = p_;", "    }"]
            out.append(f"    anvil_rowpro_sum<{W}, {TM}>(rv{n}_, anvil_kp_lds);")
        e = self.elem
        scope_for(e, (e.domain[0], e.domain[1]))
        lines = []
        em = Emitter(sc, lines, "            ", prefix="y_")
        val = em.ex(e.stores[0].value)
        out += loop_head + lines + [f"            xa_[i_][q_] = {val};", "        }", "    }"]
        sc.canon, sc.fwd, sc.names = saved
        # the first tile column's workgroups store what later kernels read
        stores = []
        for n, st in enumerate(self.stages):
            b = st.stores[0].buf.root
            if self.stored(b):
                stores.append(f"        if (wave == 0 && hh_ == 0) {sc.buf(b)}[row_ + ({st.stores[0].offset.const})] = rv{n}_[i_];")
        if self.stored(self.y):
            ystore = self.elem.stores[0]
            stores += ["#pragma unroll", f"        for (int c_ = 0; c_ < {Q // 4}; c_++) {{",
                       f"            const int k_ = anvil_rowpro_k<{NCH}, {G}>(4 * c_);",
                       "            anvil_f32x4 v_ = {xa_[i_][4 * c_], xa_[i_][4 * c_ + 1], xa_[i_][4 * c_ + 2], xa_[i_][4 * c_ + 3]};",
                       f"            *(anvil_f32x4 *)({sc.buf(self.y)} + (long long)row_ * {self.D} + k_ + ({ystore.offset.const})) = v_;",
                       "        }"]
        if stores:
            out += ["    if (n0 == 0) {", "#pragma unroll", f"        for (int i_ = 0; i_ < {TM}; i_++) {{",
                    "        const int row_ = m0 + 32 * i_ + rr_;"]
            if chkm == "true":
                out.append(f"        if (row_ >= {self.R}) continue;")
            out += ["    " + s for s in stores] + ["        }", "    }"]
        return out


def _reduction_stage(k, R, D):
    """(r, j) of a row sum kernel storing one value per row, else None."""
    if (k.red is None or k.red.op != "sum" or len(k.domain) != 1 or len(k.red.vars) != 1
            or k.domain[0].extent != R or k.red.vars[0].extent != D or len(k.stmts) != 1):
        return None
    st = k.stmts[0]
    r = k.domain[0]
    if (not isinstance(st, ir.Store) or st.accumulate or not isinstance(st.value, ir.Acc)
            or st.offset.terms != {r: 1} or st.offset.gathers() or st.buf.root.numel != R + st.offset.const):
        return None
    return r, k.red.vars[0]


def _elem_stage(k, R, D):
    if k.red is not None or len(k.domain) != 2 or len(k.stmts) != 1:
        return None
    r, j = k.domain
    st = k.stmts[0]
    if (r.extent != R or j.extent != D or not isinstance(st, ir.Store) or st.accumulate
            or st.offset.terms != {r: D, j: 1} or st.offset.const % 4):
        return None
    return r, j


def _loads_ok(k, rvars, x, xconst, D, rowvecs, written) -> bool:
    r, j = rvars
    for e in k.exprs():
        for ld in ir.loads_in(e):
            b = ld.buf.root
            if not b.shape:
                continue                                   # a scalar (host or device)
            if ld.offset.gathers() or ld.offset.scalars():
                return False
            terms = ld.offset.terms
            if b is x and terms == {r: D, j: 1} and ld.offset.const == xconst:
                continue
            if b.id in rowvecs and terms == {r: 1} and ld.offset.const == rowvecs[b.id]:
                continue
            if b.id in written or b is x or r in terms:
                return False
            if any(t is not j for t in terms):
                return False
    return True


def match(gen, stmts, i):
    """(plan, statements taken) for a row chain at stmts[i] and the product after it, or None."""
    if gen.emulate or gen.check or os.environ.get("ANVIL_HIP_ROWPRO", "1") == "0" or gen.gemm is None:
        return None
    k0 = stmts[i].kernel
    if k0.red is None or len(k0.domain) != 1 or not k0.red.vars:
        return None
    R, D = k0.domain[0].extent, k0.red.vars[0].extent
    if D % 32 or R < 32:
        return None
    stages, j = [], i
    while j < len(stmts) and isinstance(stmts[j], KernelStmt) and _reduction_stage(stmts[j].kernel, R, D):
        stages.append(stmts[j].kernel)
        j += 1
    if not stages or j + 1 >= len(stmts) or not isinstance(stmts[j], KernelStmt) \
            or not isinstance(stmts[j + 1], KernelStmt):
        return None
    elem = stmts[j].kernel
    if _elem_stage(elem, R, D) is None:
        return None
    # the row input: the first x[r, j] load of the first reduction
    r0, j0 = _reduction_stage(stages[0], R, D)
    xs = [ld for ld in ir.loads_in(stages[0].red.body)
          if ld.buf.root.shape and ld.offset.terms == {r0: D, j0: 1} and not ld.offset.gathers()]
    if not xs:
        return None
    x, xconst = xs[0].buf.root, xs[0].offset.const
    written = {st.buf.root.id for k in stages + [elem] for st in k.stores}
    if x.id in written:
        return None
    rowvecs: dict = {}
    for k in stages:
        if not _loads_ok(k, _reduction_stage(k, R, D), x, xconst, D, rowvecs, written):
            return None
        rowvecs[k.stores[0].buf.root.id] = k.stores[0].offset.const
    if not _loads_ok(elem, _elem_stage(elem, R, D), x, xconst, D, rowvecs, written):
        return None
    y, yst = elem.stores[0].buf.root, elem.stores[0]
    g_kernel = stmts[j + 1].kernel
    if A.is_host_kernel(g_kernel, gen.hosts):
        return None
    g = gen.gemm.match(gen, g_kernel, f"k{g_kernel.id}")
    if g is None or type(g).__name__ != "GemmPlan":
        return None
    s = g.s
    if (s.la.buf.root is not y or s.ea is not s.la or s.a_gather is not None or s.k_multi or s.batch
            or s.M != R or s.K != D or s.a_rs != D or s.a_ks != 1 or s.la.offset.const != yst.offset.const
            or s.lb.buf.root.id in written):
        return None
    used = 1 + gen.absorb_followers(g, stmts, j + 2)
    g.settle()
    W, G = g.waves, g.kgroup
    if (not g.pipe or g.sched != "ksplit" or g.kslices != 1 or g.slab or g.amode != "ANVIL_LD_KC"
            or D % (8 * G * W) or g.tn > int(os.environ.get("ANVIL_HIP_ROWPRO_COLS", "4"))):
        return None
    # nothing but the product's A operand reads the chain's outputs inside the launch
    for k in g.kernels:
        reads = {b.id for b in A.kernel_reads(k)}
        if k is g.k:
            reads -= {y.id}
        if reads & written:
            return None
    pro = RowPrologue(gen, stages, elem, x, xconst, R, D)
    g.rowpro = pro
    g.kernels = stages + [elem] + g.kernels
    g.label = " + ".join(k.label or k.name for k in stages + [elem]) + " → " + g.label
    return g, (j + 1 - i) + used

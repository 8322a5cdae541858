"""Algorithmic work of kernels and generated kernels: the numbers a roofline is computed from.

The conventions are the reference's cost model (anvil/cost.py:22-52): a multiply-add is 2 FLOPs,
every other arithmetic node 1 (exp, log and the like included; casts and detach are free), the
accumulation of a reduction 1 per element; memory traffic counts each tensor a kernel reads once (no
more elements than its loads can reach) and each element it writes once.

For a generated kernel that runs several IR kernels as stages, values passed between stages in
registers cost nothing: a buffer the kernel itself wrote is not read again, and a store that was
dropped (its buffer is only read by the kernel's own later stages) writes nothing.
"""
from __future__ import annotations

from .. import ir
from ..ir import Binary, Select, Unary

FREE_UNARY = {"detach", "f32", "i32"}


def expr_ops(e) -> int:
    n = 0
    for x in ir.iter_expr(e):
        if isinstance(x, (Binary, Select)) or (isinstance(x, Unary) and x.op not in FREE_UNARY):
            n += 1
    return n


def kernel_flops(k: ir.Kernel) -> int:
    dom = ir.prod(v.extent for v in k.domain)
    per = 0
    if k.red is not None:
        per += ir.prod(v.extent for v in k.red.vars) * (expr_ops(k.red.body) + 1)
    per += sum(expr_ops(st.value) for st in k.stmts)
    return dom * per


def kernel_reach(k: ir.Kernel) -> dict:
    """buffer root -> elements the kernel's loads can reach."""
    dom = ir.prod(v.extent for v in k.domain)
    red = ir.prod(v.extent for v in k.red.vars) if k.red is not None else 1
    reach: dict = {}
    parts = ([(k.red.body, dom * red)] if k.red is not None else []) + [(st.value, dom) for st in k.stmts]
    for e, n in parts:
        for ld in ir.loads_in(e):
            b = ld.buf.root
            if not b.shape:
                continue                                # a scalar argument
            reach[b] = reach.get(b, 0) + min(n, _distinct(ld.offset))
    return reach


def _distinct(off: ir.Affine) -> int:
    """At most how many different elements an offset addresses: the product of the extents of the
    loop variables it depends on (through gathered indices too)."""
    vs: dict = {}

    def walk(a):
        for t in a.terms:
            if isinstance(t, ir.Var):
                vs[t.id] = t.extent or 1
            elif isinstance(t, ir.Gather):
                walk(t.load.offset)
    walk(off)
    return ir.prod(vs.values())


def kernel_bytes(k: ir.Kernel) -> int:
    dom = ir.prod(v.extent for v in k.domain)
    read = sum(4 * min(b.numel, n) for b, n in kernel_reach(k).items())
    return read + sum(4 * dom for _ in k.stores)


def plan_cost(plan) -> tuple[int, int]:
    """(FLOPs, bytes) of one launch of a generated kernel. A matrix product counts 2·M·N·K (per batch)
    for its contraction, the matrix-core work, whatever scale factors the IR multiplies inside the
    sum (they are applied once per output); launches of several kernels side by side add up."""
    if hasattr(plan, "cost"):                           # a plan that knows its own work
        return plan.cost()
    if plan.kind == "fused":
        fl = by = 0
        for p in plan.parts:
            f, b = plan_cost(p)
            fl, by = fl + f, by + b
        return fl, by
    if plan.kind == "attention":                        # the two products; scores never stored
        return 4 * plan.B * plan.Lq * plan.Lk * plan.D, 4 * (plan.Q.numel + plan.K.numel + plan.V.numel +
                                                             plan.O.numel)
    if plan.kind == "gemm":
        s = plan.s
        flops = 2 * s.M * s.N * s.K * s.B + sum(kernel_flops(k) for k in plan.kernels[1:])
        flops += ir.prod(v.extent for v in plan.kernels[0].domain) * sum(expr_ops(st.value)
                                                                         for st in plan.kernels[0].stmts)
    else:
        flops = sum(kernel_flops(k) for k in plan.kernels)
    written: set = set()
    reach: dict = {}
    out_bytes = 0
    for k in plan.kernels:
        for b, n in kernel_reach(k).items():
            if b.id not in written:
                reach[b] = reach.get(b, 0) + n
        dom = ir.prod(v.extent for v in k.domain)
        for i, st in enumerate(k.stmts):
            if isinstance(st, ir.Store):
                written.add(st.buf.root.id)
                if (k.id, i) not in plan.skip_stores:
                    out_bytes += 4 * dom
    read = sum(4 * min(b.numel, n) for b, n in reach.items())
    return flops, read + out_bytes

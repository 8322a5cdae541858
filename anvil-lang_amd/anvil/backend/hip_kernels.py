"""Kernel schedules: how one IR kernel (or a run of them) becomes one HIP kernel.

  map     no reduction: a grid-stride loop, one output element per lane and step.
  serial  a kernel whose outputs must be produced in order (cuda.py:380-395): one lane does all.
  rows    L lanes per output row (L = 1, 64 = one wavefront, or 256 = one workgroup). The row's
          elements are split over the lanes, each lane reduces its share, and the lanes' partial
          results are combined with cross-lane shuffles (and LDS across the four waves of a
          workgroup). Several consecutive IR kernels over the same rows (softmax's max, exp-sum and
          divide; layer norm's mean, variance and normalize; cross-entropy's log-softmax) become
          the stages of one kernel: per-row results stay in registers, and each lane keeps its
          share of a row in registers between stages, so the row is read from memory once.
  split   a reduction whose elements are strided in memory (a bias gradient, Σ_i dY[i, j]): the
          lanes of a wavefront take neighbouring outputs (coalesced loads) and a workgroup splits
          each output's reduction TY ways, combining the partial results through LDS in a fixed
          order.
  rowblock  a chain of kernels that work row by row (logits, log-softmax, its gradient, the next
          layer's input gradient): one workgroup per row runs every stage of the chain.
  fused   independent kernels (no data between them) launched as one grid, side by side.

Each plan produces the kernel's source and the host-side launch: grid, block and arguments.
"""
from __future__ import annotations

import os
import re

from .. import ir
from ..ir import F32, I32, Gather, Load, ScalarRef, Var
from . import hip_analysis as A
from .hip_emit import Emitter, Scope, ctype, flit, ilit

THREADS = 256
MAX_BLOCKS = 1 << 16
QMAX = 16                       # register-cached elements per lane and row
CACHE_REGS = 96                 # register budget for cached row elements, per lane
CU_WAVES = 256 * 4              # waves that fill the chip once (256 CUs x 4 SIMDs)
# The interpreter evaluates a reduction with no output index over more than CHUNK elements in
# chunks of its first reduction variable (interp.py:25, 392-406, 484-516); argmax / argmin combine
# the chunks' picks by a rule of their own (arg_chunk).
CHUNK = 1 << 22


def index_type(n: int) -> str:
    return "uint32_t" if n < (1 << 31) else "uint64_t"


def decode(vars_, src: str, it: str) -> list[str]:
    """C declarations of each var from a flattened row-major index."""
    out = []
    strides = ir.row_major_strides([v.extent for v in vars_])
    for k, (v, s) in enumerate(zip(vars_, strides)):
        expr = src if s == 1 else f"({src}) / {s}u"
        if k > 0 and v.extent > 1:
            expr = f"({expr}) % {v.extent}u"
        if v.extent == 1:
            expr = "0"
        out.append(f"const int v{v.id} = (int)({expr});")
    return out


def unit_stride(k: ir.Kernel, v) -> bool:
    """Does every memory access of k step by 0 or 1 element along v (so that 4 consecutive values
    of v touch 4 consecutive floats: one wide load or store)?"""
    for ld in A.kernel_loads(k):
        if ld.offset.coef(v) not in (0, 1):
            return False
    for st in k.stores:
        if st.offset.coef(v) not in (0, 1):
            return False
    return True


def epilogue_loads(stages):
    """(stage index, load) pairs of kernels' statements that may be issued before their reduction:
    plain loads of buffers that no earlier statement stores to. stages: [(kernel, forwarded loads)]."""
    stored: set = set()
    out, seen = [], set()
    for si, (e, fwd) in enumerate(stages):
        fwd_ids = {id(ld) for ld in fwd}
        canon = {v: ("e", v.id) for v in e.domain}
        for st in e.stmts:
            for ld in ir.loads_in(st.value):
                b = ld.buf.root
                if id(ld) in fwd_ids or not b.shape or b.id in stored or ld.offset.gathers():
                    continue
                if any(isinstance(t, ScalarRef) for t in ld.offset.terms):
                    continue
                key = (si, canon_key(ld.buf, ld.offset, canon))
                if key not in seen:
                    seen.add(key)
                    out.append((si, ld))
            if isinstance(st, ir.Store):
                stored.add(st.buf.root.id)
    return out


def red_init(op: str, dtype: str) -> str:
    if op in ("sum",):
        return "0.0f" if dtype == F32 else "0"
    if op == "prod":
        return "1.0f" if dtype == F32 else "1"
    if op in ("max", "argmax"):
        return "(-__builtin_inff())" if dtype == F32 else "(-2147483647 - 1)"
    return "__builtin_inff()" if dtype == F32 else "2147483647"


def red_combine(op: str, dtype: str, a: str, b: str) -> str:
    if op == "sum":
        return f"({a} + {b})" if dtype == F32 else f"anvil_wrap_add({a}, {b})"
    if op == "prod":
        return f"({a} * {b})" if dtype == F32 else f"anvil_wrap_mul({a}, {b})"
    if op == "max":
        return f"anvil_maxf({a}, {b})" if dtype == F32 else f"anvil_maxi({a}, {b})"
    return f"anvil_minf({a}, {b})" if dtype == F32 else f"anvil_mini({a}, {b})"


RED_CODE = {"sum": "ANVIL_RED_SUM", "prod": "ANVIL_RED_PROD", "max": "ANVIL_RED_MAX", "min": "ANVIL_RED_MIN"}


def arg_pick(op: str, val: str, idx: str, best: str, at: str) -> str:
    """C that lets element (val, idx) replace the running argmax / argmin pick (best, at)."""
    mx = "true" if op == "argmax" else "false"
    return f"if (anvil_arg_better<{mx}>({val}, {idx}, {best}, {at})) {{ {best} = {val}; {at} = {idx}; }}"


def arg_chunk(k: ir.Kernel) -> int:
    """Elements per interpreter chunk for an argmax / argmin with no output index over more than
    CHUNK elements (0: evaluated whole): ranges of `per` values of the first reduction variable."""
    if k.red is None or k.red.op not in ("argmax", "argmin") or k.domain:
        return 0
    n = ir.prod(v.extent for v in k.red.vars)
    if n <= CHUNK:
        return 0
    inner = n // k.red.vars[0].extent
    return max(1, CHUNK // max(1, inner)) * inner


class KernelScope(Scope):
    """Device code of one plan: buffers and host scalars become parameters as they are used."""

    def __init__(self, plan: "Plan"):
        self.plan = plan
        self.names: dict = {}
        self.acc_name = "acc"
        self.rand = "u"
        self.stream_name = "anvil_rs0"
        self.fwd: dict = {}               # canonical (buffer id, offset) -> C expression of its value
        self.canon = None                 # var -> canonical symbol, for forwarding

    def var(self, v):
        return self.names.get(v, f"v{v.id}")

    def buf(self, b):
        return self.plan.use_buf(b.root)

    def host_scalar(self, b):
        if b.root.id in self.plan.gen.hosts:
            return self.plan.use_host(b.root)
        return None

    def acc(self):
        return self.acc_name

    def rand_index(self):
        return self.rand

    def stream(self):
        return self.stream_name

    def fault(self, message):
        return self.plan.gen.fault(message)

    def override_load(self, ld):
        if self.canon is None or not self.fwd:
            return None
        key = canon_key(ld.buf, ld.offset, self.canon)
        if key is None:
            return None
        got = self.fwd.get(key)
        if callable(got):
            return got(ld)
        return got


def _subst(off: ir.Affine, m: dict):
    """off with each loop variable replaced by its affine function in m (None if off has a gather
    or a variable m does not map)."""
    out = ir.Affine(off.const)
    for t, c in off.terms.items():
        if isinstance(t, Var) and t in m:
            out = out + m[t] * c
        elif isinstance(t, ScalarRef):
            out = out + ir.Affine(0, {t: c})
        else:
            return None
    return out


def canon_key(buf, off: ir.Affine, canon: dict):
    terms = []
    for t, c in off.terms.items():
        if not isinstance(t, Var) or t not in canon:
            return None
        terms.append((canon[t], c))
    return (buf.root.id, off.const, tuple(sorted(terms)))


class Plan:
    """One generated kernel: its name, source and launch."""

    kind = "?"

    def __init__(self, gen, kernels, name: str):
        self.gen = gen
        self.kernels = kernels
        self.name = name
        self.bufs: dict[int, ir.Buffer] = {}
        self.hosts: dict[int, ir.Buffer] = {}
        self.streams = [k for k in kernels if k.uses_rand()]
        self.skip_stores: set = set()      # (kernel id, store index) of dead stores
        self.label = " + ".join(k.label or k.name for k in kernels)

    # parameters
    def use_buf(self, b) -> str:
        self.bufs.setdefault(b.id, b)
        return f"b{b.id}"

    def use_host(self, b) -> str:
        self.hosts.setdefault(b.id, b)
        return f"h{b.id}"

    def by_value(self) -> bool:
        """Host scalars reach the kernel as arguments (eager launches), or from the device copy that
        the host's scalar kernels' twins keep current (graph replay: arguments are frozen)."""
        return not self.gen.graphs

    def params(self) -> str:
        ps = [f"uint32_t anvil_rs{i}" for i in range(max(1, len(self.streams)))] + ["uint32_t anvil_seed"]
        if self.by_value():
            ps += [f"{ctype(b.dtype)} h{b.id}" for b in self.hosts.values()]
        elif self.hosts:
            ps.append("uint32_t *__restrict__ anvil_hsd")
        ps += [f"{ctype(b.dtype)} *__restrict__ b{b.id}" for b in self.bufs.values()]
        return ", ".join(ps)

    def launch_args(self, stream_vars: list) -> list:
        sv = stream_vars or ["0u"]
        args = list(sv) + ["anvil_hs.seed"]
        if self.by_value():
            args += [f"anvil_h{b.id}" for b in self.hosts.values()]
        elif self.hosts:
            args.append("anvil_hsd")
        args += [f"anvil_b{b.id}" for b in self.bufs.values()]
        return args

    def host_prologue(self, mutable: bool = False) -> list[str]:
        """Graph mode: host scalars, read from the device copy."""
        out = []
        if self.by_value():
            return out
        q = "" if mutable else "const "
        for b in self.hosts.values():
            slot = self.gen.hsd_slot(b)
            v = f"(int)anvil_hsd[{slot}]" if b.dtype == I32 else f"anvil_f32_of(anvil_hsd[{slot}])"
            out.append(f"    {q}{ctype(b.dtype)} h{b.id} = {v};")
        return out

    def stream_param(self, k) -> str:
        return f"anvil_rs{self.streams.index(k)}" if k in self.streams else "anvil_rs0"

    def writes(self) -> set:
        out = set()
        for k in self.kernels:
            out |= A.kernel_writes(k)
        return out

    def comment(self) -> str:
        parts = []
        for k in self.kernels:
            d = " x ".join(f"{v.name}<{v.extent}" for v in k.domain) or "scalar"
            r = f" reduce {k.red.op} " + " x ".join(f"{v.name}<{v.extent}" for v in k.red.vars) if k.red else ""
            parts.append(f"{k.name} [{d}]{r}")
        return f"// {self.kind}: " + "; ".join(parts)

    def header(self, threads: int) -> str:
        """The kernel's signature, its opening brace, and its host-scalar declarations."""
        return "\n".join([f"__global__ void __launch_bounds__({threads}) {self.name}({self.params()}) {{"]
                         + self.host_prologue())

    def sole_writer(self, k: ir.Kernel, st) -> bool:
        """Is `st` the only store of this launch to its buffer that can reach a given element, so
        that its `+=` needs no atomic? (Other kernels of the plan must not write the buffer.)"""
        return A.sole_writer(k, st) and not any(
            o.buf.root is st.buf.root for k2 in self.kernels if k2 is not k for o in k2.stores)

    # body helpers
    def statements(self, em: Emitter, k: ir.Kernel, scope: KernelScope, parallel: bool, guard: str | None = None,
                   on_store=None) -> None:
        for i, st in enumerate(k.stmts):
            if isinstance(st, ir.Let):
                em.let(st)
                continue
            val = em.store_value(st)
            if (k.id, i) in self.skip_stores:
                if on_store:
                    on_store(st, val)
                em.reset_memo()
                continue
            off = em.affine(st.offset, st.buf)
            target = f"{scope.buf(st.buf)}[{off}]"
            if st.accumulate:
                if parallel and not self.sole_writer(k, st):
                    line = f"atomicAdd(&{target}, {val});"
                elif st.buf.dtype == I32:
                    line = f"{target} = anvil_wrap_add({target}, {val});"
                else:
                    line = f"{target} += {val};"
            elif st.buf.root.kind == "output" and st.buf.dtype == F32:
                line = f"anvil_store_out(&{target}, {val});"
            else:
                line = f"{target} = {val};"
            em.emit(f"if ({guard}) {line}" if guard else line)
            if on_store:
                on_store(st, val)
            em.reset_memo()


# ----------------------------------------------------------------------------- map

class MapPlan(Plan):
    """One lane per element of the domain (grid-stride), with the elementwise kernels that follow it
    over the same elements (each reads what this one just stored at that element: the gradient of
    a max-pool, then ReLU's) run in the same lane on the value in a register; a store that only
    those followers read is dropped."""

    kind = "map"

    def __init__(self, gen, k, name):
        super().__init__(gen, [k], name)
        self.k = k
        self.total = ir.prod(v.extent for v in k.domain)
        self.threads = THREADS
        self.followers = []             # (kernel, var map, forwarded loads), run per element after k
        self.vector_width()

    def vector_width(self):
        # four consecutive elements per lane and step when every access is unit-stride along the
        # innermost variable, or (pairs) when the innermost variable has extent 2 and the one before
        # it an even extent (a 2-wide window's elements: two windows per lane); the accesses that
        # the lane's four elements make side by side then go out as one 16-byte (or, shared by two
        # elements each, 8-byte) access (`vector_accesses`)
        k = self.k
        inner = k.domain[-1] if k.domain else None
        unit = inner is not None and unit_stride(k, inner)
        for e, m, _ in self.followers:
            for off in [ld.offset for ld in A.kernel_loads(e)] + [st.offset for st in e.stores]:
                sub = _subst(off, m)
                unit = unit and sub is not None and sub.coef(inner) in (0, 1)
        self.pairs = False
        self.V = 4 if (unit and not self.gen.emulate and inner.extent % 4 == 0) else 1
        if (self.V == 1 and not self.gen.emulate and len(k.domain) >= 2 and inner.extent == 2
                and k.domain[-2].extent % 2 == 0 and os.environ.get("ANVIL_HIP_MAP_PAIRS", "1") != "0"):
            self.pairs, self.V = True, 4
            loads, stores = self.vector_accesses()
            if not loads and not stores:
                self.pairs, self.V = False, 1
        self.blocks = max(1, min(-(-self.total // (THREADS * self.V)), MAX_BLOCKS))

    def _vector_kind(self, off) -> str | None:
        """For an access at `off` (over this kernel's domain variables) by the four elements of a
        lane: "x4" when they lie side by side from a multiple of 4 (one 16-byte access, buffers
        being 16-byte aligned), "x2" when pairs of them share each of two adjacent elements from an
        even one (pairs mode: one 8-byte access), else None."""
        if off is None or off.gathers() or off.scalars() or any(not isinstance(t, Var) for t in off.terms):
            return None
        inner = self.k.domain[-1]
        lead = {inner}
        if self.pairs:
            j = self.k.domain[-2]
            lead.add(j)
            steps = tuple((e >> 1) * off.coef(j) + (e & 1) * off.coef(inner) for e in range(4))
        else:
            steps = tuple(e * off.coef(inner) for e in range(4))

        def aligned(m):
            return off.const % m == 0 and all(t in lead or c % m == 0 for t, c in off.terms.items())
        if steps == (0, 1, 2, 3) and aligned(4):
            return "x4"
        if self.pairs and steps == (0, 0, 1, 1) and aligned(2):
            return "x2"
        return None

    def vector_accesses(self):
        """(loads, stores) that the lane's four elements make as one access: loads [(name, kind,
        load, offset over the lead's variables, [Load nodes it serves])] of f32 buffers the plan does
        not write; stores {id(store): (name, store, offset)}, plain f32 stores of buffers no load of
        the plan reads (they leave after the lane's four elements are computed)."""
        if self.V != 4 or self.gen.check or os.environ.get("ANVIL_HIP_VEC_MAP", "1") == "0":
            return [], {}
        parts = [(self.k, None)] + [(e, m) for e, m, _ in self.followers]
        written = {b.id for p, _ in parts for b in A.kernel_writes(p)}
        read = set()
        loads, by_key = [], {}
        for p, m in parts:
            for ld in A.kernel_loads(p):
                b = ld.buf.root
                read.add(b.id)
                off = ld.offset if m is None else _subst(ld.offset, m)
                kind = self._vector_kind(off) if b.dtype == F32 and b.shape and b.id not in written else None
                if kind is None:
                    continue
                key = (b.id, off.key())
                if key not in by_key:
                    by_key[key] = len(loads)
                    loads.append((f"{'qv' if kind == 'x4' else 'pv'}{len(loads)}_", kind, ld, off, []))
                loads[by_key[key]][4].append(ld)
        stores = {}
        for p, m in parts:
            for i, st in enumerate(p.stmts):
                if (not isinstance(st, ir.Store) or (p.id, i) in self.skip_stores or st.accumulate
                        or st.buf.root.dtype != F32 or st.buf.root.id in read):
                    continue
                off = st.offset if m is None else _subst(st.offset, m)
                if self._vector_kind(off) == "x4":
                    stores[id(st)] = (f"sv{len(stores)}_", st, off, (p.id, i))
        return loads, stores

    def absorb(self, e, how):
        """Take elementwise kernel e as a follower (how: its var map and forwarded loads, from
        hip_gemm.follower), unless it writes a buffer this plan writes (two lanes' elements could
        then land on one element in either order)."""
        m, fwd = how
        written = {b.id for p in [self.k] + [f[0] for f in self.followers] for b in A.kernel_writes(p)}
        if {b.id for b in A.kernel_writes(e)} & written:
            return False
        self.followers.append((e, m, fwd))
        self.kernels.append(e)
        self.label += " + " + (e.label or e.name)
        self.vector_width()
        return True

    def source(self) -> str:
        k = self.k
        it = index_type(self.total)
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        body: list[str] = []
        ind = "        " if self.V == 1 else "            "
        em = Emitter(sc, body, ind)
        vloads, vstores = self.vector_accesses()
        picks = {id(ld): f"{name}[e]" if kind == "x4" else f"{name}[e >> 1]"
                 for name, kind, _, _, served in vloads for ld in served}
        if picks:
            def override(x, sc=sc):
                got = picks.get(id(x))
                return got if got is not None else KernelScope.override_load(sc, x)
            sc.override_load = override
        deferred = {key for _, _, _, key in vstores.values()}
        self.skip_stores |= deferred
        for line in decode(k.domain, "u", it):
            em.emit(line)
        stored = {}

        def on_store(st, val):
            if id(st) in vstores:
                em.emit(f"{vstores[id(st)][0]}[e] = {val};")
            if not st.accumulate:
                stored[st.buf.root.id] = val
        self.statements(em, k, sc, parallel=True, on_store=on_store)
        for e, m, fwd in self.followers:
            em.reset_memo()
            for ev, aff in m.items():
                em.emit(f"const int v{ev.id} = (int)({em.affine(aff)});")
            canon = {v: ("e", v.id) for v in e.domain}
            sc.canon = canon
            sc.fwd = {canon_key(ld.buf, ld.offset, canon): stored[ld.buf.root.id] for ld in fwd}
            self.statements(em, e, sc, parallel=True, on_store=on_store)
            sc.canon, sc.fwd = None, {}
        self.skip_stores -= deferred
        n = self.total // self.V
        what = (" · two 2-wide windows (4 elements) per lane" if self.pairs else
                f" · {self.V} elements per lane" if self.V > 1 else "")
        if vloads or vstores:
            what += f", {len(vloads)} loads and {len(vstores)} stores as one access each"
        pre: list[str] = []
        tail: list[str] = []
        if vloads or vstores:
            # the lane's first element's variables, for the wide accesses' addresses
            pem = Emitter(sc, pre, "            ")
            pem.emit(f"const {it} u = {self.V}u * w;")
            for line in decode(k.domain, "u", it):
                pem.emit(line)
            for name, kind, ld, off, _ in vloads:
                T = "anvil_f32x4" if kind == "x4" else "anvil_f32x2"
                pem.emit(f"const {T} {name} = *(const {T} *)&{sc.buf(ld.buf)}[{pem.affine(off, ld.buf)}];")
            if vstores:
                pem.emit(f"anvil_f32x4 {', '.join(v[0] for v in vstores.values())};")
            pre.insert(0, "        {")
            post: list[str] = []
            tem = Emitter(sc, post, "            ")
            for name, st, off, _ in vstores.values():
                target = f"{sc.buf(st.buf)}[{tem.affine(off, st.buf)}]"
                if st.buf.root.kind == "output":
                    tem.emit(f"__builtin_nontemporal_store({name}, (anvil_f32x4 *)&{target});")
                else:
                    tem.emit(f"*(anvil_f32x4 *)&{target} = {name};")
            tail = post + ["        }"]
        # (the header last: the buffers the kernel takes are known once every access is emitted)
        head = [self.comment() + what, self.header(self.threads),
                f"    for ({it} w = ({it})blockIdx.x * {self.threads}u + threadIdx.x; w < {n}u; "
                f"w += ({it})gridDim.x * {self.threads}u) {{"]
        if self.V == 1:
            head.append("        const auto u = w;")
            return "\n".join(head + body + ["    }", "}"])
        head += pre + ["#pragma unroll", f"        for ({it} e = 0; e < {self.V}u; e++) {{",
                 f"            const {it} u = {self.V}u * w + e;"]
        return "\n".join(head + body + ["        }"] + tail + ["    }", "}"])

    def grid(self):
        return self.blocks, self.threads


# ----------------------------------------------------------------------------- gather-sum

def scatter_targets(k: ir.Kernel):
    """For an elementwise kernel whose one store adds (`+=`) to elements that several domain points
    share, as the gradient of an im2col copy does (dX[n, c, i+u, j+v] += dP[n, i, j, c, u, v]):
    (targets, summed vars) or None. Domain variables with the same coefficient in the store's
    offset form one target coordinate y = their sum (extent: the sum of their extents less one
    each), of which the widest member is then solved for (i = y - u); variables with coefficient 0
    are summed whole. targets: (coefficient, extent, members, solved member) per coordinate, outer
    to inner; None unless distinct coordinates reach distinct elements."""
    if k.red is not None or k.uses_rand() or not k.domain or len(k.stores) != 1:
        return None
    st = k.stores[0]
    if not st.accumulate or st.buf.dtype != F32 or any(not isinstance(t, Var) for t in st.offset.terms):
        return None
    if any(ld.buf.root is st.buf.root for ld in A.kernel_loads(k)):
        return None
    groups: dict = {}
    free = []
    for v in k.domain:
        if v.extent <= 1:
            continue
        c = st.offset.coef(v)
        if c == 0:
            free.append(v)
        else:
            groups.setdefault(c, []).append(v)
    if not free and all(len(g) == 1 for g in groups.values()):
        return None
    targets = []
    for c, g in groups.items():
        if len(g) == 1:
            targets.append((c, g[0].extent, g, None))
        else:
            solved = max(g, key=lambda v: (v.extent, k.domain.index(v)))
            targets.append((c, sum(v.extent - 1 for v in g) + 1, g, solved))
    reach = 0
    for c, ext, _, _ in sorted(targets, key=lambda t: abs(t[0])):
        if abs(c) <= reach:
            return None
        reach += abs(c) * (ext - 1)
    solved = {t[3] for t in targets if t[3] is not None}
    summed = [v for v in k.domain if v.extent > 1 and (v in free or (st.offset.coef(v) and v not in solved
                                                                       and len(groups[st.offset.coef(v)]) > 1))]
    # lanes step along the coordinate the loads are densest in (they carry the traffic: each target
    # element takes several loads); the rest outer to inner as the store's offset runs
    targets.sort(key=lambda t: -abs(t[0]))
    loads = A.kernel_loads(k)

    def load_stride(t):
        v = t[3] if t[3] is not None else t[2][0]
        return sum(abs(ld.offset.coef(v)) for ld in loads)
    dense = [t for t in targets if load_stride(t)]
    if dense:
        inner = min(dense, key=load_stride)
        targets = [t for t in targets if t is not inner] + [inner]
    return targets, summed


class GatherSumPlan(Plan):
    """The scatter of a `+=` kernel turned into a gather: one lane per element of the target
    region, which loops over the domain points that add to it (in the domain's own order, so each
    element takes the same additions in the same order as the sequential `+=`), skips those whose
    solved variable falls outside its range, and writes the element once. No atomics, and every
    element is read and written once."""

    kind = "gather-sum"

    def __init__(self, gen, k, name, targets, summed):
        super().__init__(gen, [k], name)
        self.k = k
        self.targets, self.summed = targets, summed
        self.total = ir.prod(t[1] for t in targets)
        self.blocks = max(1, min(-(-self.total // THREADS), MAX_BLOCKS))

    def source(self) -> str:
        k, st = self.k, self.k.stores[0]
        it = index_type(self.total)
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        body: list[str] = []
        em = Emitter(sc, body, "        ")
        ys = [A.new_var(900_000_000 + i, f"y{i}", t[1]) for i, t in enumerate(self.targets)]
        for line in decode(ys, "w", it):
            em.emit(line)
        for y, (_, _, members, solved) in zip(ys, self.targets):
            if solved is None:
                em.emit(f"const int v{members[0].id} = v{y.id};")
        for v in k.domain:
            if v.extent <= 1:
                em.emit(f"const int v{v.id} = 0;")
        off = ir.Affine(st.offset.const, {y: t[0] for y, t in zip(ys, self.targets)})
        target = f"{sc.buf(st.buf)}[{em.affine(off, st.buf)}]"
        em.emit(f"float acc = {target};")
        saved = em.memo
        em.memo = dict(saved)
        bound = set()
        for v in self.summed:
            em.emit(f"for (int v{v.id} = 0; v{v.id} < {v.extent}; v{v.id}++) {{")
            em.ind += "    "
            bound.add(v)
            for y, (_, ext, members, solved) in zip(ys, self.targets):
                if solved is None or v not in members or any(m not in bound for m in members if m is not solved):
                    continue
                rest = " - ".join([f"v{y.id}"] + [f"v{m.id}" for m in members if m is not solved])
                em.emit(f"const int v{solved.id} = {rest};")
                em.emit(f"if ((unsigned)v{solved.id} >= {solved.extent}u) continue;")
        for stmt in k.stmts:
            if isinstance(stmt, ir.Let):
                em.let(stmt)
            else:
                em.emit(f"acc += {em.store_value(stmt)};")
        for _ in self.summed:
            em.ind = em.ind[:-4]
            em.emit("}")
        em.memo = saved
        em.emit(f"{target} = acc;")
        head = [self.comment() + " · the scatter as a gather: one lane per target element",
                self.header(THREADS),
                f"    for ({it} w = ({it})blockIdx.x * {THREADS}u + threadIdx.x; w < {self.total}u; "
                f"w += ({it})gridDim.x * {THREADS}u) {{"]
        return "\n".join(head + body + ["    }", "}"])

    def grid(self):
        return self.blocks, THREADS


# ----------------------------------------------------------------------------- index scatter

INDEX_SCATTER_MAX_POS = 8192        # positions a workgroup's lanes hold in registers while they scan
INDEX_SCATTER_MAX_ROWS = 1024       # every workgroup scans every position: R x P index loads


def index_scatter(k: ir.Kernel):
    """For a `+=` into rows of a small table picked by an index array (an embedding's gradient:
    dE[tok[n, t], d] += dX[n, t, d]): (column vars, position vars, the gather, row width W, rows R,
    positions P), or None. The store's offset is W·idx[...] plus a row-major index over [0, W) of
    the column variables, which the index load does not use; the other domain variables are the
    positions. Only where positions collide (P >= 2R, a few rows, a bounded scan)."""
    if k.red is not None or k.uses_rand() or not k.domain or len(k.stores) != 1:
        return None
    if not all(isinstance(x, (ir.Let, ir.Store)) for x in k.stmts):
        return None
    st = k.stores[0]
    off = st.offset
    if not st.accumulate or st.buf.dtype != F32 or off.const != 0 or off.scalars() or len(off.gathers()) != 1:
        return None
    g = off.gathers()[0]
    W = off.coef(g)
    if W <= 0 or g.rest is not None or g.load.offset.gathers() or g.load.offset.scalars():
        return None
    cols = sorted((v for v in off.terms if isinstance(v, Var)), key=lambda v: -off.coef(v))
    if any(v not in k.domain for v in cols) or ir.prod(v.extent for v in cols) != W:
        return None
    stride = W
    for v in cols:
        stride //= v.extent
        if off.coef(v) != stride:
            return None
    if any(g.load.offset.coef(v) for v in cols):
        return None
    if any(ld.buf.root is st.buf.root for ld in A.kernel_loads(k)):
        return None
    pos = [v for v in k.domain if v not in cols]
    P = ir.prod(v.extent for v in pos)
    lo, R = g.check_range()
    if lo != 0 or not 0 < R <= INDEX_SCATTER_MAX_ROWS or P > INDEX_SCATTER_MAX_POS or P < 2 * R:
        return None
    if R * W > st.buf.root.numel:
        return None
    return cols, pos, g, W, R, P


class IndexScatterPlan(Plan):
    """The `+=` of `index_scatter` without atomics: one workgroup per table row r. Its four
    wavefronts each scan a quarter of the positions (the index loads, with their bounds check, in
    registers); a ballot per 64 positions counts those whose index is r, and once the wavefronts'
    counts are known each writes its hits, in position order, into one list in LDS. Then each lane
    takes a column of the row and adds the listed positions' values to the table's element in
    list order (the order of the sequential `+=`), BATCH positions' loads in flight at a time, and
    writes the element once."""

    kind = "index-scatter"
    BATCH = 16

    def __init__(self, gen, k, name, cols, pos, g, W, R, P):
        super().__init__(gen, [k], name)
        self.k = k
        self.cols, self.pos, self.g, self.W, self.R, self.P = cols, pos, g, W, R, P
        self.S = -(-P // THREADS)                    # positions per lane in the scan
        self.Q = 64 * self.S                         # positions per wavefront
        self.blocks = R
        self.batch = int(os.environ.get("ANVIL_SCATTER_BATCH", str(self.BATCH)))

    def source(self) -> str:
        k, st = self.k, self.k.stores[0]
        T, S, Q, P, W, R, B = THREADS, self.S, self.Q, self.P, self.W, self.R, self.batch
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        body: list[str] = []
        em = Emitter(sc, body, "        ")
        # the index loads first, all in flight, then their bounds checks (a check's branch to the
        # fault report between two loads would hold the second back until the first arrives)
        g = self.g
        lo, hi = g.check_range()
        code = sc.fault(f"index out of bounds ({g.where or 'gather'}; dimension size {g.bound})")
        em.emit(f"int idx_[{S}];")
        em.emit("#pragma unroll")
        em.emit(f"for (int s = 0; s < {S}; s++) {{")
        em.emit(f"    const uint32_t p = wave * {Q}u + 64u * (uint32_t)s + lane;")
        em.emit(f"    idx_[s] = {ilit(lo)};")
        em.emit(f"    if (p < {P}u) {{")
        em.ind += "        "
        for line in decode(self.pos, "p", "uint32_t"):
            em.emit(line)
        em.emit(f"idx_[s] = {em.ex(g.load)};")
        em.ind = em.ind[:-8]
        em.emit("    }")
        em.emit("}")
        em.reset_memo()
        em.emit("#pragma unroll")
        em.emit(f"for (int s = 0; s < {S}; s++) {{")
        em.emit(f"    if (idx_[s] < {ilit(lo)} || idx_[s] >= {ilit(hi)}) {{ anvil_fault({code}, idx_[s]); idx_[s] = {ilit(lo)}; }}")
        em.emit(f"    if (wave * {Q}u + 64u * (uint32_t)s + lane >= {P}u) idx_[s] = -1;      // past the last position")
        em.emit("}")
        em.emit("int cnt = 0;")
        em.emit("#pragma unroll")
        em.emit(f"for (int s = 0; s < {S}; s++) cnt += __popcll(__ballot(idx_[s] == (int)row));")
        em.emit("if (lane == 0) anvil_nhit[wave] = cnt;")
        em.emit("__syncthreads();")
        em.emit("int base = 0;")
        em.emit("for (uint32_t w = 0; w < wave; w++) base += anvil_nhit[w];")
        em.emit("const int nh = anvil_nhit[0] + anvil_nhit[1] + anvil_nhit[2] + anvil_nhit[3];")
        em.emit("#pragma unroll")
        em.emit(f"for (int s = 0; s < {S}; s++) {{")
        em.emit("    const unsigned long long m = __ballot(idx_[s] == (int)row);")
        em.emit("    if (idx_[s] == (int)row)")
        em.emit(f"        anvil_hits[base + __popcll(m & ((1ull << lane) - 1ull))] = "
                f"(int)(wave * {Q}u + 64u * (uint32_t)s + lane);")
        em.emit("    base += __popcll(m);")
        em.emit("}")
        em.emit("__syncthreads();")
        rv = A.new_var(900_000_200, "r", R)
        em.emit(f"const int v{rv.id} = (int)row;")
        em.emit(f"for (uint32_t col = threadIdx.x; col < {W}u; col += {T}u) {{")
        em.ind += "    "
        for line in decode(self.cols, "col", "uint32_t"):
            em.emit(line)
        target_off = ir.Affine(0, {rv: W, **{v: st.offset.coef(v) for v in self.cols}})
        target = f"{sc.buf(st.buf)}[{em.affine(target_off, st.buf)}]"
        em.emit(f"float acc = {target};")
        em.emit(f"for (int h0 = 0; h0 < nh; h0 += {B}) {{")
        em.ind += "    "
        em.emit(f"float x_[{B}];")
        saved = em.memo
        for j in range(B):
            em.emit(f"x_[{j}] = 0.0f;")
            em.emit(f"if (h0 + {j} < nh) {{")
            em.ind += "    "
            em.emit(f"const uint32_t p = (uint32_t)anvil_hits[h0 + {j}];")
            em.memo = dict(saved)
            for line in decode(self.pos, "p", "uint32_t"):
                em.emit(line)
            val = None
            for stmt in k.stmts:
                if isinstance(stmt, ir.Let):
                    em.let(stmt)
                else:
                    val = em.store_value(stmt)
            em.emit(f"x_[{j}] = {val};")
            em.ind = em.ind[:-4]
            em.emit("}")
        em.memo = saved
        em.emit("#pragma unroll")
        em.emit(f"for (int j = 0; j < {B}; j++)")
        em.emit("    if (h0 + j < nh) acc += x_[j];")
        em.ind = em.ind[:-4]
        em.emit("}")
        em.emit(f"{target} = acc;")
        em.ind = em.ind[:-4]
        em.emit("}")
        em.emit("__syncthreads();")
        head = [self.comment() + f" · one workgroup per table row ({R} rows of {W}), {P} positions scanned in order",
                self.header(T),
                f"    __shared__ int anvil_hits[{4 * Q}];",
                "    __shared__ int anvil_nhit[4];",
                "    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;",
                f"    for (uint32_t row = blockIdx.x; row < {R}u; row += gridDim.x) {{"]
        return "\n".join(head + body + ["    }", "}"])

    def grid(self):
        return self.blocks, THREADS


# ----------------------------------------------------------------------------- serial

class SerialPlan(Plan):
    kind = "serial"

    def __init__(self, gen, k, name):
        super().__init__(gen, [k], name)
        self.k = k
        self.total = ir.prod(v.extent for v in k.domain)

    def source(self) -> str:
        k = self.k
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        body: list[str] = []
        em = Emitter(sc, body, "        ")
        for line in decode(k.domain, "u", "uint64_t"):
            em.emit(line)
        if k.red is not None:
            serial_reduction(em, sc, k, "        ")
        self.statements(em, k, sc, parallel=False)
        head = [self.comment(), self.header(1),
                f"    for (uint64_t u = 0; u < {self.total}ull; u++) {{"]
        return "\n".join(head + body + ["    }", "}"])

    def grid(self):
        return 1, 1


def serial_reduction(em: Emitter, sc: KernelScope, k: ir.Kernel, ind: str, unroll: bool = False) -> None:
    """The reduction as nested loops in one lane (element order = the flattened row-major order).
    unroll: unroll the loops (short ones fully), so that their loads are in flight together."""
    red = k.red
    op, dt = red.op, red.body.dtype
    T = ctype(dt)
    arg = op in ("argmax", "argmin")
    P = arg_chunk(k)
    n = ir.prod(v.extent for v in red.vars)
    if arg:
        em.emit(f"{T} best = {red_init(op, dt)}; int acc = 2147483647; int ridx = 0;")
        if P:
            em.emit(f"{T} cbest = {red_init(op, dt)}; int cat = 2147483647;")
    else:
        em.emit(f"{T} acc = {red_init(op, dt)};")
    saved_ind = em.ind
    for v in red.vars:
        if unroll:
            em.emit("#pragma unroll" if v.extent <= 64 else "#pragma unroll 8")
        em.emit(f"for (int v{v.id} = 0; v{v.id} < {v.extent}; v{v.id}++) {{")
        em.ind += "    "
    saved = em.memo
    em.memo = dict(saved)
    val = em.ex(red.body)
    if arg and P:
        # one lane walks the elements in order: close each interpreter chunk as it ends
        em.emit(arg_pick(op, val, "ridx", "cbest", "cat"))
        em.emit("ridx++;")
        em.emit(f"if (ridx % {P} == 0 || ridx == {n}) {{")
        em.emit(f"    if (ridx <= {P} || anvil_chunk_better<{'true' if op == 'argmax' else 'false'}>(cbest, best)) "
                "{ best = cbest; acc = cat; }")
        em.emit(f"    cbest = {red_init(op, dt)}; cat = 2147483647;")
        em.emit("}")
    elif arg:
        em.emit(arg_pick(op, val, "ridx", "best", "acc"))
        em.emit("ridx++;")
    else:
        em.emit(f"acc = {red_combine(op, dt, 'acc', val)};")
    em.memo = saved
    for _ in red.vars:
        em.ind = em.ind[:-4]
        em.emit("}")
    em.ind = saved_ind


# ----------------------------------------------------------------------------- rows

class PoolPlan(Plan):
    """A reduction over a 2-wide window along the output's innermost index (a 2 x 2 max-pool:
    out[r, j] = max_{u, v} f(x[r, u, 2j + v])): each lane computes two adjacent outputs j = 2p,
    2p + 1, whose windows' elements along v lie side by side, so for each value of the window's
    other variables one 16-byte load gives the lane all four, and each store of the pair is one
    8-byte store. (One lane per output made four 4-byte loads and two 4-byte stores per output:
    C5's max-pool 9.6 us; two outputs per lane measured 3.7 us less per step.)

    Taken when every load of the reduction's body has coefficient 2 on j and 1 on the window's
    innermost variable (extent 2), its other coefficients and its constant multiples of 4, and every
    store is a plain f32 store of the result at coefficient 1 on j with its other coefficients and
    constant even (buffers being 16-byte aligned)."""

    kind = "rows"

    def __init__(self, gen, k, name):
        super().__init__(gen, [k], name)
        self.k = k
        self.R = ir.prod(v.extent for v in k.domain)
        self.blocks = max(1, min(-(-(self.R // 2) // THREADS), MAX_BLOCKS))
        self.label = "window pairs: " + self.label

    @staticmethod
    def match(gen, k):
        if (gen.emulate or gen.check or os.environ.get("ANVIL_HIP_POOL", "1") == "0" or k.red is None
                or k.red.op not in ("max", "min", "sum") or not k.domain or len(k.red.vars) < 1
                or k.red.body.dtype != F32 or k.uses_rand()):
            return None
        j, v = k.domain[-1], k.red.vars[-1]
        if j.extent % 2 or v.extent != 2:
            return None
        loads = ir.loads_in(k.red.body)
        if not loads:
            return None
        for x in ir.iter_expr(k.red.body):
            if not isinstance(x, (ir.Const, ir.Unary, ir.Binary, Load)):
                return None
        for ld in loads:
            off = ld.offset
            if (ld.buf.root.dtype != F32 or off.gathers() or off.scalars() or off.const % 4
                    or off.coef(j) != 2 or off.coef(v) != 1
                    or any(not isinstance(t, Var) or (t is not j and t is not v and c % 4) for t, c in off.terms.items())):
                return None
        for st in k.stmts:
            if isinstance(st, ir.Let):
                continue
            off = st.offset
            if (st.accumulate or st.buf.dtype != F32 or off.gathers() or off.scalars() or off.const % 2
                    or off.coef(j) != 1 or any(not isinstance(t, Var) or (t is not j and c % 2) for t, c in off.terms.items())):
                return None
        return PoolPlan(gen, k, f"k{k.id}")

    def grid(self):
        return self.blocks, THREADS

    def source(self) -> str:
        k = self.k
        j, v = k.domain[-1], k.red.vars[-1]
        others = list(k.red.vars[:-1])
        op, T = k.red.op, ctype(F32)
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        body: list[str] = []
        em = Emitter(sc, body, "        ")
        half = j.extent // 2
        em.emit(f"const uint32_t p_ = w % {half}u, rest_ = w / {half}u;")
        for line in decode(k.domain[:-1], "rest_", "uint32_t"):
            em.emit(line)
        em.emit(f"const int v{j.id} = 2 * (int)p_;")
        loads, seen = [], {}
        for ld in ir.loads_in(k.red.body):
            kk = (ld.buf.root.id, ld.offset.key())
            if kk not in seen:
                seen[kk] = len(loads)
                loads.append(ld)
        em.emit(f"{T} acc0 = {red_init(op, F32)}, acc1 = {red_init(op, F32)};")
        import itertools
        for vals in itertools.product(*[range(x.extent) for x in others]):
            for x, val in zip(others, vals):
                sc.names[x] = str(val)
            sc.names[v] = "0"
            em.reset_memo()
            quads = {}
            for n, ld in enumerate(loads):
                name = f"w{n}_" + "_".join(str(x) for x in vals)
                em.emit(f"const anvil_f32x4 {name} = *(const anvil_f32x4 *)&{sc.buf(ld.buf)}[{em.affine(ld.offset, ld.buf)}];")
                quads[id(ld)] = name
            for e in (0, 1):
                for dv in (0, 1):
                    em.reset_memo()
                    fwd = {(ld.buf.root.id, ld.offset.key()): quads[id(ld)] for ld in loads}

                    def pick(x, e=e, dv=dv, fwd=fwd):
                        return f"{fwd[(x.buf.root.id, x.offset.key())]}[{2 * e + dv}]"
                    saved = em.s.override_load
                    em.s.override_load = lambda x, pick=pick: pick(x) if isinstance(x, Load) else None
                    val = em.ex(k.red.body)
                    em.s.override_load = saved
                    em.emit(f"acc{e} = {red_combine(op, F32, f'acc{e}', val)};")
        for x in others + [v]:
            sc.names.pop(x, None)
        # the statements for both outputs, then each store as one 8-byte store
        vals = {}
        for e in (0, 1):
            em.reset_memo()
            em.lets = {}
            sc.acc_name = f"acc{e}"
            em.prefix = f"o{e}_"
            for i, st in enumerate(k.stmts):
                if isinstance(st, ir.Let):
                    em.let(st)
                    continue
                vals[(i, e)] = em.store_value(st)
        for i, st in enumerate(k.stmts):
            if isinstance(st, ir.Let) or (k.id, i) in self.skip_stores:
                continue
            target = f"{sc.buf(st.buf)}[{em.affine(st.offset, st.buf)}]"
            em.emit(f"*(float2 *)&{target} = make_float2({vals[(i, 0)]}, {vals[(i, 1)]});")
        head = [self.comment() + f" · two outputs of the 2-wide window per lane, {self.R // 2} pairs",
                self.header(THREADS),
                f"    for (uint32_t w = blockIdx.x * {THREADS}u + threadIdx.x; w < {self.R // 2}u; w += gridDim.x * {THREADS}u) {{"]
        return "\n".join(head + body + ["    }", "}"])


class RowsPlan(Plan):
    """Stages over the same rows; stage 0 is a reduction whose domain is the rows."""

    kind = "rows"

    def __init__(self, gen, kernels, name, lanes: int, emulate: bool):
        super().__init__(gen, kernels, name)
        head = kernels[0]
        self.outer = list(head.domain)
        self.inner_extents = [v.extent for v in head.red.vars]
        self.R = ir.prod(v.extent for v in self.outer)
        self.n = ir.prod(self.inner_extents)
        self.L = lanes
        inner = head.red.vars[-1]
        self.V = 4 if (lanes > 1 and not emulate and self.n % (4 * lanes) == 0 and inner.extent % 4 == 0
                       and all(self._unit(k) for k in kernels)) else 1
        self.Q = -(-self.n // (lanes * self.V))
        self.rpb = THREADS // lanes if lanes < THREADS else 1
        self.threads = THREADS if lanes > 1 else min(THREADS, max(64, 64 * -(-self.R // 64)))
        if lanes == 1:
            self.rpb = self.threads
        # rows within one wavefront: sixteen wavefronts per CU (four per SIMD) when that gives each
        # wavefront two rows (C3's layernorm over 8192 rows of 1024: 2048 workgroups 12.3 µs, 1024
        # 11.8 µs, 512 12.9; four rows each of 256 (C4's) measured no better). A row spread over a
        # workgroup (its reductions cross the wavefronts through LDS) keeps one workgroup per row:
        # C3's softmax over rows of 4096 was 42.6 µs so and 45-47 µs with the cap.
        want = -(-self.R // self.rpb)
        cap = int(os.environ.get("ANVIL_ROWS_BLOCKS", str(16 * 256 * 64 // self.threads)))
        if 1 < lanes <= 64 and want <= 2 * cap:
            want = min(want, cap)
        self.blocks = max(1, min(want, MAX_BLOCKS))
        self.cached = self.Q <= QMAX and (lanes > 1 or self.n <= 32)
        self.cache_arrays: dict = {}       # canonical key -> array name
        self.emulate = emulate
        self.plan_cache()

    def _unit(self, k) -> bool:
        inner = k.red.vars[-1] if k.red is not None else (k.domain[-1] if len(k.domain) > len(self.outer) else None)
        return inner is None or unit_stride(k, inner)

    @property
    def slot(self) -> str:
        """The register-cache index of the current element."""
        return "q" if self.V == 1 else f"(q * {self.V} + e)"

    # which element-level values live in registers between stages
    def stage_vars(self, k):
        if k.red is not None:
            return list(k.domain), list(k.red.vars)
        no = len(self.outer)
        return list(k.domain[:no]), list(k.domain[no:])

    def canon_map(self, k) -> dict:
        outer, inner = self.stage_vars(k)
        m = {v: ("o", i) for i, v in enumerate(outer)}
        m.update({v: ("i", i) for i, v in enumerate(inner)})
        return m

    def plan_cache(self):
        if not self.cached:
            return
        seen: dict = {}
        written: dict = {}
        for si, k in enumerate(self.kernels):
            cm = self.canon_map(k)
            _, inner = self.stage_vars(k)
            inner_set = set(inner)
            for ld in A.kernel_loads(k):
                key = canon_key(ld.buf, ld.offset, cm)
                if key is None or not any(v in inner_set for v in ld.offset.direct_vars()):
                    continue
                seen.setdefault(key, set()).add(si)
            if k.red is None:
                for st in k.stores:
                    key = canon_key(st.buf, st.offset, cm)
                    if key is not None:
                        written[key] = si
        budget = CACHE_REGS // max(1, self.Q)
        for key, stages in sorted(seen.items(), key=lambda kv: (min(kv[1]), repr(kv[0]))):
            if len(self.cache_arrays) >= budget:
                break
            if key in written or len(stages) >= 2:
                self.cache_arrays[key] = f"c{len(self.cache_arrays)}"
        for key in written:
            if key not in self.cache_arrays and len(self.cache_arrays) < budget:
                self.cache_arrays[key] = f"c{len(self.cache_arrays)}"

    def source(self) -> str:
        L, Q, n = self.L, self.Q, self.n
        out = [self.comment() + f" · {L} lane(s) per row, {self.R} rows of {n}"]
        body: list[str] = []
        ind = "        "
        shared: list[str] = []
        sc = KernelScope(self)
        em = Emitter(sc, body, ind)
        if L == THREADS:
            row0, rstep = "blockIdx.x", "gridDim.x"
            pre = ["    const int lane = threadIdx.x;"]
        elif L == 1:
            row0, rstep = f"blockIdx.x * {self.rpb}u + threadIdx.x", f"gridDim.x * {self.rpb}u"
            pre = ["    const int lane = 0;"]
        else:
            row0, rstep = f"blockIdx.x * {self.rpb}u + (threadIdx.x / {L}u)", f"gridDim.x * {self.rpb}u"
            pre = [f"    const int lane = threadIdx.x % {L}u;"]
        pre.append("    (void)lane;")
        for line in decode(self.outer, "row", "uint32_t"):
            em.emit(line)
        for key, name in self.cache_arrays.items():
            em.emit(f"{ctype(self._key_dtype(key))} {name}[{Q * self.V}];")
        populated: set = set()
        fwd: dict = {}
        self.vector_preload(em, sc, populated)
        for si, k in enumerate(self.kernels):
            em.reset_memo()
            cm = self.canon_map(k)
            # the canonical symbols of this stage's own vars: outer vars keep the head's names
            for i, v in enumerate(self.stage_vars(k)[0]):
                sc.names[v] = f"v{self.outer[i].id}"
            sc.canon = cm
            sc.stream_name = self.stream_param(k)
            self.populated_now = set()
            if k.red is not None:
                self.reduction_stage(em, sc, k, si, shared, fwd, populated)
            else:
                self.map_stage(em, sc, k, si, fwd, populated)
            populated |= self.populated_now
        if L == THREADS:
            em.emit("__syncthreads();")
        text = out + [self.header(self.threads)] + pre + shared
        text.append(f"    for (uint32_t row = {row0}; row < {self.R}u; row += {rstep}) {{")
        return "\n".join(text + body + ["    }", "}"])

    def _key_dtype(self, key):
        bid = key[0]
        for k in self.kernels:
            for ld in A.kernel_loads(k):
                if ld.buf.root.id == bid:
                    return ld.buf.root.dtype
            for st in k.stores:
                if st.buf.root.id == bid:
                    return st.buf.root.dtype
        return F32

    def element_loop(self, em: Emitter, inner_vars, body_fn, after_e=None, before_e=None):
        """for q: j = lane + L*q; decode the inner vars; body_fn(q). after_e / before_e: called in
        each q trip once its V elements are done / before they start (cached rows with V > 1 only)."""
        L, Q, n, V = self.L, self.Q, self.n, self.V
        saved_memo = em.memo
        if self.cached:
            em.emit("#pragma unroll")
            em.emit(f"for (int q = 0; q < {Q}; q++) {{")
            em.ind += "    "
            if V > 1 and before_e is not None:
                em.memo = dict(saved_memo)
                before_e()
                em.memo = saved_memo
            if V > 1:
                em.emit("#pragma unroll")
                em.emit(f"for (int e = 0; e < {V}; e++) {{")
                em.ind += "    "
                em.emit(f"const uint32_t j = {V}u * ((uint32_t)lane + {L}u * (uint32_t)q) + (uint32_t)e;")
            else:
                em.emit(f"const uint32_t j = (uint32_t)lane + {L}u * (uint32_t)q;")
            if n % (L * V):
                em.emit(f"if (j < {n}u) {{")
                em.ind += "    "
        else:
            if V > 1:
                em.emit(f"for (uint32_t jv = (uint32_t)lane; jv < {n // V}u; jv += {L}u) {{")
                em.ind += "    "
                em.emit("#pragma unroll")
                em.emit(f"for (uint32_t e = 0; e < {V}u; e++) {{")
                em.ind += "    "
                em.emit(f"const uint32_t j = {V}u * jv + e;")
            else:
                em.emit("#pragma unroll 8")
                em.emit(f"for (uint32_t j = (uint32_t)lane; j < {n}u; j += {L}u) {{")
                em.ind += "    "
        em.memo = dict(saved_memo)
        for line in decode(inner_vars, "j", "uint32_t"):
            em.emit(line)
        body_fn()
        em.memo = saved_memo
        if self.cached and n % (L * V):
            em.ind = em.ind[:-4]
            em.emit("}")
        if V > 1:
            em.ind = em.ind[:-4]
            em.emit("}")
            if after_e is not None and self.cached:
                em.memo = dict(saved_memo)
                after_e()
                em.memo = saved_memo
        em.ind = em.ind[:-4]
        em.emit("}")

    def install_cache(self, sc: KernelScope, cm, fwd: dict, populated: set, em: Emitter):
        """Forwarded row values, and cached element values (loaded on first use)."""
        table = dict(fwd)
        for key, name in self.cache_arrays.items():
            if key in populated or key in fwd:
                table[key] = fwd.get(key, f"{name}[{self.slot}]")
            else:
                def first_load(ld, name=name, key=key):
                    v = em.build(ld)
                    em.emit(f"{name}[{self.slot}] = {v};")
                    sc.fwd[key] = f"{name}[{self.slot}]"
                    self.populated_now.add(key)
                    return f"{name}[{self.slot}]"
                table[key] = first_load
        sc.fwd = table

    def reduction_stage(self, em, sc, k, si, shared, fwd, populated):
        red = k.red
        op, dt = red.op, red.body.dtype
        T = ctype(dt)
        arg = op in ("argmax", "argmin")
        cm = self.canon_map(k)
        sc.rand = "row"
        self.install_cache(sc, cm, fwd, populated, em)
        if arg:
            em.emit(f"{T} best{si} = {red_init(op, dt)}; int acc{si} = 2147483647;")
        else:
            em.emit(f"{T} acc{si} = {red_init(op, dt)};")
        mx = "true" if op == "argmax" else "false"
        if arg and arg_chunk(k):
            self.chunked_arg_stage(em, sc, k, si, shared, arg_chunk(k))
            sc.acc_name = f"acc{si}"
            sc.fwd = dict(fwd)
            self.row_statements(em, sc, k, cm, fwd)
            return

        def body():
            val = em.ex(red.body)
            if arg:
                em.emit(arg_pick(op, val, "(int)j", f"best{si}", f"acc{si}"))
            else:
                em.emit(f"acc{si} = {red_combine(op, dt, f'acc{si}', val)};")
        ql = self.quad_loads(em, sc, k, cm, list(red.vars))
        if ql is not None:
            sc.fwd.update(ql[1])
        self.element_loop(em, list(red.vars), body, None, ql[0] if ql else None)
        if self.L == 64:
            if arg:
                em.emit(f"anvil_wave_arg<{mx}, {T}>(best{si}, acc{si});")
            else:
                em.emit(f"acc{si} = anvil_wave_all<{RED_CODE[op]}, {T}>(acc{si});")
        elif self.L == THREADS:
            if arg:
                shared.append(f"    __shared__ {T} sv{si}[4]; __shared__ int si{si}[4];")
                em.emit(f"anvil_block_arg<{mx}, {T}>(best{si}, acc{si}, sv{si}, si{si});")
            else:
                shared.append(f"    __shared__ {T} sv{si}[4];")
                em.emit(f"acc{si} = anvil_block_all<{RED_CODE[op]}, {T}>(acc{si}, sv{si});")
        sc.acc_name = f"acc{si}"
        sc.fwd = dict(fwd)
        self.row_statements(em, sc, k, cm, fwd)

    def chunked_arg_stage(self, em, sc, k, si, shared, P: int):
        """argmax / argmin with no output index over more than CHUNK elements: the row's lanes pick
        within each interpreter chunk of P elements (nan first, then the extreme, ties to the
        smaller index), combine the chunk's pick across the lanes, and the chunk picks meet in
        chunk order by the interpreter's rule (anvil_chunk_better)."""
        red = k.red
        op, dt = red.op, red.body.dtype
        T = ctype(dt)
        mx = "true" if op == "argmax" else "false"
        L, n = self.L, self.n
        em.emit(f"for (uint32_t c0 = 0; c0 < {n}u; c0 += {P}u) {{")
        em.ind += "    "
        em.emit(f"const uint32_t c1 = c0 + {P}u < {n}u ? c0 + {P}u : {n}u;")
        em.emit(f"{T} cb = {red_init(op, dt)}; int ca = 2147483647;")
        em.emit(f"for (uint32_t j = c0 + (uint32_t)lane; j < c1; j += {L}u) {{")
        em.ind += "    "
        saved_memo = em.memo
        em.memo = dict(saved_memo)
        for line in decode(list(red.vars), "j", "uint32_t"):
            em.emit(line)
        val = em.ex(red.body)
        em.emit(arg_pick(op, val, "(int)j", "cb", "ca"))
        em.memo = saved_memo
        em.ind = em.ind[:-4]
        em.emit("}")
        if L == 64:
            em.emit(f"anvil_wave_arg<{mx}, {T}>(cb, ca);")
        elif L == THREADS:
            shared.append(f"    __shared__ {T} sv{si}[4]; __shared__ int si{si}[4];")
            em.emit(f"anvil_block_arg<{mx}, {T}>(cb, ca, sv{si}, si{si});")
            em.emit("__syncthreads();                  // the slots are written again for the next chunk")
        em.emit(f"if (c0 == 0 || anvil_chunk_better<{mx}>(cb, best{si})) {{ best{si} = cb; acc{si} = ca; }}")
        em.ind = em.ind[:-4]
        em.emit("}")

    def row_statements(self, em, sc, k, cm, fwd):
        def on_store(st, val):
            key = canon_key(st.buf, st.offset, cm)
            if key is not None and not st.accumulate:
                fwd[key] = val
                sc.fwd = dict(fwd)
        self.statements(em, k, sc, parallel=True, guard="lane == 0" if self.L > 1 else None, on_store=on_store)

    def map_stage(self, em, sc, k, si, fwd, populated):
        cm = self.canon_map(k)
        _, inner = self.stage_vars(k)
        if not inner:                                   # a per-row scalar stage
            sc.rand = "row"
            sc.fwd = dict(fwd)
            self.row_statements(em, sc, k, cm, fwd)
            return
        sc.rand = f"(row * {self.n}u + j)"
        self.install_cache(sc, cm, fwd, populated, em)
        vec = self.vector_stores(k, cm, inner)
        self.skip_stores |= {(k.id, i) for i, _ in vec}
        ql = self.quad_loads(em, sc, k, cm, inner)
        if ql is not None:
            sc.fwd.update(ql[1])

        def after_e():
            # the V values of each vector store, kept in their cache array, as one 16-byte store
            self.quad_head(em, inner)
            for i, st in vec:
                name = self.cache_arrays[canon_key(st.buf, st.offset, cm)]
                target = f"{sc.buf(st.buf)}[{em.affine(st.offset, st.buf)}]"
                vals = ", ".join(f"{name}[q * 4 + {e}]" for e in range(4))
                em.emit(f"{{ const anvil_f32x4 w_ = {{{vals}}};")
                if st.buf.root.kind == "output":
                    em.emit(f"  __builtin_nontemporal_store(w_, (anvil_f32x4 *)&{target}); }}")
                else:
                    em.emit(f"  *(anvil_f32x4 *)&{target} = w_; }}")
            self.quad_tail(em)

        def body():
            def on_store(st, val):
                key = canon_key(st.buf, st.offset, cm)
                if key is None or st.accumulate:
                    return
                name = self.cache_arrays.get(key)
                if name is not None:
                    em.emit(f"{name}[{self.slot}] = {val};")
                    fwd[key] = f"{name}[{self.slot}]"
                    sc.fwd[key] = f"{name}[{self.slot}]"
                    self.populated_now.add(key)
            self.statements(em, k, sc, parallel=True, on_store=on_store)
        self.element_loop(em, inner, body, after_e if vec else None, ql[0] if ql else None)
        self.skip_stores -= {(k.id, i) for i, _ in vec}

    # 16-byte loads and stores of a cached row (V = 4: lane l holds elements 4(l + L·q) .. + 3)
    @staticmethod
    def quad_aligned(off, inner_last) -> bool:
        """Are the 4 elements a lane holds side by side in memory, the first at a multiple of 4
        (so, buffers being 16-byte aligned, one 16-byte access)?"""
        if off.gathers() or off.scalars() or off.const % 4 or off.terms.get(inner_last) != 1:
            return False
        return all(isinstance(t, Var) and (t is inner_last or c % 4 == 0) for t, c in off.terms.items())

    def quad_enabled(self) -> bool:
        return self.cached and self.V == 4 and os.environ.get("ANVIL_HIP_VEC_ROWS", "1") != "0"

    def quad_head(self, em, inner):
        em.emit("{")
        em.ind += "    "
        em.emit(f"const uint32_t j = 4u * ((uint32_t)lane + {self.L}u * (uint32_t)q);")
        if self.n % (self.L * 4):
            em.emit(f"if (j < {self.n}u) {{")
            em.ind += "    "
        for line in decode(inner, "j", "uint32_t"):
            em.emit(line)

    def quad_tail(self, em):
        if self.n % (self.L * 4):
            em.ind = em.ind[:-4]
            em.emit("}")
        em.ind = em.ind[:-4]
        em.emit("}")

    def quad_loads(self, em, sc, k, cm, inner):
        """A before_e hook for stage k: its loads of buffers the plan does not write, held in no
        cache array, 4 side by side (a per-column scale or shift), one 16-byte load per lane and q
        trip; the element loop then reads them from there."""
        if not self.quad_enabled() or not inner:
            return None
        written = {b.id for kk in self.kernels for b in A.kernel_writes(kk)}
        picks, seen = [], set()
        for ld in A.kernel_loads(k):
            b = ld.buf.root
            key = canon_key(ld.buf, ld.offset, cm)
            if (key is None or key in seen or key in self.cache_arrays or b.id in written or b.dtype != F32
                    or not b.shape or not self.quad_aligned(ld.offset, inner[-1])):
                continue
            seen.add(key)
            picks.append((key, ld))
        if not picks:
            return None
        names = {key: f"qv{n}_" for n, (key, _) in enumerate(picks)}

        def hook():
            em.emit(f"anvil_f32x4 {', '.join(names.values())};")
            self.quad_head(em, inner)
            for key, ld in picks:
                em.emit(f"{names[key]} = *(const anvil_f32x4 *)&{sc.buf(ld.buf)}[{em.affine(ld.offset, ld.buf)}];")
            self.quad_tail(em)
        return hook, {key: f"{name}[e]" for key, name in names.items()}

    def vector_stores(self, k, cm, inner):
        """(index, store) of k's stores that go out 16 bytes at a time: plain f32 stores whose value
        the row's cache array holds, 4 elements side by side."""
        if not self.quad_enabled() or not inner:
            return []
        out = []
        for i, st in enumerate(k.stmts):
            if (not isinstance(st, ir.Store) or st.accumulate or st.buf.dtype != F32 or (k.id, i) in self.skip_stores
                    or canon_key(st.buf, st.offset, cm) not in self.cache_arrays
                    or not self.quad_aligned(st.offset, inner[-1])):
                continue
            out.append((i, st))
        return out

    def vector_preload(self, em, sc, populated):
        """Cached row values of buffers the plan does not write, loaded 16 bytes at a time before the
        first stage (the stages then read them from the cache)."""
        if not self.quad_enabled():
            return
        written = {b.id for k in self.kernels for b in A.kernel_writes(k)}
        done: set = set()
        for k in self.kernels:
            cm = self.canon_map(k)
            outer, inner = self.stage_vars(k)
            if not inner:
                continue
            for ld in A.kernel_loads(k):
                b = ld.buf.root
                key = canon_key(ld.buf, ld.offset, cm)
                if (key is None or key in done or key in populated or key not in self.cache_arrays or b.id in written
                        or b.dtype != F32 or not b.shape or not self.quad_aligned(ld.offset, inner[-1])):
                    continue
                done.add(key)
                for i, v in enumerate(outer):
                    sc.names[v] = f"v{self.outer[i].id}"
                name = self.cache_arrays[key]
                em.reset_memo()
                em.emit("#pragma unroll")
                em.emit(f"for (int q = 0; q < {self.Q}; q++) {{")
                em.ind += "    "
                self.quad_head(em, inner)
                em.emit(f"const anvil_f32x4 w_ = *(const anvil_f32x4 *)&{sc.buf(ld.buf)}[{em.affine(ld.offset, ld.buf)}];")
                em.emit(" ".join(f"{name}[q * 4 + {e}] = w_[{e}];" for e in range(4)))
                self.quad_tail(em)
                em.ind = em.ind[:-4]
                em.emit("}")
                populated.add(key)
        em.reset_memo()

    def grid(self):
        return self.blocks, self.threads


# ----------------------------------------------------------------------------- split

class SplitPlan(Plan):
    """TX outputs per workgroup, each reduced TY ways (lane t: output t % TX, share t / TX)."""

    kind = "split"

    def __init__(self, gen, k, name, ty: int, threads: int = THREADS):
        super().__init__(gen, [k], name)
        self.k = k
        self.R = ir.prod(v.extent for v in k.domain)
        self.n = ir.prod(v.extent for v in k.red.vars)
        self.TY = ty
        self.threads = threads
        self.TX = threads // ty
        self.blocks = max(1, min(-(-self.R // self.TX), MAX_BLOCKS))

    def source(self) -> str:
        k = self.k
        red = k.red
        op, dt = red.op, red.body.dtype
        T = ctype(dt)
        TX, TY = self.TX, self.TY
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        sc.rand = "row"
        body: list[str] = []
        em = Emitter(sc, body, "        ")
        for line in decode(k.domain, "row", "uint32_t"):
            em.emit(line)
        # the statements' own operands (an optimizer's state) are loaded before the reduction
        pre = epilogue_loads([(k, [])])[:8]
        canon = {v: ("e", v.id) for v in k.domain}
        if pre:
            em.emit(" ".join(f"float pre{i} = 0.0f;" if ld.buf.dtype == F32 else f"int pre{i} = 0;"
                             for i, (_, ld) in enumerate(pre)))
            em.emit(f"if (ty == 0 && row < {self.R}u) {{")
            for i, (_, ld) in enumerate(pre):
                em.emit(f"    pre{i} = {em.build(ld)};")
            em.emit("}")
        em.emit(f"{T} acc = {red_init(op, dt)};")
        em.emit(f"if (row < {self.R}u) {{")
        em.ind += "    "
        em.emit("#pragma unroll 8")
        em.emit(f"for (uint32_t j = ty; j < {self.n}u; j += {TY}u) {{")
        em.ind += "    "
        saved = em.memo
        em.memo = dict(saved)
        for line in decode(list(red.vars), "j", "uint32_t"):
            em.emit(line)
        val = em.ex(red.body)
        em.emit(f"acc = {red_combine(op, dt, 'acc', val)};")
        em.memo = saved
        em.ind = em.ind[:-4]
        em.emit("}")
        em.ind = em.ind[:-4]
        em.emit("}")
        em.emit("part[ty][tx] = acc;")
        em.emit("__syncthreads();")
        em.emit(f"if (ty == 0 && row < {self.R}u) {{")
        em.ind += "    "
        em.emit("acc = part[0][tx];")
        em.emit(f"for (int p = 1; p < {TY}; p++) acc = {red_combine(op, dt, 'acc', 'part[p][tx]')};")
        if pre:
            sc.canon = canon
            sc.fwd = {canon_key(ld.buf, ld.offset, canon): f"pre{i}" for i, (_, ld) in enumerate(pre)}
        em.reset_memo()
        self.statements(em, k, sc, parallel=True)
        sc.canon, sc.fwd = None, {}
        em.ind = em.ind[:-4]
        em.emit("}")
        em.emit("__syncthreads();")
        head = [self.comment() + f" · {TX} outputs x {TY}-way split per workgroup",
                self.header(self.threads),
                f"    __shared__ {T} part[{TY}][{TX}];",
                f"    const uint32_t tx = threadIdx.x % {TX}u, ty = threadIdx.x / {TX}u;",
                f"    for (uint32_t rb = blockIdx.x * {TX}u; rb < {self.R}u; rb += gridDim.x * {TX}u) {{",
                "        const uint32_t row = rb + tx;"]
        return "\n".join(head + body + ["    }", "}"])

    def grid(self):
        return self.blocks, self.threads


# ----------------------------------------------------------------------------- row blocks

def row_local(off: ir.Affine, k: ir.Kernel, R: int, S: int | None) -> bool:
    """Does `off` (an access of kernel k, whose first domain variable walks R rows of f0 values
    each) stay inside row r's slice [r S, (r + 1) S) of its buffer, for every row r?"""
    if S is None or off.scalars():
        return False
    v0 = k.domain[0]
    f0 = v0.extent // R
    if off.coef(v0) * f0 != S:
        return False
    lo = hi = off.const
    for t, c in off.terms.items():
        if isinstance(t, Var):
            ext = f0 if t is v0 else (t.extent or 1)
            span = c * (ext - 1)
        elif isinstance(t, Gather):
            g0, g1 = t.check_range()
            lo += min(c * g0, c * (g1 - 1))
            hi += max(c * g0, c * (g1 - 1))
            continue
        else:
            return False
        if span >= 0:
            hi += span
        else:
            lo += span
    return lo >= 0 and hi < S


class RowBlockBuilder:
    """A chain of consecutive kernels that all work row by row over the same R rows (the first
    domain variable of each walks the rows), where every buffer the chain writes is only ever
    touched in the row being processed: then one workgroup can run the whole chain for a row,
    stage after stage, with a barrier in between and no launch between the stages."""

    MAX_ROW_WORK = 1 << 15          # outputs x reduction length per row and stage

    MIN_ROW_FOR_PRIOR = 128         # see `prior` below

    def __init__(self, R: int, prior: set = frozenset()):
        self.R = R
        self.kernels: list = []
        self.written: dict = {}     # buffer id -> row slice
        self.far: set = set()       # buffers some stage reads outside its row
        self.before: set = set()    # buffers read before the chain writes them (their old values)
        self.prior = prior          # buffers an earlier kernel of the same block wrote

    def slice_of(self, b):
        n = b.root.numel
        return n // self.R if n % self.R == 0 else None

    def fits(self, k: ir.Kernel, hosts: set) -> bool:
        if not k.domain or A.is_host_kernel(k, hosts) or not A.parallel_safe(k):
            return False
        if k.domain[0].extent % self.R:
            return False
        E = ir.prod(v.extent for v in k.domain) // self.R
        n = ir.prod(v.extent for v in k.red.vars) if k.red is not None else 1
        if E * n > self.MAX_ROW_WORK:
            return False
        # a buffer whose old contents a stage reads is not written by the chain: the chain's
        # launch is one position of the program for the arena, where the reads of buffers the
        # launch writes are taken to be of the launch's own values. Unless an earlier kernel of the
        # same block wrote it: its lifetime then began before the launch (a gradient a product
        # wrote and a stage adds to, layer norm's input gradient). That is taken only for rows of
        # MIN_ROW_FOR_PRIOR elements or more: a workgroup per row of 64 (C4's softmax gradient at
        # T = 64, 4096 rows) measured 17.8 µs against 7.8 for its three launches.
        before = self.before | {b.id for b in A.kernel_reads(k) if b.id not in self.written}
        written = dict(self.written)
        long_rows = E >= self.MIN_ROW_FOR_PRIOR
        for st in k.stores:
            b = st.buf.root
            S = self.slice_of(b)
            if (b.id in self.far or (b.id in before and not (long_rows and b.id in self.prior))
                    or not row_local(st.offset, k, self.R, S)):
                return False
            written[b.id] = S
        far = set()
        for ld in A.kernel_loads(k):
            b = ld.buf.root
            local = row_local(ld.offset, k, self.R, self.slice_of(b))
            if b.id in written and not local:
                return False
            if not local:
                far.add(b.id)
        scal: set = set()
        for e in k.exprs():
            for x in ir.iter_expr(e):
                if isinstance(x, Load):
                    A.affine_scalars(x.offset, scal)
        if any(b.id in written for b in scal):
            return False
        self.written = written
        self.far |= far
        self.before = before
        self.kernels.append(k)
        return True


class RowBlockScope(KernelScope):
    """Loads of the chain's own row slices kept in LDS read the LDS copy; operands the plan keeps
    in registers (hoisted per-row loads, values forwarded from an earlier stage, the components of
    a vector load a block stage's outputs share) read those."""

    def __init__(self, plan):
        super().__init__(plan)
        self.em = None
        self.part = "stmts"             # which part of the stage is being emitted: "body" / "stmts"
        self.q = None                   # a block stage's output being accumulated (its body)
        self.red_index = "0"            # a serial stage's flat reduction index (its body)
        self.hoisted: dict = {}         # load key -> register
        self.targets: dict = {}         # (part, load key) -> (slot, map from the index to the slot's)
        self.sources: dict = {}         # (part, load key) -> slot
        self.vectors: dict = {}         # block stage's body load key -> (array, width): one vector load

    def inner(self) -> str:
        """The index of the current load among the part's I (see RowBlockPlan.addresses)."""
        if self.part != "body":
            return "0"
        return self.red_index if self.q is None else str(self.q)

    def override_load(self, ld):
        b = ld.buf.root
        if b.id in self.plan.shadow and self.em is not None:
            S = self.plan.shadow[b.id]
            return f"sh{b.id}[{self.em.affine(ld.offset, ld.buf)} - (int)row * {S}]"
        key = ld.key()
        if key in self.hoisted and self.part == "stmts":
            return self.hoisted[key]
        if key in self.vectors and self.part == "body" and self.q is not None:
            name, w = self.vectors[key]
            val = f"{name}[{self.q // w}].{'xyzw'[self.q % w]}"
            slot = self.sources.get(("body", key))
            if slot is not None and self.em is not None:
                self.em.emit(f"fw{slot}[it_][{self.q}] = {val};")
            return val
        got = self.targets.get((self.part, key))
        if got is not None:
            slot, qmap = got
            q = str(qmap[0]) if len(set(qmap)) == 1 else self.red_index      # one element, or the same index
            return f"fw{slot}[it_][{q}]"
        return super().override_load(ld)

    def loaded(self, ld, name):
        slot = self.sources.get((self.part, ld.key()))
        if slot is not None and self.em is not None:
            self.em.emit(f"fw{slot}[it_][{self.inner()}] = {name};")


class RowStage:
    """How RowBlockPlan.source() runs one kernel of the chain: "block" (every lane accumulates a
    share of the reduction for all E outputs of the row, the shares then combined), "wave" (a
    wavefront per output), "serial" (a lane per output, its reduction in the lane) or "map". The
    lanes walk their index (the reduction's for "block", the outputs' otherwise: N of them) in
    steps of T, `trips` times; a block stage's outputs are finished by lanes 0 .. E-1 (its tail)."""

    def __init__(self, k, R: int, T: int):
        self.k = k
        self.E = ir.prod(v.extent for v in k.domain) // R
        red = k.red
        self.n = ir.prod(v.extent for v in red.vars) if red is not None else 1
        if red is not None and red.op in RED_CODE and self.E <= 16 and self.n >= 256:
            self.form = "block"
        elif red is not None and red.op in RED_CODE and self.E < 64 and self.n > 64:
            self.form = "wave"
        else:
            self.form = "serial" if red is not None else "map"
        self.N = self.n if self.form == "block" else self.E
        self.trips = -(-self.N // T)
        self.split = _row_lane_rules(k.domain, self.E)
        self.itform = False             # the lane loop counts its trips (it_), for forwarding

    def parts(self) -> dict:
        """Each part's loads (with the gathers' index loads): the body is the reduction's
        expression (a block stage's lanes evaluate it for each of the E outputs, a serial stage's
        lane for each reduction element), the statements run once per output."""
        body, stmts = [], []
        if self.k.red is not None:
            _loads_of(self.k.red.body, body)
        for st in self.k.stmts:
            _loads_of(st.value, stmts)
            if isinstance(st, ir.Store):
                A.offset_loads(st.offset, stmts)
        return {"body": body, "stmts": stmts}


def _loads_of(e, out: list) -> None:
    for x in ir.iter_expr(e):
        if isinstance(x, Load):
            out.append(x)
            A.offset_loads(x.offset, out)
        elif isinstance(x, ir.Index):
            A.offset_loads(x.affine, out)


def _row_lane_rules(vars_, E: int):
    """How each variable decoded from row·E + e (e < E) splits into a part that depends on the row
    and one that depends on e: (row divisor, row modulus, row scale, e divisor, e modulus), the
    value being (row // rd) % rm · rs + (e // ed) % em; None if some variable mixes the two."""
    out = []
    for v, P in zip(vars_, ir.row_major_strides([v.extent for v in vars_])):
        X = v.extent
        if P % E == 0:                              # counts rows only
            out.append((P // E, X, 1, 1, 1))
        elif E % P == 0 and (X * P) % E == 0:        # rows (mod X·P/E) above, e // P below
            out.append((1, X * P // E, E // P, P, E // P))
        elif E % P == 0 and E % (X * P) == 0:        # within a row only
            out.append((1, 1, 0, P, X))
        else:
            return None
    return out


def _digits(flat, vars_):
    """Row-major digits of the flattened index (a NumPy array) over vars_."""
    strides = ir.row_major_strides([v.extent for v in vars_])
    return [(flat // s) % v.extent for v, s in zip(vars_, strides)]


class RowBlockPlan(Plan):
    """One workgroup per row (of R) runs a chain of kernels stage by stage. A stage's outputs for
    the row are spread over the workgroup: lane t takes outputs t, t + 256, ... and reduces each one
    alone; a stage with a few outputs and a long reduction instead has every lane accumulate a
    share of the reduction for all of the outputs (so an operand row is read once), the shares
    then combined by shuffles and LDS in a fixed order. Each buffer the chain writes is written in
    the row's own slice; a slice of up to SHADOW elements is also kept in LDS, where later stages
    read it (and a buffer no kernel outside the chain reads is not written to memory at all). A
    barrier separates the stages.

    Operands that no stage writes are loaded once where they can be: a load that a later stage
    repeats in the same lane and trip (C2's logits stage reads h2 and W3 for the row, and the
    input-gradient stages after the softmax read the same h2 and W3 elements again) is forwarded
    in registers (FORWARD_REGS per lane at most), and the loads of one-trip stages (a bias, the
    row's label) are issued before the first stage instead of after the stages before them."""

    kind = "rowblock"
    SHADOW = 2048                   # elements of a row slice kept in LDS
    FORWARD_REGS = 64               # registers per lane holding operands forwarded between stages
    HOIST = 8                       # per-row operand loads issued before the first stage

    def __init__(self, gen, kernels, name, R: int, before: set = frozenset()):
        super().__init__(gen, kernels, name)
        self.R = R
        # 256 lanes per row, or 128 when there are more rows than 256-lane workgroups fit on the
        # chip at once (8 per CU: 2048): all rows then run in one round (C4's 4096-row layer-norm
        # gradients 14.6 -> 10.6 ms over 200 steps; C2's 256 rows lose 1.6 µs a step with 128)
        self.threads = int(os.environ.get("ANVIL_ROWBLOCK_THREADS", "128" if R > 2048 else str(THREADS)))
        self.blocks = min(R, MAX_BLOCKS)
        self.shadow: dict = {}      # buffer id -> row slice (kept in LDS)
        self.before_ids = set(before)
        self.dead: set = set()      # buffers only the chain reads: no memory copy
        readers_in: dict = {}
        for k in kernels:
            for b in A.kernel_reads(k):
                readers_in[b.id] = readers_in.get(b.id, 0) + 1
        total = 0
        for k in kernels:
            for st in k.stores:
                b = st.buf.root
                if b.id in self.shadow:
                    continue
                S = b.numel // R
                # a buffer some stage reads before the chain writes it (`before`: the values of a
                # kernel ahead of the launch, or the target of a `+=`) keeps its memory copy as the
                # only one: an LDS shadow starts empty, so those reads would see no values
                if b.id in before:
                    continue
                dead = (b.kind in A.SHARED_KINDS and not gen.is_host(b) and not getattr(b, "heap", False)
                        and gen.readers.get(b.id, 0) == readers_in.get(b.id, 0))
                accum = any(s2.accumulate and s2.buf.root is b for k2 in kernels for s2 in k2.stores)
                if S > self.SHADOW or total + S > 8192 or (accum and not dead) or not readers_in.get(b.id):
                    continue
                self.shadow[b.id] = S
                total += S
                if dead:
                    self.dead.add(b.id)
        self.stages = [RowStage(k, R, self.threads) for k in kernels]
        self.plan_reuse()
        self.plan_vectors()

    def plan_vectors(self) -> None:
        """In a block stage, the E outputs' loads of one operand that sit side by side in memory
        (C2's logits: lane j reads W3[j, 0..9], 40 contiguous bytes) become E/2 (or E/4) 8- (or
        16-) byte loads, issued before the outputs' blocks: half (a quarter) of the load
        instructions, each touching the same cache lines. Only for the arena's buffers (256-byte
        aligned), when every lane's first element is 2- (4-) aligned in every row and trip."""
        import numpy as np
        n = 0
        for st in self.stages:
            st.vectors = {}
            if st.form != "block" or st.split is None or st.trips > 8 or st.E % 2 or st.E > 16:
                continue
            seen = set()
            for ld in st.parts()["body"]:
                key = ld.key()
                b = ld.buf.root
                if key in seen or b.kind in ir.EXTERN_KINDS or not self.reusable(st, ld, "body"):
                    continue
                seen.add(key)
                row, x, act = self.addresses(st, ld, "body")
                x = np.broadcast_to(x, (self.threads, st.trips, st.E))
                q = np.arange(st.E)
                if not ((x - x[:, :, :1] == q) | ~act[:, :, None]).all():
                    continue                                # not consecutive along the outputs
                first = (row[:, None, None] + x[None, :, :, 0])[:, act]
                for w in (4, 2):
                    if st.E % w == 0 and (first % w == 0).all():
                        st.vectors[key] = (f"vl{n}", w, ld)
                        n += 1
                        break

    # ------------------------------------------------------------------ operand reuse
    def reusable(self, st: RowStage, ld, part: str) -> bool:
        """A load the analysis may move: of memory no stage writes, at an affine offset of the
        stage's own variables."""
        b = ld.buf.root
        if not b.shape or b.id in self.chain_writes or b.id in self.shadow:
            return False
        ok = set(st.k.domain) | (set(st.k.red.vars) if part == "body" and st.k.red is not None else set())
        return all(isinstance(t, Var) and t in ok for t in ld.offset.terms)

    def addresses(self, st: RowStage, ld, part: str):
        """The element each lane loads, split as row part (R,) + lane part (T, trips, I) (I: the
        block stage's outputs, or the serial stage's reduction elements, for the body), with the
        lanes that run the part (T, trips)."""
        import numpy as np
        T, R, k = self.threads, self.R, st.k
        coef = ld.offset.terms
        rows = np.arange(R, dtype=np.int64)
        row = np.full(R, ld.offset.const, dtype=np.int64)
        idx = np.arange(T, dtype=np.int64)[:, None] + T * np.arange(st.trips, dtype=np.int64)[None, :]
        act = idx < st.N
        x = np.zeros(idx.shape + (1,), dtype=np.int64)
        # the domain's variables: e is the output q (a block stage's body) or the lane's index
        e = np.arange(st.E, dtype=np.int64)[None, None, :] if st.form == "block" else idx[:, :, None]
        for v, (rd, rm, rs, ed, em) in zip(k.domain, st.split):
            c = coef.get(v, 0)
            if c:
                row = row + c * rs * ((rows // rd) % rm)
                x = x + c * ((e // ed) % em)
        if st.form == "block":                      # the body: reduction index idx
            for v, d in zip(k.red.vars, _digits(idx, k.red.vars)):
                x = x + coef.get(v, 0) * d[:, :, None]
        else:
            if part == "body":
                r = np.arange(st.n, dtype=np.int64)
                for v, d in zip(k.red.vars, _digits(r, k.red.vars)):
                    x = x + coef.get(v, 0) * d[None, None, :]
        return row, x, act

    def plan_reuse(self) -> None:
        """Choose the forwarded and the hoisted loads (see the class docstring)."""
        import numpy as np
        self.chain_writes = {b.id for k in self.kernels for b in A.kernel_writes(k)}
        T = self.threads
        self.slots: list = []                       # (C type, trips, I) of each forwarding array
        used: dict = {}                             # slot -> {(trip, index)} that later stages read
        cand: list = []                             # loads a later stage may take from registers
        for st in self.stages:
            st.targets, st.sources, st.hoisted = {}, {}, {}
        for si, st in enumerate(self.stages):
            if st.form == "wave" or st.split is None or st.trips > 8:
                continue
            mine = []
            for part, loads in st.parts().items():
                if st.form == "block" and part == "stmts":
                    continue                        # the tail: lanes 0 .. E-1 once (hoisted below)
                I = st.E if st.form == "block" else (st.n if part == "body" else 1)
                if I > 16:
                    continue
                seen = set()
                for ld in loads:
                    key = ld.key()
                    if key in seen or not self.reusable(st, ld, part):
                        continue
                    seen.add(key)
                    row, x, act = self.addresses(st, ld, part)
                    x = np.broadcast_to(x, (T, st.trips, I))
                    match = None
                    for c in cand:
                        if c["buf"] is not ld.buf.root or c["stage"].trips < st.trips:
                            continue
                        d = c["row"] - row
                        if not (d == d[0]).all() or not (c["act"][:, :st.trips] | ~act).all():
                            continue
                        xs = c["x"][:, :st.trips, :] + d[0]
                        qmap = []
                        for r in range(I):
                            ok = ((xs == x[:, :, r][:, :, None]) | ~act[:, :, None]).all(axis=(0, 1))
                            if not ok.any():
                                break
                            qmap.append(int(np.argmax(ok)))
                        # the register is the same element for every index, or the index itself
                        if len(qmap) == I and (len(set(qmap)) == 1 or qmap == list(range(I))):
                            match = (c, qmap)
                            break
                    if match is None:
                        mine.append({"stage": st, "part": part, "key": key, "buf": ld.buf.root, "dtype": ld.dtype,
                                     "row": row, "x": x, "act": act, "slot": None})
                        continue
                    c, qmap = match
                    need = {(t, q) for t in range(st.trips) for q in qmap}
                    slot = c["slot"]
                    extra = need - used.get(slot, set())
                    if sum(len(u) for u in used.values()) + len(extra) > self.FORWARD_REGS:
                        continue
                    if slot is None:
                        slot = c["slot"] = len(self.slots)
                        self.slots.append((ctype(c["dtype"]), c["stage"].trips, c["x"].shape[2]))
                        c["stage"].sources[(c["part"], c["key"])] = slot
                        c["stage"].itform = True
                    used.setdefault(slot, set()).update(need)
                    st.targets[(part, key)] = (slot, qmap)
                    st.itform = True
            cand += mine                            # sources for later stages only
        # per-row operands of one-trip parts: loaded before the first stage
        n = 0
        for si, st in enumerate(self.stages):
            one = st.form == "block" or (st.form in ("map", "serial") and st.trips == 1)
            if not one or st.split is None:
                continue
            for ld in st.parts()["stmts"]:
                key = ld.key()
                if (n >= self.HOIST or key in st.hoisted or ("stmts", key) in st.targets
                        or ("stmts", key) in st.sources or not self.reusable(st, ld, "stmts")):
                    continue
                st.hoisted[key] = (f"hz{n}", ld)
                n += 1

    def grid(self):
        return self.blocks, self.threads

    def row_owned(self, b) -> bool:
        """Does each element of buffer b belong to one lane of one row's workgroup, so that a `+=`
        to it needs no atomic? Every store of the launch to b is at the row-major index of its
        kernel's domain, which is b's size: row r then writes only its own slice of b, one lane per
        element within a stage, and the workgroup's barriers between stages order the stages."""
        for k in self.kernels:
            for o in k.stores:
                if o.buf.root is not b:
                    continue
                off = o.offset
                if off.gathers() or off.scalars() or off.const != 0 or len(off.terms) != len(k.domain):
                    return False
                if ir.prod(v.extent for v in k.domain) != b.numel:
                    return False
                stride = 1
                for v in reversed(k.domain):
                    if off.coef(v) != stride:
                        return False
                    stride *= v.extent
        return True

    def stage_statements(self, em, k, sc, guard=None):
        for st in k.stmts:
            if isinstance(st, ir.Let):
                em.let(st)
                continue
            val = em.store_value(st)
            b = st.buf.root
            off = em.affine(st.offset, st.buf)
            lines = []
            if b.id in self.shadow:
                sh = f"sh{b.id}[{off} - (int)row * {self.shadow[b.id]}]"
                lines.append(f"atomicAdd(&{sh}, {val});" if st.accumulate else f"{sh} = {val};")
            if b.id not in self.dead:
                target = f"{sc.buf(st.buf)}[{off}]"
                if not st.accumulate:
                    lines.append(f"{target} = {val};")
                elif not self.row_owned(b):
                    lines.append(f"atomicAdd(&{target}, {val});")
                elif b.dtype == I32:
                    lines.append(f"{target} = anvil_wrap_add({target}, {val});")
                else:
                    lines.append(f"{target} += {val};")
            for line in lines:
                em.emit(f"if ({guard}) {line}" if guard else line)
            em.reset_memo()

    def wave_only(self, si: int) -> bool:
        """Does stage si run on the first wavefront's lanes alone (one lane per element, at most
        64 of them: a row's 10 logits, its one loss)? Only with $ANVIL_ROWBLOCK_WAVESYNC=1: the
        wave-level fences between such stages measured no faster than the workgroup barriers (C2
        53.2 -> 53.0 us per step, C5 184.3 -> 185.0)."""
        if si >= len(self.stages) or os.environ.get("ANVIL_ROWBLOCK_WAVESYNC", "0") != "1":
            return False
        st = self.stages[si]
        return st.form not in ("block", "wave") and st.N <= 64

    def lane_loop(self, em, st: RowStage, var: str, stride: int, start: str = "threadIdx.x") -> None:
        """The loop of a lane over its share of the stage's index (`var` < N, in steps of stride);
        with itform, a counted loop (it_) whose trips index the forwarding registers."""
        if st.itform:
            em.emit("#pragma unroll")
            em.emit(f"for (int it_ = 0; it_ < {st.trips}; it_++) {{")
            em.emit(f"    const uint32_t {var} = {start} + {stride}u * (uint32_t)it_;")
            if st.N % stride:
                em.emit(f"    if ({var} >= {st.N}u) break;")
            return
        trips = -(-st.N // stride)
        if trips > 1:
            em.emit(f"#pragma unroll {min(4, trips)}")
        em.emit(f"for (uint32_t {var} = {start}; {var} < {st.N}u; {var} += {stride}u) {{")

    def source(self) -> str:
        T = self.threads
        body: list[str] = []
        shared: list[str] = []
        for si, (k, st) in enumerate(zip(self.kernels, self.stages)):
            sc = RowBlockScope(self)
            sc.stream_name = self.stream_param(k)
            sc.targets, sc.sources = st.targets, st.sources
            sc.hoisted = {key: name for key, (name, ld) in st.hoisted.items()}
            sc.vectors = {key: (name, w) for key, (name, w, ld) in getattr(st, "vectors", {}).items()}
            em = Emitter(sc, body, "        ")
            sc.em = em
            E, n, red = st.E, st.n, k.red
            sc.rand = f"(row * {E}u + e)"
            em.emit(f"// stage {si}: {k.name} ({E} per row" + (f", reduce {red.op} of {n}" if red else "") + ")")
            if st.form == "block":
                self.block_stage(em, sc, st, si, shared)
                em.emit("__syncthreads();")
                continue
            wave = st.form == "wave"
            if wave:
                em.emit(f"for (uint32_t e = threadIdx.x >> 6; e < {E}u; e += {T // 64}u) {{")
            else:
                self.lane_loop(em, st, "e", T)
            em.ind += "    "
            for line in decode(k.domain, f"row * {E}u + e", "uint32_t"):
                em.emit(line)
            if red is None:
                self.stage_statements(em, k, sc)
            elif wave:
                dt = red.body.dtype
                ty = ctype(dt)
                em.emit(f"{ty} acc = {red_init(red.op, dt)};")
                em.emit("#pragma unroll 8")
                em.emit(f"for (uint32_t j = lane; j < {n}u; j += 64u) {{")
                em.ind += "    "
                saved = em.memo
                em.memo = dict(saved)
                for line in decode(list(red.vars), "j", "uint32_t"):
                    em.emit(line)
                val = em.ex(red.body)
                em.emit(f"acc = {red_combine(red.op, dt, 'acc', val)};")
                em.memo = saved
                em.ind = em.ind[:-4]
                em.emit("}")
                em.emit(f"acc = anvil_wave_all<{RED_CODE[red.op]}, {ty}>(acc);")
                self.stage_statements(em, k, sc, guard="lane == 0")
            else:
                strides = ir.row_major_strides([v.extent for v in red.vars])
                sc.red_index = " + ".join(f"{s} * v{v.id}" if s != 1 else f"v{v.id}"
                                          for v, s in zip(red.vars, strides)) or "0"
                sc.part = "body"
                serial_reduction(em, sc, k, em.ind, unroll=True)
                sc.part = "stmts"
                self.stage_statements(em, k, sc)
            em.ind = em.ind[:-4]
            em.emit("}")
            if self.wave_only(si) and self.wave_only(si + 1):
                # two stages that only the first wavefront's lanes run: its own lanes' writes are
                # ordered before its later reads without a workgroup barrier (the other waves meet
                # the barrier after the last such stage)
                em.emit("__builtin_amdgcn_fence(__ATOMIC_RELEASE, \"workgroup\"); __builtin_amdgcn_wave_barrier(); "
                        "__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, \"workgroup\");")
            else:
                em.emit("__syncthreads();")
        for bid, S in self.shadow.items():
            shared.append(f"    __shared__ {ctype(self.gen.by_id[bid].dtype)} sh{bid}[{S}];")
        prologue = self.row_prologue()          # before the header: its loads add parameters
        head = [self.comment() + f" · one workgroup per row, {self.R} rows", self.header(T)] + shared + [
                "    const uint32_t lane = threadIdx.x & 63u;",
                "    (void)lane;",
                f"    for (uint32_t row = blockIdx.x; row < {self.R}u; row += gridDim.x) {{"]
        return "\n".join(head + prologue + body + ["    }", "}"])

    def row_prologue(self) -> list[str]:
        """Declarations of the forwarding registers, and the hoisted loads, at the top of a row."""
        out: list[str] = []
        for slot, (ty, trips, I) in enumerate(self.slots):
            out.append(f"        {ty} fw{slot}[{trips}][{I}];")
        for si, st in enumerate(self.stages):
            for key, (name, ld) in st.hoisted.items():
                sc = RowBlockScope(self)
                em = Emitter(sc, out, "        ", prefix=f"p{name}_")
                sc.em = em
                ty = ctype(ld.dtype)
                em.emit(f"{ty} {name} = {'0.0f' if ty == 'float' else '0'};")
                em.emit(f"if (threadIdx.x < {st.E}u) {{      // stage {si}'s lanes")
                em.ind += "    "
                em.emit("const uint32_t e = threadIdx.x;")
                for line in decode(st.k.domain, f"row * {st.E}u + e", "uint32_t"):
                    em.emit(line)
                em.emit(f"{name} = {em.build(ld)};")
                em.ind = em.ind[:-4]
                em.emit("}")
        return out

    def block_stage(self, em, sc, st: RowStage, si, shared):
        """Every lane accumulates its share of the reduction for each of the E outputs; wave
        shuffles, then LDS across the four waves (in wave order), give the sums; lane e finishes
        output e."""
        T = self.threads
        k, E, n = st.k, st.E, st.n
        red = k.red
        dt = red.body.dtype
        ty = ctype(dt)
        shared.append(f"    __shared__ {ty} part{si}[{T // 64}][{E}];")
        em.emit("{")
        em.ind += "    "
        em.emit(f"{ty} acc[{E}];")
        em.emit(f"for (int q = 0; q < {E}; q++) acc[q] = {red_init(red.op, dt)};")
        if st.itform:
            self.lane_loop(em, st, "j", T)
        else:
            em.emit("#pragma unroll 4")
            em.emit(f"for (uint32_t j = threadIdx.x; j < {n}u; j += {T}u) {{")
        em.ind += "    "
        for line in decode(list(red.vars), "j", "uint32_t"):
            em.emit(line)
        for key, (name, w, ld) in getattr(st, "vectors", {}).items():
            vt = f"{ctype(ld.dtype)}{w}"
            em.emit(f"{vt} {name}[{E // w}];")
            em.emit("{")
            em.emit("    const uint32_t e = 0u;")
            for line in decode(k.domain, f"row * {E}u + e", "uint32_t"):
                em.emit("    " + line)
            em.emit(f"    const {vt} *p_ = (const {vt} *)&{sc.buf(ld.buf)}[{em.affine(ld.offset, ld.buf)}];")
            em.emit(f"    for (int u = 0; u < {E // w}; u++) {name}[u] = p_[u];")
            em.emit("}")
        sc.part = "body"
        for q in range(E):
            em.emit("{")
            em.ind += "    "
            saved = em.memo
            em.memo = {}
            sc.q = q
            em.emit(f"const uint32_t e = {q}u;")
            for line in decode(k.domain, f"row * {E}u + e", "uint32_t"):
                em.emit(line)
            val = em.ex(red.body)
            em.emit(f"acc[{q}] = {red_combine(red.op, dt, f'acc[{q}]', val)};")
            em.memo = saved
            em.ind = em.ind[:-4]
            em.emit("}")
        sc.part = "stmts"
        em.ind = em.ind[:-4]
        em.emit("}")
        em.emit(f"for (int q = 0; q < {E}; q++) {{")
        em.emit(f"    const {ty} w_ = anvil_wave_all<{RED_CODE[red.op]}, {ty}>(acc[q]);")
        em.emit(f"    if (lane == 0) part{si}[threadIdx.x >> 6][q] = w_;")
        em.emit("}")
        em.emit("__syncthreads();")
        em.emit(f"if (threadIdx.x < {E}u) {{")
        em.ind += "    "
        em.emit("const uint32_t e = threadIdx.x;")
        for line in decode(k.domain, f"row * {E}u + e", "uint32_t"):
            em.emit(line)
        em.emit(f"{ty} acc_s = part{si}[0][e];")
        em.emit(f"for (int w = 1; w < {T // 64}; w++) acc_s = {red_combine(red.op, dt, 'acc_s', f'part{si}[w][e]')};")
        sc.acc_name = "acc_s"
        em.reset_memo()
        self.stage_statements(em, k, sc)
        em.ind = em.ind[:-4]
        em.emit("}")
        em.ind = em.ind[:-4]
        em.emit("}")


# ----------------------------------------------------------------------------- side by side

def lds_bytes(plan) -> int:
    """Static LDS of a plan's kernel: its own __shared__ arrays plus what its library templates use."""
    src = plan._source if hasattr(plan, "_source") else plan.source()
    plan._source = src
    total = 0
    for typ, dims in re.findall(r"__shared__\s+(\w+)\s+\w+((?:\[\d+\])+)", src):
        total += 4 * ir.prod(int(d) for d in re.findall(r"\d+", dims))
    return total + getattr(plan, "template_lds", lambda: 0)()


KP_LDS = re.compile(r"__shared__ float anvil_kp_lds\[(\d+)\];")
LDS_PER_CU = 160 * 1024


def fused_target(parts):
    """Workgroups per CU for a side-by-side launch of products, or None to keep each part's LDS its
    own (the launch then holds the sum of the parts' arrays). A workgroup runs one part, so the
    parts' partial-tile arrays can share one; the launch's LDS then sets how many workgroups a CU
    holds, chosen by the longest K a workgroup of the launch sums. Measured on the weight-gradient
    launches (step loops): K = 4096 (C4 at T = 256) with one workgroup per CU (the arrays apart)
    1394 us per step, two 1390, three 1421, four 1455; K = 1320 (C5's convolution weight gradient)
    three 201 us, four 197.4, five 199.6, eight 215.6; K = 1024 (C4 at T = 64) one to three 542 us,
    four 537, five 527.5, six 526.8; K = 256 (C2) four 53.2 us (the arrays apart), two 57.8, three
    54.4, five 53.4, seven 54.1.
    A launch with fewer than two such arrays keeps its own. $ANVIL_HIP_FUSED_WGS=<n> sets the
    target, 0 keeps the arrays apart."""
    force = os.environ.get("ANVIL_HIP_FUSED_WGS")
    if force is not None:
        return int(force) or None
    if sum(1 for p in parts if KP_LDS.search(p._source if hasattr(p, "_source") else p.source())) < 2:
        return None                                     # nothing to share
    kwg = max((getattr(p, "kslice", 0) for p in parts if p.kind == "gemm"), default=0)
    if kwg >= 4096:
        return 2
    if kwg > 1024:
        return 4
    if kwg > 512:
        return 6
    return None


def fused_lds(parts) -> int:
    """LDS of parts side by side, as the budget for joining them counts it: the sum of their arrays
    unless they share one at more than two workgroups per CU (C4 at T = 256, two per CU: 1390 us
    per step with the launches the sum allows, 1397.5 with the longer ones the shared size
    allows)."""
    target = fused_target(parts)
    if target is None or target <= 2:
        return sum(lds_bytes(p) for p in parts)
    kp = rest = 0
    for p in parts:
        total = lds_bytes(p)
        m = KP_LDS.search(p._source)
        own = 4 * int(m.group(1)) if m else 0
        kp, rest = max(kp, own), rest + total - own
    return max(kp + rest, lds_for(target))


def lds_for(target: int) -> int:
    """LDS bytes per workgroup that let a CU hold `target` workgroups and no more: the middle of the
    range (160 KB / (target + 1), 160 KB / target]."""
    lo, hi = LDS_PER_CU // (target + 1), LDS_PER_CU // target
    return (lo + hi) // 2 // 256 * 256


def barrier_free(plan) -> bool:
    src = plan._source if hasattr(plan, "_source") else plan.source()
    plan._source = src
    return "__syncthreads" not in src and "__shared__" not in src


def split_params(params: str) -> list[tuple[str, str]]:
    out = []
    for prm in params.split(", "):
        typ, name = prm.rsplit(" ", 1)
        out.append((typ, name))
    return out


class FusedPlan(Plan):
    """Kernels with no data between them (none writes what another reads or writes) launched as one
    grid: workgroup b runs workgroup b - start_j of part j, the part whose range of workgroups holds
    b. Each part's kernel becomes a device function of its workgroup and grid coordinates. The
    launch fills the chip with one part's tail and the next one's start instead of draining it
    between launches, and a short part (a bias gradient) runs beside a long one (a weight gradient).
    Parts use the fused workgroup's lanes; one with fewer lanes runs on the first ones, which it
    may only do if it has no barrier."""

    kind = "fused"

    def __init__(self, gen, parts, name, hoisted):
        super().__init__(gen, [k for p in parts for k in p.kernels], name)
        self.parts = parts
        self.streams = [k for p in parts for k in p.streams]
        self.label = " | ".join(f"{p.name} {p.kind}: {p.label}" for p in parts)
        self.threads = max(p.grid()[1] for p in parts)
        self.hoisted = hoisted
        for p in parts:
            self.skip_stores |= p.skip_stores
        # parts that finish in a second launch (partial tiles or slices, then their sum): those
        # second launches follow this one, side by side in turn
        self.kslices = max(getattr(p, "kslices", 1) for p in parts)
        self.joined_reads: set = set()      # what a second launch that joined this one reads

    def extra_reads(self) -> set:
        """Buffers read beyond the IR kernels of the parts: those of an earlier plan whose second
        launch runs here."""
        return set(self.joined_reads)

    def second(self):
        seconds = [p.second() for p in self.parts if getattr(p, "kslices", 1) > 1]
        return seconds[0] if len(seconds) == 1 else FusedPlan(self.gen, seconds, self.name + "r", [])

    @staticmethod
    def dims(p):
        blocks, _ = p.grid()
        return blocks if isinstance(blocks, tuple) else (blocks, 1, 1)

    def part_params(self, j, p):
        """(fused parameter name, type) of part j's parameters, in its order."""
        out = []
        for typ, name in split_params(p.params()):
            out.append((f"{name}_{j}" if name.startswith("anvil_rs") else name, typ))
        return out

    def params(self) -> str:
        seen: dict = {}
        for j, p in enumerate(self.parts):
            for name, typ in self.part_params(j, p):
                seen.setdefault(name, typ)
        return ", ".join(f"{typ} {name}" for name, typ in seen.items())

    def launch_args(self, stream_vars: list) -> list:
        seen: dict = {}
        at = 0
        for j, p in enumerate(self.parts):
            sv = stream_vars[at:at + len(p.streams)]
            at += len(p.streams)
            for (name, _), arg in zip(self.part_params(j, p), p.launch_args(sv)):
                seen.setdefault(name, arg)
        return list(seen.values())

    def grid(self):
        return sum(ir.prod(self.dims(p)) for p in self.parts), self.threads

    def source(self) -> str:
        texts, calls = [], []
        pool, rest = 0, 0
        target = fused_target(self.parts)
        for j, p in enumerate(self.parts):
            src = p._source if hasattr(p, "_source") else p.source()
            m = KP_LDS.search(src)
            if target is not None:
                rest += lds_bytes(p) - (4 * int(m.group(1)) if m else 0)
            if m and target is not None:
                # a workgroup runs one part: the parts' partial tiles share one LDS array
                pool = max(pool, int(m.group(1)))
                src = src.replace(m.group(0), f"float *const anvil_kp_lds = anvil_fl_{self.name};", 1)
            _, t = p.grid()
            head = f"__global__ void __launch_bounds__({t}) {p.name}("
            assert head in src, p.name
            src = src.replace(head, f"__device__ __forceinline__ void {self.name}_{p.name}(const uint3 anvil_b, "
                                    f"const uint3 anvil_g, ", 1)
            src = src.replace("blockIdx.", "anvil_b.").replace("gridDim.", "anvil_g.")
            texts.append(src)
            gx, gy, gz = self.dims(p)
            n = gx * gy * gz
            args = ", ".join(name for name, _ in self.part_params(j, p))
            guard = "" if t == self.threads else f"if (threadIdx.x < {t}u) "
            calls += [f"    if (b < {n}u) {{",
                      f"        {guard}{self.name}_{p.name}(make_uint3(b % {gx}u, b / {gx}u % {gy}u, b / {gx * gy}u), "
                      f"make_uint3({gx}u, {gy}u, {gz}u), {args});",
                      "        return;",
                      "    }",
                      f"    b -= {n}u;"]
        for p in self.parts:
            self.bufs.update(p.bufs)
            self.hosts.update(p.hosts)
        if pool:
            # sized for the launch's workgroups per CU (fused_target)
            pool = max(pool, (lds_for(target) - rest) // 4)
            texts.insert(0, f"__shared__ float anvil_fl_{self.name}[{pool}];   // the parts' partial tiles, "
                            f"{target} workgroups per CU")
        head = [f"// fused: {', '.join(p.name for p in self.parts)} side by side",
                f"__global__ void __launch_bounds__({self.threads}) {self.name}({self.params()}) {{",
                "    uint32_t b = blockIdx.x;"]
        return "\n\n".join(texts) + "\n" + "\n".join(head + calls[:-1] + ["}"])


# ----------------------------------------------------------------------------- choosing

def inner_contiguous(k: ir.Kernel) -> bool:
    """Do the reduction's loads walk memory with unit stride along its innermost variable?"""
    if k.red is None or not k.red.vars:
        return False
    v = k.red.vars[-1]
    unit = other = 0
    for ld in ir.loads_in(k.red.body):
        if not ld.buf.root.shape:
            continue
        c = ld.offset.coef(v)
        if c == 1:
            unit += 1
        elif c != 0:
            other += 1
    return unit > 0 and unit >= other


def rows_lanes(k: ir.Kernel, emulate: bool) -> int:
    n = ir.prod(v.extent for v in k.red.vars)
    R = ir.prod(v.extent for v in k.domain)
    if emulate or n <= 32 or not inner_contiguous(k):
        return 1
    if n > 1024 or R < CU_WAVES // 4:
        return THREADS
    return 64


def split_ways(k: ir.Kernel, emulate: bool) -> int:
    """TY for a strided reduction (1: a plain rows kernel with one lane per output)."""
    if emulate or k.red is None or k.red.op in ("argmax", "argmin"):
        return 1
    n = ir.prod(v.extent for v in k.red.vars)
    R = ir.prod(v.extent for v in k.domain)
    if n < 64 or inner_contiguous(k) or R >= 64 * CU_WAVES:
        return 1
    for ty in (16, 8, 4, 2):
        if n >= 16 * ty:
            return ty
    return 1


# ----------------------------------------------------------------------------- slices

def slice_count(k: ir.Kernel, emulate: bool) -> int:
    """S for a reduction with few outputs and a long, contiguous sum (a convolution's bias or weight
    gradient: 32 outputs of 86528 terms), reduced in S slices per output by as many workgroups and
    the slices then added in order (the reference's two-pass split, cuda.py:282-345); 1: not so."""
    if emulate or k.red is None or k.red.op not in RED_CODE or k.uses_rand() or not k.domain:
        return 1
    n = ir.prod(v.extent for v in k.red.vars)
    R = ir.prod(v.extent for v in k.domain)
    if R > 1024 or n < 8192 or not inner_contiguous(k):
        return 1
    S = max(2, min(2048 // R, n // 2048))
    return S if R * S <= MAX_BLOCKS else 1


class SlicePlan(Plan):
    """Workgroup (r, s) reduces slice s of output r's terms (256 lanes, then across the workgroup)
    into partial[s][r]; SliceSumPlan, the next launch, adds each output's S partials in slice order
    (the result does not depend on timing) and runs the kernel's statements."""

    kind = "slices"

    def __init__(self, gen, k, name, S):
        super().__init__(gen, [k], name)
        self.k = k
        self.R = ir.prod(v.extent for v in k.domain)
        self.n = ir.prod(v.extent for v in k.red.vars)
        self.kslices = S
        self.chunk = -(-self.n // S)

    def ws_buffer(self):
        """The partials, [slice][output]."""
        if not hasattr(self, "_ws"):
            self._ws = A.new_buffer(810_000_000 + self.k.id, f"{self.name}.partials", (self.kslices * self.R,),
                                    self.k.red.body.dtype, "scratch")
        return self._ws

    def second(self):
        return SliceSumPlan(self)

    def source(self) -> str:
        k, red = self.k, self.k.red
        T, dt = ctype(red.body.dtype), red.body.dtype
        sc = KernelScope(self)
        sc.stream_name = self.stream_param(k)
        body: list[str] = []
        em = Emitter(sc, body, "    ")
        em.emit(f"__shared__ {T} sv[4];")
        em.emit(f"const uint32_t r = blockIdx.x % {self.R}u, s = blockIdx.x / {self.R}u;")
        for line in decode(k.domain, "r", "uint32_t"):
            em.emit(line)
        em.emit(f"{T} acc = {red_init(red.op, dt)};")
        em.emit(f"const uint32_t jb = s * {self.chunk}u, je = min({self.n}u, jb + {self.chunk}u);")
        em.emit("#pragma unroll 4")
        em.emit("for (uint32_t j = jb + threadIdx.x; j < je; j += 256u) {")
        em.ind += "    "
        saved = em.memo
        em.memo = dict(saved)
        for line in decode(list(red.vars), "j", "uint32_t"):
            em.emit(line)
        val = em.ex(red.body)
        em.emit(f"acc = {red_combine(red.op, dt, 'acc', val)};")
        em.memo = saved
        em.ind = em.ind[:-4]
        em.emit("}")
        em.emit(f"acc = anvil_block_all<{RED_CODE[red.op]}, {T}>(acc, sv);")
        em.emit(f"if (threadIdx.x == 0) {sc.buf(self.ws_buffer())}[s * {self.R}u + r] = acc;")
        head = [self.comment() + f" · {self.R} outputs x {self.kslices} slices of {self.chunk}, added by "
                f"{self.name}s", self.header(THREADS)]
        return "\n".join(head + body + ["}"])

    def grid(self):
        return self.R * self.kslices, THREADS


class SliceSumPlan(Plan):
    """The second launch of a sliced reduction: each output's partials added in slice order, then
    the kernel's statements with that sum as the reduction's value."""

    kind = "slices-sum"

    def __init__(self, first: SlicePlan):
        super().__init__(first.gen, [], first.name + "s")
        self.first = first
        self.label = "slice sum + " + first.label
        self.blocks = max(1, min(-(-first.R // THREADS), MAX_BLOCKS))
        self.streams = list(first.streams)

    def source(self) -> str:
        f, k = self.first, self.first.k
        red = k.red
        T, dt = ctype(red.body.dtype), red.body.dtype
        self.skip_stores = f.skip_stores
        sc = KernelScope(self)
        sc.stream_name = f.stream_param(k)
        ws = sc.buf(f.ws_buffer())
        body: list[str] = []
        em = Emitter(sc, body, "        ")
        em.emit(f"{T} sum = {ws}[e];")
        em.emit(f"for (uint32_t sl = 1; sl < {f.kslices}u; sl++) "
                f"sum = {red_combine(red.op, dt, 'sum', f'{ws}[sl * {f.R}u + e]')};")
        for line in decode(k.domain, "e", "uint32_t"):
            em.emit(line)
        sc.acc_name = "sum"
        sc.rand = "e"
        self.statements(em, k, sc, parallel=True)
        head = [f"// slices-sum: {f.name}: the {f.kslices} partials of each of {f.R} outputs added in order, "
                "then the kernel's statements", self.header(THREADS),
                f"    for (uint32_t e = blockIdx.x * {THREADS}u + threadIdx.x; e < {f.R}u; "
                f"e += gridDim.x * {THREADS}u) {{"]
        return "\n".join(head + body + ["    }", "}"])

    def grid(self):
        return self.blocks, THREADS


# ----------------------------------------------------------------------------- row groups

class GroupBuilder:
    """Decides which consecutive kernels can be stages of one rows kernel."""

    def __init__(self, head: ir.Kernel):
        self.kernels = [head]
        self.outer_ext = [v.extent for v in head.domain]
        self.inner_ext = [v.extent for v in head.red.vars]
        self.stores: dict = {}          # buffer id -> canonical offset key of its stores
        self.reads: dict = {}           # buffer id -> set of canonical offset keys read
        self._note(head)

    def canon(self, k):
        if k.red is not None:
            outer, inner = list(k.domain), list(k.red.vars)
        else:
            no = len(self.outer_ext)
            outer, inner = list(k.domain[:no]), list(k.domain[no:])
        m = {v: ("o", i) for i, v in enumerate(outer)}
        m.update({v: ("i", i) for i, v in enumerate(inner)})
        return m

    def _note(self, k):
        cm = self.canon(k)
        for ld in A.kernel_loads(k):
            self.reads.setdefault(ld.buf.root.id, set()).add(canon_key(ld.buf, ld.offset, cm))
        for st in k.stores:
            self.stores[st.buf.root.id] = canon_key(st.buf, st.offset, cm)

    def fits(self, k: ir.Kernel, hosts: set) -> bool:
        if A.is_host_kernel(k, hosts) or not A.parallel_safe(k):
            return False
        if any(st.accumulate or st.offset.gathers() for st in k.stores):
            return False
        if k.red is not None:
            if [v.extent for v in k.domain] != self.outer_ext or [v.extent for v in k.red.vars] != self.inner_ext:
                return False
        else:
            no = len(self.outer_ext)
            ext = [v.extent for v in k.domain]
            if ext[:no] != self.outer_ext or ext[no:] not in ([], self.inner_ext):
                return False
        cm = self.canon(k)
        # reads of what the group wrote must be the elements this lane wrote
        for ld in A.kernel_loads(k):
            bid = ld.buf.root.id
            if bid in self.stores:
                key = canon_key(ld.buf, ld.offset, cm)
                if key is None or key != self.stores[bid]:
                    return False
        scal: set = set()
        for e in k.exprs():
            for x in ir.iter_expr(e):
                if isinstance(x, Load):
                    A.affine_scalars(x.offset, scal)
        for st in k.stores:
            A.affine_scalars(st.offset, scal)
        if any(b.id in self.stores for b in scal):
            return False
        # no earlier stage may read what this one writes, and one place per buffer
        for st in k.stores:
            bid = st.buf.root.id
            if bid in self.reads:
                return False
            key = canon_key(st.buf, st.offset, cm)
            if key is None or (bid in self.stores and self.stores[bid] != key):
                return False
        return True

    def add(self, k):
        self.kernels.append(k)
        self._note(k)


# ----------------------------------------------------------------------------- twins

class TwinPlan(Plan):
    """The device twin of a scalar kernel the host runs: it updates the device copy of the host
    scalars (the array kernels read them from), so that a captured graph needs no host values."""

    kind = "twin"

    def by_value(self) -> bool:
        return False

    def __init__(self, gen, k, name):
        super().__init__(gen, [k], name)
        self.k = k

    def source(self) -> str:
        k = self.k
        sc = KernelScope(self)
        body: list[str] = []
        em = Emitter(sc, body, "    ")
        for st in k.stmts:
            if isinstance(st, ir.Let):
                em.let(st)
                continue
            val = em.store_value(st)
            b = st.buf.root
            h = sc.host_scalar(b)
            slot = self.gen.hsd_slot(b)
            bits = f"(uint32_t)({val})" if b.dtype == I32 else f"anvil_bits_of({val})"
            em.emit(f"{h} = {val}; anvil_hsd[{slot}] = {bits};")
            em.reset_memo()
        for st in k.stores:                               # make sure it is a parameter
            sc.host_scalar(st.buf.root)
        head = [f"// twin of the host's {k.name}",
                f"__global__ void __launch_bounds__(64) {self.name}({self.params()}) {{"] + self.host_prologue(True)
        return "\n".join(head + ["    if (threadIdx.x != 0 || blockIdx.x != 0) return;"] + body + ["}"])

    def grid(self):
        return 1, 64

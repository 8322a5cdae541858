"""Attention as one kernel: the IR chain S = scale·Q Kᵀ → softmax over S's rows → O = P V becomes
anvil_attention_tile (hip_rt/anvil_mfma.h), which never writes S or P.

The chain is what the reference's front end lowers `softmax(q @ kᵀ · scale) @ v` into
(prelude.anvil softmax: m = detach(max), e = exp(s - m), e / Σe; ops.py:366-469): six kernels,

    s[b, i, j] = Σ_c scale · q[b, i, c] · k[b, j, c]      (a batched product, K = D)
    m[r]       = max_j s[r, j]                            (r = b·Lq + i)
    e[r, j]    = exp(s[r, j] - m[r])
    t[r]       = Σ_j e[r, j]
    p[r, j]    = e[r, j] / t[r]
    o[b, i, d] = Σ_j p[b, i, j] · v[b, j, d]              (a batched product, K = Lk)

matched on the IR's structure, and only when no other statement reads s, m, e, t or p (they then
take no memory at all). Every buffer is row-major and contiguous; D is 64 or 128; Lq is a multiple
of 32 and Lk of 128 (four waves × 32-key tiles).
"""
from __future__ import annotations

from .. import ir
from ..ir import Binary, KernelStmt, Load, Unary, Var
from . import hip_analysis as A
from .hip_emit import flit
from .hip_kernels import Plan


def _strides_ok(off: ir.Affine, vars_and_strides) -> bool:
    want = ir.Affine(0, {v: s for v, s in vars_and_strides if v.extent > 1})
    return off == want


def _row_major(k: ir.Kernel, shape):
    """(row var, col var) form check: the kernel's domain walks a row-major [R, C] array, either as
    two variables or one flattened one. Returns a function offset -> (is the element (r, c) at
    r·C + c, is the row r) tests, or None."""
    return None


def _acc_only(e) -> bool:
    """An expression that is the reduction's value, possibly through lets and detach."""
    if isinstance(e, ir.Acc):
        return True
    if isinstance(e, ir.LetRef):
        return _acc_only(e.let.value)
    if isinstance(e, Unary) and e.op == "detach":
        return _acc_only(e.a)
    return False


def _only_store(k: ir.Kernel):
    stores = [st for st in k.stmts if isinstance(st, ir.Store)]
    if len(stores) != 1 or stores[0].accumulate:
        return None
    return stores[0]


def _elementwise_rows(k: ir.Kernel, R: int, C: int):
    """For a kernel over an [R, C] row-major domain (two variables, or one of extent R·C): the
    affine of element (r, c) and of row r, in the kernel's variables; else None."""
    if len(k.domain) == 2 and [v.extent for v in k.domain] == [R, C]:
        r, c = k.domain
        return ir.Affine(0, {r: C, c: 1}) if C > 1 else ir.Affine(0, {r: 1}), ir.Affine(0, {r: 1})
    if len(k.domain) == 1 and k.domain[0].extent == R * C:
        return None                      # a flattened domain: the row is not affine
    return None


def match(gen, stmts: list, i: int):
    """An AttnPlan for stmts[i:i+6], or None."""
    from .hip_gemm import analyse
    if gen.emulate or i + 6 > len(stmts):
        return None
    if not all(isinstance(st, KernelStmt) for st in stmts[i:i + 6]):
        return None
    ks, km, ke, kt, ko, kpv = (st.kernel for st in stmts[i:i + 6])
    if any(A.is_host_kernel(k, gen.hosts) for k in (ks, km, ke, kt, ko, kpv)):
        return None
    s = analyse(ks)
    if s is None or len(s.batch) > 1 or len(s.m_vars) != 1 or len(s.n_vars) != 1 or len(s.k_vars) != 1:
        return None
    if s.a_gather or s.b_gather or s.ea is not s.la or s.eb is not s.lb:
        return None
    D, Lq, Lk, B = s.K, s.M, s.N, s.B
    if D not in (64, 128) or Lq % 32 or Lk % 128 or s.a_ks != 1 or s.b_ks != 1 or s.a_rs != D or s.b_rs != D:
        return None
    Q, K = s.la.buf.root, s.lb.buf.root
    bv = s.batch[0] if s.batch else None
    iv, jv = s.m_vars[0], s.n_vars[0]
    if s.la.offset != ir.Affine(0, {**({bv: Lq * D} if bv is not None and B > 1 else {}), iv: D, s.k_vars[0]: 1}):
        return None
    if s.lb.offset != ir.Affine(0, {**({bv: Lk * D} if bv is not None and B > 1 else {}), jv: D, s.k_vars[0]: 1}):
        return None
    st = _only_store(ks)
    if st is None or not _acc_only(st.value):
        return None
    S = st.buf.root
    if st.offset != ir.Affine(0, {**({bv: Lq * Lk} if bv is not None and B > 1 else {}), iv: Lk, jv: 1}):
        return None
    R = B * Lq
    # m[r] = max_j s[r, j]
    if km.red is None or km.red.op != "max" or len(km.domain) != 1 or km.domain[0].extent != R:
        return None
    if len(km.red.vars) != 1 or km.red.vars[0].extent != Lk:
        return None
    r0, j0 = km.domain[0], km.red.vars[0]
    body = km.red.body
    if not (isinstance(body, Load) and body.buf.root is S and body.offset == ir.Affine(0, {r0: Lk, j0: 1})):
        return None
    st = _only_store(km)
    if st is None or not _acc_only(st.value) or st.offset != ir.Affine(0, {r0: 1}):
        return None
    M = st.buf.root
    # e[r, j] = exp(s[r, j] - m[r])
    rows = _elementwise_rows(ke, R, Lk)
    st = _only_store(ke)
    if rows is None or st is None or ke.red is not None:
        return None
    el, row = rows
    x = st.value
    if not (isinstance(x, Unary) and x.op == "exp" and isinstance(x.a, Binary) and x.a.op == "sub"):
        return None
    a, b = x.a.a, x.a.b
    if not (isinstance(a, Load) and a.buf.root is S and a.offset == el
            and isinstance(b, Load) and b.buf.root is M and b.offset == row and st.offset == el):
        return None
    E = st.buf.root
    # t[r] = Σ_j e[r, j]
    if kt.red is None or kt.red.op != "sum" or len(kt.domain) != 1 or kt.domain[0].extent != R:
        return None
    if len(kt.red.vars) != 1 or kt.red.vars[0].extent != Lk:
        return None
    r1, j1 = kt.domain[0], kt.red.vars[0]
    body = kt.red.body
    if not (isinstance(body, Load) and body.buf.root is E and body.offset == ir.Affine(0, {r1: Lk, j1: 1})):
        return None
    st = _only_store(kt)
    if st is None or not _acc_only(st.value) or st.offset != ir.Affine(0, {r1: 1}):
        return None
    T = st.buf.root
    # p[r, j] = e[r, j] / t[r]
    rows = _elementwise_rows(ko, R, Lk)
    st = _only_store(ko)
    if rows is None or st is None or ko.red is not None:
        return None
    el, row = rows
    x = st.value
    if not (isinstance(x, Binary) and x.op == "div" and isinstance(x.a, Load) and x.a.buf.root is E
            and x.a.offset == el and isinstance(x.b, Load) and x.b.buf.root is T and x.b.offset == row
            and st.offset == el):
        return None
    P = st.buf.root
    # o[b, i, d] = Σ_j p[b, i, j] · v[b, j, d]
    s2 = analyse(kpv)
    if s2 is None or s2.a_gather or s2.b_gather or s2.alpha != 1.0 or s2.ea is not s2.la or s2.eb is not s2.lb:
        return None
    if (s2.M, s2.N, s2.K, s2.B) != (Lq, D, Lk, B) or s2.la.buf.root is not P:
        return None
    if len(s2.batch) > 1 or len(s2.m_vars) != 1 or len(s2.n_vars) != 1 or len(s2.k_vars) != 1:
        return None
    b2 = s2.batch[0] if s2.batch else None
    i2, d2, l2 = s2.m_vars[0], s2.n_vars[0], s2.k_vars[0]
    bt = lambda n: {b2: n} if b2 is not None and B > 1 else {}
    if s2.la.offset != ir.Affine(0, {**bt(Lq * Lk), i2: Lk, l2: 1}):
        return None
    V = s2.lb.buf.root
    if s2.lb.offset != ir.Affine(0, {**bt(Lk * D), l2: D, d2: 1}):
        return None
    st = _only_store(kpv)
    if st is None or not _acc_only(st.value) or st.offset != ir.Affine(0, {**bt(Lq * D), i2: D, d2: 1}):
        return None
    O = st.buf.root
    # s, m, e, t, p: only this chain reads them
    chain = (ks, km, ke, kt, ko, kpv)
    for X in (S, M, E, T, P):
        inside = sum(1 for k in chain if X in A.kernel_reads(k))
        if gen.readers.get(X.id, 0) != inside or X.kind not in A.SHARED_KINDS or gen.is_host(X):
            return None
    if len({Q.id, K.id, V.id, O.id}) != 4 and O.id in (Q.id, K.id, V.id):
        return None
    return AttnPlan(gen, list(chain), f"k{ks.id}", Q, K, V, O, s.alpha, B, Lq, Lk, D)


class AttnPlan(Plan):
    kind = "attention"

    def __init__(self, gen, kernels, name, Q, K, V, O, scale, B, Lq, Lk, D):
        super().__init__(gen, kernels, name)
        self.Q, self.K, self.V, self.O = Q, K, V, O
        self.scale, self.B, self.Lq, self.Lk, self.D = scale, B, Lq, Lk, D
        # every store but the output's is dropped
        for k in kernels[:-1]:
            for idx, st in enumerate(k.stmts):
                if isinstance(st, ir.Store):
                    self.skip_stores.add((k.id, idx))
        self.threads = 256

    def grid(self):
        return (self.Lq // 32, self.B, 1), self.threads

    def source(self) -> str:
        q, k, v, o = (self.use_buf(b) for b in (self.Q, self.K, self.V, self.O))
        D, Lq, Lk = self.D, self.Lq, self.Lk
        return "\n".join([
            f"// attention: {' + '.join(k.name for k in self.kernels)} · {self.B} x ({Lq} x {Lk}, D = {D}) · "
            "S and P stay in registers",
            self.header(self.threads),
            "    const long long b = blockIdx.y;",
            f"    anvil_attention_tile<{D}>({q} + b * {Lq * D}LL, {k} + b * {Lk * D}LL, {v} + b * {Lk * D}LL, "
            f"{o} + b * {Lq * D}LL, {flit(self.scale)}, {Lq}, {Lk}, blockIdx.x * 32);",
            "}"])

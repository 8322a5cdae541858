"""Causal self-attention for training in three launches (hip_rt/anvil_attn_train.h), with the scores,
the probabilities and their gradients never in memory.

The reference's transformer (examples/transformer.anvil:29-36: `s = q @ kᵀ · scale − 1e9 · (u > t)`,
`p = softmax(s)`, `mix = p @ v`, softmax as prelude.anvil:28-32 defines it) reaches the backend as
two runs of kernels, the forward six (ops.py's kernels for a batched product, a max, exp, a sum, a
division, a batched product)

    score[n, h, t, u] = Σ_c alpha · Q[n, t, h, c] · K[n, u, h, c] − C · (u > t)
    m[r]    = max_j score[r, j]                   r = (n, h, t) flattened
    e[r, j] = exp(score[r, j] − m[r])
    l[r]    = Σ_j e[r, j]
    p[r, j] = e[r, j] / l[r]
    O[n, t, h, c] = Σ_u p[n, h, t, u] · V[n, u, h, c]

and, where the program trains, their adjoints (autodiff.py) as eight more, in this order:

    G = 0                                         G: the gradient of the buffer holding Q, K, V
    G[V][n, u, h, c] += Σ_t dO[n, t, h, c] · p[n, h, t, u]
    dp[n, h, t, u] = Σ_c dO[n, t, h, c] · V[n, u, h, c];   de = dp · (1 / l[r])
    dl[r] = Σ_j dp[r, j] · (−p[r, j] / l[r])
    de[r, j] += dl[r]
    ds = de · e
    G[Q][n, t, h, c] += Σ_u ds[n, h, t, u] · (alpha · K[n, u, h, c])
    G[K][n, u, h, c] += Σ_t ds[n, h, t, u] · (alpha · Q[n, t, h, c])

Both runs are matched on the IR's structure (expression trees, the layouts of every access, and
that no other statement reads score, m, e, p, dp, de, dl or ds), only together, only where T is a
multiple of 32 no larger than 256 and a head's width D is 32 or 64, and only with C ≥ 1e6 (so that
exp of a masked score is 0 in float32, as the kernels assume). The forward launch then writes O, m
(in base 2) and l; the backward's two launches write all of G (its zeroing is not needed) from Q,
K, V, O, dO, m and l. Q, K, V and G share one layout (element (n, t, h, c) at a fixed offset plus
n·qn + t·qs + h·qh + c), as do O and dO.
"""
from __future__ import annotations

import os

import numpy as np

from .. import ir
from ..ir import Binary, KernelStmt, Load, Unary
from . import hip_analysis as A
from .hip_emit import flit
from .hip_kernels import Plan

MIN_MASK = 1e6


# ------------------------------------------------------------------------------ expression shapes

def _see(e):
    """e through lets (a kernel's named values are the expressions they name)."""
    while isinstance(e, ir.LetRef):
        e = e.let.value
    return e


def _unify(e, pat, env) -> bool:
    """Does expression e have the shape pat? Patterns: ("load", key) binds a Load, ("const", key) a
    constant, ("index", key) an index expression; ("acc",) is the reduction's value; ("?detach", p)
    matches p with or without a detach around it; (op, p, q...) a unary or binary operation (mul
    either way round). A key bound twice must bind equal things."""
    e = _see(e)
    tag = pat[0]
    if tag == "?detach":
        if isinstance(e, Unary) and e.op == "detach":
            e = _see(e.a)
        return _unify(e, pat[1], env)
    if tag in ("load", "const", "index"):
        cls = {"load": Load, "const": ir.Const, "index": ir.Index}[tag]
        if not isinstance(e, cls) or (tag != "index" and e.dtype != ir.F32):
            return False
        key = pat[1]
        if key in env:
            old = env[key]
            if tag == "load":
                return old.buf.root is e.buf.root and old.offset == e.offset
            if tag == "const":
                return old.value == e.value
            return old.affine == e.affine
        env[key] = e
        return True
    if tag == "acc":
        return isinstance(e, ir.Acc)
    if len(pat) == 2:
        return isinstance(e, Unary) and e.op == tag and _unify(e.a, pat[1], env)
    if not (isinstance(e, Binary) and e.op == tag):
        return False
    for a, b in ((e.a, e.b), (e.b, e.a)) if tag == "mul" else ((e.a, e.b),):
        trial = dict(env)
        if _unify(a, pat[1], trial) and _unify(b, pat[2], trial):
            env.clear()
            env.update(trial)
            return True
    return False


def _stores(k: ir.Kernel):
    return [st for st in k.stmts if isinstance(st, ir.Store)]


def _terms(off: ir.Affine) -> dict:
    return dict(off.terms)


def _is(off: ir.Affine, const: int, terms: dict) -> bool:
    return off.const == const and _terms(off) == {v: c for v, c in terms.items() if c != 0}


def _by_coef(k_vars, off: ir.Affine, coefs: list):
    """The variables of k_vars whose coefficients in off are coefs (in order), or None."""
    t = _terms(off)
    out = []
    for c in coefs:
        hit = [v for v in k_vars if t.get(v) == c and v not in out]
        if len(hit) != 1:
            return None
        out.append(hit[0])
    return out


# ------------------------------------------------------------------------------ matching

class _Shape:
    """B, H, T, D and the layouts found so far."""


def _score_kernel(k: ir.Kernel, sh: _Shape):
    """score = Σ_c alpha · Q · K − C · (u > t), stored row-major [n, h, t, u]."""
    if k.red is None or k.red.op != "sum" or len(k.red.vars) != 1 or len(k.domain) != 4:
        return None
    (c,) = k.red.vars
    env: dict = {}
    if not _unify(k.red.body, ("mul", ("const", "alpha"), ("mul", ("load", "x"), ("load", "y"))), env):
        return None
    sts = _stores(k)
    if len(sts) != 1 or sts[0].accumulate:
        return None
    st = sts[0]
    if not _unify(st.value, ("sub", ("acc",), ("mul", ("const", "C"), ("gt", ("index", "key"), ("index", "query")))), env):
        return None
    if env["C"].value < MIN_MASK:
        return None
    kv, qv = _terms(env["key"].affine), _terms(env["query"].affine)
    if env["key"].affine.const or env["query"].affine.const or len(kv) != 1 or len(qv) != 1:
        return None
    (u, cu), = kv.items()
    (t, ct), = qv.items()
    if cu != 1 or ct != 1 or u is t or u not in k.domain or t not in k.domain:
        return None
    T, D = t.extent, c.extent
    if u.extent != T:
        return None
    rest = [v for v in k.domain if v is not t and v is not u]
    S = st.buf.root
    st_t = _terms(st.offset)
    if st.offset.const or st_t.get(u) != 1 or st_t.get(t) != T:
        return None
    hv = [v for v in rest if st_t.get(v) == T * T]
    if len(hv) != 1:
        return None
    h = hv[0]
    H = h.extent
    nv = [v for v in rest if v is not h]
    n = nv[0]
    B = n.extent
    if st_t.get(n) != H * T * T or len(st_t) != 4:
        return None
    # Q is the load over t, K the one over u
    x, y = env["x"], env["y"]
    if t in _terms(y.offset):
        x, y = y, x
    lay = []
    for ld, row in ((x, t), (y, u)):
        tt = _terms(ld.offset)
        if set(tt) != {n, h, row, c} or tt[c] != 1:
            return None
        lay.append((ld.buf.root, ld.offset.const, tt[n], tt[h], tt[row]))
    (qb, q0, qn, qh, qs), (kb, k0, kn, kh, ks) = lay
    if qb is not kb or (qn, qh, qs) != (kn, kh, ks):
        return None
    sh.B, sh.H, sh.T, sh.D = B, H, T, D
    sh.alpha = env["alpha"].value
    sh.QKV, sh.q0, sh.k0, sh.qn, sh.qh, sh.qs = qb, q0, k0, qn, qh, qs
    sh.S = S
    return sh


def _row_reduce(k: ir.Kernel, op: str, src, R: int, T: int):
    """out[r] = op_j src[r·T + j]: the output buffer, or None."""
    if k.red is None or k.red.op != op or len(k.domain) != 1 or k.domain[0].extent != R:
        return None
    if len(k.red.vars) != 1 or k.red.vars[0].extent != T:
        return None
    r, j = k.domain[0], k.red.vars[0]
    body = _see(k.red.body)
    if not (isinstance(body, Load) and body.buf.root is src and _is(body.offset, 0, {r: T, j: 1})):
        return None
    sts = _stores(k)
    if len(sts) != 1 or sts[0].accumulate or not isinstance(_see(sts[0].value), ir.Acc):
        return None
    if not _is(sts[0].offset, 0, {r: 1}):
        return None
    return sts[0].buf.root


def _rows_map(k: ir.Kernel, R: int, T: int, pat, binds: dict):
    """A kernel over (r, j) of R x T storing pat (whose ("load", "el"/"row") keys are the element and
    row of the domain) at element (r, j); binds[key] = buffer for each other load key. Returns the
    stored buffer."""
    if k.red is not None or len(k.domain) != 2 or [v.extent for v in k.domain] != [R, T]:
        return None
    r, j = k.domain
    sts = _stores(k)
    if len(sts) != 1 or sts[0].accumulate or not _is(sts[0].offset, 0, {r: T, j: 1}):
        return None
    env: dict = {}
    if not _unify(sts[0].value, pat, env):
        return None
    for key, ld in env.items():
        want = binds.get(key)
        if not isinstance(ld, Load) or want is None:
            continue
        buf, kind = want
        off = {r: T, j: 1} if kind == "el" else {r: 1}
        if ld.buf.root is not buf or not _is(ld.offset, 0, off):
            return None
    if any(key not in env for key in binds):
        return None
    return sts[0].buf.root


def _pv_kernel(k: ir.Kernel, sh: _Shape, P):
    """O[n, t, h, c] = Σ_u P[n, h, t, u] · V[n, u, h, c]."""
    B, H, T, D = sh.B, sh.H, sh.T, sh.D
    if k.red is None or k.red.op != "sum" or len(k.red.vars) != 1 or len(k.domain) != 4:
        return None
    (u,) = k.red.vars
    env: dict = {}
    if not _unify(k.red.body, ("mul", ("load", "p"), ("load", "v")), env):
        return None
    p, v = env["p"], env["v"]
    if p.buf.root is not P:
        p, v = v, p
    if p.buf.root is not P or u.extent != T:
        return None
    got = _by_coef(k.domain, p.offset, [H * T * T, T * T, T])
    if got is None or p.offset.const or _terms(p.offset).get(u) != 1 or len(_terms(p.offset)) != 4:
        return None
    n, h, t = got
    c = [x for x in k.domain if x not in (n, h, t)][0]
    if (n.extent, h.extent, t.extent, c.extent) != (B, H, T, D):
        return None
    vt = _terms(v.offset)
    if v.buf.root is not sh.QKV or vt != {x: y for x, y in ((n, sh.qn), (h, sh.qh), (u, sh.qs), (c, 1))}:
        return None
    sts = _stores(k)
    if len(sts) != 1 or sts[0].accumulate or not isinstance(_see(sts[0].value), ir.Acc):
        return None
    ot = _terms(sts[0].offset)
    if set(ot) != {n, h, t, c} or ot[c] != 1:
        return None
    sh.v0 = v.offset.const
    sh.O, sh.o0, sh.on, sh.oh, sh.os = sts[0].buf.root, sts[0].offset.const, ot[n], ot[h], ot[t]
    return sh


def _qkv_at(sh, off: ir.Affine, n, h, row, c, base) -> bool:
    return _is(off, base, {n: sh.qn, h: sh.qh, row: sh.qs, c: 1})


def _o_at(sh, off: ir.Affine, n, h, t, c) -> bool:
    return _is(off, sh.o0, {n: sh.on, h: sh.oh, t: sh.os, c: 1})


def _s_at(sh, off: ir.Affine, n, h, t, u) -> bool:
    T = sh.T
    return _is(off, 0, {n: sh.H * T * T, h: T * T, t: T, u: 1})


def _vars4(k: ir.Kernel, red_extent: int):
    """(domain vars, the reduction var) of a product over a 4-variable domain."""
    if k.red is None or k.red.op != "sum" or len(k.red.vars) != 1 or len(k.domain) != 4:
        return None
    if k.red.vars[0].extent != red_extent:
        return None
    return list(k.domain), k.red.vars[0]


def _slices_tile(sh: _Shape, numel: int) -> bool:
    """Do the Q, K and V slices of QKV cover each of its numel elements exactly once? The fused
    backward writes dQ, dK and dV with plain stores at those offsets of G (same layout as QKV) in
    place of the chain's `G = 0` and its three `+=`: with two slices at one place (Q and K read
    from the same columns) their gradients would overwrite each other instead of adding, and an
    element no slice covers (a fourth, unused slice) would keep stale memory instead of 0."""
    B, H, T, D = sh.B, sh.H, sh.T, sh.D
    rel = (np.arange(B, dtype=np.int64)[:, None, None, None] * sh.qn
           + np.arange(H, dtype=np.int64)[None, :, None, None] * sh.qh
           + np.arange(T, dtype=np.int64)[None, None, :, None] * sh.qs
           + np.arange(D, dtype=np.int64)[None, None, None, :]).reshape(-1)
    hits = np.zeros(numel, dtype=np.int64)
    for base in (sh.q0, sh.k0, sh.v0):
        at = rel + base
        if at.min() < 0 or at.max() >= numel:
            return False
        hits += np.bincount(at, minlength=numel)
    return bool((hits == 1).all())


def _backward(gen, stmts: list, j: int, sh: _Shape):
    """The eight backward kernels at stmts[j:j+8] for the forward described by sh, or None."""
    if j + 8 > len(stmts) or not all(isinstance(st, KernelStmt) for st in stmts[j:j + 8]):
        return None
    k0, k1, k2, k3, k4, k5, k6, k7 = (st.kernel for st in stmts[j:j + 8])
    if any(A.is_host_kernel(k, gen.hosts) for k in (k0, k1, k2, k3, k4, k5, k6, k7)):
        return None
    B, H, T, D = sh.B, sh.H, sh.T, sh.D
    R = B * H * T
    # G = 0 over all of G
    sts = _stores(k0)
    if k0.red is not None or len(sts) != 1 or sts[0].accumulate:
        return None
    cv = _see(sts[0].value)
    G = sts[0].buf.root
    if not (isinstance(cv, ir.Const) and cv.value == 0.0) or not A._full_write(k0, G) or G.dtype != ir.F32:
        return None
    if G.numel != sh.QKV.numel or G is sh.QKV or not _slices_tile(sh, G.numel):
        return None
    # G[V] += Σ_t dO · P
    got = _vars4(k1, T)
    if got is None:
        return None
    dom, t = got
    env: dict = {}
    if not _unify(k1.red.body, ("mul", ("load", "a"), ("load", "b")), env):
        return None
    a, b = env["a"], env["b"]
    if b.buf.root is not sh.P:
        a, b = b, a
    if b.buf.root is not sh.P:
        return None
    vs = _by_coef(dom, b.offset, [H * T * T, T * T, 1])
    if vs is None:
        return None
    n, h, u = vs
    c = [x for x in dom if x not in (n, h, u)][0]
    if not _s_at(sh, b.offset, n, h, t, u) or not _o_at(sh, a.offset, n, h, t, c):
        return None
    dO = a.buf.root
    sts = _stores(k1)
    if (len(sts) != 1 or not sts[0].accumulate or sts[0].buf.root is not G or not isinstance(_see(sts[0].value), ir.Acc)
            or not _qkv_at(sh, sts[0].offset, n, h, u, c, sh.v0)):
        return None
    # dp = Σ_c dO · V;  de = dp · (1 / l)
    got = _vars4(k2, D)
    if got is None:
        return None
    dom, c = got
    env = {}
    if not _unify(k2.red.body, ("mul", ("load", "a"), ("load", "b")), env):
        return None
    a, b = env["a"], env["b"]
    if a.buf.root is not dO:
        a, b = b, a
    if a.buf.root is not dO or b.buf.root is not sh.QKV:
        return None
    ta, tb = _terms(a.offset), _terms(b.offset)
    t = [x for x in dom if ta.get(x) == sh.os]
    u = [x for x in dom if tb.get(x) == sh.qs]
    if len(t) != 1 or len(u) != 1:
        return None
    t, u = t[0], u[0]
    n = [x for x in dom if ta.get(x) == sh.on and x not in (t, u)]
    h = [x for x in dom if ta.get(x) == sh.oh and x not in (t, u)]
    if len(n) != 1 or len(h) != 1:
        return None
    n, h = n[0], h[0]
    if not _o_at(sh, a.offset, n, h, t, c) or not _qkv_at(sh, b.offset, n, h, u, c, sh.v0):
        return None
    sts = _stores(k2)
    if len(sts) != 2 or any(s.accumulate for s in sts):
        return None
    if not isinstance(_see(sts[0].value), ir.Acc) or not _s_at(sh, sts[0].offset, n, h, t, u):
        return None
    dP = sts[0].buf.root
    env = {}
    if not _unify(sts[1].value, ("mul", ("acc",), ("div", ("const", "one"), ("load", "l"))), env):
        return None
    if env["one"].value != 1.0 or env["l"].buf.root is not sh.L:
        return None
    if not _is(env["l"].offset, 0, {n: H * T, h: T, t: 1}) or not _s_at(sh, sts[1].offset, n, h, t, u):
        return None
    DE = sts[1].buf.root
    # dl[r] = Σ_j dp · (−p / l)
    if k3.red is None or k3.red.op != "sum" or len(k3.domain) != 1 or k3.domain[0].extent != R:
        return None
    if len(k3.red.vars) != 1 or k3.red.vars[0].extent != T:
        return None
    r, jv = k3.domain[0], k3.red.vars[0]
    env = {}
    if not _unify(k3.red.body, ("mul", ("load", "dp"), ("div", ("neg", ("load", "p")), ("load", "l"))), env):
        return None
    if (env["dp"].buf.root is not dP or env["p"].buf.root is not sh.P or env["l"].buf.root is not sh.L
            or not _is(env["dp"].offset, 0, {r: T, jv: 1}) or not _is(env["p"].offset, 0, {r: T, jv: 1})
            or not _is(env["l"].offset, 0, {r: 1})):
        return None
    sts = _stores(k3)
    if len(sts) != 1 or sts[0].accumulate or not isinstance(_see(sts[0].value), ir.Acc) or not _is(sts[0].offset, 0, {r: 1}):
        return None
    DL = sts[0].buf.root
    # de[r, j] += dl[r]
    if k4.red is not None or len(k4.domain) != 2 or [x.extent for x in k4.domain] != [R, T]:
        return None
    r, jv = k4.domain
    sts = _stores(k4)
    if len(sts) != 1 or not sts[0].accumulate or sts[0].buf.root is not DE or not _is(sts[0].offset, 0, {r: T, jv: 1}):
        return None
    x = _see(sts[0].value)
    if not (isinstance(x, Load) and x.buf.root is DL and _is(x.offset, 0, {r: 1})):
        return None
    # ds = de · e
    if k5.red is not None or len(k5.domain) != 1 or k5.domain[0].extent != R * T:
        return None
    z = k5.domain[0]
    sts = _stores(k5)
    env = {}
    if len(sts) != 1 or sts[0].accumulate or not _is(sts[0].offset, 0, {z: 1}):
        return None
    if not _unify(sts[0].value, ("mul", ("load", "de"), ("load", "e")), env):
        return None
    if (env["de"].buf.root is not DE or env["e"].buf.root is not sh.E or not _is(env["de"].offset, 0, {z: 1})
            or not _is(env["e"].offset, 0, {z: 1})):
        return None
    DS = sts[0].buf.root
    # G[Q] += Σ_u ds · (alpha · K);  G[K] += Σ_t ds · (alpha · Q)
    for kk, base_out, base_in, out_is_query in ((k6, sh.q0, sh.k0, True), (k7, sh.k0, sh.q0, False)):
        got = _vars4(kk, T)
        if got is None:
            return None
        dom, red = got
        env = {}
        if not _unify(kk.red.body, ("mul", ("load", "ds"), ("mul", ("const", "alpha"), ("load", "x"))), env):
            return None
        if env["alpha"].value != sh.alpha or env["ds"].buf.root is not DS or env["x"].buf.root is not sh.QKV:
            return None
        vs = _by_coef(dom + [red], env["ds"].offset, [H * T * T, T * T, T, 1])
        if vs is None:
            return None
        n, h, t, u = vs
        if (red is not u) if out_is_query else (red is not t):
            return None
        c = [x for x in dom if x not in (n, h, t, u)]
        if len(c) != 1:
            return None
        c = c[0]
        own, other = (t, u) if out_is_query else (u, t)
        if not _s_at(sh, env["ds"].offset, n, h, t, u) or not _qkv_at(sh, env["x"].offset, n, h, other, c, base_in):
            return None
        sts = _stores(kk)
        if (len(sts) != 1 or not sts[0].accumulate or sts[0].buf.root is not G
                or not isinstance(_see(sts[0].value), ir.Acc) or not _qkv_at(sh, sts[0].offset, n, h, own, c, base_out)):
            return None
    kernels = [k0, k1, k2, k3, k4, k5, k6, k7]
    # nothing else reads the chain's temporaries (the forward's included)
    inside = list(sh.fwd) + kernels
    for X in (sh.S, sh.M, sh.E, sh.P, sh.L, dP, DE, DL, DS):
        n_in = sum(1 for k in inside if X in A.kernel_reads(k))
        if gen.readers.get(X.id, 0) != n_in or X.kind not in A.SHARED_KINDS or gen.is_host(X):
            return None
    if sh.L in A.kernel_writes(k3) or dO is G or any(gen.is_host(b) for b in (sh.QKV, sh.O, dO, G)):
        return None
    sh.G, sh.dO = G, dO
    sh.DL = DL                          # [B·H·T]: holds Drow between the two backward launches
    return kernels


def match(gen, stmts: list, i: int):
    """(plan, statements taken) for the forward chain at stmts[i] (its backward found later in the
    same block and registered), or for a registered backward chain at stmts[i]; else None."""
    if gen.emulate or not isinstance(stmts[i], KernelStmt):
        return None
    reg = gen.attn_train.get(stmts[i].kernel.id)
    if reg is not None:
        return reg
    if i + 6 > len(stmts) or not all(isinstance(st, KernelStmt) for st in stmts[i:i + 6]):
        return None
    ks, km, ke, kt, ko, kpv = (st.kernel for st in stmts[i:i + 6])
    if any(A.is_host_kernel(k, gen.hosts) for k in (ks, km, ke, kt, ko, kpv)):
        return None
    sh = _score_kernel(ks, _Shape())
    if sh is None:
        return None
    B, H, T, D = sh.B, sh.H, sh.T, sh.D
    if T % 32 or T > 256 or D not in (32, 64):
        return None
    R = B * H * T
    sh.M = _row_reduce(km, "max", sh.S, R, T)
    if sh.M is None:
        return None
    sh.E = _rows_map(ke, R, T, ("exp", ("sub", ("load", "s"), ("?detach", ("load", "m")))),
                     {"s": (sh.S, "el"), "m": (sh.M, "row")})
    if sh.E is None:
        return None
    sh.L = _row_reduce(kt, "sum", sh.E, R, T)
    if sh.L is None:
        return None
    sh.P = _rows_map(ko, R, T, ("div", ("load", "e"), ("load", "l")), {"e": (sh.E, "el"), "l": (sh.L, "row")})
    if sh.P is None or _pv_kernel(kpv, sh, sh.P) is None:
        return None
    if len({sh.S.id, sh.M.id, sh.E.id, sh.L.id, sh.P.id, sh.O.id, sh.QKV.id}) != 7:
        return None
    # alignment of the 16-byte accesses
    if any(x % 4 for x in (sh.q0, sh.k0, sh.v0, sh.qn, sh.qh, sh.qs, sh.o0, sh.on, sh.oh, sh.os)):
        return None
    sh.fwd = [ks, km, ke, kt, ko, kpv]
    j = i + 6
    while j < len(stmts):
        if isinstance(stmts[j], KernelStmt) and sh.P in A.kernel_reads(stmts[j].kernel):
            break
        j += 1
    if j >= len(stmts):
        return None
    bwd = _backward(gen, stmts, j - 1, sh)
    if bwd is None:
        return None
    if sh.dO is sh.O or any(x % 4 for x in (sh.on, sh.oh, sh.os)):
        return None
    fwd_plan = AttnTrainFwdPlan(gen, sh.fwd, f"k{ks.id}", sh)
    bwd_plan = AttnTrainBwdPlan(gen, bwd, f"k{bwd[0].id}", sh)
    gen.attn_train[bwd[0].id] = (bwd_plan, 8)
    gen.attn_train[ks.id] = (fwd_plan, 6)
    return fwd_plan, 6


# ------------------------------------------------------------------------------ plans

class _AttnTrainPlan(Plan):
    alone = True                     # never joins a side-by-side launch (its own LDS and lane count)

    def __init__(self, gen, kernels, name, sh):
        super().__init__(gen, kernels, name)
        self.sh = sh
        for k in kernels:
            for idx, st in enumerate(k.stmts):
                if isinstance(st, ir.Store):
                    self.skip_stores.add((k.id, idx))
        self.NT = sh.T // 32
        # a workgroup per tile where a head has at most two (T ≤ 64: more workgroups, each wavefront
        # one pair of tiles); else per pair of tiles p, NT − 1 − p (equal work per workgroup)
        self.TI = int(os.environ.get("ANVIL_ATTN_TI", "0")) or (1 if self.NT <= 2 else 2)
        self.threads = 256 * self.TI
        self.groups = self.NT if self.TI == 1 else (self.NT + 1) // 2
        # the backward as one launch whose workgroups alternate between dQ and dK/dV (each
        # computing Drow) up to five tiles per head, where the two launches are mostly fixed cost;
        # two launches (dQ writing Drow for dK/dV) above
        self.combined = self.NT <= 5

    def grid(self):
        return self.groups * self.sh.B * self.sh.H, self.threads

    def io(self, backward: bool) -> list[str]:
        sh = self.sh
        qkv = self.use_buf(sh.QKV)
        o = self.use_buf(sh.O)
        m, l = self.use_buf(sh.M), self.use_buf(sh.L)
        lines = ["    anvil_attn_io a;",
                 f"    a.q = {qkv} + {sh.q0}LL; a.k = {qkv} + {sh.k0}LL; a.v = {qkv} + {sh.v0}LL;",
                 f"    a.qn = {sh.qn}LL; a.qh = {sh.qh}LL; a.qs = {sh.qs}LL;",
                 f"    a.o = {o} + {sh.o0}LL; a.on = {sh.on}LL; a.oh = {sh.oh}LL; a.os = {sh.os}LL;",
                 f"    a.m = {m}; a.l = {l};",
                 f"    a.H = {sh.H}; a.BH = {sh.B * sh.H}; a.alpha = {flit(sh.alpha)};"]
        if backward:
            g, do = self.use_buf(sh.G), self.use_buf(sh.dO)
            dr = "nullptr" if self.combined else self.use_buf(sh.DL)
            lines += [f"    a.dout = {do} + {sh.o0}LL; a.drow = {dr};",
                      f"    a.dq = {g} + {sh.q0}LL; a.dk = {g} + {sh.k0}LL; a.dv = {g} + {sh.v0}LL;"]
        else:
            lines += ["    a.dout = nullptr; a.drow = nullptr; a.dq = a.dk = a.dv = nullptr;"]
        return lines

    def units(self) -> int:
        """(query tile, key tile) pairs met under the causal mask, over all heads."""
        return self.sh.B * self.sh.H * self.NT * (self.NT + 1) // 2

    def tensor_bytes(self, n: int) -> int:
        sh = self.sh
        return 4 * n * sh.B * sh.T * sh.H * sh.D


class AttnTrainFwdPlan(_AttnTrainPlan):
    kind = "attention-train"

    def writes(self) -> set:
        return {self.sh.O, self.sh.M, self.sh.L}

    def full_writes(self) -> set:
        return {self.sh.O.id, self.sh.M.id, self.sh.L.id}

    def cost(self):
        sh = self.sh
        return (self.units() * 2 * 2 * 32 * 32 * sh.D,
                self.tensor_bytes(4) + 4 * 2 * sh.B * sh.H * sh.T)

    def source(self) -> str:
        sh = self.sh
        io = self.io(False)                          # before the signature: it names the buffers
        return "\n".join(
            [f"// attention-train forward: {' + '.join(k.name for k in self.kernels)} · {sh.B * sh.H} heads of "
             f"{sh.T} x {sh.T}, D = {sh.D}, causal · writes O, m (base 2), l; S and P stay in registers",
             self.header(self.threads)] + io +
            [f"    anvil_attn_fwd<{sh.D}, {self.NT}, {self.TI}>(a);", "}"])


class AttnTrainBwdPlan(_AttnTrainPlan):
    """The backward: one launch of both kinds of workgroup, or the dQ launch with second() the
    dK/dV launch that follows it."""
    kind = "attention-train-dq"

    def __init__(self, gen, kernels, name, sh):
        super().__init__(gen, kernels, name, sh)
        self.two_launches = not self.combined
        if self.combined:
            self.kind = "attention-train-bwd"

    def grid(self):
        blocks, threads = super().grid()
        return (2 * blocks if self.combined else blocks), threads

    def writes(self) -> set:
        return {self.sh.G} if self.combined else {self.sh.G, self.sh.DL}

    def full_writes(self) -> set:
        return {b.id for b in self.writes()}

    def extra_reads(self) -> set:
        """What the launches read beyond the IR kernels they replace: the forward's row maxima and
        output (the IR's backward reads p and e instead)."""
        return {self.sh.M, self.sh.O}

    def cost(self):
        sh = self.sh
        if self.combined:                  # both kinds of workgroup: dQ's 3 products, dK/dV's 4
            return self.units() * 7 * 2 * 32 * 32 * sh.D, self.tensor_bytes(13) + 4 * 4 * sh.B * sh.H * sh.T
        return self.units() * 3 * 2 * 32 * 32 * sh.D, self.tensor_bytes(6) + 4 * 2 * sh.B * sh.H * sh.T

    def second(self):
        return AttnTrainBwdKVPlan(self)

    def source(self) -> str:
        sh = self.sh
        io = self.io(True)
        if self.combined:
            return "\n".join(
                [f"// attention-train backward: {' + '.join(k.name for k in self.kernels)} · {sh.B * sh.H} heads of "
                 f"{sh.T} x {sh.T}, D = {sh.D}, causal · dQ and dK/dV workgroups side by side, P and dS never stored",
                 self.header(self.threads)] + io +
                [f"    anvil_attn_bwd<{sh.D}, {self.NT}, {self.TI}, false>(a);", "}"])
        return "\n".join(
            [f"// attention-train dQ: {' + '.join(k.name for k in self.kernels)} · {sh.B * sh.H} heads of "
             f"{sh.T} x {sh.T}, D = {sh.D}, causal · P recomputed from Q, K, m, l; dS stays in registers",
             self.header(self.threads)] + io +
            [f"    anvil_attn_bwd_q<{sh.D}, {self.NT}, {self.TI}, false>(a);", "}"])


class AttnTrainBwdKVPlan(_AttnTrainPlan):
    kind = "attention-train-dkdv"

    def __init__(self, first: AttnTrainBwdPlan):
        super().__init__(first.gen, [], first.name + "kv", first.sh)
        self.first = first
        self.label = "dK, dV + " + first.label

    def writes(self) -> set:
        return {self.sh.G}

    def cost(self):
        sh = self.sh
        return self.units() * 4 * 2 * 32 * 32 * sh.D, self.tensor_bytes(7) + 4 * 2 * sh.B * sh.H * sh.T

    def source(self) -> str:
        sh = self.sh
        io = self.io(True)
        return "\n".join(
            [f"// attention-train dK, dV: {self.first.label} · {sh.B * sh.H} heads of {sh.T} x {sh.T}, D = {sh.D}, "
             "causal · P and dS recomputed, never stored",
             self.header(self.threads)] + io +
            [f"    anvil_attn_bwd_kv<{sh.D}, {self.NT}, {self.TI}, false>(a);", "}"])

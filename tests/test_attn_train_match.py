"""The training-attention chains (backend/hip_attn_train.py) are found where the reference's
transformer makes them, and only there.

C4 (the reference's examples/transformer.anvil: causal `softmax(q @ kᵀ · scale − 1e9 · (u > t)) @ v`
per layer, trained with Adam) lowers to six forward and eight backward kernels per layer; each pair
of runs becomes the forward launch and the backward as one launch (up to five 32-row tiles per head:
dQ and dK/dV workgroups side by side) or two (dQ, then dK/dV). A chain whose mask constant is too small for
exp to be exactly 0 in float32, or whose probabilities another statement reads, keeps its kernels.
The arena keeps the row maxima and the attention output (which the fused backward reads and the
IR's backward does not) alive up to the backward. The GPU results of the fused launches are held to
the reference's own vectors by the C4 programs of tests/test_hip_gpu.py (c4_mid, c4_full2,
c4_t160: pairs of tiles with an odd middle one, c4_t256_2).
"""
import pytest

from fixtures import load_ir

LAYERS = {"c4_full2": 4, "c4_t256_2": 4, "c4_mid": 1, "c4_small": 0, "c4_t160": 1}
SHAPES = {"c4_full2": (16, 4, 64, 64), "c4_t256_2": (16, 4, 256, 64), "c4_mid": (4, 2, 32, 32),
          "c4_t160": (2, 2, 160, 64)}


def _gen(prog, data):
    from anvil.backend import hip
    g = hip.HipGen(prog, seed=data.get("seed", 0))
    src = g.generate()
    return g, src


@pytest.mark.parametrize("name", sorted(LAYERS))
def test_each_layer_becomes_two_or_three_launches(name):
    prog, data = load_ir(name)
    g, src = _gen(prog, data)
    kinds = [p.kind for p in g.plans]
    L = LAYERS[name]
    assert kinds.count("attention-train") == L
    if L:
        B, H, T, D = SHAPES[name]
        NT = T // 32
        TI = 1 if NT <= 2 else 2                  # a workgroup per tile, or per pair of tiles
        one = NT <= 5                             # the backward as one launch
        assert kinds.count("attention-train-bwd") == (L if one else 0)
        assert kinds.count("attention-train-dq") == (0 if one else L)
        assert kinds.count("attention-train-dkdv") == (0 if one else L)
        assert src.count(f"anvil_attn_fwd<{D}, {NT}, {TI}>(a);") == L
        if one:
            assert src.count(f"anvil_attn_bwd<{D}, {NT}, {TI}, false>(a);") == L
        else:
            assert src.count(f"anvil_attn_bwd_q<{D}, {NT}, {TI}, false>(a);") == L
            assert src.count(f"anvil_attn_bwd_kv<{D}, {NT}, {TI}, false>(a);") == L
        assert src.count(f"__launch_bounds__({256 * TI})") >= (2 if one else 3) * L
    else:
        assert not any(k.startswith("attention-train") for k in kinds)
        fwd = [p for p in g.plans if p.kind == "attention-train"]
        for p in fwd:
            assert (p.sh.B, p.sh.H, p.sh.T, p.sh.D) == (B, H, T, D)
            # scores, probabilities and their gradients get no device memory at all
            for X in (p.sh.S, p.sh.E, p.sh.P):
                assert X.id not in g.device_bufs


def test_no_header_without_the_chain():
    """Programs without the chain generate exactly the source they did: the header is left out."""
    prog, data = load_ir("c2_small")
    _, src = _gen(prog, data)
    assert "anvil_attn_fwd" not in src


def _first_score_const(prog):
    from anvil import ir
    for k in ir.all_kernels(prog):
        for st in k.stmts:
            for e in ir.iter_expr(st.value):
                if isinstance(e, ir.Const) and e.value == 1e9:
                    return e
    return None


def test_small_mask_constant_keeps_the_chain():
    prog, data = load_ir("c4_mid")
    c = _first_score_const(prog)
    assert c is not None
    c.value = 1000.0                  # exp(−1000 + s − m) is 0, but not for every score's size
    g, _ = _gen(prog, data)
    assert "attention-train" not in [p.kind for p in g.plans]


def test_another_reader_of_p_keeps_the_chain():
    """A print of the probabilities after the backward: they must then exist in memory."""
    from anvil import ir
    prog, data = load_ir("c4_mid")
    g0, _ = _gen(prog, data)
    (fwd,) = [p for p in g0.plans if p.kind == "attention-train"]
    P = fwd.sh.P
    prog, data = load_ir("c4_mid")
    Pb = [b for b in prog.buffers if b.id == P.id][0]
    r = ir.Var("r", Pb.numel)
    k = ir.Kernel([r], [ir.Store(Pb, ir.Affine(0, {r: 1}), ir.Binary("mul", ir.Load(Pb, ir.Affine(0, {r: 1})),
                                                                     ir.Const(1.0)))])
    prog.main.stmts.append(ir.KernelStmt(k))
    g, _ = _gen(prog, data)
    assert "attention-train" not in [p.kind for p in g.plans]


@pytest.mark.parametrize("name", ["c4_full2", "c4_mid"])
def test_row_maxima_and_output_live_until_the_backward(name):
    prog, data = load_ir(name)
    g, _ = _gen(prog, data)
    spans = g.arena.spans
    for p in g.plans:
        if p.kind not in ("attention-train-dq", "attention-train-bwd"):
            continue
        G = p.sh.G
        assert G.id in spans or G.id in g.arena.offsets
        if G.id not in spans:
            continue
        start = spans[G.id][0]
        for X in (p.sh.M, p.sh.O):
            if X.id in spans:               # shared: its bytes are not reused before the backward
                assert spans[X.id][1] >= start, (X.name, spans[X.id], start)


@pytest.mark.parametrize("name", ["c4_full2", "c4_t256_2"])
def test_costs_count_the_causal_tile_pairs(name):
    """FLOPs of the launches: 2 products of 32 x 32 x D per (query tile, key tile) pair the causal
    mask leaves for the forward, 3 for dQ, 4 for dK/dV, 7 for the backward as one launch, counted
    here by walking the pairs."""
    from anvil.backend import hip_cost
    prog, data = load_ir(name)
    g, _ = _gen(prog, data)
    B, H, T, D = SHAPES[name]
    pairs = sum(1 for qt in range(T // 32) for kt in range(T // 32) if kt <= qt) * B * H
    tile = 2 * 32 * 32 * D
    want = {"attention-train": 2 * tile * pairs, "attention-train-dq": 3 * tile * pairs,
            "attention-train-dkdv": 4 * tile * pairs, "attention-train-bwd": 7 * tile * pairs}
    seen = 0
    for p in g.plans:
        if p.kind in want:
            assert hip_cost.plan_cost(p)[0] == want[p.kind]
            seen += 1
    assert seen == (12 if T > 160 else 8)


@pytest.mark.parametrize("name", ["attn_same_qk", "attn_four_slices"])
def test_slices_that_do_not_tile_the_gradient_keep_the_chain(name):
    """The fused backward stores dQ, dK and dV at the Q, K and V slices of G in place of `G = 0` and
    three `+=`: only right when the slices cover G once each. Queries and keys read from the same
    columns (attn_same_qk: their gradients must add) and a projection with a fourth, unread slice
    (attn_four_slices: its gradient must be 0) keep the generated kernels, forward and backward;
    tests/test_hip_gpu.py runs both against the reference interpreter's vectors."""
    prog, data = load_ir(name)
    g, src = _gen(prog, data)
    assert not any(p.kind.startswith("attention-train") for p in g.plans)
    assert "anvil_attn_fwd" not in src


def test_slice_cover_rule():
    """_slices_tile on hand-made layouts: C4's [n, t, 3, h, c] (q0, k0, v0 = 0, H·D, 2·H·D)
    tiles; two slices at one offset, a gap, a slice past the end and an overlap by one do not."""
    from anvil.backend.hip_attn_train import _Shape, _slices_tile
    sh = _Shape()
    sh.B, sh.H, sh.T, sh.D = 2, 2, 4, 8
    HD = sh.H * sh.D
    sh.qh, sh.qs = sh.D, 3 * HD
    sh.qn = sh.T * sh.qs
    n = sh.B * sh.qn
    for (q0, k0, v0), ok in (((0, HD, 2 * HD), True), ((2 * HD, 0, HD), True), ((0, 0, 2 * HD), False),
                             ((0, HD, HD), False), ((0, HD, 2 * HD + 1), False), ((0, HD - 1, 2 * HD), False)):
        sh.q0, sh.k0, sh.v0 = q0, k0, v0
        assert _slices_tile(sh, n) is ok, (q0, k0, v0)
    sh.q0, sh.k0, sh.v0 = 0, HD, 2 * HD
    assert not _slices_tile(sh, n + 1)           # one element of G no slice covers

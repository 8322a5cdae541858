"""The HIP generator's IR rewrites keep each program's meaning: the oracle (oracle/interp.py, pinned
to the reference interpreter by test_oracle.py) runs the program before and after each rewrite and
must print and store the same thing. The rewrites only move or re-address work, so integers and the
printed text are identical; floats are identical where the sums keep their order and within 1e-5
where a rewrite splits one summed variable into several (NumPy then sums over more axes).
"""
import numpy as np

from fixtures import load_ir, run_oracle
from hiprun import kept_buffers, outputs_match, tensors_match

from anvil import ir
from anvil.backend import hip_analysis as A
from anvil.backend import hip_conv, hip_gemm


def kernels(prog):
    return [st.kernel for blk in ir.walk_blocks(prog.main) for st in blk.stmts if isinstance(st, ir.KernelStmt)]


def run(prog, data, keep):
    m, out = run_oracle(prog, data)
    by_name = {b.name: b for b in prog.buffers}
    return out, {k: m.arr(by_name[k])[:by_name[k].numel].reshape(by_name[k].shape).copy() for k in keep}


def test_implicit_convolution_rewrite_keeps_the_program():
    """c5_mid: both products over the second convolution's im2col copy read the copy's source
    through the window (their merged variables split back out), and the copy is dropped."""
    prog, data = load_ir("c5_mid")
    new = hip_conv.forward_im2col_copies(prog, A.IdSource(prog))
    before, after = kernels(prog), kernels(new)
    assert len(after) == len(before) - 1                          # the im2col copy of conv2 is gone
    split = [k for k in after if k not in before and k.red is not None]
    assert len(split) == 2 and all(len(k.domain) + len(k.red.vars) > 4 for k in split)
    keep = kept_buffers("c5_mid")
    out0, bufs0 = run(prog, data, keep)
    out1, bufs1 = run(new, data, keep)
    assert outputs_match(out0, out1, rtol=1e-5) is None
    for k in keep:
        assert tensors_match(bufs0[k], bufs1[k], rtol=1e-5) is None, k


def test_gathered_batch_rows_keep_the_program():
    """c2_small: the first product reads X[perm[s·B + i], ·] instead of the gathered batch copy;
    the same values, summed in the same order."""
    prog, data = load_ir("c2_small")
    new = hip_gemm.forward_gather_copies(prog, A.host_scalars(prog))

    def gathered_products(p):
        return [k for k in kernels(p) if k.red is not None and k.red.op == "sum"
                and any(ld.offset.gathers() for ld in ir.loads_in(k.red.body))]
    assert len(gathered_products(new)) == len(gathered_products(prog)) + 1
    keep = kept_buffers("c2_small")
    out0, bufs0 = run(prog, data, keep)
    out1, bufs1 = run(new, data, keep)
    assert out0 == out1
    for k in keep:
        np.testing.assert_array_equal(bufs0[k], bufs1[k], err_msg=k)


def test_sunk_scalar_kernels_keep_the_program():
    """c2_small: the loss (a one-value reduction) moves past the kernels it commutes with."""
    prog, data = load_ir("c2_small")
    new = A.sink_scalar_kernels(prog)
    assert [k.id for k in kernels(new)] != [k.id for k in kernels(prog)]
    keep = kept_buffers("c2_small")
    out0, bufs0 = run(prog, data, keep)
    out1, bufs1 = run(new, data, keep)
    assert out0 == out1
    for k in keep:
        np.testing.assert_array_equal(bufs0[k], bufs1[k], err_msg=k)


def test_split_vars_is_the_row_major_index():
    """A variable t of extent 12 split into (a, b) of extents (3, 4): every offset 5·t becomes
    20·a + 5·b, in the domain's place of t."""
    t, i = ir.Var("t", 12), ir.Var("i", 7)
    buf = ir.Buffer("x", (7, 12), "f32", "temp")
    k = ir.Kernel([i, t], [ir.Store(buf, ir.Affine(0, {i: 12, t: 1}), ir.Load(buf, ir.Affine(3, {t: 5})))])
    a, b = ir.Var("a", 3), ir.Var("b", 4)
    k2 = hip_conv.split_vars(k, {t: [a, b]})
    assert k2.domain == [i, a, b]
    st = k2.stmts[0]
    assert st.offset == ir.Affine(0, {i: 12, a: 4, b: 1})
    assert st.value.offset == ir.Affine(3, {a: 20, b: 5})


def row_block_plans(name):
    from anvil.backend import hip
    prog, data = load_ir(name)
    gen = hip.HipGen(prog, seed=int(data.get("seed", 0)))
    gen.generate()
    out = []
    for p in gen.plans:
        for q in getattr(p, "parts", [p]):
            if q.kind == "rowblock":
                out.append(q)
    return out


def lane_addresses(plan, st, ld, part, rows):
    """The element each (row, lane, trip, inner index) of a row-block stage loads, by decoding the
    flat index row·E + e over the whole domain (as the generated code does)."""
    T = plan.threads
    k = st.k
    rows = np.asarray(rows)[:, None, None, None]
    idx = np.arange(T)[None, :, None, None] + T * np.arange(st.trips)[None, None, :, None]

    def digits(flat, vars_):
        strides = ir.row_major_strides([v.extent for v in vars_])
        return {v: (flat // s) % v.extent for v, s in zip(vars_, strides)}
    if st.form == "block":
        vals = digits(rows * st.E + np.arange(st.E)[None, None, None, :], k.domain)
        vals.update(digits(idx, k.red.vars))
    else:
        vals = digits(rows * st.E + idx, k.domain)
        if part == "body":
            vals.update(digits(np.arange(st.n)[None, None, None, :], k.red.vars))
    addr = ld.offset.const + sum(c * vals[v] for v, c in ld.offset.terms.items())
    return np.broadcast_to(addr + 0 * idx, np.broadcast_shapes(np.shape(addr), idx.shape)), idx < st.N


def test_row_block_forwarding_reads_the_same_elements():
    """Every operand a row-block stage takes from registers (loaded by an earlier stage of the same
    lane and trip) is the element that stage would load itself: checked against a decode of the
    whole flat index, for every row, lane and trip. C2's block forwards W3 and h2 from the logits
    stage to the input-gradient stages and hoists the bias and label loads. Loads that a block stage
    makes as one vector for several outputs read consecutive, aligned elements (C2: W3's row j as
    5 8-byte loads)."""
    total = 0
    for name in ["c2_wide_mlp", "c1_mlp", "c4_transformer", "c5_small", "mnist_like", "attention_fit"]:
        for plan in row_block_plans(name):
            slots = {}
            for st in plan.stages:
                for (part, key), slot in st.sources.items():
                    slots[slot] = (st, part, key)
            for t, st in enumerate(plan.stages):
                for (part, key), (slot, qmap) in st.targets.items():
                    src, spart, skey = slots[slot]
                    assert plan.stages.index(src) < t
                    ld = next(x for x in st.parts()[part] if x.key() == key)
                    ld2 = next(x for x in src.parts()[spart] if x.key() == skey)
                    assert ld.buf.root is ld2.buf.root and ld.buf.root.id not in plan.chain_writes
                    rows = range(plan.R) if plan.R <= 512 else [0, 1, 2, plan.R // 2, plan.R - 1]
                    a, act = lane_addresses(plan, st, ld, part, rows)
                    b, act2 = lane_addresses(plan, src, ld2, spart, rows)
                    b = b[:, :, :st.trips, :][..., qmap]
                    act2 = act2[:, :, :st.trips, :]
                    assert (act2 | ~act).all()
                    assert ((a == b) | ~act).all(), (name, plan.name, t, key)
                    total += 1
            for st in plan.stages:
                for key, (vname, w, ld) in getattr(st, "vectors", {}).items():
                    # one w-wide load per w outputs: consecutive elements from a w-aligned first one
                    rows = range(plan.R) if plan.R <= 512 else [0, 1, 2, plan.R // 2, plan.R - 1]
                    a, act = lane_addresses(plan, st, ld, "body", rows)
                    q = np.arange(st.E)
                    assert ((a == a[..., :1] + q) | ~act).all(), (name, plan.name, key)
                    assert ((a[..., 0] % w == 0) | ~act[..., 0]).all(), (name, plan.name, key)
                    assert ld.buf.root.kind not in ir.EXTERN_KINDS
                    total += 1
            if name == "c2_wide_mlp":
                assert [w for st in plan.stages for (_, w, _) in getattr(st, "vectors", {}).values()] == [2]
                assert sum(len(st.targets) for st in plan.stages) == 2
                assert sum(len(st.hoisted) for st in plan.stages) == 2
    assert total >= 30


def test_generated_source_does_not_depend_on_earlier_programs():
    """The passes' new loop variables are named by ids that follow the program's own, so the same
    program gives the same source (and library name) after other programs were generated in the
    same process, as in a build pool."""
    from anvil.backend import hip
    prog, data = load_ir("c5_mid")          # its ids end at 819, far below mnist_like's
    alone = hip.generate(prog, seed=int(data.get("seed", 0)))
    other, odata = load_ir("mnist_like")
    hip.generate(other, seed=int(odata.get("seed", 0)))
    again, _ = load_ir("c5_mid")
    assert hip.generate(again, seed=int(data.get("seed", 0))) == alone

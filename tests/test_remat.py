"""Rematerialization (hip_analysis.rematerialize): temporaries that are a cheap elementwise function
of another buffer are recomputed where they are read, and no longer stored.

The rewritten program must compute exactly what the original does: the NumPy oracle runs both
(same seed) and their printed output and parameters must be identical, byte for byte. Hand-built
programs pin each condition under which a temporary has to stay in memory.
"""
import io

import numpy as np
import pytest

from fixtures import load_ir

from anvil import ir
from anvil.backend import hip_analysis as A


def _stored(prog):
    return {st.buf.name for k in ir.all_kernels(prog) for st in k.stores}


def _reads(prog):
    return {b.name for k in ir.all_kernels(prog) for b in A.kernel_reads(k)}


def test_gelu_intermediates_are_recomputed_in_the_backward():
    """C4's feed-forward GELU: the tanh and 0.044715·x² that the reference's autodiff saves for the
    backward are dropped from the forward's stores; the backward reads x instead. The GELU output
    itself (an operand of the next product, read inside its reduction) stays in memory."""
    prog, _ = load_ir("c4_small")
    new = A.rematerialize(prog)
    gone = _stored(prog) - _stored(new)
    assert gone == {"t16", "t20", "t41", "t45"}             # two per layer, two layers
    assert not gone & _reads(new)
    assert {"t22", "t47"} <= _stored(new)                   # the GELU outputs
    assert len(ir.all_kernels(new)) == len(ir.all_kernels(prog))
    # the caller's program is unchanged
    assert _stored(load_ir("c4_small")[0]) == _stored(prog)


def test_no_candidates_in_programs_without_them():
    for name in ("c2_small", "c5_small", "logreg"):
        prog, _ = load_ir(name)
        assert A.rematerialize(prog) is prog


@pytest.mark.parametrize("name", ["c4_small", "c4_t160"])
def test_oracle_output_is_identical(name):
    """The oracle interpreter on the rewritten program prints the same bytes and leaves the same
    parameters, bit for bit, as on the original."""
    from oracle import interp
    prog, data = load_ir(name)
    new = A.rematerialize(prog)
    assert new is not prog
    runs = []
    for p in (prog, new):
        out = io.StringIO()
        m = interp.Machine(p, out=out, seed=int(data.get("seed", 0)))
        m.run()
        params = {b.name: m.arr(b)[:b.numel].copy() for b in p.buffers if b.kind == "param"}
        runs.append((out.getvalue(), params))
    assert runs[0][0] == runs[1][0]
    for k, v in runs[0][1].items():
        np.testing.assert_array_equal(runs[1][1][k], v, err_msg=k)


# --------------------------------------------------------------------------- hand-built programs

N = 64


def _program(*, second_writer=False, shifted=False, in_reduction=False, before=False, print_t=False):
    """x (data) -> z = 2x -> t = tanh(z) (+ 1 in the same kernel: u) -> y = t + u, by default.
    The options break one condition each."""
    x = ir.Buffer("x", (N + 1,), "f32", "data")
    z = ir.Buffer("z", (N + 1,), "f32", "temp")
    t = ir.Buffer("t", (N,), "f32", "temp")
    u = ir.Buffer("u", (N,), "f32", "temp")
    y = ir.Buffer("y", (N,) if not in_reduction else (), "f32", "temp")
    i, j, k, r = ir.Var("i", N + 1), ir.Var("j", N), ir.Var("k", N), ir.Var("r", N)
    at = lambda v, c=0: ir.Affine(c, {v: 1})
    wz = ir.Kernel([i], [ir.Store(z, at(i), ir.Binary("mul", ir.Const(2.0), ir.Load(x, at(i))))], name="wz")
    th = ir.Unary("tanh", ir.Load(z, at(j, 1) if shifted else at(j)))
    m = ir.Kernel([j], [ir.Store(t, at(j), th), ir.Store(u, at(j), ir.Binary("add", ir.Load(z, at(j)), ir.Const(1.0)))],
                  name="m")
    if in_reduction:
        c = ir.Kernel([], [ir.Store(y, ir.Affine(0), ir.Acc())], red=ir.Reduction([r], "sum", ir.Load(t, at(r))),
                      name="c")
    else:
        c = ir.Kernel([k], [ir.Store(y, at(k), ir.Binary("add", ir.Load(t, at(k)), ir.Load(u, at(k))))], name="c")
    stmts = [ir.KernelStmt(wz), ir.KernelStmt(m), ir.KernelStmt(c)]
    if before:                                    # a reader of t before its writer
        k2 = ir.Var("k2", N)
        stmts.insert(1, ir.KernelStmt(ir.Kernel([k2], [ir.Store(u, at(k2), ir.Load(t, at(k2)))], name="early")))
    if second_writer:                             # z written again later
        i2 = ir.Var("i2", N + 1)
        stmts.append(ir.KernelStmt(ir.Kernel([i2], [ir.Store(z, at(i2), ir.Const(0.0))], name="wz2")))
    if print_t:
        stmts.append(ir.Print([ir.PrintItem("tensor", buf=t)]))
    return ir.Program(ir.Block(stmts), [x, z, t, u, y])


def test_simple_case_is_rewritten():
    prog = _program()
    new = A.rematerialize(prog)
    assert "t" not in _stored(new) and "t" not in _reads(new)
    # u = z + 1 (the writer's other store) qualifies too: the writer then stores nothing and goes,
    # and y = tanh(z) + (z + 1) reads z alone
    assert "u" not in _stored(new) and [k.name for k in ir.all_kernels(new)] == ["wz", "c"]
    c = ir.all_kernels(new)[1]
    assert {b.name for b in A.kernel_reads(c)} == {"z"}


@pytest.mark.parametrize("how", ["print", "shifted", "reduction", "before", "second_writer"])
def test_t_stays_in_memory(how):
    prog = _program(print_t=how == "print", shifted=how == "shifted", in_reduction=how == "reduction",
                    before=how == "before", second_writer=how == "second_writer")
    new = A.rematerialize(prog)
    assert "t" in _stored(new)

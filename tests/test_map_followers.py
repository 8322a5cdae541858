"""Elementwise kernels run in the lane of the kernel before them (hip_kernels.MapPlan followers, and
the convolution input gradient's follower in hip_conv.DgradPlan), pinned on the generated source
and, for a hand-built program, on its CPU build against the unfused one.

A follower walks the same elements in the same row-major order and reads what its leader stored
only at its own element, so each element gets the same operations on the same values: the results
are the same bits either way. On the GPU the fused C5 kernels are held to the reference's vectors
by c5_small, c5_mid, c5_step1, c5_conv12 and c5_full3 (tests/test_hip_gpu.py).
"""
import json
import os
import re
import subprocess
import sys

import pytest

from fixtures import ROOT_PKG, load_ir

from anvil import ir, irjson
from anvil.backend import hip

N = 1000


def _source(prog, **env):
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return hip.generate(prog)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _costly(v):
    """exp(tanh(exp(tanh(v)))): more work than the backend recomputes in place of a stored value."""
    for op in ("tanh", "exp", "tanh", "exp"):
        v = ir.Unary(op, v)
    return v


def _program(*, clash=False):
    """x = 0.001 i; print x; t = f(x); y = t + x; print y. With clash: the last kernel also writes t,
    at the mirrored element (another lane's)."""
    x = ir.Buffer("x", (N,), "f32", "data")
    t = ir.Buffer("t", (N,), "f32", "temp")
    y = ir.Buffer("y", (N,), "f32", "temp")
    i, j = ir.Var("i", N), ir.Var("j", N)
    at = lambda v: ir.Affine(0, {v: 1})
    fill = ir.Kernel([i], [ir.Store(x, at(i), ir.Binary("mul", ir.Const(0.001), ir.Unary("f32", ir.Index(at(i)))))],
                     name="fill")
    a = ir.Kernel([i], [ir.Store(t, at(i), _costly(ir.Load(x, at(i))))], name="a")
    stmts = [ir.Store(y, at(j), ir.Binary("add", ir.Load(t, at(j)), ir.Load(x, at(j))))]
    if clash:
        stmts.append(ir.Store(t, ir.Affine(N - 1, {j: -1}), ir.Const(1.0)))
    b = ir.Kernel([j], stmts, name="b")
    body = [ir.KernelStmt(fill), ir.Print([ir.PrintItem("tensor", buf=x)]), ir.KernelStmt(a), ir.KernelStmt(b),
            ir.Print([ir.PrintItem("tensor", buf=y)])]
    return ir.Program(ir.Block(body), [x, t, y])


def _maps(src):
    return re.findall(r"^// map: (.*)$", src, re.M)


def test_follower_runs_in_the_leaders_lane_and_its_input_is_not_stored():
    src = _source(_program())
    maps = _maps(src)
    fused = [m for m in maps if "; " in m]
    assert len(fused) == 1, maps
    kernel = src[src.index("// map: " + fused[0]):].split("\n}\n", 1)[0]
    # t is read only by the follower, from a register: y is the kernel's one store
    # (a plain store, or the lane's four elements as one 16-byte store)
    assert len(re.findall(r"^\s+(?:\*\(anvil_f32x4 \*\)&)?b\d+\[.*\] = ", kernel, re.M)) == 1     # y alone
    assert not any("; " in m for m in _maps(_source(_program(), ANVIL_HIP_MAP_FUSE="0")))


def test_a_follower_that_writes_what_the_leader_writes_stays_apart():
    maps = _maps(_source(_program(clash=True)))
    assert not any("; " in m for m in maps), maps


def _chain(shift):
    """x -> t = f(x) -> u = f(t) -> y = u[i + shift] + t: a second follower that reads the first
    follower's output at another lane's element when shift != 0."""
    M = N + 8
    x = ir.Buffer("x", (M,), "f32", "data")
    t = ir.Buffer("t", (M,), "f32", "temp")
    u = ir.Buffer("u", (M,), "f32", "temp")
    y = ir.Buffer("y", (M,), "f32", "temp")
    i, j, k = ir.Var("i", N), ir.Var("j", N), ir.Var("k", N)
    at = lambda v, c=0: ir.Affine(c, {v: 1})
    a = ir.Kernel([i], [ir.Store(t, at(i), _costly(ir.Load(x, at(i))))], name="a")
    b = ir.Kernel([j], [ir.Store(u, at(j), _costly(ir.Load(t, at(j))))], name="b")
    c = ir.Kernel([k], [ir.Store(y, at(k), ir.Binary("add", ir.Load(u, at(k, shift)), ir.Load(t, at(k))))], name="c")
    body = [ir.KernelStmt(a), ir.KernelStmt(b), ir.KernelStmt(c), ir.Print([ir.PrintItem("tensor", buf=y)])]
    return ir.Program(ir.Block(body), [x, t, u, y])


def test_a_second_follower_reads_the_first_ones_output_only_at_its_own_element():
    assert any(m.count("; ") == 2 for m in _maps(_source(_chain(0))))            # a; b; c in one lane
    maps = _maps(_source(_chain(3)))
    assert not any(m.count("; ") == 2 for m in maps), maps                       # c reads u[k + 3]: apart


@pytest.mark.slow
def test_fused_and_unfused_cpu_builds_print_the_same(tmp_path):
    path = tmp_path / "p.json"
    with open(path, "w") as f:
        json.dump(irjson.dump(_program()), f)
    outs = []
    for env in ({}, {"ANVIL_HIP_MAP_FUSE": "0"}):
        r = subprocess.run([sys.executable, "-m", "anvil", "run", str(path), "--emulate"], capture_output=True,
                           text=True, timeout=600, env=dict(os.environ, PYTHONPATH=ROOT_PKG, **env))
        assert r.returncode == 0, r.stderr
        outs.append(r.stdout)
    assert outs[0] == outs[1] and outs[0].strip()


def test_c5_gradients_fuse_their_relu_masks():
    """C5's backward: the max-pool gradient and ReLU's gradient in one map (the pooled-gradient
    intermediate never stored), and conv1's ReLU gradient in the input gradient's epilogue (its dX
    never stored): two launches fewer per step."""
    prog, data = load_ir("c5_cnn")
    src = _source(prog)
    unfused = _source(prog, ANVIL_HIP_MAP_FUSE="0")
    assert src.count("__global__") == unfused.count("__global__") - 2
    assert any(re.match(r"k\d+ \[nci<98304 x u<2 x j<12 x v<2\]; k\d+ \[ijkl<4718592\]", m) for m in _maps(src))
    dgrad = src[src.index("// conv-dgrad"):].split("\n}\n", 1)[0]
    assert "const float dx_ =" in dgrad and "= dx_;" not in dgrad
    assert re.search(r"pre0\[ijq\] = b\d+\[", dgrad)                      # z1 loaded before the product

"""The arena's lifetime sharing and the cost model, checked independently of how they are computed.

Arena (hip_analysis.plan_arena, the reference's arena.py:121-144 rule): programs built with the
sharing on and off (ANVIL_HIP_SHARE=0) print the same text and end with bit-identical kept
buffers, in the CPU build of the generated file, and the shared arena is smaller (reference
tests/test_arena.py: sharing keeps the output, and memory goes down).

Cost model (backend/hip_cost.py, the reference's cost.py:22-52 conventions): the FLOPs and bytes a
kernel and a generated kernel report equal closed forms of the operation (reference
tests/test_cost.py: a product's 2·M·N·K).
"""
import ctypes

import numpy as np
import pytest

from fixtures import load_ir
from hiprun import kept_buffers, run_program


@pytest.mark.parametrize("name", ["c2_small", "c4_small", "c5_small", "attention_fit"])
def test_sharing_keeps_the_output(name):
    keep = kept_buffers(name)
    runs = []
    for share in ("1", "0"):
        rc, out, err, arrays = run_program(name, emulate=True, keep=keep, timeout=600,
                                           env_extra={"ANVIL_HIP_SHARE": share})
        assert rc == 0, err
        runs.append((out, arrays))
    (out1, a1), (out0, a0) = runs
    assert out1 == out0
    for k in keep:
        np.testing.assert_array_equal(a1[k].view(np.int32), a0[k].view(np.int32), err_msg=k)


@pytest.mark.parametrize("name", ["c2_small", "c4_small"])
def test_sharing_shrinks_the_arena(name):
    from anvil.backend import hip
    prog, data = load_ir(name)
    src = hip.generate(prog, seed=data.get("seed", 0), emulate=True)
    lib = ctypes.CDLL(hip.compile_source(src, emulate=True))
    lib.anvil_arena_bytes.restype = lib.anvil_arena_unshared_bytes.restype = ctypes.c_longlong
    shared, unshared = lib.anvil_arena_bytes(), lib.anvil_arena_unshared_bytes()
    assert 0 < shared < unshared, (shared, unshared)


def _plans(name):
    from anvil.backend import hip
    prog, data = load_ir(name)
    g = hip.HipGen(prog, seed=data.get("seed", 0), library=True)
    g.generate()
    return prog, g.plans


def test_linear_costs_2mnk_plus_the_bias():
    """y[i, j] = Σ_c W[j, c] x[i, c] + b[j] at [96, 80] × [72, 80]ᵀ: 2·M·N·K FLOPs for the product and one
    per output for the bias; x, W and b read once, y written once."""
    from anvil import ir
    from anvil.backend import hip_cost
    M, N, K = 96, 72, 80
    flops, nbytes = 2 * M * N * K + M * N, 4 * (M * K + N * K + N + M * N)
    prog, plans = _plans("c3_linear_small")
    (k,) = list(ir.all_kernels(prog))
    assert (hip_cost.kernel_flops(k), hip_cost.kernel_bytes(k)) == (flops, nbytes)
    gemm = [p for p in plans if p.kind == "gemm"]
    assert len(gemm) == 1 and hip_cost.plan_cost(gemm[0]) == (flops, nbytes)


def test_softmax_rows_count_each_tensor_once():
    """Softmax over rows of [64, 300] as one row kernel: max (1 per element), exp(x - m) (2), the sum
    (1), the division (1); the input read once and the output written once (the row's max,
    exponentials and sum stay in the kernel)."""
    from anvil.backend import hip_cost
    R, C = 64, 300
    _, plans = _plans("c3_softmax_small")
    rows = [p for p in plans if len(p.kernels) == 4]
    assert len(rows) == 1
    assert hip_cost.plan_cost(rows[0]) == (5 * R * C, 4 * (R * C + R * C))

"""The index-scatter schedule (hip_kernels.index_scatter / IndexScatterPlan): a `+=` into rows of a
small table picked by an index array, run without atomics, one workgroup per table row.

Which kernels take it, and the kernel it generates, are checked here; the results are checked on
the GPU against the reference's vectors by the programs that use it (the `scatter` fixture's
histogram; `scatter_rows`: 300 columns, more than a workgroup's lanes, 999 positions, 7 rows; C4's
token-embedding gradient in c4_t160, c4_full2 and c4_t256_2).
"""
import re

import pytest

from fixtures import load_ir

from anvil import ir
from anvil.backend import hip
from anvil.backend import hip_kernels as HK


def _kernels(name):
    prog, _ = load_ir(name)
    return [k for k in ir.all_kernels(prog) if HK.index_scatter(k) is not None]


def test_embedding_gradient_is_found():
    """C4 at T = 256: dE[tok[n, t], d] += dX[n, t, d], 96 rows of 256, 16 x 256 positions."""
    ks = _kernels("c4_t256_2")
    assert len(ks) == 1
    cols, pos, g, W, R, P = HK.index_scatter(ks[0])
    assert [v.extent for v in cols] == [256] and [v.extent for v in pos] == [16, 256]
    assert (W, R, P) == (256, 96, 4096)
    assert g.load.buf.dtype == "i32"


def test_histogram_is_found():
    ks = _kernels("scatter")
    assert len(ks) == 1
    cols, pos, g, W, R, P = HK.index_scatter(ks[0])
    assert cols == [] and (W, R, P) == (1, 10, 1000)


def test_few_positions_per_row_keep_the_atomic_map():
    """c4_small has 16 positions for 96 rows: the scan would cost more than the collisions."""
    assert _kernels("c4_small") == []


def _scatter_kernel(col_in_index=False):
    tab = ir.Buffer("tab", (8, 4), "f32", "temp")
    idx = ir.Buffer("idx", (64,), "i32", "data")
    x = ir.Buffer("x", (64, 4), "f32", "data")
    i, d = ir.Var("i", 64), ir.Var("d", 4)
    g = ir.Gather(ir.Load(idx, ir.Affine(0, {i: 1, d: 1} if col_in_index else {i: 1})), 8)
    st = ir.Store(tab, ir.Affine(0, {g: 4, d: 1}), ir.Load(x, ir.Affine(0, {i: 4, d: 1})), accumulate=True)
    return ir.Kernel([i, d], [st], name="k")


def test_hand_built_scatter():
    cols, pos, g, W, R, P = HK.index_scatter(_scatter_kernel())
    assert [v.name for v in cols] == ["d"] and [v.name for v in pos] == ["i"] and (W, R, P) == (4, 8, 64)


def test_column_used_by_the_index_is_rejected():
    assert HK.index_scatter(_scatter_kernel(col_in_index=True)) is None


@pytest.mark.parametrize("name", ["c4_t160", "scatter", "scatter_rows"])
def test_generated_kernel(name):
    """The generated kernel: no atomics, the bounds check kept in the scan, the LDS list sized for
    every position, and the adds in list order."""
    prog, data = load_ir(name)
    src = hip.generate(prog, seed=data.get("seed", 0))
    m = re.search(r"// index-scatter: .*?\n(__global__.*?\n)}\n", src, re.S)
    assert m is not None
    body = m.group(0)
    assert "atomicAdd" not in body
    assert "anvil_fault(" in body
    P = int(re.search(r"(\d+) positions scanned", body).group(1))
    hits = int(re.search(r"__shared__ int anvil_hits\[(\d+)\]", body).group(1))
    assert hits >= P
    assert "if (h0 + j < nh) acc += x_[j];" in body
    # the emulation build keeps the plain map (it has no wavefronts to ballot over)
    assert "// index-scatter" not in hip.generate(prog, seed=data.get("seed", 0), emulate=True)

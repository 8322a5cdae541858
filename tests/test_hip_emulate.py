"""The HIP generator's output, built for the CPU (-DANVIL_EMULATE), against the reference.

The generated file's host program (control flow, host scalars, the shuffle, printing, checkpoints,
faults) and its kernels' per-element code are the same in this build as in the gfx950 one; the
GPU-only kernel shapes (cross-lane reductions, split reductions, MFMA products) are replaced by
one-lane-per-row loops. The golden vectors were written by the reference interpreter
(tests/golden/make_fixtures.py).
"""
import os

import numpy as np
import pytest

from fixtures import stdout_of, vectors
from hiprun import check_program_run, function_call, kept_buffers, outputs_match, run_program, tensors_match

PROGRAMS = ["greet", "logreg", "attention_fit", "split", "scatter", "integers", "formats", "control",
            "products", "c1_small", "c2_small", "c2_steps100", "mnist_like", "c4_small", "c4_mid", "c5_small", "c5_mid",
            "files", "picks", "ckpt_write", "ckpt_read", "serial", "draws", "board", "c5_conv12", "c4_t160",
            "scatter_rows", "argpick", "attn_same_qk", "attn_four_slices", "rowblock_prior"]
FUNCTIONS = ["c3_softmax_small", "c3_layernorm_small", "c3_linear_small", "c3_linear_tall", "c3_attention_small",
             "c3_attention_d64", "c3_attention_d128"]
TRAINED = {"c2_steps100", "c2_small", "c1_small", "mnist_like", "logreg", "attention_fit", "c5_mid", "c4_mid",
           "c5_conv12", "c4_t160", "attn_same_qk", "attn_four_slices"}


@pytest.mark.parametrize("name", PROGRAMS)
def test_program_matches_reference(name, tmp_path):
    check_program_run(name, emulate=True, tmp_path=tmp_path, rtol=1e-3 if name in TRAINED else 1e-4)


@pytest.mark.parametrize("name", FUNCTIONS)
def test_function_matches_reference(name):
    got, want = function_call(name, emulate=True)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(w))))


def test_bounds_check_reports_the_value():
    rc, out, err, _ = run_program("bounds", emulate=True)
    assert rc == 1
    assert out.split() == [str(i) for i in range(10)]
    assert "index out of bounds (size 10) (got 10)" in err


def test_gather_fault_is_latched_and_reported():
    rc, out, err, _ = run_program("gather_oob", emulate=True)
    assert rc == 1 and out == ""
    assert "runtime error: index out of bounds (E[idx[i], d]; dimension size 5) (got 7)" in err


def test_failed_assert_exits_with_status_1():
    rc, out, err, _ = run_program("assert_fail", emulate=True)
    assert rc == 1 and "x is too big" in err and "unreachable" not in out


def test_checkpoint_save_then_load(tmp_path):
    """The same library run twice with its checkpoint in tmp_path ($ANVIL_OUT): the first run finds
    none and saves, the second loads what the first saved."""
    rc1, out1, err1, _ = run_program("save_load", emulate=True, out_dir=tmp_path)
    rc2, out2, err2, _ = run_program("save_load", emulate=True, out_dir=tmp_path)
    assert rc1 == 0 and rc2 == 0, err1 + err2
    assert out1.startswith("loaded 0.0000") and out2.startswith("loaded 1.0000")
    assert out1.split("sum")[1] == out2.split("sum")[1]
    raw = (tmp_path / "CKPT").read_bytes()
    assert raw[:4] == b"EINW" and int.from_bytes(raw[4:8], "little") == 2 and len(raw) == 16 + 8 + 4 * 12


@pytest.mark.parametrize("name", ["c2_small", "logreg", "control"])
def test_graph_mode_matches_reference(name):
    """Loop bodies captured as graph segments: host scalars reach kernels through their device copy,
    kept current by the host scalar kernels' device twins (here run eagerly, on the CPU)."""
    keep = kept_buffers(name)
    rc, out, err, arrays = run_program(name, emulate=True, keep=keep, env_extra={"ANVIL_HIP_GRAPHS": "1"})
    assert rc == 0, err
    z = vectors(name)
    problem = outputs_match(stdout_of(z), out, rtol=1e-3)
    assert problem is None, problem
    for k in keep:
        assert tensors_match(z[f"buf:{k}"], arrays[k], rtol=1e-3) is None, k


def test_loop_marks_window():
    """The loop marks bench.py times with: every iteration of the selected loop counted, an event
    only at the two iterations of the window, and no elapsed time for a mark outside it."""
    from anvil.backend import hip
    from fixtures import load_ir
    prog, data = load_ir("c2_small")
    src = hip.generate(prog, seed=data.get("seed", 0), emulate=True)
    lib = hip.HipLibrary(hip.compile_source(src, emulate=True), src)
    lib.lib.anvil_marks_select(b"x_batch")
    assert lib.lib.anvil_marks_window(3, 1) == -1 and lib.lib.anvil_marks_window(-1, 4) == -1
    assert lib.lib.anvil_marks_window(2, 9) == 0
    assert lib.main() == 0
    n = lib.lib.anvil_marks_count()
    assert n == 41          # 32 batches of the first epoch, 9 of the second (the ninth breaks at STEPS = 40)
    assert lib.lib.anvil_marks_elapsed_ms(2, 9) >= 0
    assert lib.lib.anvil_marks_elapsed_ms(0, 9) == -1 and lib.lib.anvil_marks_elapsed_ms(2, 5) == -1
    lib.lib.anvil_marks_select(b"x_batch")           # a new selection: every iteration again
    assert lib.main() == 0
    assert lib.lib.anvil_marks_count() == n and lib.lib.anvil_marks_elapsed_ms(0, n - 1) >= 0

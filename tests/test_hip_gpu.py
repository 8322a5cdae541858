"""Parity of the gfx950 libraries with the reference, on the GPU.

The same programs and functions as the CPU-build tests, now compiled with hipcc for MI355X and run
on the device: every kernel schedule (cross-lane row reductions, split reductions, fp32 MFMA
products with fused epilogues), the device arena, host scalars and the fault latch. Golden outputs
were written by the reference interpreter (tests/golden/make_fixtures.py); the libraries are built
by __graft_entry__.build() (they are looked up by the hash of their source).
"""
import json
import os
import re

import numpy as np
import pytest

import closed_forms
from fixtures import GOLDEN, load_ir, stdout_of, vectors
from hiprun import (accuracy_tokens, check_program_run, function_call, kept_buffers, outputs_match, run_program,
                    tensors_match)
from test_hip_emulate import FUNCTIONS, PROGRAMS, TRAINED

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", PROGRAMS)
def test_gpu_program_matches_reference(name, tmp_path):
    print(f"gpu program {name}", flush=True)
    check_program_run(name, emulate=False, tmp_path=tmp_path, rtol=1e-3 if name in TRAINED else 1e-4, timeout=300)


@pytest.mark.parametrize("name", ["c1_full", "c2_full", "c2_full10", "c4_full2", "c5_full3"])
def test_gpu_full_size_program_matches_reference(name):
    """C1, C2, C4 and C5 as BASELINE.json states them, against the reference interpreter's own runs
    (C4 at T = 64 for 2 of its 200 steps: the loss and weights of the first and last blocks and the
    output layer, to the same Adam bar as C2's 10 steps)
    (C5 for 3 of its 300 steps: the loss and the trained weights, through the implicit-GEMM
    convolutions, the fused input gradient and the sliced bias gradients; its first steps raise the
    loss from 2.3 to 5.7, and a ReLU or max-pool choice that flips between two nearly equal values
    sends a whole gradient elsewhere, so a different summation order shows up in a few weights:
    the loss must agree to 1e-3, 99 % of every tensor to 0.5 % of its largest value and all of it
    to 2 %; measured 0.09 %, and 0.12 % / 0.9 % at the worst tensor).
    C1 (784-128-10 MLP, SGD, batch 64, one epoch and the test accuracy): the printed loss and
    accuracy and the last layer's trained weights. C2 (784-1024-1024-10 MLP, Adam, batch 256, 500
    steps over 65,536 samples): the printed loss, to 2e-3 (the last batch's loss after 500 Adam
    steps depends on the order of every sum before it: the same kernels summing K in 8-k or 16-k
    chunks printed 2.3053, 2.3026 and 2.3072 against the reference's 2.3037). C2 for 10 steps at full size: the printed loss and
    trained weights and biases, measured against how far Adam moves a parameter (at most about lr
    per step, whatever its gradient's size: a gradient that crosses zero near a step takes a full
    step either way, so summing the batch in another order — the matrix cores' vs NumPy's — moves
    such a parameter differently). Every parameter must agree to 5 % of lr·steps and 99 % of them to
    0.2 % (measured: at most 0.9 %, 99th percentile 0.09 %). A bar relative to the tensor's largest
    value does not hold for biases, which start at 0. (Over 500 steps the differences compound and
    the weights drift apart while the loss still agrees; the north star bounds trained weights after
    100 steps.)"""
    print(f"gpu full-size program {name}", flush=True)
    keep = kept_buffers(name) if name != "c2_full" else []
    rc, out, err, arrays = run_program(name, emulate=False, keep=keep, timeout=300)
    assert rc == 0, err
    z = vectors(name)
    problem = outputs_match(stdout_of(z), out, rtol=2e-3 if name == "c2_full" else 1e-3)
    assert problem is None, problem
    if _step1_loss(stdout_of(z)) is not None:
        want, got = _step1_loss(stdout_of(z)), _step1_loss(out)
        assert abs(got - want) <= 1e-4 * abs(want), f"step-1 loss {got} vs {want}"
    assert accuracy_tokens(out) == accuracy_tokens(stdout_of(z)), "test accuracy differs"
    for k in keep:
        ref, got = z[f"buf:{k}"].astype(np.float64), arrays[k].astype(np.float64)
        if name == "c5_full3":
            err = np.abs(got - ref) / np.abs(ref).max()
            assert err.max() <= 0.02, f"{k}: max |error| {err.max():.3g} of the largest value"
            assert np.percentile(err, 99) <= 0.005, f"{k}: 99th percentile {np.percentile(err, 99):.3g}"
        elif name in ("c2_full10", "c4_full2"):
            moved = 1e-3 * (10 if name == "c2_full10" else 2)       # lr · steps
            err = np.abs(got - ref) / moved
            print(f"  {k}: |error| / (lr·steps): median {np.median(err):.2e} p99 {np.percentile(err, 99):.3g} "
                  f"max {err.max():.3g}", flush=True)
            assert err.max() <= 0.05, f"{k}: max |error| {err.max():.3g} of lr·steps"
            assert np.percentile(err, 99) <= 0.002, f"{k}: 99th percentile {np.percentile(err, 99):.3g} of lr·steps"
        else:
            problem = tensors_match(z[f"buf:{k}"], arrays[k], rtol=1e-3)
            assert problem is None, f"{k}: {problem}"


def _step1_loss(text):
    m = re.search(r"step 1 loss (\S+)", text)
    return None if m is None else float(m.group(1))


def _noise_floor(name):
    with open(os.path.join(GOLDEN, "noise_floor.json")) as f:
        return json.load(f)[name]


@pytest.mark.parametrize("name", ["c2_full100", "c4_t256_2", "c5_step1"])
def test_gpu_north_star_tolerances(name):
    """BASELINE.json's north-star bars at full size, against the reference interpreter's runs:
      - the first training step's loss of C2, C4 (at T = 256) and C5, printed to 7 digits, within
        rel 1e-4 (c2_full100, c4_t256_2, c5_step1; every C2/C4 fixture prints it too);
      - C2's parameters after 100 full-size Adam steps. Rel 1e-3 of each tensor's largest value
        cannot hold there for any float32 implementation that adds in another order than NumPy:
        the reference's own algorithm (the oracle) with its float sums merely reversed lands 1.4 %
        (W1), 3.5 % (W2) and 8 % (W3) of the largest weight from the reference at the 99th
        percentile (Adam moves a parameter by about lr whatever its gradient's size, so a gradient
        near zero whose sign depends on rounding takes a full step either way, and 100 steps
        compound it). The bar is that spread (tests/golden/noise_floor.json, written by
        tests/golden/make_noise_floor.py): for every parameter tensor, the median, 99th percentile
        and largest |error| over lr·steps within twice the larger of the reordered runs';
      - C4 at T = 256 for 2 steps: the weights of the first and last layers and the output layer
        against lr·steps, 99 % to 0.2 % and all to 5 % (as c4_full2 at T = 64).
    The measured errors are printed (pytest -s) for the record."""
    print(f"gpu north star {name}", flush=True)
    keep = kept_buffers(name)
    rc, out, err, arrays = run_program(name, emulate=False, keep=keep, timeout=300)
    assert rc == 0, err
    z = vectors(name)
    want_text = stdout_of(z)
    want, got = _step1_loss(want_text), _step1_loss(out)
    assert want is not None and got is not None, out
    print(f"{name}: step-1 loss {got!r} vs {want!r}: rel {abs(got - want) / abs(want):.2e}", flush=True)
    assert abs(got - want) <= 1e-4 * abs(want)
    problem = outputs_match(want_text, out, rtol=1e-3)
    assert problem is None, problem
    steps = {"c2_full100": 100, "c4_t256_2": 2}.get(name)
    floor = _noise_floor(name)["orders"] if name == "c2_full100" else None
    problems = []
    for k in keep:
        ref, val = z[f"buf:{k}"].astype(np.float64), arrays[k].astype(np.float64)
        by_max = np.abs(val - ref) / np.abs(ref).max()
        by_lr = np.abs(val - ref) / (1e-3 * steps)
        got_q = {"lr_p50": np.median(by_lr), "lr_p99": np.percentile(by_lr, 99), "lr_max": by_lr.max()}
        print(f"  {k}: |error| / max|w|: median {np.median(by_max):.2e} p99 {np.percentile(by_max, 99):.2e} "
              f"max {by_max.max():.2e}; / (lr·steps): median {got_q['lr_p50']:.2e} p99 {got_q['lr_p99']:.3g} "
              f"max {got_q['lr_max']:.3g}", flush=True)
        if floor is not None:
            for q, v in got_q.items():
                bar = 2 * max(o[k][q] for o in floor.values())
                if v > bar:
                    problems.append(f"{k} {q} {v:.3g} > {bar:.3g}")
        elif got_q["lr_max"] > 0.05 or got_q["lr_p99"] > 0.002:
            problems.append(f"{k}: p99 {got_q['lr_p99']:.3g} max {got_q['lr_max']:.3g} of lr·steps")
    assert not problems, f"parameters off by more than the bar: {problems}"


@pytest.mark.parametrize("name", FUNCTIONS)
def test_gpu_function_matches_reference(name):
    print(f"gpu function {name}", flush=True)
    got, want = function_call(name, emulate=False)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(w))))


def test_gpu_attention_at_full_size_matches_closed_form():
    """C3's attention, Q, K, V [4, 2048, 128]: the one-kernel path (scores never stored) against
    softmax(Q Kᵀ / √128) V computed in float64."""
    print("gpu attention full size", flush=True)
    prog, data = load_ir("c3_attention")
    assert any("attention:" in line for line in _source_lines(prog, data)), "not the one-kernel schedule"
    args, want = closed_forms.attention_case()
    got = _full_size_call("c3_attention", args)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(want))))


def _full_size_call(name, args):
    from anvil.hip_function import Compiled, Lowered
    prog, data = load_ir(name)
    low = Lowered.from_fixture(prog, data)
    assert [tuple(b.shape) for b in low.inputs] == [a.shape for a in args]
    return Compiled(low.name, low, seed=data.get("seed", 0)).call(args)


def test_gpu_softmax_at_full_size_matches_closed_form():
    """C3's softmax over the rows of [8192, 4096] (inputs ~N(0,1), seed 2) against float64 NumPy;
    every row also sums to 1."""
    print("gpu softmax full size", flush=True)
    args, want = closed_forms.softmax_case()
    got = _full_size_call("c3_softmax", args)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(got.astype(np.float64).sum(axis=1), 1.0, rtol=0, atol=1e-4)


def test_gpu_layernorm_at_full_size_matches_closed_form():
    """C3's layer_norm(x)·γ + β at [8192, 1024] (eps 1e-5, biased variance) against float64 NumPy."""
    print("gpu layernorm full size", flush=True)
    args, want = closed_forms.layernorm_case()
    got = _full_size_call("c3_layernorm", args)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


def test_gpu_linear_at_full_size_matches_closed_form():
    """C3's linear y = x·Wᵀ + b at [8192, 4096] × [4096, 4096]: one row of each of the 64 row tiles
    of 128 rows, at a different place in each tile, against float64 NumPy."""
    print("gpu linear full size", flush=True)
    args, want = closed_forms.linear_case()
    got = _full_size_call("c3_linear", args)
    np.testing.assert_allclose(got[closed_forms.LINEAR_ROWS], want, rtol=1e-4,
                               atol=1e-5 * float(np.max(np.abs(want))))


def test_gpu_linear_batch256_matches_closed_form():
    """x·Wᵀ + b at C2's layer shape, [256, 1024] × [1024, 1024]ᵀ (both operands contiguous in k, C2's
    input-gradient layout): 32 x 32 tiles with K split across the four wavefronts of a workgroup.
    Every output against float64 NumPy."""
    print("gpu linear 256x1024x1024", flush=True)
    prog, data = load_ir("c3_linear_b256")
    assert any("ksplit 32x32" in line for line in _source_lines(prog, data)), "not the K-split schedule"
    rng = np.random.default_rng(7)
    x = rng.standard_normal((256, 1024)).astype(np.float32)
    w = rng.standard_normal((1024, 1024)).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    got = _full_size_call("c3_linear_b256", [x, w, b])
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(want))))


def test_gpu_linear_2x2_tiles_matches_closed_form():
    """A linear layer of C4's MLP shape, [4096, 256] × [1024, 256]ᵀ, which takes one wavefront of
    2 x 2 MFMA tiles per workgroup: one row of each 64-row tile against float64 NumPy."""
    print("gpu linear 4096x1024x256", flush=True)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4096, 256)).astype(np.float32)
    w = rng.standard_normal((1024, 256)).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    got = _full_size_call("c3_linear_mid", [x, w, b])
    rows = 64 * np.arange(64) + (29 * np.arange(64)) % 64
    want = x[rows].astype(np.float64) @ w.astype(np.float64).T + b
    np.testing.assert_allclose(got[rows], want, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(want))))


def test_gpu_batched_2x2_tiles_matches_closed_form():
    """A batched product of C4's attention shape, 64 × ([256, 64] · [64, 256]), in 2 x 2 MFMA tiles
    per wavefront with the batch in the grid: every batch's outputs against float64 NumPy."""
    print("gpu bmm 64 x 256x256x64", flush=True)
    rng = np.random.default_rng(6)
    a = rng.standard_normal((64, 256, 64)).astype(np.float32)
    w = rng.standard_normal((64, 64, 256)).astype(np.float32)
    got = _full_size_call("c3_bmm", [a, w])
    want = np.matmul(a.astype(np.float64), w.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(want))))


def _source_lines(prog, data):
    from anvil.backend import hip
    return hip.generate(prog, seed=data.get("seed", 0), library=True).splitlines()


def test_gpu_bounds_check_reports_the_value():
    rc, out, err, _ = run_program("bounds", emulate=False, timeout=120)
    assert rc == 1
    assert out.split() == [str(i) for i in range(10)]
    assert "index out of bounds (size 10) (got 10)" in err


def test_gpu_gather_fault_is_latched_and_reported():
    rc, out, err, _ = run_program("gather_oob", emulate=False, timeout=120)
    assert rc == 1 and out == ""
    assert "runtime error: index out of bounds (E[idx[i], d]; dimension size 5) (got 7)" in err


def test_gpu_failed_assert_exits_with_status_1():
    rc, out, err, _ = run_program("assert_fail", emulate=False, timeout=120)
    assert rc == 1 and "x is too big" in err and "unreachable" not in out


def test_gpu_checkpoint_save_then_load(tmp_path):
    rc1, out1, err1, _ = run_program("save_load", emulate=False, timeout=120, out_dir=tmp_path)
    rc2, out2, err2, _ = run_program("save_load", emulate=False, timeout=120, out_dir=tmp_path)
    assert rc1 == 0 and rc2 == 0, err1 + err2
    assert out1.startswith("loaded 0.0000") and out2.startswith("loaded 1.0000")
    assert out1.split("sum")[1] == out2.split("sum")[1]


@pytest.mark.parametrize("name", ["c2_small", "logreg", "c4_small", "c4_mid", "c4_t160"])
def test_gpu_graph_replay_matches_reference(name):
    """The same programs with loop bodies captured once as HIP graphs and replayed (c4_mid and
    c4_t160: with the training attention's launches among the captured ones)."""
    print(f"gpu graphs {name}", flush=True)
    keep = kept_buffers(name)
    rc, out, err, arrays = run_program(name, emulate=False, keep=keep, timeout=300, env_extra={"ANVIL_HIP_GRAPHS": "1"})
    assert rc == 0, err
    z = vectors(name)
    problem = outputs_match(stdout_of(z), out, rtol=1e-3)
    assert problem is None, problem
    for k in keep:
        assert tensors_match(z[f"buf:{k}"], arrays[k], rtol=1e-3) is None, k


@pytest.mark.parametrize("name", ["c4_full200", "c5_full300"])
def test_gpu_full_runs_within_the_noise_floor(name):
    """C4 (T = 64, its 200 Adam steps) and C5 (its 300 SGD steps) run whole, against the oracle's
    runs of the same programs (tests/golden/make_long_runs.py: the oracle reproduces the reference
    interpreter bit for bit on the first steps of both, c4_full2 and c5_full3). Over a whole run
    every float32 implementation that adds in another order drifts from the reference's trajectory;
    the bar is how far the reference's own algorithm drifts when only its sums are reordered
    (tests/golden/noise_floor.json, the reversed and sequential runs of make_noise_floor.py):
      - the first step's loss within rel 1e-4 (nothing has drifted yet);
      - each later printed loss within twice the larger reordered run's relative error at the same
        print, or 1e-3, whichever is larger;
      - every kept parameter's median, 99th percentile and largest |error| over lr·steps within
        twice the larger reordered run's.
    C4 stays on the reference's trajectory (losses to 6-7 digits; the reordered runs too). C5 is
    chaotic where its loss falls off the plateau (steps 30-90): the reordered runs alone move the
    printed losses there by up to 76 %, the last one by 3-7 %; the HIP run, in the same regime,
    measured 8-81 % there and 10 % at the end. The measured errors are printed (pytest -s)."""
    print(f"gpu full run {name}", flush=True)
    keep = kept_buffers(name)
    rc, out, err, arrays = run_program(name, emulate=False, keep=keep, timeout=300)
    assert rc == 0, err
    z = vectors(name)
    floor = _noise_floor(name)
    want_text = stdout_of(z)
    want = [float(v) for v in re.findall(r"loss\s+(\S+)", want_text)]
    got = [float(v) for v in re.findall(r"loss\s+(\S+)", out)]
    assert want and len(got) == len(want), (out, want_text)
    assert abs(got[0] - want[0]) <= 1e-4 * abs(want[0]), (got[0], want[0])
    problems = []
    for i, (g, w) in enumerate(zip(got, want)):
        bar = max(1e-3, 2 * max(o["losses"][i] for o in floor["orders"].values()))
        rel = abs(g - w) / abs(w)
        print(f"  loss {i}: {g!r} vs {w!r}: rel {rel:.2e} (bar {bar:.2e})", flush=True)
        if rel > bar:
            problems.append(f"loss {i}: rel {rel:.3g} > {bar:.3g}")
    lr, steps = floor["lr"], floor["steps"]
    for k in keep:
        ref, val = z[f"buf:{k}"].astype(np.float64), arrays[k].astype(np.float64)
        by_lr = np.abs(val - ref) / (lr * steps)
        got_q = {"lr_p50": np.median(by_lr), "lr_p99": np.percentile(by_lr, 99), "lr_max": by_lr.max()}
        print(f"  {k}: / (lr·steps): median {got_q['lr_p50']:.2e} p99 {got_q['lr_p99']:.3g} "
              f"max {got_q['lr_max']:.3g}", flush=True)
        for q, v in got_q.items():
            bar = 2 * max(o[k][q] for o in floor["orders"].values())
            if v > bar:
                problems.append(f"{k} {q} {v:.3g} > {bar:.3g}")
    assert not problems, f"off by more than the noise floor: {problems}"

"""The oracle (oracle/interp.py) pinned against the reference interpreter and closed forms.

Golden vectors: every fixture in tests/golden/vectors was written by the reference interpreter
(anvil/interp.py) itself; the oracle must reproduce its stdout byte for byte and every kept buffer
bit for bit (RNG data, He-initialised weights after training, shuffled permutations, function
outputs). Closed forms: float64 NumPy restatements of softmax, layer norm, the linear layer and
attention (prelude.anvil:28-43, pyapi.py test style), and the shuffle against brute force.
"""
import io
import os

import numpy as np
import pytest

from fixtures import load_ir, load_ir_writing_to, run_oracle, stdin_of, stdout_of, vector_names, vectors, written_files
from oracle import interp


@pytest.mark.parametrize("name", vector_names(slow=os.environ.get("ANVIL_SLOW_ORACLE") == "1"))
def test_oracle_matches_reference_interpreter(name, tmp_path):
    z = vectors(name)
    files = written_files(z)
    prog, data = load_ir_writing_to(name, tmp_path) if files else load_ir(name)
    m, out = run_oracle(prog, data, z, stdin=stdin_of(name))
    assert out == stdout_of(z)
    for f in files:                                   # save_npy / save: the same bytes
        assert (tmp_path / f).read_bytes() == bytes(z[f"file:{f}"]), f
    if "check_error" in z.files:                       # --check: the same element, tensor and message
        assert m.check_error == bytes(z["check_error"]).decode()
        return
    by_name = {b.name: b for b in prog.buffers}
    by_id = {b.id: b for b in prog.buffers}
    for key in z.files:
        if key.startswith("buf:"):
            b = by_name[key[4:]]
            np.testing.assert_array_equal(m.arr(b)[:b.numel].reshape(b.shape), z[key], err_msg=key)
        elif key.startswith("output"):
            b = by_id[data["function"]["outputs"][int(key[6:])]]
            np.testing.assert_array_equal(m.arr(b)[:b.numel].reshape(b.shape), z[key], err_msg=key)


def _function_output(name):
    prog, data = load_ir(name)
    z = vectors(name)
    m, _ = run_oracle(prog, data, z)
    b = {b.id: b for b in prog.buffers}[data["function"]["outputs"][0]]
    return m.arr(b)[:b.numel].reshape(b.shape), z


def test_softmax_closed_form():
    got, z = _function_output("c3_softmax_small")
    x = z["input0"].astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(got, e / e.sum(axis=1, keepdims=True), rtol=1e-5, atol=1e-7)


def test_layernorm_closed_form():
    got, z = _function_output("c3_layernorm_small")
    x, g, b = (z[f"input{k}"].astype(np.float64) for k in range(3))
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    np.testing.assert_allclose(got, (x - mu) / np.sqrt(var + 1e-5) * g + b, rtol=1e-4, atol=1e-5)


def test_linear_closed_form():
    got, z = _function_output("c3_linear_small")
    x, W, b = (z[f"input{k}"].astype(np.float64) for k in range(3))
    np.testing.assert_allclose(got, x @ W.T + b, rtol=1e-4, atol=1e-4)


def test_attention_closed_form():
    got, z = _function_output("c3_attention_small")
    q, k, v = (z[f"input{i}"].astype(np.float64) for i in range(3))
    s = q @ k.transpose(0, 2, 1) / np.sqrt(q.shape[-1])
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    np.testing.assert_allclose(got, p @ v, rtol=1e-4, atol=1e-5)


def test_lowbias32_known_values():
    """lowbias32 (hash-prospector, constants 0x7feb352d / 0x846ca68b) is a bijection on uint32
    with h(0) = 0; its values on a few inputs computed with Python integers, step by step."""
    def ref(x):
        x ^= x >> 16
        x = (x * 0x7FEB352D) & 0xFFFFFFFF
        x ^= x >> 15
        x = (x * 0x846CA68B) & 0xFFFFFFFF
        x ^= x >> 16
        return x
    xs = np.array([0, 1, 2, 0xFFFFFFFF, 0x12345678, 0x9E3779B1], dtype=np.uint64)
    assert [int(v) for v in interp.lowbias32(xs)] == [ref(int(v)) for v in xs]
    assert int(interp.lowbias32(np.array([0]))[0]) == 0
    # a bijection: no collisions on a dense block of inputs
    block = interp.lowbias32(np.arange(1 << 16, dtype=np.uint64))
    assert len(np.unique(block)) == 1 << 16


def test_uniform_is_24_bit_grid():
    bits = interp.rand_bits(np.arange(4096), 3, 0, 17)
    u = interp.rand_uniform(bits, False)
    assert u.dtype == np.float32 and u.min() >= 0 and u.max() < 1
    assert np.all(u * (1 << 24) == np.floor(u * (1 << 24)))
    v = interp.rand_uniform(bits, True)
    assert v.min() > 0 and v.max() <= 1


@pytest.mark.parametrize("n", range(1, 8))
def test_shuffle_is_fisher_yates(n):
    """Brute force: the permutation equals swapping p[i] with p[draw_k % (i+1)] for i = n-1 .. 1,
    and every permutation of n <= 4 elements is reachable over seeds."""
    p = np.arange(n, dtype=np.int32)
    interp.shuffle_inplace(p, n, 5, 123)
    q = list(range(n))
    draws = [int(d) for d in interp.rand_bits(np.arange(max(n - 1, 0)), 5, 7, 123)]
    for k in range(n - 1):
        i = n - 1 - k
        j = draws[k] % (i + 1)
        q[i], q[j] = q[j], q[i]
    assert p.tolist() == q
    assert sorted(p.tolist()) == list(range(n))
    if n <= 4:
        seen = set()
        for seed in range(400):
            r = np.arange(n, dtype=np.int32)
            interp.shuffle_inplace(r, n, 0, seed)
            seen.add(tuple(r.tolist()))
        import math
        assert len(seen) == math.factorial(n)


def test_print_format_rules():
    assert interp.fmt_f32(0.0) == "0.0000"
    assert interp.fmt_f32(1e-5) == "1.0000e-05"
    assert interp.fmt_f32(123456.0) == "123456.0000"
    assert interp.fmt_f32(1e6) == "1.0000e+06"
    assert interp.fmt_f32(float("nan")) == "nan"
    assert interp.format_tensor(np.arange(8), (8,), True) == "[0, 1, 2, 3, 4, 5, 6, 7]"
    s = interp.format_tensor(np.arange(2000), (2000,), True)
    assert s == "[0, 1, 2, ..., 1997, 1998, 1999]"


def test_oracle_catches_a_planted_mistake():
    """A plausible mistake in the oracle (a sum reduction that drops its last element) must be
    caught by the golden vectors."""
    prog, data = load_ir("c3_softmax_small")
    z = vectors("c3_softmax_small")

    class Broken(interp.Machine):
        def reduce(self, op, body, nd):
            if op == "sum":
                body = body[..., :-1]
            return super().reduce(op, body, nd)
    m = Broken(prog, out=io.StringIO())
    by_id = {b.id: b for b in prog.buffers}
    m.arr(by_id[data["function"]["inputs"][0]])[:] = z["input0"].reshape(-1)
    m.run()
    b = by_id[data["function"]["outputs"][0]]
    assert not np.array_equal(m.arr(b)[:b.numel].reshape(b.shape), z["output0"])


def _linear_with_order(order):
    prog, data = load_ir("c3_linear_small")
    z = vectors("c3_linear_small")
    m = interp.Machine(prog, out=io.StringIO(), sum_order=order)
    by_id = {b.id: b for b in prog.buffers}
    for k, bid in enumerate(data["function"]["inputs"]):
        m.arr(by_id[bid])[:] = z[f"input{k}"].reshape(-1)
    m.run()
    b = by_id[data["function"]["outputs"][0]]
    return m.arr(b)[:b.numel].reshape(b.shape).copy(), z


def test_reordered_sums_change_only_the_rounding():
    """The oracle's other summation orders (used to measure the reorder spread of trained weights,
    tests/golden/make_noise_floor.py): the same sums up to float32 rounding, against float64 NumPy,
    and really another order (some results differ from NumPy's in the last bits); the reversed and
    sequential sums of 1, 2**-24, 2**-24 have closed forms (2**-24 is half an ulp of 1)."""
    x, w, bias = (vectors("c3_linear_small")[f"input{k}"].astype(np.float64) for k in range(3))
    exact = x @ w.T + bias
    base, _ = _linear_with_order("numpy")
    for order in ("reversed", "sequential"):
        got, _ = _linear_with_order(order)
        np.testing.assert_allclose(got, exact, rtol=0, atol=1e-5 * np.abs(exact).max())
        assert not np.array_equal(got, base), order
    body = np.array([[1.0, 2.0 ** -24, 2.0 ** -24]], np.float32)
    m = interp.Machine(load_ir("c3_linear_small")[0], out=io.StringIO(), sum_order="sequential")
    assert m.reduce("sum", body, 1)[0] == np.float32(1.0)             # 1 + h rounds to 1, twice
    m.sum_order = "reversed"
    assert m.reduce("sum", body, 1)[0] == np.float32(1.0 + 2.0 ** -23)  # h + h = ulp(1), then exact
    with pytest.raises(ValueError):
        interp.Machine(load_ir("c3_linear_small")[0], sum_order="pairwise")

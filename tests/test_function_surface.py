"""anvil.function's surface through the HIP library ABI (`anvil.hip_function.Compiled`, the twin of
the reference's pyapi.Compiled), as the reference's own tests use it (tests/test_pyapi.py:32-134):

  - an i32 argument, and a Python number passed as a compile-time constant: one lowering per value
    (fn_pick with scale 2.0, fn_pick_half with 0.5), and a constant that sets a shape (fn_shifted);
  - a loss-and-gradient tuple whose first item is a 0-d result (a NumPy scalar);
  - a scalar result, and a compile-time result beside a tensor one (the reference's `consts`);
  - a function that assigns into its argument leaves the caller's array unchanged;
  - float64 and transposed (non-contiguous) arguments are taken as contiguous float32;
  - eight threads calling one Compiled (the lock serializes the library's buffers);
  - causal attention.

Each function was lowered by the reference's pyapi.lower (tests/golden/make_fixtures.py). The
results are held to the reference interpreter's outputs on the same inputs and to the closed forms
the reference's tests use. The CPU build (-DANVIL_EMULATE) runs the same generated file.
"""
import threading

import numpy as np
import pytest

from fixtures import load_ir, vectors


def compiled(name, emulate):
    from anvil.hip_function import Compiled, Lowered
    prog, data = load_ir(name)
    low = Lowered.from_fixture(prog, data)
    return Compiled(low.name, low, seed=int(data.get("seed", 0)), emulate=emulate), vectors(name)


def np_softmax(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


MODES = [pytest.param(True, id="cpu"), pytest.param(False, id="gpu", marks=pytest.mark.gpu)]


@pytest.mark.parametrize("emulate", MODES)
def test_integer_argument_and_compile_time_constants(emulate):
    print(f"function surface: pick (emulate={emulate})", flush=True)
    for name, scale in (("fn_pick", 2.0), ("fn_pick_half", 0.5)):
        f, z = compiled(name, emulate)
        x, idx = z["input0"], z["input1"]
        assert idx.dtype == np.int32
        got = f.call([x, idx])
        np.testing.assert_array_equal(got, z["output0"])
        np.testing.assert_array_equal(got, x[idx] * np.float32(scale))
        # Python lists and int64 arrays are taken as i32
        np.testing.assert_array_equal(f.call([x, list(map(int, idx))]), got)
        np.testing.assert_array_equal(f.call([x, idx.astype(np.int64)]), got)
    f, z = compiled("fn_shifted", emulate)
    x = z["input0"]
    np.testing.assert_array_equal(f.call([x]), x[2:])


@pytest.mark.parametrize("emulate", MODES)
def test_loss_and_gradient_tuple(emulate):
    print(f"function surface: loss_and_grad (emulate={emulate})", flush=True)
    f, z = compiled("fn_loss_grad", emulate)
    w, x, y = z["input0"], z["input1"], z["input2"]
    loss, g = f.call([w, x, y])
    assert isinstance(loss, np.float32)
    np.testing.assert_allclose(loss, z["output0"], rtol=1e-5)
    np.testing.assert_allclose(g, z["output1"], rtol=1e-4, atol=1e-6)
    r = x.astype(np.float64) @ w - y
    np.testing.assert_allclose(loss, (r ** 2).mean(), rtol=1e-5)
    np.testing.assert_allclose(g, 2 * x.T @ r / 32, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("emulate", MODES)
def test_scalar_and_constant_results(emulate):
    print(f"function surface: scalar results (emulate={emulate})", flush=True)
    f, z = compiled("fn_total", emulate)
    t = f.call([z["input0"]])
    assert np.ndim(t) == 0 and t == pytest.approx(float(z["output0"]), rel=1e-5)
    assert f.call([np.arange(10.0)]) == 45.0
    g, z = compiled("fn_sizes", emulate)
    n, s = g.call([np.ones((3, 4))])
    assert n == 12 and s == 12.0
    n, s = g.call([z["input0"]])
    assert n == 12 and s == pytest.approx(float(z["output1"]), rel=1e-5)


@pytest.mark.parametrize("emulate", MODES)
def test_the_callers_arrays_are_not_modified(emulate):
    print(f"function surface: caller's arrays (emulate={emulate})", flush=True)
    f, z = compiled("fn_keeps_args", emulate)
    a = np.zeros(4, np.float32)
    np.testing.assert_array_equal(f.call([a]), [2, 0, 0, 0])
    np.testing.assert_array_equal(a, 0)
    x = z["input0"].copy()
    np.testing.assert_array_equal(f.call([x]), z["output0"])
    np.testing.assert_array_equal(x, z["input0"])


@pytest.mark.parametrize("emulate", MODES)
def test_non_contiguous_and_float64_arguments(emulate):
    print(f"function surface: float64, transposed (emulate={emulate})", flush=True)
    f, z = compiled("fn_double", emulate)
    x = np.arange(12.0).reshape(3, 4).T                     # float64, transposed: shape (4, 3)
    out = f.call([x])
    assert out.dtype == np.float32 and out.shape == (4, 3)
    np.testing.assert_array_equal(out, x * 2)
    np.testing.assert_array_equal(f.call([z["input0"]]), z["output0"])


@pytest.mark.parametrize("emulate", MODES)
def test_calls_from_threads(emulate):
    print(f"function surface: threads (emulate={emulate})", flush=True)
    f, z = compiled("fn_scaled", emulate)
    x = z["input0"]
    np.testing.assert_array_equal(f.call([x, z["input1"]]), z["output0"])
    f.call([x, np.float32(1)])
    results = {}

    def work(k):
        results[k] = f.call([x, np.float32(k)])
    ts = [threading.Thread(target=work, args=(k,)) for k in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    for k in range(8):
        np.testing.assert_array_equal(results[k], x * np.float32(k))


@pytest.mark.parametrize("emulate", MODES)
def test_causal_attention(emulate):
    print(f"function surface: causal attention (emulate={emulate})", flush=True)
    f, z = compiled("fn_causal", emulate)
    q, k, v = (z[f"input{i}"].astype(np.float64) for i in range(3))
    got = f.call([z["input0"], z["input1"], z["input2"]])
    np.testing.assert_allclose(got, z["output0"], rtol=1e-5, atol=1e-6)
    s = q @ k.transpose(0, 2, 1) / 2 + np.where(np.arange(7)[None, :] <= np.arange(7)[:, None], 0, -1e9)
    np.testing.assert_allclose(got, np_softmax(s) @ v, rtol=1e-5, atol=1e-6)

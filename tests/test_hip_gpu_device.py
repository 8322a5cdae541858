"""The device-pointer ABI (anvil_entry_device, hip_function.Compiled.call_device) that the C3
kernel timings go through: the same full-size functions as the host-array tests, with inputs and
results in device memory allocated through the HIP runtime (DeviceArray), against the same float64
closed forms. Inputs stay resident across two calls; the results of both calls must agree bit for
bit (the kernels sum in a fixed order)."""
import numpy as np
import pytest

import closed_forms
from fixtures import load_ir

pytestmark = pytest.mark.gpu

CASES = {
    "c3_softmax": (closed_forms.softmax_case, None, dict(rtol=1e-4, atol=1e-7)),
    "c3_layernorm": (closed_forms.layernorm_case, None, dict(rtol=1e-4, atol=1e-4)),
    "c3_linear": (closed_forms.linear_case, closed_forms.LINEAR_ROWS, None),
    "c3_attention": (closed_forms.attention_case, None, None),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_gpu_device_resident_call_matches_closed_form(name):
    print(f"gpu call_device {name}", flush=True)
    from anvil.hip_function import Compiled, DeviceArray, Lowered
    make, rows, tol = CASES[name]
    args, want = make()
    prog, data = load_ir(name)
    low = Lowered.from_fixture(prog, data)
    fn = Compiled(low.name, low, seed=data.get("seed", 0))
    dev_args = [DeviceArray.from_host(a) for a in args]
    dev_out = [DeviceArray(b.shape) for b in low.outputs]
    try:
        fn.call_device(dev_args, dev_out)
        first = dev_out[0].to_host()
        fn.call_device(dev_args, dev_out)
        second = dev_out[0].to_host()
    finally:
        for d in dev_args + dev_out:
            d.free()
    np.testing.assert_array_equal(first, second)
    got = first if rows is None else first[rows]
    tol = tol or dict(rtol=1e-4, atol=1e-5 * float(np.max(np.abs(want))))
    np.testing.assert_allclose(got, want, **tol)

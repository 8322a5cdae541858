"""The C ABI of generated libraries, on a machine without a GPU: a gfx950 library loads, exports
every symbol include/anvil_hip.h declares (and its per-function slots), and refuses to run without a
device instead of falling back to anything."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from fixtures import ROOT, load_ir


def declared_functions():
    with open(os.path.join(ROOT, "include", "anvil_hip.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^[a-z][\w \*]*?\b(anvil_\w+)\(", text, re.M)))


def gpu_library(name):
    from anvil.backend import hip
    prog, data = load_ir(name)
    return hip.compile_source(hip.generate(prog, seed=data.get("seed", 0), library="function" in data))


def test_header_declares_the_abi():
    names = declared_functions()
    for must in ("anvil_main", "anvil_entry", "anvil_entry_device", "anvil_init", "anvil_sync_device",
                 "anvil_profile_ms", "anvil_marks_elapsed_ms", "anvil_buffer_read", "anvil_arena_bytes"):
        assert must in names


def test_gpu_library_exports_every_declared_symbol():
    path = gpu_library("c3_softmax_small")
    lib = ctypes.CDLL(path)                     # loads without a GPU (nothing runs at load time)
    for name in declared_functions():
        assert hasattr(lib, name), name
    for slot in ("anvil_input0", "anvil_output0", "anvil_dinput0", "anvil_doutput0"):
        ctypes.c_void_p.in_dll(lib, slot)
    lib.anvil_target.restype = ctypes.c_char_p
    assert lib.anvil_target() == b"gfx950"


def test_without_a_gpu_the_library_refuses_to_run():
    path = gpu_library("greet")
    code = f"import ctypes, sys; sys.exit(ctypes.CDLL({path!r}).anvil_main())"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120,
                       env=dict(os.environ, HIP_VISIBLE_DEVICES=os.environ.get("HIP_VISIBLE_DEVICES", "")))
    if r.returncode == 0 and r.stdout:
        pytest.skip("a GPU is present here")
    assert r.returncode == 1 and "no HIP device" in r.stderr


def test_generation_is_deterministic():
    from anvil.backend import hip
    prog, _ = load_ir("c2_small")
    a = hip.generate(prog, seed=0)
    prog2, _ = load_ir("c2_small")
    assert a == hip.generate(prog2, seed=0)


def _emulated_function(name):
    from anvil.backend import hip
    from anvil.hip_function import Lowered
    prog, data = load_ir(name)
    src = hip.generate(prog, seed=data.get("seed", 0), library=True, emulate=True)
    return hip.HipLibrary(hip.compile_source(src, emulate=True), src), Lowered.from_fixture(prog, data)


@pytest.mark.parametrize("name", ["c3_attention_small", "c3_layernorm_small"])
def test_entry_device_gives_what_entry_gives_on_the_cpu_build(name):
    """anvil_entry_device with host arrays standing in for device pointers (in the CPU build device
    memory is host memory): the same results as anvil_entry's copy-in/copy-out call, bit for bit,
    and the library's own buffers are back in place afterwards (a later anvil_entry still works)."""
    import numpy as np
    from fixtures import vectors
    lib, low = _emulated_function(name)
    z = vectors(name)
    args = [np.ascontiguousarray(z[f"input{k}"]) for k in range(len(low.inputs))]

    def run(entry, prefix):
        outs = [np.full(b.shape, np.nan, np.float32) for b in low.outputs]
        for b, a in zip(low.inputs, args):
            lib.slot(prefix + b.name).value = a.ctypes.data
        for b, o in zip(low.outputs, outs):
            lib.slot(prefix + b.name).value = o.ctypes.data
        assert getattr(lib.lib, entry)() == 0
        for b in low.inputs + low.outputs:
            lib.slot(prefix + b.name).value = None
        return outs
    host = run("anvil_entry", "")
    dev = run("anvil_entry_device", "d")
    again = run("anvil_entry", "")
    for h, d, a, w in zip(host, dev, again, [z[f"output{k}"] for k in range(len(low.outputs))]):
        np.testing.assert_array_equal(h, d)
        np.testing.assert_array_equal(h, a)
        np.testing.assert_allclose(d, w, rtol=1e-4, atol=1e-5 * float(np.max(np.abs(w))))


class _FakeTensor:
    """What device_pointer reads of a torch tensor."""

    def __init__(self, shape, dtype="torch.float32", cuda=True, contiguous=True, ptr=1 << 20):
        self.shape, self.dtype, self.is_cuda, self._c, self._p = shape, dtype, cuda, contiguous, ptr
        self.device = "cuda:0" if cuda else "cpu"

    def is_contiguous(self):
        return self._c

    def data_ptr(self):
        return self._p


def test_call_device_refuses_arrays_that_do_not_fit():
    from anvil import ir
    from anvil.hip_function import device_pointer
    b = ir.Buffer("input0", (64, 300), "f32", "input")
    assert device_pointer(_FakeTensor((64, 300)), b) == 1 << 20
    bad = [_FakeTensor((64, 301)), _FakeTensor((64, 300), dtype="torch.float16"),
           _FakeTensor((64, 300), cuda=False), _FakeTensor((64, 300), contiguous=False),
           _FakeTensor((64, 300), ptr=(1 << 20) + 4), 12345]
    for t in bad:
        with pytest.raises((TypeError, ValueError)):
            device_pointer(t, b)

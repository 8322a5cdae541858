"""anvil_entry_noalloc, the entry point that allocates nothing, against anvil_entry_device.

Both run one call of a lowered function on device buffers the caller allocated; the no-allocation
entry keeps the function's other buffers (the attention scores and probabilities of the three-kernel
schedule, the host-scalar copy) in the library's static `anvil_scratch` array instead of the arena
that anvil_entry_device's first call allocates. Results must be bit-identical: the same kernels run
in the same order, only the temporaries' addresses differ. Every call is compared, on two calls in a
row with different inputs into one library, and on a call of a second library whose shapes are
smaller (shapes are fixed when a function is lowered, so a smaller input is a smaller compilation).
Refused calls (wrong argument count or size) must return their status and leave the outputs alone.
"""
import ctypes

import numpy as np
import pytest

from fixtures import load_ir

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p
LL = ctypes.c_longlong


def _library(name):
    from anvil.hip_function import Compiled, Lowered
    prog, data = load_ir(name)
    low = Lowered.from_fixture(prog, data)
    fn = Compiled(low.name, low, seed=data.get("seed", 0))
    entry = fn.lib.lib.anvil_entry_noalloc
    entry.restype = ctypes.c_int
    entry.argtypes = [ctypes.POINTER(P), ctypes.POINTER(LL), ctypes.c_int, ctypes.POINTER(P),
                      ctypes.POINTER(LL), ctypes.c_int, P]
    return fn, low, entry


def _noalloc(entry, args, outs, n_in=None, bytes_in=None, stream=None):
    ins = (P * len(args))(*[a.data_ptr() for a in args])
    nin = (LL * len(args))(*[a.nbytes if bytes_in is None else bytes_in for a in args])
    ous = (P * len(outs))(*[o.data_ptr() for o in outs])
    nou = (LL * len(outs))(*[o.nbytes for o in outs])
    return entry(ins, nin, len(args) if n_in is None else n_in, ous, nou, len(outs), stream)


def _inputs(low, seed):
    from anvil.hip_function import DeviceArray
    rng = np.random.default_rng(seed)
    return [DeviceArray.from_host(rng.standard_normal(b.shape).astype(np.float32)) for b in low.inputs]


def _compare(name, seeds):
    from anvil.hip_function import DeviceArray
    fn, low, entry = _library(name)
    for seed in seeds:
        print(f"no-alloc {name} seed {seed}", flush=True)
        args = _inputs(low, seed)
        want = [DeviceArray(b.shape) for b in low.outputs]
        got = [DeviceArray(b.shape) for b in low.outputs]
        fn.call_device(args, want)
        assert _noalloc(entry, args, got) == 0
        for w, g in zip(want, got):
            np.testing.assert_array_equal(g.to_host(), w.to_host())
        for d in args + want + got:
            d.free()


def test_noalloc_matches_entry_device_on_two_calls_then_a_smaller_function():
    # c3_attention_small keeps s and p in scratch (three kernels); then the same function compiled
    # for half the keys and head size, in a second library
    _compare("c3_attention_small", seeds=[11, 12])
    _compare("c3_attention_tiny", seeds=[13])


def test_noalloc_refuses_mismatched_arguments_without_running():
    from anvil.hip_function import DeviceArray
    fn, low, entry = _library("c3_attention_small")
    args = _inputs(low, 14)
    sentinel = np.full(low.outputs[0].shape, 7.0, np.float32)
    out = DeviceArray.from_host(sentinel)
    print("no-alloc refusals", flush=True)
    assert _noalloc(entry, args, [out], n_in=2) == -1
    assert _noalloc(entry, args, [out], bytes_in=args[0].nbytes - 4) == -2
    np.testing.assert_array_equal(out.to_host(), sentinel)
    for d in args + [out]:
        d.free()


def test_noalloc_on_a_stream_of_the_callers():
    from anvil.hip_function import DeviceArray
    hip = ctypes.CDLL("libamdhip64.so")
    stream = P()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    fn, low, entry = _library("c3_attention_small")
    args = _inputs(low, 15)
    want = [DeviceArray(b.shape) for b in low.outputs]
    got = [DeviceArray(b.shape) for b in low.outputs]
    print("no-alloc on a created stream", flush=True)
    fn.call_device(args, want)
    assert _noalloc(entry, args, got, stream=stream) == 0
    assert hip.hipStreamSynchronize(stream) == 0
    np.testing.assert_array_equal(got[0].to_host(), want[0].to_host())
    assert hip.hipStreamDestroy(stream) == 0
    for d in args + want + got:
        d.free()

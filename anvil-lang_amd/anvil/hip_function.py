"""`anvil.function` on the GPU: a lowered function compiled by the HIP backend and called through
the library-mode C ABI.

`Compiled` is the HIP twin of the reference's pyapi.Compiled (pyapi.py:237-299): it takes what
pyapi.lower returns (a program whose arguments are `input<k>` buffers and whose results are
`output<k>` buffers), builds the library once (cached by the hash of the generated source), and on
each call points the `anvil_input<k>` / `anvil_output<k>` slots at the caller's arrays, calls
`anvil_entry()` under a lock, and clears the slots. Results are new arrays, as in the reference.

NumPy arguments live in host memory, so each call copies them to the device and the results back
(the slots hold host pointers, exactly as in the reference's ABI). `call_device` is the extension
for arrays that already live on the GPU (ROCm torch tensors, or `DeviceArray`s): the
same program reads and writes them in place through the `anvil_dinput<k>` / `anvil_doutput<k>`
slots, with no copies.

A run-time error in the compiled code (an index out of bounds) ends the process, as in the
reference (pyapi.py:25-26).
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import ir
from .backend import hip


class Lowered:
    """A function as a program of its own (the fields pyapi.Lowered has, pyapi.py:100-111)."""

    def __init__(self, prog, inputs, outputs, consts=(), tuple_result=False, name="fn"):
        self.prog = prog
        self.inputs = list(inputs)
        self.outputs = list(outputs)
        self.consts = list(consts)
        self.tuple_result = tuple_result
        self.name = name

    @staticmethod
    def from_fixture(prog, data) -> "Lowered":
        """From an irjson document with a "function" entry (input and output buffer ids)."""
        by_id = {b.id: b for b in prog.buffers}
        fn = data["function"]
        outs = [None if i is None else by_id[i] for i in fn["outputs"]]
        return Lowered(prog, [by_id[i] for i in fn["inputs"]], outs, consts=fn.get("consts", ()),
                       name=fn.get("name", "fn"), tuple_result=fn.get("tuple_result", len(outs) > 1))


class Compiled:
    """emulate: the generated file built as plain C++ for the CPU (a test build, never a fallback;
    call_device then has no device to use)."""

    def __init__(self, name, lowered: Lowered, seed: int = 0, emulate: bool = False):
        self.name = name
        self.prog = lowered.prog
        self.inputs = lowered.inputs
        self.outputs = lowered.outputs
        self.consts = lowered.consts
        self.tuple_result = lowered.tuple_result
        self.source = hip.generate(self.prog, seed=seed, library=True, emulate=emulate)
        self.lib = hip.HipLibrary(hip.compile_source(self.source, emulate=emulate), self.source)
        exported = set()
        for b in self.inputs + [o for o in self.outputs if o is not None]:
            try:
                self.lib.slot(b.name)
                exported.add(b.id)
            except ValueError:
                pass
        # an argument the function never reads has no slot (pyapi.py:270-275)
        self.in_slots = [self.lib.slot(b.name) if b.id in exported else None for b in self.inputs]
        self.out_slots = [self.lib.slot(b.name) if b is not None and b.id in exported else None
                          for b in self.outputs]
        self.din_slots = [self.lib.slot("d" + b.name) if b.id in exported else None for b in self.inputs]
        self.dout_slots = [self.lib.slot("d" + b.name) if b is not None and b.id in exported else None
                           for b in self.outputs]
        self.lock = threading.Lock()

    @property
    def ir(self) -> str:
        return "\n".join(ir.fmt_kernel(k) for k in ir.all_kernels(self.prog))

    def _check(self, arrays):
        if len(arrays) != len(self.inputs):
            raise TypeError(f"{self.name} takes {len(self.inputs)} tensor arguments, got {len(arrays)}")

    def call(self, arrays):
        self._check(arrays)
        args = []
        for a, b in zip(arrays, self.inputs):
            a = np.ascontiguousarray(a, dtype=np.int32 if b.dtype == "i32" else np.float32)
            if a.shape != b.shape:
                raise ValueError(f"argument {b.name} has shape {a.shape}; this version was compiled for {b.shape}")
            args.append(a)
        results = [None if b is None else np.empty(b.shape, np.float32 if b.dtype == "f32" else np.int32)
                   for b in self.outputs]
        with self.lock:
            for slot, a in zip(self.in_slots, args):
                if slot is not None:
                    slot.value = a.ctypes.data
            for slot, r in zip(self.out_slots, results):
                if slot is not None:
                    slot.value = r.ctypes.data
            self.lib.lib.anvil_entry()
            for slot in self.in_slots + self.out_slots:
                if slot is not None:
                    slot.value = None
        return self._result(results)

    def call_device(self, tensors, outputs=None):
        """Device arrays in and out: ROCm torch tensors, or DeviceArray (below). Each must have the
        shape and dtype the function was compiled for and be contiguous on the GPU; anything else is
        refused before the library sees its address (the kernels would read or write past it).
        `outputs` are preallocated device arrays for the results (torch tensors are made if None)."""
        self._check(tensors)
        if outputs is None:
            import torch
            dev = next((t.device for t in tensors if hasattr(t, "device")), "cuda")
            outputs = [None if b is None else torch.empty(b.shape, device=dev,
                                                          dtype=torch.float32 if b.dtype == "f32" else torch.int32)
                       for b in self.outputs]
        if len(outputs) != len(self.outputs):
            raise TypeError(f"{self.name} has {len(self.outputs)} results, got {len(outputs)} output arrays")
        in_ptrs = [device_pointer(t, b) for t, b in zip(tensors, self.inputs)]
        out_ptrs = [None if b is None else device_pointer(t, b) for t, b in zip(outputs, self.outputs)]
        with self.lock:
            for slot, p in zip(self.din_slots, in_ptrs):
                if slot is not None:
                    slot.value = p
            for slot, p in zip(self.dout_slots, out_ptrs):
                if slot is not None:
                    slot.value = p
            self.lib.lib.anvil_entry_device()
            for slot in self.din_slots + self.dout_slots:
                if slot is not None:
                    slot.value = None
        return self._result(outputs)

    def _result(self, results):
        consts = iter(self.consts)
        out = [next(consts) if r is None else (r[()] if getattr(r, "ndim", 1) == 0 else r) for r in results]
        return tuple(out) if self.tuple_result else out[0]


def device_pointer(t, b) -> int:
    """The device address of t, after checking that t can stand for buffer b: same shape and dtype,
    contiguous, on the GPU, 16-byte aligned (the kernels load 16 bytes at a time)."""
    want = "float32" if b.dtype == "f32" else "int32"
    if hasattr(t, "is_cuda"):                                           # a torch tensor
        if not t.is_cuda:
            raise ValueError(f"{b.name}: a device array is needed, got a tensor on {t.device}")
        if str(t.dtype) != f"torch.{want}":
            raise TypeError(f"{b.name}: dtype {t.dtype}, compiled for {want}")
        if tuple(t.shape) != tuple(b.shape):
            raise ValueError(f"{b.name}: shape {tuple(t.shape)}, compiled for {tuple(b.shape)}")
        if not t.is_contiguous():
            raise ValueError(f"{b.name}: the tensor is not contiguous")
        p = t.data_ptr()
    elif isinstance(t, DeviceArray):
        if t.dtype != want or tuple(t.shape) != tuple(b.shape):
            raise ValueError(f"{b.name}: {t.dtype}{list(t.shape)}, compiled for {want}{list(b.shape)}")
        p = t.data_ptr()
    else:
        raise TypeError(f"{b.name}: expected a torch tensor on the GPU or a DeviceArray, got {type(t).__name__}")
    if p % 16:
        raise ValueError(f"{b.name}: device address {p:#x} is not 16-byte aligned")
    return p


class DeviceArray:
    """A contiguous f32/i32 array in device memory, allocated through the HIP runtime itself (no
    framework needed): for callers that keep their data on the GPU between calls."""

    _hip = None

    def __init__(self, shape, dtype="float32"):
        if DeviceArray._hip is None:
            DeviceArray._hip = ctypes.CDLL("libamdhip64.so")
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype).name
        if self.dtype not in ("float32", "int32"):
            raise TypeError(f"DeviceArray holds float32 or int32, not {self.dtype}")
        self.nbytes = 4 * int(np.prod(self.shape, dtype=np.int64))
        self.ptr = ctypes.c_void_p()
        rc = DeviceArray._hip.hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(max(self.nbytes, 16)))
        if rc != 0:
            raise MemoryError(f"hipMalloc of {self.nbytes} bytes failed (status {rc})")

    @classmethod
    def from_host(cls, a) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d._copy(d.ptr, a.ctypes.data_as(ctypes.c_void_p), 1)
        return d

    def to_host(self):
        a = np.empty(self.shape, self.dtype)
        self._copy(a.ctypes.data_as(ctypes.c_void_p), self.ptr, 2)
        return a

    def _copy(self, dst, src, kind):
        rc = DeviceArray._hip.hipMemcpy(dst, src, ctypes.c_size_t(self.nbytes), kind)
        if rc != 0:
            raise RuntimeError(f"hipMemcpy failed (status {rc})")

    def data_ptr(self) -> int:
        return self.ptr.value

    def free(self):
        if self.ptr.value:
            DeviceArray._hip.hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

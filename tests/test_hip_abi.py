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
    path = gpu_library("hello")
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

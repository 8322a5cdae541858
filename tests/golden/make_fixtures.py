"""Write the golden fixtures: kernel IR and interpreter vectors from the reference.

Run in the development container only (the reference checkout is not on the GPU box):

    python tests/golden/make_fixtures.py [/root/reference] [NAME ...] [--route-only]

(--route-only: the IR and the reference-route source hashes, without running the interpreter.)

The reference numbers IR objects from one counter per process (ir.py:37-41), so a program's ids
depend on the programs compiled before it in the same run; a program marked `own_process` is
written by a child process of its own, which gives it the same ids whether it is written alone or
in a full run.

For each program in `programs.py` (Anvil source written for this repository's tests and
workloads) it writes:
  - ir/<name>.json       the optimized kernel IR that the reference front end produces
                          (driver.compile_text: parse -> elaborate -> autodiff -> optimize,
                          driver.py:33-41), or for a function, pyapi.lower (pyapi.py:114-181);
  - vectors/<name>.npz    for programs marked `interp`: what the reference interpreter
                          (interp.py:118-644) prints and the final contents of chosen buffers.

Nothing here is imported by the product, the oracle or the GPU tests; they read the JSON and
NPZ files. The reference's own code is imported only by this script.
"""
from __future__ import annotations

import hashlib
import importlib.util
import io
import subprocess
import json
import os
import shutil
import sys

import numpy as np

sys.dont_write_bytecode = True
HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))


def _irjson():
    """This package's serializer, loaded by file path (its dump needs no package import)."""
    path = os.path.join(REPO, "anvil-lang_amd", "anvil", "irjson.py")
    spec = importlib.util.spec_from_file_location("_fixture_irjson", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _backend_on_reference():
    """This repository's HIP backend modules loaded as members of the reference's own
    `anvil.backend` package, so that their `from .. import ir` is the reference's ir module and
    `generate` receives the reference's own Program objects (the drop-in route)."""
    import anvil.backend as ref_backend
    ours = os.path.join(REPO, "anvil-lang_amd", "anvil", "backend")
    if ours not in ref_backend.__path__:
        ref_backend.__path__.append(ours)
    import anvil.backend.hip as hip
    assert hip.ir.__file__.startswith(os.path.dirname(ref_backend.__file__).rsplit(os.sep, 1)[0])
    return hip


ROUTE = os.path.join(HERE, "reference_route.json")


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from anvil.driver import compile_text          # the reference front end
    from anvil.interp import Interpreter
    from anvil import pyapi
    sys.path.insert(0, HERE)
    import programs

    irjson = _irjson()
    hip = _backend_on_reference()
    os.makedirs(os.path.join(HERE, "ir"), exist_ok=True)
    os.makedirs(os.path.join(HERE, "vectors"), exist_ok=True)
    args = sys.argv[2:]
    route_only = "--route-only" in args
    only = set(a for a in args if not a.startswith("--"))
    route = {}
    if os.path.exists(ROUTE):
        with open(ROUTE) as f:
            route = json.load(f)
    for spec in programs.PROGRAMS:
        name = spec["name"]
        if only and name not in only:
            continue
        if spec.get("own_process") and only != {name}:
            with open(ROUTE, "w") as f:                  # what this run has so far, for the child to extend
                json.dump(dict(sorted(route.items())), f, indent=1)
            subprocess.run([sys.executable, os.path.abspath(__file__), ref_root, name]
                           + (["--route-only"] if route_only else []), check=True)
            with open(ROUTE) as f:
                route[name] = json.load(f)[name]
            continue
        path = spec.get("path") or os.path.join(HERE, "programs", f"{name}.anvil")
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        if spec.get("function"):
            fn = spec["function"]
            # a tensor argument is (shape, dtype); a Python number passed to the function is
            # ("const", its Anvil text), a compile-time constant (pyapi.arguments)
            sig = tuple(("const", a[1]) if a[0] == "const" else ("tensor", tuple(a[0]), a[1]) for a in fn["args"])
            low = pyapi.lower(spec["source"], path, fn["name"], sig, seed=spec.get("seed", 0))
            prog = low.prog
            data = irjson.dump(prog)
            data["function"] = {"name": fn["name"], "inputs": [b.id for b in low.inputs],
                                "outputs": [None if b is None else b.id for b in low.outputs],
                                "arg_names": list(low.arg_names), "out_names": list(low.out_names),
                                "consts": [c.item() if hasattr(c, "item") else c for c in low.consts],
                                "tuple_result": bool(low.tuple_result)}
        else:
            prog = compile_text(spec["source"], path=path, consts=spec.get("consts"),
                                optimize=spec.get("optimize", True)).program
            data = irjson.dump(prog)
            if spec.get("check"):
                # what --check says about each kernel (the reference's aarch64.check_description)
                from anvil.backend.aarch64 import check_description
                from anvil import ir as ref_ir
                descs = {k.id: check_description(k) for k in ref_ir.all_kernels(prog)}
                for kd in _kernels(data["main"]):
                    kd["kernel"]["desc"] = descs[kd["kernel"]["id"]]
        data["seed"] = spec.get("seed", 0)
        if spec.get("check"):
            data["check"] = spec["check"]                # built and run with --check=<mode>
        # the source the backend generates from the reference's own objects (sha256): the JSON
        # route must give the same bytes (tests/test_reference_route.py)
        src = hip.generate(prog, seed=data["seed"], library=bool(spec.get("function")), graphs=False,
                           check=spec.get("check"))
        route[name] = {"sha256": hashlib.sha256(src.encode()).hexdigest(), "library": bool(spec.get("function")),
                       "bytes": len(src)}
        with open(os.path.join(HERE, "ir", f"{name}.json"), "w") as f:
            json.dump(data, f, separators=(",", ":"))
        nk = sum(1 for _ in _kernels(data["main"]))
        print(f"{name}: {nk} kernels, source {route[name]['sha256'][:12]}", flush=True)
        # --check vectors quote kernel names (k<id>), which a new dump renumbers: always rerun those
        if not spec.get("interp") or (route_only and not spec.get("check")):
            continue
        out = io.StringIO()
        it = Interpreter(prog, out=out, seed=spec.get("seed", 0), inp=io.StringIO(spec.get("stdin", "")),
                         check=spec.get("check"))
        arrays = {}
        if spec.get("function"):
            rng = np.random.default_rng(spec["function"].get("input_seed", 2))
            tensor_args = [a for a in spec["function"]["args"] if a[0] != "const"]
            for k, (b, (shape, dtype)) in enumerate(zip(low.inputs, tensor_args)):
                x = (rng.standard_normal(shape).astype(np.float32) if dtype == "f32"
                     else rng.integers(0, spec["function"].get("int_hi", 10), shape).astype(np.int32))
                it.arr(b)[:b.numel] = x.reshape(-1)
                arrays[f"input{k}"] = x
        arrays["check_error"] = np.frombuffer(b"", dtype=np.uint8)
        try:
            it.run()
        except Exception as e:                           # --check: the interpreter's message
            if not spec.get("check") or type(e).__name__ != "AnvilRuntimeError":
                raise
            arrays["check_error"] = np.frombuffer(str(e).encode(), dtype=np.uint8)
        if not spec.get("check"):
            del arrays["check_error"]
        by_name = {b.name: b for b in prog.buffers}
        for bname in spec.get("keep", []):
            b = by_name[bname]
            arrays[f"buf:{bname}"] = it.arr(b)[:b.numel].reshape(b.shape).copy()
        if spec.get("function"):
            for k, b in enumerate(low.outputs):
                if b is not None:
                    arrays[f"output{k}"] = it.arr(b)[:b.numel].reshape(b.shape).copy()
        # files the program wrote (save_npy, save), kept byte for byte; a checkpoint the reference
        # wrote may also be published as a data file for a program that loads it
        for fname in spec.get("files", []):
            written = os.path.join(os.path.dirname(path), fname)
            with open(written, "rb") as f:
                arrays[f"file:{fname}"] = np.frombuffer(f.read(), dtype=np.uint8)
            if fname in spec.get("publish", {}):
                shutil.copyfile(written, os.path.join(HERE, "data", spec["publish"][fname]))
            os.remove(written)
        arrays["stdout"] = np.frombuffer(out.getvalue().encode(), dtype=np.uint8)
        np.savez_compressed(os.path.join(HERE, "vectors", f"{name}.npz"), **arrays)
    with open(ROUTE, "w") as f:
        json.dump(dict(sorted(route.items())), f, indent=1)


def _kernels(stmts):
    for s in stmts:
        if s["t"] == "kernel":
            yield s
        for key in ("body", "then", "else", "cond_block"):
            if key in s:
                yield from _kernels(s[key])


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

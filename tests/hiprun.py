"""Running generated libraries in tests, and comparing their results with the reference's.

Whole programs run in a child process (`python -m anvil run`), so that a program that ends with
a run-time error (exit status 1, as compiled Anvil programs do) ends only that child. Functions
run in this process through the library-mode ABI (anvil.hip_function.Compiled).

Comparison rules (the bar the backend is held to):
  - printed text must be identical apart from numbers;
  - integers (and so shuffled permutations, gathered indices, argmax results, counts, device-drawn
    randint values) bit for bit: a token printed without a point or exponent must be the same text;
  - a printed float within `rtol` of the reference's, or within one unit of its last printed digit,
    and printed the same way (same decimals, same fixed or scientific notation, except for two
    values that straddle the default format's switch at 1e6 or 1e-4);
  - a float tensor within `rtol` of the reference's, relative to the tensor's largest magnitude.
"""
from __future__ import annotations

import json
import os
import re
import subprocess
import sys
import tempfile

import numpy as np

from fixtures import ROOT_PKG, ir_path, load_ir, vectors

NUMBER = re.compile(r"[-+]?(?:\d+\.\d*|\.\d+|\d+)(?:[eE][-+]?\d+)?|[-+]?inf|nan")


def run_program(name_or_path: str, emulate: bool, keep=(), timeout: int = 600, cwd=None, env_extra=None,
                check=None, stdin: str = "", out_dir=None, extra_args=()):
    """(exit status, stdout, stderr, {buffer name: final contents}). stdin: what `input` reads;
    out_dir: where the files the program writes go ($ANVIL_OUT; the library is the same build);
    extra_args: more options of `anvil run` (--profile)."""
    path = name_or_path if name_or_path.endswith(".json") else ir_path(name_or_path)
    with tempfile.TemporaryDirectory() as d:
        dump = os.path.join(d, "out.npz")
        cmd = [sys.executable, "-u", "-m", "anvil", "run", path]
        if emulate:
            cmd.append("--emulate")
        if check:
            cmd.append(f"--check={check}")
        if keep:
            cmd += ["--dump", dump, "--keep", ",".join(keep)]
        cmd += list(extra_args)
        env = dict(os.environ, PYTHONPATH=ROOT_PKG + os.pathsep + os.environ.get("PYTHONPATH", ""))
        env.update(env_extra or {})
        if out_dir is not None:
            env["ANVIL_OUT"] = str(out_dir)
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, cwd=cwd or d, env=env,
                           input=stdin)
        arrays = {}
        if keep and os.path.exists(dump):
            z = np.load(dump)
            arrays = {k[4:]: z[k] for k in z.files if k.startswith("buf:")}
        return r.returncode, r.stdout, r.stderr, arrays


def _unit(token: str) -> float:
    """One unit of the last printed digit of a number."""
    mant, _, exp = token.lower().partition("e")
    dec = len(mant.split(".")[1]) if "." in mant else 0
    return 10.0 ** (-dec) * (10.0 ** int(exp) if exp else 1.0)


def _is_integer(token: str) -> bool:
    """A printed integer: digits with an optional sign, no point, no exponent (`%d`, i32 tensors)."""
    return token.lstrip("+-").isdigit()


def _form(token: str) -> tuple:
    """How a float was printed: decimals after the point, and fixed (%.Nf) or scientific (%.Ne)."""
    mant, e, _ = token.lower().partition("e")
    return (len(mant.split(".")[1]) if "." in mant else 0, bool(e))


def number_mismatch(x: str, y: str, rtol: float) -> bool:
    """True if the printed number y does not stand for the reference's x under the rules above."""
    if x == y:
        return False
    if _is_integer(x) or _is_integer(y):
        return True                                    # integers (and argmax, counts) bit for bit
    fx, fy = float(x), float(y)
    if np.isnan(fx) and np.isnan(fy):
        return False
    if _form(x) != _form(y):
        # the default format switches between %.4f and %.4e at |v| = 1e6 and 1e-4: two values
        # within rtol of each other may straddle that line, and nothing else changes the form
        near = any(abs(abs(fx) - edge) <= rtol * edge for edge in (1e6, 1e-4))
        return not (near and abs(fx - fy) <= rtol * abs(fx))
    return abs(fx - fy) > max(rtol * abs(fx), 1.01 * _unit(x))


def outputs_match(want: str, got: str, rtol: float) -> str | None:
    """None if the texts match under the rules above, else a description of the first difference."""
    wl, gl = want.splitlines(), got.splitlines()
    if len(wl) != len(gl):
        return f"{len(gl)} lines, expected {len(wl)}:\n{got[-800:]}"
    for i, (a, b) in enumerate(zip(wl, gl)):
        if a == b:
            continue
        ta, tb = NUMBER.split(a), NUMBER.split(b)
        na, nb = NUMBER.findall(a), NUMBER.findall(b)
        if ta != tb or len(na) != len(nb):
            return f"line {i + 1}: {b!r}, expected {a!r}"
        for x, y in zip(na, nb):
            if number_mismatch(x, y, rtol):
                return f"line {i + 1}: {y} where the reference printed {x} ({b!r})"
    return None


def accuracy_tokens(text: str) -> list[str]:
    """The printed test accuracies (`accuracy X`): a count of argmax hits over the test set divided
    by its size, so it must be the same text as the reference's, not merely close."""
    return re.findall(r"accuracy\s+(\S+)", text)


def tensors_match(want: np.ndarray, got: np.ndarray, rtol: float) -> str | None:
    if want.shape != got.shape:
        return f"shape {got.shape}, expected {want.shape}"
    if want.dtype.kind in "iu":
        bad = np.flatnonzero(want.reshape(-1) != got.reshape(-1))
        return None if bad.size == 0 else f"{bad.size} integers differ (first at {bad[0]})"
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    err = float(np.max(np.abs(want.astype(np.float64) - got))) if want.size else 0.0
    if not np.isfinite(got).all() and np.isfinite(want).all():
        return "non-finite values"
    return None if err <= rtol * max(scale, 1e-30) else f"max |error| {err:.3g} > {rtol} x max |value| {scale:.3g}"


def kept_buffers(name: str) -> list[str]:
    return [k[4:] for k in vectors(name).files if k.startswith("buf:")]


# fixtures whose kept buffers hold values the device computes exactly (random draws, copies of
# them, gathered stores): compared bit for bit, not to a tolerance
BIT_EXACT = {"draws", "serial"}


def same_bits(want: np.ndarray, got: np.ndarray) -> str | None:
    if want.shape != got.shape or want.dtype.itemsize != 4:
        return f"shape {got.shape}, expected {want.shape}"
    w, g = np.ascontiguousarray(want).view(np.uint32), np.ascontiguousarray(got).astype(want.dtype).view(np.uint32)
    bad = np.flatnonzero(w.reshape(-1) != g.reshape(-1))
    return None if bad.size == 0 else f"{bad.size} elements differ in their bits (first at {bad[0]})"


def check_program_run(name: str, emulate: bool, tmp_path, rtol: float, timeout: int = 600):
    """Run a fixture program (its scripted stdin, its output files into tmp_path) and hold it to the
    rules above: stdout, kept buffers, printed accuracies, and the bytes of every file it wrote."""
    from fixtures import stdin_of, stdout_of, written_files
    keep = kept_buffers(name)
    z = vectors(name)
    files = written_files(z)
    rc, out, err, arrays = run_program(name, emulate=emulate, keep=keep, timeout=timeout, stdin=stdin_of(name),
                                       out_dir=tmp_path if files else None)
    assert rc == 0, err
    problem = outputs_match(stdout_of(z), out, rtol=rtol)
    assert problem is None, problem
    assert accuracy_tokens(out) == accuracy_tokens(stdout_of(z)), "test accuracy differs"
    for k in keep:
        problem = (same_bits if name in BIT_EXACT else lambda w, g: tensors_match(w, g, rtol=1e-3))(z[f"buf:{k}"], arrays[k])
        assert problem is None, f"{k}: {problem}"
    for f in files:
        got = (tmp_path / f).read_bytes()
        assert got == bytes(z[f"file:{f}"]), f"{f}: {len(got)} bytes differ from the reference's"


def patched_program(name: str, directory: str, **replace) -> str:
    """A copy of a fixture's IR with strings in its run-time calls replaced (e.g. file paths)."""
    with open(ir_path(name)) as f:
        text = f.read()
    for old, new in replace.items():
        text = text.replace(old, new)
    path = os.path.join(directory, f"{name}.json")
    with open(path, "w") as f:
        f.write(text)
    return path


def function_call(name: str, emulate: bool = False):
    """(outputs of the generated library, golden outputs) for a function fixture."""
    from anvil.backend import hip
    from anvil.hip_function import Compiled, Lowered
    prog, data = load_ir(name)
    z = vectors(name)
    low = Lowered.from_fixture(prog, data)
    if emulate:
        src = hip.generate(prog, seed=data.get("seed", 0), library=True, emulate=True)
        lib = hip.HipLibrary(hip.compile_source(src, emulate=True), src)
        slots = [lib.slot(b.name) for b in low.inputs]
        args = [np.ascontiguousarray(z[f"input{k}"]) for k in range(len(low.inputs))]
        outs = [np.empty(b.shape, np.float32 if b.dtype == "f32" else np.int32) for b in low.outputs]
        for s, a in zip(slots, args):
            s.value = a.ctypes.data
        for b, o in zip(low.outputs, outs):
            lib.slot(b.name).value = o.ctypes.data
        lib.lib.anvil_entry()
        got = outs
    else:
        fn = Compiled(low.name, low, seed=data.get("seed", 0))
        got = fn.call([z[f"input{k}"] for k in range(len(low.inputs))])
        got = list(got) if isinstance(got, tuple) else [got]
    want = [z[f"output{k}"] for k in range(len(got))]
    return got, want

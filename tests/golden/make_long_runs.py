"""Writes tests/golden/vectors/<name>.npz for the full-length runs of C4 (200 Adam steps) and C5
(300 SGD steps): the parameters programs.py keeps, and everything the program prints.

The vectors come from the oracle (oracle/interp.py) in the reference's summation order. The oracle
reproduces the reference interpreter (reference anvil/interp.py) bit for bit on every fixture the
reference itself wrote, among them the first steps of these same programs at the same sizes
(c4_full2, c4_small, c5_full3, c5_step1; tests/test_oracle.py), so the long runs are taken from the
pinned restatement instead of running the reference again. tests/golden/make_noise_floor.py then
measures how far the same runs move when only the order of the float32 sums changes.

Usage: python tests/golden/make_long_runs.py [NAME ...]   (C4 about 2.6 hours, C5 about 2.9, one core each)
"""
from __future__ import annotations

import io
import os
import sys
import time
from concurrent.futures import ProcessPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
NAMES = ("c4_full200", "c5_full300")


def one(name):
    sys.path[:0] = [ROOT, os.path.join(ROOT, "anvil-lang_amd"), os.path.join(ROOT, "tests"), HERE]
    from fixtures import GOLDEN, load_ir
    from oracle import interp
    import programs
    spec = next(s for s in programs.PROGRAMS if s["name"] == name)
    prog, data = load_ir(name)
    t0 = time.time()
    out = io.StringIO()
    m = interp.Machine(prog, out=out, seed=data.get("seed", 0)).run()
    by_name = {b.name: b for b in prog.buffers}
    arrays = {}
    for bname in spec.get("keep", []):
        b = by_name[bname]
        arrays[f"buf:{bname}"] = m.arr(b)[:b.root.numel].reshape(b.shape).copy()
    arrays["stdout"] = np.frombuffer(out.getvalue().encode(), dtype=np.uint8)
    path = os.path.join(GOLDEN, "vectors", f"{name}.npz")
    np.savez_compressed(path + ".tmp.npz", **arrays)
    os.replace(path + ".tmp.npz", path)
    print(f"{name}: {time.time() - t0:.0f} s", flush=True)
    return name


def main():
    names = sys.argv[1:] or list(NAMES)
    with ProcessPoolExecutor(len(names)) as ex:
        for name in ex.map(one, names):
            print(f"wrote vectors/{name}.npz", flush=True)


if __name__ == "__main__":
    main()

"""Writes tests/golden/noise_floor.json: how far C2's trained parameters move from the reference's
when only the order of the float32 additions changes.

The oracle (oracle/interp.py, the reference interpreter restated) runs C2 at full size for 10 and
for 100 Adam steps twice more, with every float sum taken in another order ("reversed": last
element first; "sequential": one running sum in index order) and nothing else changed, and each run's
kept parameters are compared with the reference's own (tests/golden/vectors/<name>.npz). The
spread it records is what any correct float32 implementation that sums in its own order can be
expected to show; the GPU tests hold the HIP libraries to it.

Usage: python tests/golden/make_noise_floor.py   (about 25 minutes on 4 cores)
"""
from __future__ import annotations

import io
import json
import os
import sys
import time
from concurrent.futures import ProcessPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "noise_floor.json")
LR = 1e-3                     # C2's adam(lr = 1e-3)
RUNS = [("c2_full10", 10), ("c2_full100", 100)]
ORDERS = ("reversed", "sequential")


def spread(val, ref, steps):
    """Percentiles of |val - ref| over lr·steps and over the tensor's largest |ref|."""
    d = np.abs(val.astype(np.float64) - ref.astype(np.float64))
    by_lr = d / (LR * steps)
    by_max = d / np.abs(ref).max()
    q = lambda a, p: float(np.percentile(a, p))
    return {"lr_p50": q(by_lr, 50), "lr_p99": q(by_lr, 99), "lr_max": float(by_lr.max()),
            "max_p50": q(by_max, 50), "max_p99": q(by_max, 99), "max_max": float(by_max.max())}


def one(job):
    name, steps, order = job
    sys.path[:0] = [ROOT, os.path.join(ROOT, "anvil-lang_amd"), os.path.join(ROOT, "tests")]
    from fixtures import load_ir, vectors
    from oracle import interp
    prog, data = load_ir(name)
    t0 = time.time()
    m = interp.Machine(prog, out=io.StringIO(), seed=data.get("seed", 0), sum_order=order).run()
    z = vectors(name)
    by_name = {b.name: b for b in prog.buffers}
    res = {}
    for key in z.files:
        if key.startswith("buf:"):
            b = by_name[key[4:]]
            res[key[4:]] = spread(m.arr(b)[:b.root.numel].reshape(b.shape), z[key], steps)
    print(f"{name} {order}: {time.time() - t0:.0f} s", flush=True)
    return name, steps, order, res


def main():
    out = {"about": "per kept parameter: |oracle run with the float sums reordered - reference| over "
                    "lr·steps (lr_*) and over the tensor's largest |value| (max_*); written by "
                    "tests/golden/make_noise_floor.py"}
    jobs = [(n, s, o) for n, s in RUNS for o in ORDERS]
    with ProcessPoolExecutor(max_workers=len(jobs)) as pool:
        for name, steps, order, res in pool.map(one, jobs):
            out.setdefault(name, {"steps": steps, "lr": LR, "orders": {}})["orders"][order] = res
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()

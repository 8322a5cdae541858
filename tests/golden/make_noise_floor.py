"""Writes tests/golden/noise_floor.json: how far trained parameters and printed losses move from the
reference's when only the order of the float32 additions changes.

The oracle (oracle/interp.py, the reference interpreter restated) runs C2 at full size for 10 and
for 100 Adam steps, C4 for its 200 steps and C5 for its 300, twice more each, with every float sum
taken in another order ("reversed": last element first; "sequential": one running sum in index
order) and nothing else changed, and each run's kept parameters and printed losses are compared
with the reference's own (tests/golden/vectors/<name>.npz). The spread it records is what any
correct float32 implementation that sums in its own order can be expected to show; the GPU tests
hold the HIP libraries to it.

Usage: python tests/golden/make_noise_floor.py [--orders reversed[,sequential]] [NAME ...]
  (C2: about 25 minutes on 4 cores; C4 and C5 whole: about 3 hours reversed, longer sequential.
  Named runs are added to the existing file, each order as soon as it finishes. A run whose
  reference vectors make_fixtures.py is still writing waits for them.)
"""
from __future__ import annotations

import io
import json
import os
import re
import sys
import time
from concurrent.futures import ProcessPoolExecutor, as_completed

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "noise_floor.json")
# (fixture, steps, learning rate): C2 and C4 train with adam(lr = 1e-3), C5 with sgd(lr = 0.05)
RUNS = [("c2_full10", 10, 1e-3), ("c2_full100", 100, 1e-3), ("c4_full200", 200, 1e-3), ("c5_full300", 300, 0.05)]
ORDERS = ("reversed", "sequential")
LOSS = re.compile(r"loss\s+(\S+)")


def spread(val, ref, steps, lr):
    """Percentiles of |val - ref| over lr·steps and over the tensor's largest |ref|."""
    d = np.abs(val.astype(np.float64) - ref.astype(np.float64))
    by_lr = d / (lr * steps)
    by_max = d / np.abs(ref).max()
    q = lambda a, p: float(np.percentile(a, p))
    return {"lr_p50": q(by_lr, 50), "lr_p99": q(by_lr, 99), "lr_max": float(by_lr.max()),
            "max_p50": q(by_max, 50), "max_p99": q(by_max, 99), "max_max": float(by_max.max())}


def one(job):
    name, steps, lr, order = job
    sys.path[:0] = [ROOT, os.path.join(ROOT, "anvil-lang_amd"), os.path.join(ROOT, "tests")]
    from fixtures import GOLDEN, load_ir, stdout_of, vectors
    from oracle import interp
    prog, data = load_ir(name)
    t0 = time.time()
    out = io.StringIO()
    m = interp.Machine(prog, out=out, seed=data.get("seed", 0), sum_order=order).run()
    path = os.path.join(GOLDEN, "vectors", f"{name}.npz")
    while not os.path.exists(path):                      # make_fixtures.py still running the reference
        time.sleep(60)
    time.sleep(5)
    z = vectors(name)
    by_name = {b.name: b for b in prog.buffers}
    res = {}
    for key in z.files:
        if key.startswith("buf:"):
            b = by_name[key[4:]]
            res[key[4:]] = spread(m.arr(b)[:b.root.numel].reshape(b.shape), z[key], steps, lr)
    # every printed loss: |reordered - reference| / |reference|, in print order
    want = [float(v) for v in LOSS.findall(stdout_of(z))]
    got = [float(v) for v in LOSS.findall(out.getvalue())]
    if len(want) == len(got) and want:
        res["losses"] = [abs(g - w) / abs(w) for g, w in zip(got, want)]
    print(f"{name} {order}: {time.time() - t0:.0f} s", flush=True)
    return name, steps, lr, order, res


ABOUT = ("per kept parameter: |oracle run with the float sums reordered - reference| over "
         "lr·steps (lr_*) and over the tensor's largest |value| (max_*); losses: each printed "
         "loss's |reordered - reference| / |reference|; written by tests/golden/make_noise_floor.py")


def record(name, steps, lr, order, res, fresh):
    """Merge one finished run into the file (re-read, so runs finishing elsewhere are kept)."""
    out = {}
    if os.path.exists(OUT):
        with open(OUT) as f:
            out = json.load(f)
    out["about"] = ABOUT
    if name in fresh:                                    # this invocation's first result for name
        out.pop(name, None)
        fresh.discard(name)
    out.setdefault(name, {"steps": steps, "lr": lr, "orders": {}})["orders"][order] = res
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", name, order, "to", OUT, flush=True)


def main():
    args = sys.argv[1:]
    orders = ORDERS
    if args[:1] == ["--orders"]:
        orders, args = tuple(args[1].split(",")), args[2:]
    only = set(args)
    jobs = [(n, s, lr, o) for n, s, lr in RUNS for o in orders if not only or n in only]
    # a name's old entry goes when its first run here finishes, unless only some orders are rerun
    fresh = {j[0] for j in jobs} if orders == ORDERS else set()
    with ProcessPoolExecutor(max_workers=len(jobs)) as pool:
        for fut in as_completed([pool.submit(one, j) for j in jobs]):
            record(*fut.result(), fresh)


if __name__ == "__main__":
    main()

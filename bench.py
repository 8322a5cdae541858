#!/usr/bin/env python3
"""Benchmark: config C2 of BASELINE.json through the HIP backend on one MI355X.

The workload is the kernel IR of the 784-1024-1024-10 MLP training program (ReLU, cross-entropy,
adam(lr=1e-3), batch 256, shuffled batches, 500 steps; X f32[65536, 784] ~ U[0,1), labels ~
U{0..9}, Linear-default init after seed(1)) as the reference front end produces it
(tests/golden/ir/c2_wide_mlp.json). The program generates its own synthetic data on the device.

A step is one training iteration: the batch gather, forward, backward and Adam update. The library
records a device event at the start of iterations W and W + K of the batch loop (it counts the
others and records nothing for them); the timed region is the K iterations between, all on the
library's stream, with the device synchronized before and after. `value` is samples/s over those K
steps.

The roofline object is for the generated kernel that takes the most device time in a second,
profiled run of the same program (HIP events around every launch on the library's stream):
achieved = its algorithmic FLOPs (or bytes) per launch / its mean launch time. step_roofline puts
the whole step beside its serial roofline: every launch of a step at its own bound, summed.

cpu_baseline: this repository's NumPy interpreter of the same IR (oracle/interp.py, which follows
the reference interpreter anvil/interp.py) timed on this host for a few full-size steps.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "anvil-lang_amd"))

WORKLOAD = os.path.join(ROOT, "tests", "golden", "ir", "c2_wide_mlp.json")
BATCH = 256
STEPS_IN_PROGRAM = 500
LOOP_COUNTER = "x_batch"
PEAK_FP32_MFMA = 157.3e12
PEAK_HBM = 8.0e12
METRIC = "train samples/s (784-1024-1024-10 MLP, batch 256) + % of fp32-MFMA/HBM roofline"


def load_program():
    from anvil import irjson
    with open(WORKLOAD) as f:
        data = json.load(f)
    return irjson.load(data), data


class quiet_stdout:
    """The program prints (its loss); bench.py's stdout carries only the JSON line."""

    def __enter__(self):
        sys.stdout.flush()
        self.saved = os.dup(1)
        self.null = os.open(os.devnull, os.O_WRONLY)
        os.dup2(self.null, 1)

    def __exit__(self, *exc):
        libc = ctypes.CDLL(None)
        libc.fflush(None)
        os.dup2(self.saved, 1)
        os.close(self.null)
        os.close(self.saved)


def gpu_run(prog, data, steps: int, warmup: int, graphs: bool = False):
    from anvil.backend import hip
    lib = hip.load(prog, seed=int(data.get("seed", 0)), graphs=graphs)
    # timed run
    lib.lib.anvil_marks_select(LOOP_COUNTER.encode())
    lib.lib.anvil_marks_window(warmup, warmup + steps)     # events at the timed region's two ends only
    lib.lib.anvil_sync_device()
    t0 = time.perf_counter()
    with quiet_stdout():
        rc = lib.main()
        lib.lib.anvil_sync_device()
    wall = time.perf_counter() - t0
    if rc != 0:
        raise SystemExit(f"bench: the program exited with status {rc}")
    n = lib.lib.anvil_marks_count()
    if warmup + steps >= n:
        raise SystemExit(f"bench: the program marks {n} iteration starts; warmup + steps must be below that")
    ms = lib.lib.anvil_marks_elapsed_ms(warmup, warmup + steps)
    # profiled run: per-kernel device time
    lib.lib.anvil_marks_select(b"")
    lib.lib.anvil_profile_enable(1)
    lib.lib.anvil_profile_reset()
    with quiet_stdout():
        lib.main()
        lib.lib.anvil_sync_device()
    prof = lib.profile()
    lib.lib.anvil_profile_enable(0)
    return ms, wall, prof, lib


TRAFFIC = os.path.join(ROOT, "profiles", "c2_mlp_train_step_traffic.txt")


def measured_traffic(library: str, kernel: str):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, calibrated with a copy kernel),
    from the committed counter profile, if it was taken on this very library build; else None."""
    try:
        with open(TRAFFIC) as f:
            lines = f.read().splitlines()
    except OSError:
        return None
    if f"library {library}" not in lines:
        return None
    for line in lines:
        parts = line.split()
        if len(parts) == 3 and parts[0] == kernel:
            return int(parts[1]) + int(parts[2])
    return None


def roofline(prof, library: str):
    """The kernel with the most device time among those launched once per step."""
    rows = [r for r in prof if r[2] >= STEPS_IN_PROGRAM]
    label, ms, calls, flops, nbytes = max(rows, key=lambda r: r[1])
    t = ms / calls * 1e-3
    traffic = measured_traffic(library, label.split()[0])
    if flops / max(nbytes, 1) > PEAK_FP32_MFMA / PEAK_HBM:
        achieved = flops / t / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA / 1e12,
                "unit": "TFLOP/s", "frac": round(achieved / (PEAK_FP32_MFMA / 1e12), 4), "traffic": traffic,
                "kernel": label, "mean_us": round(t * 1e6, 3), "flops_per_launch": flops,
                "algorithmic_bytes_per_launch": nbytes}
    achieved = nbytes / t / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(achieved / (PEAK_HBM / 1e9), 4), "traffic": traffic, "kernel": label,
            "mean_us": round(t * 1e6, 3), "bytes_per_launch": nbytes}


def step_roofline(prof, ms_per_step: float):
    """The whole step against its serial roofline: each launch of a step at its own bound (its
    FLOPs at the fp32 MFMA peak or its bytes at the HBM peak, whichever takes longer), summed, over
    the measured step time."""
    t = 0.0
    for label, ms, calls, flops, nbytes in prof:
        if calls >= STEPS_IN_PROGRAM:
            t += calls / STEPS_IN_PROGRAM * max(flops / PEAK_FP32_MFMA, nbytes / PEAK_HBM)
    return {"t_roofline_us": round(t * 1e6, 2), "t_step_us": round(ms_per_step * 1e3, 2),
            "frac": round(t * 1e3 / ms_per_step, 4)}


COPY_ELEMS = 1 << 24          # the calibration copy: 64 MiB read, 64 MiB written per launch
COPY_LAUNCHES = 50


def copy_program():
    """An IR program whose loop is one plain copy kernel B[i] = A[i] of COPY_ELEMS floats: the
    known-size kernel that calibrates the FETCH_SIZE / WRITE_SIZE counters into bytes."""
    from anvil import ir

    def numbered(obj, ident):          # fixed ids: the same source, so the same built library,
        obj.id = ident                 # in every process
        return obj
    a = numbered(ir.Buffer("A", (COPY_ELEMS,), "f32", "param"), 1)
    b = numbered(ir.Buffer("B", (COPY_ELEMS,), "f32", "param"), 2)
    i, j = numbered(ir.Var("i", COPY_ELEMS), 3), numbered(ir.Var("j", COPY_ELEMS), 4)
    fill = ir.Kernel([i], [ir.Store(a, ir.Affine(0, {i: 1}), ir.Rand(0))], name="fill", label="uniform", id=5)
    copy = ir.Kernel([j], [ir.Store(b, ir.Affine(0, {j: 1}), ir.Load(a, ir.Affine(0, {j: 1})))], name="copy",
                     label="copy", id=6)
    it = numbered(ir.Buffer("it", (), "i32", "var"), 7)
    main = ir.Block([ir.KernelStmt(fill), ir.For(it, 0, COPY_LAUNCHES, 1, ir.Block([ir.KernelStmt(copy)]))])
    return ir.Program(main, [a, b, it])


def copy_run() -> dict:
    from anvil.backend import hip
    lib = hip.load(copy_program())
    lib.lib.anvil_marks_select(b"it")
    lib.lib.anvil_marks_window(5, COPY_LAUNCHES - 1)
    with quiet_stdout():
        lib.main()
        lib.lib.anvil_sync_device()
    n = lib.lib.anvil_marks_count()
    ms = lib.lib.anvil_marks_elapsed_ms(5, n - 1) / (n - 6)
    nbytes = 8 * COPY_ELEMS
    return {"metric": "copy GB/s (calibration kernel)", "value": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
            "bytes_per_launch": nbytes, "mean_us": round(ms * 1e3, 2), "launches": COPY_LAUNCHES,
            "library": os.path.basename(lib.path)}


C3 = ["c3_softmax", "c3_layernorm", "c3_linear", "c3_attention"]


def c3_run(calls: int) -> dict:
    """Config C3: each anvil.function at its BASELINE size, inputs ~N(0,1) (seed 2) already on the
    device; every generated kernel timed with dispatch events over `calls` calls."""
    import numpy as np
    from anvil import irjson
    from anvil.hip_function import Compiled, DeviceArray, Lowered
    out = {}
    for name in C3:
        with open(os.path.join(ROOT, "tests", "golden", "ir", f"{name}.json")) as f:
            data = json.load(f)
        prog = irjson.load(data)
        low = Lowered.from_fixture(prog, data)
        fn = Compiled(name, low, seed=int(data.get("seed", 0)))
        rng = np.random.default_rng(2)
        args = [DeviceArray.from_host(rng.standard_normal(b.shape).astype(np.float32)) for b in low.inputs]
        res = [DeviceArray(b.shape) for b in low.outputs]
        fn.call_device(args, res)                                                          # warm-up
        fn.lib.lib.anvil_profile_enable(1)
        fn.lib.lib.anvil_profile_reset()
        for _ in range(calls):
            fn.call_device(args, res)
        kernels = []
        for label, ms, n, flops, nbytes in fn.lib.profile():
            if n == 0:
                continue
            t = ms / n * 1e-3
            mfma = flops / max(nbytes, 1) > PEAK_FP32_MFMA / PEAK_HBM
            ach = flops / t / 1e12 if mfma else nbytes / t / 1e9
            peak = PEAK_FP32_MFMA / 1e12 if mfma else PEAK_HBM / 1e9
            kernels.append({"kernel": label, "mean_us": round(t * 1e6, 2), "bound": "mfma" if mfma else "hbm",
                            "achieved": round(ach, 2), "unit": "TFLOP/s" if mfma else "GB/s",
                            "frac": round(ach / peak, 4), "flops": flops, "bytes": nbytes})
        fn.lib.lib.anvil_profile_enable(0)
        out[name] = {"us_per_call_kernels": round(sum(k["mean_us"] for k in kernels), 2), "kernels": kernels,
                     "library": os.path.basename(fn.lib.path)}
    return {"metric": "C3 anvil.function kernels vs roofline (device-resident inputs)", "calls": calls,
            "functions": out}


C3_CALLS = 20


def c3_summary(run: dict) -> dict:
    """Per C3 function: its library, kernel time per call and every kernel's mean time and roofline
    fraction (the bench line's compact form of c3_run)."""
    out = {"calls": run["calls"], "timing": "HIP events around each launch on the library's stream, "
                                            "inputs resident in device memory"}
    for name, f in run["functions"].items():
        out[name] = {"library": f["library"], "us_per_call_kernels": f["us_per_call_kernels"],
                     "kernels": [{k: r[k] for k in ("kernel", "mean_us", "bound", "achieved", "unit", "frac")}
                                 for r in f["kernels"]]}
    return out


def host_description() -> str:
    """The host CPU (model, count) and its thread environment, for the baseline's record."""
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    env = ", ".join(f"{k}={os.environ.get(k, 'unset')}" for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS"))
    return f"{model}, {os.cpu_count()} logical CPUs; environment {env}"


ONE_THREAD = {"OMP_NUM_THREADS": "1", "OPENBLAS_NUM_THREADS": "1", "MKL_NUM_THREADS": "1"}


def oracle_leg(path: str, counter: str, stop_after: int | None) -> dict:
    """Run in a child process started with ONE_THREAD in its environment: the NumPy interpreter
    (oracle/interp.py) on the IR program at `path`, every BLAS/OpenMP pool also limited to one
    thread at run time; the perf_counter time at each start of the `counter` loop's iterations and
    at the end of the run (or when stop_after iterations have started), and the host's description."""
    import io
    sys.path.insert(0, ROOT)
    from threadpoolctl import threadpool_limits
    from anvil import irjson
    from oracle import interp
    with open(path) as f:
        data = json.load(f)
    prog = irjson.load(data)
    marks = []

    def hook(name, value):
        if name == counter:
            marks.append(time.perf_counter())
            if stop_after is not None and len(marks) > stop_after:
                raise interp.StopRun()
    m = interp.Machine(prog, out=io.StringIO(), seed=int(data.get("seed", 0)), loop_hook=hook)
    with threadpool_limits(limits=1):
        try:
            m.run()
        except interp.StopRun:
            pass
    end = time.perf_counter()
    return {"marks": [t - marks[0] for t in marks], "end": end - marks[0], "host": host_description()}


def oracle_run(path: str, counter: str, stop_after: int | None) -> dict:
    """oracle_leg in a child process whose environment pins BLAS and OpenMP to one thread (the child
    touches no GPU)."""
    cmd = [sys.executable, os.path.abspath(__file__), "--oracle-leg", path, counter, str(stop_after or 0)]
    r = subprocess.run(cmd, capture_output=True, text=True, env=dict(os.environ, **ONE_THREAD))
    if r.returncode != 0:
        raise SystemExit(f"bench: the CPU baseline failed:\n{r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def cpu_baseline(steps: int):
    """The NumPy interpreter on the same IR: set-up untimed, one warm-up step, then `steps` steps."""
    run = oracle_run(WORKLOAD, LOOP_COUNTER, steps + 1)
    marks = run["marks"]
    t = marks[-1] - marks[1]
    return {"value": round(steps * BATCH / t, 2), "unit": "samples/s", "cores": 1, "kind": "port",
            "sample": f"{steps} full-size C2 training steps (batch 256) after 1 warm-up step, NumPy "
                      f"interpreter (oracle/interp.py) in a child process with OMP_NUM_THREADS = "
                      f"OPENBLAS_NUM_THREADS = MKL_NUM_THREADS = 1 (and every thread pool limited to 1 "
                      f"at run time, threadpoolctl); host: {run['host']}; {t:.1f} s"}


# configs C4 (character transformer at T = 256, 200 Adam steps) and C5 (the CNN, 300 SGD steps):
# their own step loops at full size, reported beside the metric
STEP_CONFIGS = {
    "c4": ("c4_transformer_t256.json", 200, "C4: decoder-only char transformer, B 16, T 256, D 256, 4 heads, "
           "4 layers, MLP 4D, causal attention, layernorm, vocab 96, adam, 200-step program"),
    "c5": ("c5_cnn.json", 300, "C5: CNN conv3x3 1->32 + ReLU, conv3x3 32->64 + ReLU, 2x2 maxpool, 9216->128->10, "
           "cross_entropy, sgd(0.05), batch 128, 300-step program"),
}


def config_steps(name: str, warmup: int = 10) -> dict:
    """One of STEP_CONFIGS: ms per step over its step loop after `warmup` steps (device events at
    the loop marks of the timed region's two ends), then a profiled run for the serial roofline of
    the step (each launch at its own bound, summed) and the launch with the most device time."""
    from anvil import irjson
    from anvil.backend import hip
    fname, steps, workload = STEP_CONFIGS[name]
    with open(os.path.join(ROOT, "tests", "golden", "ir", fname)) as f:
        data = json.load(f)
    lib = hip.load(irjson.load(data), seed=int(data.get("seed", 0)))
    lib.lib.anvil_marks_select(b"step")
    lib.lib.anvil_marks_window(warmup, steps - 1)
    with quiet_stdout():
        rc = lib.main()
        lib.lib.anvil_sync_device()
    if rc != 0:
        raise SystemExit(f"bench: {name} exited with status {rc}")
    ms = lib.lib.anvil_marks_elapsed_ms(warmup, steps - 1)
    if ms < 0:
        raise SystemExit(f"bench: {name} marked {lib.lib.anvil_marks_count()} steps, fewer than {steps}")
    ms /= steps - 1 - warmup
    lib.lib.anvil_marks_select(b"")
    lib.lib.anvil_profile_enable(1)
    lib.lib.anvil_profile_reset()
    with quiet_stdout():
        lib.main()
        lib.lib.anvil_sync_device()
    prof = lib.profile()
    lib.lib.anvil_profile_enable(0)
    t_roof, top = 0.0, None
    for label, tms, calls, flops, nbytes in prof:
        if calls >= steps:
            t_roof += calls / steps * max(flops / PEAK_FP32_MFMA, nbytes / PEAK_HBM)
            if top is None or tms > top[1]:
                top = (label, tms, calls, flops, nbytes)
    label, tms, calls, flops, nbytes = top
    t = tms / calls * 1e-3
    mfma = flops / max(nbytes, 1) > PEAK_FP32_MFMA / PEAK_HBM
    achieved = flops / t / 1e12 if mfma else nbytes / t / 1e9
    peak = PEAK_FP32_MFMA / 1e12 if mfma else PEAK_HBM / 1e9
    return {"workload": workload, "ms_per_step": round(ms, 5), "steps_timed": steps - 1 - warmup,
            "timing": "HIP events at the step loop's marks, no profiling", "library": os.path.basename(lib.path),
            "step_roofline": {"t_roofline_us": round(t_roof * 1e6, 2), "frac": round(t_roof * 1e3 / ms, 4)},
            "dominant_launch": {"kernel": label, "mean_us": round(t * 1e6, 3), "bound": "mfma" if mfma else "hbm",
                                "achieved": round(achieved, 1 if not mfma else 3),
                                "unit": "TFLOP/s" if mfma else "GB/s", "frac": round(achieved / peak, 4)}}


C1_WORKLOAD = os.path.join(ROOT, "tests", "golden", "ir", "c1_mlp.json")
C1_BATCH = 64


def c1_epoch(cpu: bool) -> dict:
    """Config C1 (784-128-10 MLP, SGD 0.1, batch 64 shuffled, one epoch of 60,000 samples, then the
    10,000-sample evaluation): samples/s over the epoch's steps on the GPU (device events at each
    step) and, with cpu, through the NumPy interpreter on this host, one thread (the whole epoch
    and the evaluation after it, perf_counter)."""
    from anvil import irjson
    from anvil.backend import hip
    with open(C1_WORKLOAD) as f:
        data = json.load(f)
    prog = irjson.load(data)
    lib = hip.load(prog, seed=int(data.get("seed", 0)))
    lib.lib.anvil_marks_select(LOOP_COUNTER.encode())
    t0 = time.perf_counter()
    with quiet_stdout():
        rc = lib.main()
        lib.lib.anvil_sync_device()
    wall = time.perf_counter() - t0
    if rc != 0:
        raise SystemExit(f"bench: C1 exited with status {rc}")
    n = lib.lib.anvil_marks_count()
    ms = lib.lib.anvil_marks_elapsed_ms(0, n - 1)
    gpu = round((n - 1) * C1_BATCH / (ms / 1e3), 1)
    out = {"steps": n, "gpu_samples_per_s": gpu, "gpu_epoch_ms_steps": round(ms * n / (n - 1), 3),
           "gpu_program_wall_s": round(wall, 3), "library": os.path.basename(lib.path)}
    if cpu:
        run = oracle_run(C1_WORKLOAD, LOOP_COUNTER, None)
        marks = run["marks"]
        steps = len(marks)
        t_steps = marks[-1] - marks[0]
        out.update({"cpu_samples_per_s": round((steps - 1) * C1_BATCH / t_steps, 1),
                    "cpu_epoch_s": round(run["end"], 2),
                    "cpu": f"oracle/interp.py in a child process with OMP_NUM_THREADS = OPENBLAS_NUM_THREADS = "
                           f"MKL_NUM_THREADS = 1 (and threadpoolctl); {run['host']}",
                    "speedup": round(gpu / ((steps - 1) * C1_BATCH / t_steps), 1)})
    return out


YARDSTICK_SHAPES = {
    # C2: fwd1, fwd2, dX2 and the weight gradients dW1, dW2 (M x N x K; TN: A stored K x M)
    "c2": [(256, 1024, 784, "NN"), (256, 1024, 1024, "NN"), (256, 1024, 1024, "NT"),
           (784, 1024, 256, "TN"), (1024, 1024, 256, "TN")],
    # C4 at T = 256 (4096 tokens, width 256, feed-forward 1024): the forward products (qkv, attention
    # output, feed-forward in and out), their input gradients and their weight gradients
    "c4": [(4096, 768, 256, "NN"), (4096, 256, 256, "NN"), (4096, 1024, 256, "NN"), (4096, 256, 1024, "NN"),
           (4096, 256, 768, "NT"), (4096, 256, 1024, "NT"), (4096, 1024, 256, "NT"),
           (256, 768, 4096, "TN"), (256, 256, 4096, "TN"), (256, 1024, 4096, "TN"), (1024, 256, 4096, "TN")],
}


def yardstick(config: str = "c2", calls: int = 200) -> dict:
    """The vendor library's fp32 products (torch.mm: hipBLASLt / rocBLAS, TF32 off) on a config's
    product shapes, as a yardstick for the generated kernels. Event timing here includes the host's
    launch rate; the kernels' own durations come from `rocprofv3 --kernel-trace --stats` of this
    mode."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    out = []
    for M, N, K, lay in YARDSTICK_SHAPES[config]:
        a = torch.randn(*((K, M) if lay == "TN" else (M, K)), device="cuda")
        b = torch.randn(*((N, K) if lay == "NT" else (K, N)), device="cuda")
        c = torch.empty(M, N, device="cuda")
        x = a.t() if lay == "TN" else a
        y = b.t() if lay == "NT" else b
        for _ in range(10):
            torch.mm(x, y, out=c)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(calls):
            torch.mm(x, y, out=c)
        e.record()
        torch.cuda.synchronize()
        out.append({"shape": f"{lay} {M}x{N}x{K}", "us_per_call_events": round(s.elapsed_time(e) / calls * 1e3, 2)})
    return {"metric": f"torch.mm fp32 on {config.upper()}'s product shapes (yardstick)", "calls": calls,
            "products": out}


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=480)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-steps", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-c1", action="store_true", help="skip config C1's one-epoch run (GPU and CPU)")
    p.add_argument("--profile-table", action="store_true", help="print every kernel's time to stderr")
    p.add_argument("--graphs", action="store_true", help="replay loop bodies as HIP graphs")
    p.add_argument("--copy", action="store_true", help="run the copy kernel that calibrates HBM counters")
    p.add_argument("--c3", action="store_true", help="config C3 alone: the standalone functions, per kernel")
    p.add_argument("--no-c3", action="store_true", help="skip config C3's functions in the default line")
    p.add_argument("--no-c45", action="store_true", help="skip configs C4 and C5's step loops in the default line")
    p.add_argument("--yardstick", nargs="?", const="c2", choices=sorted(YARDSTICK_SHAPES),
                   help="torch.mm (the vendor library) on a config's product shapes (default c2)")
    p.add_argument("--oracle-leg", nargs=3, metavar=("IR", "COUNTER", "STOP"), help=argparse.SUPPRESS)
    args = p.parse_args()
    if args.oracle_leg:
        path, counter, stop = args.oracle_leg
        print(json.dumps(oracle_leg(path, counter, int(stop) or None)), flush=True)
        return 0
    if args.yardstick:
        print(json.dumps(yardstick(args.yardstick)), flush=True)
        return 0
    if args.copy:
        print(json.dumps(copy_run()), flush=True)
        return 0
    if args.c3:
        print(json.dumps(c3_run(20)), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench: this build measures one GPU only (asked for {args.gpus}); data-parallel sharding "
              "over several GPUs is designed but not run", file=sys.stderr)
        return 2
    prog, data = load_program()
    ms, wall, prof, lib = gpu_run(prog, data, args.steps, args.warmup, graphs=args.graphs)
    if args.profile_table:
        for label, tms, calls, flops, nbytes in sorted(prof, key=lambda r: -r[1]):
            if calls:
                t = tms / calls * 1e-3
                print(f"{tms:9.3f} ms {calls:6d} x {t * 1e6:9.2f} us {flops / t / 1e12:8.3f} TFLOP/s "
                      f"{nbytes / t / 1e9:8.1f} GB/s  {label}", file=sys.stderr)
    value = args.steps * BATCH / (ms / 1e3)
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (generated on the device by the program: X ~ U[0,1), labels ~ U{0..9})",
        "config": {"workload": "C2: MLP 784-1024-1024-10, ReLU, cross_entropy, adam(lr=1e-3), batch 256, "
                               "shuffled, 500-step program", "global_batch": BATCH, "n_train": 65536,
                   "parallelism": "single GPU", "library": os.path.basename(lib.path),
                   "graph_replay": args.graphs,
                   "program_wall_s": round(wall, 3)},
        "roofline": roofline(prof, os.path.basename(lib.path)),
        "step_roofline": step_roofline(prof, ms / args.steps),
    }
    # the box's measured stream-copy rate, labelled apart from the 8 TB/s published peak
    cp = copy_run()
    line["copy_ceiling"] = {"value": cp["value"], "unit": "GB/s", "frac_of_peak": round(cp["value"] / (PEAK_HBM / 1e9), 4),
                            "kernel": f"plain copy, {cp['bytes_per_launch'] // 2 >> 20} MiB read + "
                                      f"{cp['bytes_per_launch'] // 2 >> 20} MiB written per launch, "
                                      f"mean of {cp['launches'] - 6} launches"}
    if line["roofline"].get("unit") == "GB/s":
        line["roofline"]["frac_of_copy"] = round(line["roofline"]["achieved"] / cp["value"], 4)
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_steps)
        line["cpu_baseline"] = cpu
        line["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    if not args.no_c1:
        line["c1_epoch"] = c1_epoch(cpu=not args.no_cpu)
    if not args.no_c3:
        line["c3"] = c3_summary(c3_run(C3_CALLS))
    if not args.no_c45:
        for name in STEP_CONFIGS:
            line[name] = config_steps(name)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""The `anvil` command line for the HIP backend, on kernel-IR programs (JSON, `irjson`).

    python -m anvil hip   PROG.json [-o PROG.hip] [--seed N]     write the generated .hip file
    python -m anvil build PROG.json [-o PROG.so]  [--seed N]     compile it for gfx950
    python -m anvil run   PROG.json [--seed N] [--profile | --profile-rates] [--check[=inf]] [--dump OUT.npz --keep a,...]
    python -m anvil export FN.json [-o DIR] [--name LIB]        a function as lib<LIB>.so + <LIB>.h

These mirror the reference's `anvil cuda file.anvil` and `anvil run|build --cuda` (cli.py:259-270,
305-320): the same generated-file / build / run split, libraries cached by the hash of their source
(cli.py:127-136; $ANVIL_CACHE picks the directory). The reference's front end turns .anvil source
into the IR; this package starts from the IR (see `irjson`), which the reference front end can
write, and which the reference's own cli.py can hand to `hip.generate` directly.

`run` executes the program's `anvil_main` in this process: its stdout is the program's, a run-time
error prints `anvil: runtime error: ...` and exits with status 1, as a compiled Anvil program does.
`--emulate` builds the same file as plain C++ for the CPU instead (the reference's --cuda-emulate,
cuda.py:650-654): a test build of the generator's output, never chosen automatically.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np


def _load_program(path):
    from . import irjson
    with open(path) as f:
        data = json.load(f)
    return irjson.load(data), data


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="anvil", description="Anvil's MI355X (HIP) backend on kernel-IR programs")
    sub = p.add_subparsers(dest="cmd", required=True)
    for name in ("hip", "build", "run"):
        q = sub.add_parser(name)
        q.add_argument("program", help="a kernel-IR program (.json, anvil-ir/1)")
        q.add_argument("--seed", type=int, default=None, help="the random seed (default: the program's own)")
        q.add_argument("--emulate", action="store_true", help="a CPU build of the generated file (testing)")
        q.add_argument("--graphs", action="store_true", default=None,
                       help="replay loop bodies as HIP graphs (default: $ANVIL_HIP_GRAPHS)")
        q.add_argument("--check", nargs="?", const="nan", choices=["nan", "inf"], default=None,
                       help="stop at the first nan a computation makes, and say which line made it and how "
                            "(--check=inf: at the first infinity too)")
        if name in ("hip", "build"):
            q.add_argument("-o", "--output", default=None)
        if name == "run":
            q.add_argument("--profile", action="store_true",
                           help="time every launch and print the reference's breakdown at exit (stdout)")
            q.add_argument("--profile-rates", action="store_true",
                           help="time every launch; per launch ms, share, calls, GFLOP/s and GB/s on stderr")
            q.add_argument("--dump", default=None, help="write the final contents of --keep buffers here (.npz)")
            q.add_argument("--keep", default="", help="comma-separated buffer names (or #id) to dump")
            q.add_argument("--marks", default=None, help="record an event per iteration of loops with this counter")
    q = sub.add_parser("export", help="a lowered function as a C library and header (lib<name>.so, <name>.h)")
    q.add_argument("program", help="a lowered function (.json, anvil-ir/1 with a \"function\" entry)")
    q.add_argument("-o", "--output", default=None, help="the directory to write to")
    q.add_argument("--name", default=None, help="the library's name (default: the file's)")
    q.add_argument("--seed", type=int, default=None)
    args = p.parse_args(argv)
    if args.cmd == "export":
        from .export_hip import export
        for path in export(args.program, args.output, name=args.name, seed=args.seed):
            print(path)
        return 0
    from .backend import hip
    prog, data = _load_program(args.program)
    seed = args.seed if args.seed is not None else int(data.get("seed", 0))
    src = hip.generate(prog, seed=seed, emulate=args.emulate, graphs=args.graphs, check=args.check)
    if args.cmd == "hip":
        out = args.output or os.path.splitext(args.program)[0] + ".hip"
        with open(out, "w") as f:
            f.write(src)
        return 0
    if args.cmd == "build":
        out = args.output or os.path.splitext(args.program)[0] + ".so"
        hip.build(src, out, emulate=args.emulate)
        return 0
    lib = hip.HipLibrary(hip.compile_source(src, emulate=args.emulate), src)
    profiling = args.cmd == "run" and (args.profile or args.profile_rates)
    if profiling:
        lib.lib.anvil_profile_enable(1)
    if args.marks:
        lib.lib.anvil_marks_select(args.marks.encode())
    sys.stdout.flush()
    rc = lib.main()
    lib.lib.anvil_sync_device()
    if args.cmd == "run" and args.profile:
        lib.lib.anvil_profile_print()           # the reference prints its table when the program ends
    if args.cmd == "run" and args.profile_rates:
        rows = sorted(lib.profile(), key=lambda r: -r[1])
        total = sum(r[1] for r in rows) or 1.0
        sys.stderr.write(f"{'ms':>10} {'%':>6} {'calls':>8} {'GFLOP/s':>9} {'GB/s':>8}  kernel\n")
        for label, ms, calls, flops, nbytes in rows:
            if calls:
                s = ms / calls * 1e-3
                sys.stderr.write(f"{ms:10.3f} {100 * ms / total:6.1f} {calls:8d} {flops / s / 1e9:9.1f} "
                                 f"{nbytes / s / 1e9:8.1f}  {label}\n")
    if args.dump:
        keep = [k for k in args.keep.split(",") if k]
        # a name held by several buffers (a variable reassigned in place) means the last of them,
        # as the fixture writer reads it
        by_name = {b.name: b.root for b in prog.buffers}
        arrays = {}
        for k in keep:
            b = by_name[k] if not k.startswith("#") else next(x.root for x in prog.buffers if x.id == int(k[1:]))
            try:
                arrays[f"buf:{k}"] = read_buffer(lib, b)
            except KeyError:
                if k in by_name:
                    raise
        if args.marks:
            n = lib.lib.anvil_marks_count()
            arrays["marks_ms"] = np.array([lib.lib.anvil_marks_elapsed_ms(0, i) for i in range(n)])
        np.savez(args.dump, **arrays)
    return rc


def read_buffer(lib, b) -> np.ndarray:
    import ctypes
    out = np.zeros(max(1, b.numel), dtype=np.int32 if b.dtype == "i32" else np.float32)
    n = lib.lib.anvil_buffer_read(ctypes.c_int(b.id), out.ctypes.data_as(ctypes.c_void_p), ctypes.c_longlong(out.nbytes))
    if n < 0:
        raise KeyError(f"buffer {b.name} (#{b.id}) is not held by the library")
    return out[:b.numel].reshape(b.shape)


if __name__ == "__main__":
    sys.exit(main())

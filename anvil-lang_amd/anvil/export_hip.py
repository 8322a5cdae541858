"""`anvil export --hip`: an Anvil function as a C library (`lib<name>.so`, built for MI355X) and a
header, for use outside Python — the HIP twin of the reference's `anvil export` (export.py:68-161).

    python -m anvil export FUNCTION.json -o build/ [--name digits]   ->  build/digits.h, build/libdigits.so

FUNCTION.json is a lowered function (the kernel IR `pyapi.lower` produces, with its "function"
entry). Everything the function reads besides its arguments was computed when it was lowered and is
part of the library. From C:

    #include "digits.h"
    float image[DIGITS_READ_IMAGE_SIZE], probs[DIGITS_READ_OUT_SIZE];
    digits_read(image, probs);

Link with `cc app.c -Lbuild -ldigits -Wl,-rpath,build`. Arrays are row-major host memory, read and
written in place (each call copies the arguments to the GPU and the results back). Calls from
several threads take turns (a mutex around the library's one device arena), as in the reference.
The header keeps the reference's form: `<LIB>_<FN>_<ARG>_SIZE` macros and one prototype.
"""
from __future__ import annotations

import json
import os
import re

from . import irjson
from .backend import hip
from .hip_function import Lowered


def c_type(dtype) -> str:
    return "int32_t" if dtype == "i32" else "float"


def c_ident(s: str) -> str:
    s = re.sub(r"[^A-Za-z0-9_]", "_", s)
    return s if s and not s[0].isdigit() else "_" + s


def fmt_shape(shape) -> str:
    return "[" + ", ".join(str(d) for d in shape) + "]"


def export(path: str, out_dir: str | None = None, name: str | None = None, seed: int | None = None) -> list[str]:
    """Write <name>.h and lib<name>.so; returns their paths."""
    with open(path) as f:
        data = json.load(f)
    if "function" not in data:
        raise ValueError(f"{path}: not a lowered function (no \"function\" entry)")
    prog = irjson.load(data)
    low = Lowered.from_fixture(prog, data)
    fn = data["function"]
    fn_name = fn.get("name", "fn")
    arg_names = fn.get("arg_names") or [f"x{k}" for k in range(len(low.inputs))]
    outs = [b for b in low.outputs if b is not None]
    out_names = fn.get("out_names") or ([f"out{k}" for k in range(len(outs))] if len(outs) > 1 else ["out"])
    lib = c_ident(name or os.path.splitext(os.path.basename(path))[0])
    func = f"{lib}_{c_ident(fn_name)}"
    out_dir = os.path.abspath(out_dir or os.path.dirname(os.path.abspath(path)))
    os.makedirs(out_dir, exist_ok=True)
    seed = int(data.get("seed", 0)) if seed is None else seed

    args, sizes, sets, clears, doc_in, doc_out = [], [], [], [], [], []
    for b, an in zip(low.inputs, arg_names):
        arg = c_ident(an)
        args.append(f"const {c_type(b.dtype)} *{arg}")
        sizes.append(f"#define {func.upper()}_{arg.upper()}_SIZE {max(1, b.numel)}   /* {b.dtype}{fmt_shape(b.shape)} */")
        doc_in.append(f"{an}: {b.dtype}{fmt_shape(b.shape)}")
        sets.append(f"    anvil_{b.name} = (void *){arg};")
        clears.append(f"    anvil_{b.name} = 0;")
    for b, on in zip(outs, out_names):
        arg = c_ident(on)
        args.append(f"{c_type(b.dtype)} *{arg}")
        sizes.append(f"#define {func.upper()}_{arg.upper()}_SIZE {max(1, b.numel)}   /* {b.dtype}{fmt_shape(b.shape)} */")
        doc_out.append(f"{b.dtype}{fmt_shape(b.shape)}")
        sets.append(f"    anvil_{b.name} = (void *){arg};")
        clears.append(f"    anvil_{b.name} = 0;")
    proto = f"void {func}({', '.join(args)})"
    header = f"""// {lib}.h — the Anvil function `{fn_name}`, compiled for MI355X by `anvil export --hip`.
//
//     {fn_name}({', '.join(doc_in)}) -> {', '.join(doc_out)}
//
// Link with lib{lib}.so (cc app.c -L<dir> -l{lib} -Wl,-rpath,<dir>). Arrays are row-major host
// memory and are read and written in place; the library holds everything else the function needs
// (its weights included). Calls from several threads take turns.
#pragma once
#include <stdint.h>
#ifdef __cplusplus
extern "C" {{
#endif

{chr(10).join(sizes)}

{proto};

#ifdef __cplusplus
}}
#endif
"""
    wrapper = f"""
// ---------------------------------------------------------------- {lib}: the exported entry point
// Points the library's argument slots at the caller's arrays, runs the function, clears the slots.
#include <pthread.h>
static pthread_mutex_t anvil_export_lock = PTHREAD_MUTEX_INITIALIZER;
extern "C" {proto} {{
    pthread_mutex_lock(&anvil_export_lock);
{chr(10).join(sets)}
    anvil_entry();
{chr(10).join(clears)}
    pthread_mutex_unlock(&anvil_export_lock);
}}
"""
    src = hip.generate(prog, seed=seed, library=True) + wrapper
    h_path = os.path.join(out_dir, f"{lib}.h")
    so_path = os.path.join(out_dir, f"lib{lib}.so")
    with open(h_path, "w") as f:
        f.write(header)
    hip.build(src, so_path)
    return [h_path, so_path]

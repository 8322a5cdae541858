"""Helpers that read the committed golden fixtures (tests/golden/ir, tests/golden/vectors)."""
import io
import json
import os

import numpy as np

from anvil import irjson

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT_PKG = os.path.join(ROOT, "anvil-lang_amd")


def ir_path(name):
    return os.path.join(GOLDEN, "ir", f"{name}.json")


def load_ir(name):
    """(program, raw JSON dict) of a fixture."""
    with open(ir_path(name)) as f:
        data = json.load(f)
    return irjson.load(data), data


def vectors(name):
    return np.load(os.path.join(GOLDEN, "vectors", f"{name}.npz"))


# fixtures whose oracle run takes minutes (C2 whole: 500 full-size steps of the NumPy interpreter;
# C5 at full size: its im2col products broadcast over 10^9 elements a step); the oracle replays them
# only with ANVIL_SLOW_ORACLE=1, the GPU tests always compare against them
SLOW = {"c2_full", "c5_full3", "c4_full2", "c2_full100", "c4_t256_2", "c5_step1", "c2_full10"}


# the full-length C4 and C5 runs, written by the oracle itself (tests/golden/make_long_runs.py) from
# the restatement the other vectors pin: not vectors of the reference interpreter, and hours long
ORACLE_WRITTEN = {"c4_full200", "c5_full300"}


def vector_names(slow=False):
    """The fixtures the reference interpreter wrote (the oracle is checked against each)."""
    d = os.path.join(GOLDEN, "vectors")
    names = sorted(f[:-4] for f in os.listdir(d) if f.endswith(".npz"))
    return [n for n in names if (slow or n not in SLOW) and n not in ORACLE_WRITTEN]


def stdout_of(z):
    return bytes(z["stdout"]).decode()


# where make_fixtures.py placed the fixture programs: files they write (save_npy, save) are recorded
# under this directory in their IR, and kept byte for byte in the vectors as "file:<name>"
RECORDED_DIR = "/root/repo/tests/golden/programs/"


def written_files(z) -> list[str]:
    return [k[5:] for k in z.files if k.startswith("file:")]


def stdin_of(name: str) -> str:
    """What a fixture program reads with `input` (the scripted stdin of tests/golden/programs.py)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("_fixture_programs", os.path.join(GOLDEN, "programs.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return next((p.get("stdin", "") for p in mod.PROGRAMS if p["name"] == name), "")


def load_ir_writing_to(name, directory):
    """A fixture's program whose output files go to `directory` instead of RECORDED_DIR."""
    with open(ir_path(name)) as f:
        text = f.read().replace(RECORDED_DIR, os.path.join(str(directory), ""))
    data = json.loads(text)
    return irjson.load(data), data


def run_oracle(prog, data, z=None, stdin=""):
    """Run the oracle on a fixture; function inputs come from the vectors file."""
    from oracle import interp
    out = io.StringIO()
    m = interp.Machine(prog, out=out, seed=data.get("seed", 0), inp=io.StringIO(stdin), check=data.get("check"))
    if "function" in data and z is not None:
        by_id = {b.id: b for b in prog.buffers}
        for k, bid in enumerate(data["function"]["inputs"]):
            m.arr(by_id[bid])[:] = z[f"input{k}"].reshape(-1)
    m.check_error = ""
    try:
        m.run()
    except interp.RuntimeFault as e:
        if not data.get("check"):
            raise
        m.check_error = str(e)                          # --check stopped the program
    return m, out.getvalue()

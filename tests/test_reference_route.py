"""The backend as a drop-in for the reference's plugin API (reference anvil/backend/cuda.py:636-663).

tests/golden/make_fixtures.py loads anvil/backend/hip*.py as members of the reference's own
`anvil.backend` package, so that their `from .. import ir` is the reference's ir module, hands
`hip.generate` the reference front end's own Program objects, and records the sha256 of each
generated source (tests/golden/reference_route.json). Here the same programs come through the JSON
fixtures and this package's ir module: the sources must be byte-identical, so what the tests measure
is what the reference's `cli.py`/`pyapi.py` would get by calling `hip.generate` directly.
"""
import hashlib
import inspect
import json
import os

import pytest

from fixtures import GOLDEN, load_ir

with open(os.path.join(GOLDEN, "reference_route.json")) as f:
    ROUTE = json.load(f)


@pytest.mark.parametrize("name", sorted(ROUTE))
def test_json_route_generates_the_reference_route_source(name):
    from anvil.backend import hip
    prog, data = load_ir(name)
    src = hip.generate(prog, seed=int(data.get("seed", 0)), library=ROUTE[name]["library"], graphs=False,
                       check=data.get("check"))
    assert len(src) == ROUTE[name]["bytes"]
    assert hashlib.sha256(src.encode()).hexdigest() == ROUTE[name]["sha256"]


def test_ir_constructors_take_the_reference_arguments():
    """Buffer and Var as the reference declares them (anvil/ir.py:66, :103): the backend may not
    rely on extra arguments such as a chosen id."""
    from anvil import ir
    assert list(inspect.signature(ir.Buffer).parameters) == ["name", "shape", "dtype", "kind", "init", "span"]
    assert list(inspect.signature(ir.Var).parameters) == ["name", "extent"]
    for mod in ("hip", "hip_analysis", "hip_attn", "hip_attn_train", "hip_conv", "hip_cost", "hip_emit", "hip_gemm",
                "hip_kernels"):
        path = os.path.join(os.path.dirname(ir.__file__), "backend", f"{mod}.py")
        with open(path) as f:
            text = f.read()
        for name in ("restart_ids", "bump_ids", "max_id"):
            assert f"ir.{name}" not in text and f"prog.{name}" not in text, (mod, name)


def test_every_fixture_program_is_on_the_route():
    names = {f[:-5] for f in os.listdir(os.path.join(GOLDEN, "ir")) if f.endswith(".json")}
    assert names == set(ROUTE)

"""`--check` on the HIP backend (the reference's `anvil run --check`, cli.py:44-45): after each kernel
the tensors it wrote are scanned for the first nan (--check=inf: or infinity), and the program stops
with a report naming the value, the tensor and element, the computation and its source line, and
whether the computation's inputs already held nans or infinities (runtime.s _anvil_rt_check).

Pinned two ways: the reference interpreter's own --check finding for the same programs (the golden
`check_error`: value, tensor, element, description; compiled unoptimized, one kernel per operation,
as the reference does for --check) and the substrings the reference's tests assert on its native
backend's report (tests/test_native.py:292-320)."""
import re

import pytest

from fixtures import load_ir, stdout_of, vectors
from hiprun import run_program

CASES = ["check_nan", "check_inf", "check_inf_traced", "check_healthy"]
# the reference's tests/test_native.py:292-320
ASSERTED = {
    "check_nan": ["nan in `t3` (f32[4, 3]) at [0, 0]", "made by `log` at checked.anvil:3:1",
                  "y = log(x - 0.5) * w", "this computation made it"],
    "check_inf": ["nan in", "its input `z` already held 0 nan and 12 infinite values", "--check=inf"],
    "check_inf_traced": ["-inf in `z` (f32[4, 3]) at [0, 0]", "`log`"],
    "check_healthy": [],
}


def _expect(name, rc, out, err):
    _, data = load_ir(name)
    z = vectors(name)
    assert out == stdout_of(z)
    want = bytes(z["check_error"]).decode()
    if not want:
        assert rc == 0 and err == "", err
        return
    assert rc == 1, err
    head, _, desc = want.partition("\n")
    m = re.match(r"--check: (\S+) in `([^`]+)`( at \[[0-9, ]*\])?$", head)
    assert m, head
    value, tensor, where = m.group(1), m.group(2), m.group(3) or ""
    assert f"anvil: --check: {value} in `{tensor}` (" in err, err
    assert where in err and desc in err, err
    for s in ASSERTED[name]:
        assert s in err, (s, err)


@pytest.mark.parametrize("name", CASES)
def test_check_emulated(name):
    _, data = load_ir(name)
    rc, out, err, _ = run_program(name, emulate=True, check=data["check"], timeout=300)
    _expect(name, rc, out, err)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_gpu_check(name):
    print(f"gpu check {name}", flush=True)
    _, data = load_ir(name)
    rc, out, err, _ = run_program(name, emulate=False, check=data["check"], timeout=300)
    _expect(name, rc, out, err)

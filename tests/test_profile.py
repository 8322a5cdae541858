"""`anvil run --profile`: the reference's per-kernel table (its runtime's report, runtime.s:1592-1671;
rows as aarch64.py:877-881 names them; README.md:628-636), printed on stdout when the program ends:

      time%        ms      calls   kernel
      17.4%      89.4       4685   k70    copy                    mnist.anvil:26
    ...
              xxxx.x ms in kernels

One row per launch of the generated program, in program order: its share of the kernel time, its
total milliseconds and number of launches, then the launch's name (6 columns), what it computes
(the labels of the IR kernels it runs, joined by '+', 34 columns) and the source line of its first
kernel. The launch counts are held to the NumPy oracle's count of executions of the same IR
kernels (summed over the launches that hold a kernel), the labels and lines to the IR the
reference front end wrote.
"""
import io
import os
import re

import pytest

from fixtures import load_ir
from hiprun import run_program

HEAD = "\n  time%        ms      calls   kernel\n"
ROW = re.compile(r"^([ \d.]{5}\d)%  ([ \d.]{7}\d)  ([ \d]{8}\d)   (.*)$")
TOTAL = re.compile(r"^ {10}([ \d.]{7}\d) ms in kernels$")


def parse_table(out: str):
    """(program output before the table, [(percent, ms, calls, name, label, loc)], total ms)."""
    i = out.rindex(HEAD)
    lines = out[i + len(HEAD):].splitlines()
    total = TOTAL.match(lines[-1])
    assert total, lines[-1]
    rows = []
    for line in lines[:-1]:
        m = ROW.match(line)
        assert m, repr(line)
        where = m.group(4)
        name = where.split(" ", 1)[0]
        rest = where[max(6, len(name)) + 1:]
        rows.append((float(m.group(1)), float(m.group(2)), int(m.group(3)), name, rest[:34], rest[35:]))
    return out[:i], rows, float(total.group(1))


def oracle_launch_counts(name: str) -> dict:
    """How many times the oracle executes each IR kernel of the program (kernel id -> count)."""
    from oracle import interp
    prog, data = load_ir(name)
    counts: dict = {}

    class Counting(interp.Machine):
        def kernel(self, k):
            counts[k.id] = counts.get(k.id, 0) + 1
            return super().kernel(k)
    Counting(prog, out=io.StringIO(), seed=int(data.get("seed", 0))).run()
    return counts


# launches that finish another's work (partial sums added, the second half of a backward, the device
# twins of host scalars): they run the same IR kernels again and are not counted as executions
SECOND = {"gemm-reduce", "slices-sum", "attention-train-dkdv", "twin"}


def _second(p) -> bool:
    return p.kind in SECOND or (p.kind == "fused" and all(_second(q) for q in p.parts))


def expected_rows(name: str, emulate: bool):
    """(name, label, loc, IR kernel ids or None for a second launch) of each launch, in program order."""
    from anvil.backend import hip
    prog, data = load_ir(name)
    g = hip.HipGen(prog, seed=int(data.get("seed", 0)), emulate=emulate)
    g.generate()
    out = []
    for p in g.plans:
        row = hip.profile_row(p)
        nm = row.split(" ", 1)[0]
        rest = row[max(6, len(nm)) + 1:]
        out.append((nm, rest[:34], rest[35:], None if _second(p) else [k.id for k in p.kernels]))
    return out


def check_table(name: str, emulate: bool):
    rc0, plain, err0, _ = run_program(name, emulate=emulate)
    rc, out, err, _ = run_program(name, emulate=emulate, extra_args=["--profile"])
    assert rc == 0 and rc0 == 0, err + err0
    program, rows, total = parse_table(out)
    assert program == plain                                   # the program's own output is unchanged
    want = expected_rows(name, emulate)
    assert [r[3] for r in rows] == [w[0] for w in want]       # every launch, in program order
    # every IR kernel runs in the launches that hold it (a fused launch, or on the iteration that
    # leaves the loop the part of it before the exit) as often as the oracle executes it
    counts = oracle_launch_counts(name)
    ran: dict = {}
    for (pct, ms, calls, nm, label, loc), (wn, wlabel, wloc, kids) in zip(rows, want):
        assert (label, loc) == (wlabel, wloc), nm
        assert ms >= 0 and 0 <= pct <= 100
        for kid in kids or []:
            ran[kid] = ran.get(kid, 0) + calls
    assert ran and all(ran[k] == counts.get(k, 0) for k in ran), \
        {k: (ran[k], counts.get(k, 0)) for k in ran if ran[k] != counts.get(k, 0)}
    assert abs(sum(r[1] for r in rows) - total) <= 0.05 * len(rows) + 0.1
    if total > 0:
        assert abs(sum(r[0] for r in rows) - 100) <= 0.05 * len(rows) + 0.1
    return rows, total


def test_profile_table_form_cpu_build():
    """c2_small built for the CPU: header, one row per launch with the oracle's launch counts, the
    labels and source lines of the IR, the total."""
    rows, _ = check_table("c2_small", emulate=True)
    labels = [r[4].strip() for r in rows]
    assert labels[:3] == ["uniform", "randint", "normal"]     # X, labels, then the first layer's init
    assert rows[0][5] == "c2_small.anvil:8"
    assert {r[2] for r in rows} >= {1, 40}                    # set-up kernels once, the step's 40 times


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c2_small", "c4_mid", "c5_mid"])
def test_profile_table_on_the_gpu(name):
    """The same table from the gfx950 build: the launches (fused side-by-side and row-block launches
    included) in program order, each counted as often as the oracle executes its IR kernels, and
    timed with device events."""
    print(f"gpu profile table {name}", flush=True)
    rows, total = check_table(name, emulate=False)
    assert total > 0                                 # (a row prints 0.0 ms when it took under 0.05 ms)

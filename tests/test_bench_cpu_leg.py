"""bench.py's CPU baseline leg, on the CPU: the oracle runs in a child process whose environment
pins BLAS and OpenMP to one thread, and returns the times of the loop's iterations."""
import sys

from fixtures import ROOT, ir_path


def test_oracle_leg_runs_single_threaded_in_a_child():
    sys.path.insert(0, ROOT)
    import bench
    run = bench.oracle_run(ir_path("c1_small"), bench.LOOP_COUNTER, 2)
    marks = run["marks"]
    assert len(marks) == 3 and marks[0] == 0.0 and marks[1] < marks[2] <= run["end"]
    assert "OMP_NUM_THREADS=1" in run["host"] and "OPENBLAS_NUM_THREADS=1" in run["host"]

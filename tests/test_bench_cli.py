"""bench.py's command line, on the CPU: the driver's contract that a run on
more than one GPU exits with a message (this build measures one GPU), and
that the options and modes parse.  Neither touches a GPU: the GPU count is
checked before torch is imported."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2", "--steps", "3", "--warmup", "1")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout == ""   # no JSON line for a run that did not happen


def test_help_lists_the_modes():
    r = _run("--help")
    assert r.returncode == 0
    for mode in ("full", "headline", "batched-kernels", "batched-pmc", "layout", "small-shards"):
        assert mode in r.stdout, mode
    for opt in ("--gpus", "--steps", "--warmup", "--settle-ms"):
        assert opt in r.stdout, opt


def test_update_bytes_counts_parity_up_to_the_longest_changed_unit():
    """The update's algorithmic bytes: new + old of each changed unit, and m
    parity units per changed stripe read and written up to that stripe's
    longest changed unit."""
    import types
    import numpy as np
    sys.path.insert(0, ROOT)
    import bench
    # k = 3, m = 2, 100-byte units; stripe 0 full, stripe 1 with a 40-byte unit
    lay = types.SimpleNamespace(k=3, m=2, host_len=np.array([[100, 100, 100], [100, 40, 0]],
                                                             np.uint32))
    read, write = bench.update_bytes(lay, np.array([0, 2, 4]))
    # changed: unit 0 (100 B) and 2 (100 B) of stripe 0, unit 4 (40 B) of stripe 1
    assert write == 2 * 100 + 2 * 40
    assert read == 2 * (100 + 100 + 40) + write
    read, write = bench.update_bytes(lay, np.array([3, 4]))
    assert write == 2 * 100 and read == 2 * 140 + 200

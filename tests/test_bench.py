"""bench.py's contract: one GPU only, and exactly the requested timed steps.

The GPU case runs the headline at the driver's short setting (direct launches
behind the spin kernel) and the launch floor (graph-replayed), each through
`bench.py --only` in a child process, and checks what it reports."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_unknown_workload_key_is_refused():
    """Exit status 2 and nothing on stdout (on a host without a GPU at the GPU
    check, with one at the key check)."""
    r = subprocess.run([sys.executable, BENCH, "--only", "no_such_workload"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert r.stdout == ""


@pytest.mark.gpu
def test_short_run_times_exactly_the_requested_steps():
    print("bench --only gemv_q4_0_11008x4096_b1,launch_floor --steps 20 --warmup 5", flush=True)
    r = subprocess.run([sys.executable, "-u", BENCH, "--only", "gemv_q4_0_11008x4096_b1,launch_floor",
                        "--steps", "20", "--warmup", "5"], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("{")][-1]
    res = json.loads(line)["only"]
    head = res["gemv_q4_0_11008x4096_b1"]
    assert head["steps"] == 20
    assert head["alg_bytes"] == 11008 * (4096 // 32) * 18 + 4 * 4096 + 4 * 11008
    # a 25 MB read per step: between 1 and 8 TB/s (HBM peak)
    assert 1000.0 < head["value"] < 8000.0
    assert head["ms_per_step"] * 1e3 > 3.0
    # the wall clock per step (host launches included, the spin excluded) is
    # never below the GPU time
    assert head["wall_ms_per_step"] >= 0.9 * head["ms_per_step"]
    floor = res["launch_floor"]
    assert floor["steps"] >= 1000  # the other lines: graph-replayed, >= 1000 launches
    assert 0.0005 < floor["ms_per_step"] < 0.01

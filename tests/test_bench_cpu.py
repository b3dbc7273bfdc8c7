"""bench.py's contract pieces that need no GPU: the kernels whose HBM traffic and
SQ counters the roofline object reports exist under those exact names in the
committed counter summaries, and --gpus above 1 is refused."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_profiled_kernel_names_are_in_the_summaries():
    import bench

    names = [bench.K_FWD, bench.K_BWD, bench.K_RED, bench.K_NF, bench.K_NB]
    traffic = json.load(open(os.path.join(ROOT, "profiles", "hbm_traffic.json")))["kernels"]
    counters = json.load(open(os.path.join(ROOT, "profiles", "laplace_newton_counters.json")))["kernels"]
    for name in names:
        assert name in traffic, f"{name} is not in profiles/hbm_traffic.json"
        assert name in counters, f"{name} is not in profiles/laplace_newton_counters.json"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr

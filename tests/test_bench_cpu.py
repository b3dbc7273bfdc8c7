"""bench.py's contract pieces that need no GPU: the kernels whose HBM traffic the
roofline object reports exist under those exact names in the committed counter
summary, and --gpus above 1 is refused."""
import json
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_traffic_kernel_names_are_in_the_summary():
    src = open(os.path.join(ROOT, "bench.py")).read()
    calls = re.findall(r"_traffic\(((?:\s*\"[^\"]+\"\s*,?)+)\)", src)
    assert calls, "bench.py reports no traffic"
    table = json.load(open(os.path.join(ROOT, "profiles", "hbm_traffic.json")))["kernels"]
    for call in calls:
        for name in re.findall(r"\"([^\"]+)\"", call):
            assert name in table, f"{name} is not in profiles/hbm_traffic.json"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr

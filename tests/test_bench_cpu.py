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


def test_layer_floors():
    """The config-5 layer's floors, from the shapes counted by hand: 128 slices x (784 + 784 + 49)
    rows x 49 landmarks x 64 channels = 649,076,736 triples at 11 flop; 128 x 11 x 4 x 49^3
    NewtonInverse flop; six products of one fp32 [128, 784, 49] and one fp16 [128, 784, 64]
    tensor (19,668,992 + 12,845,056 bytes); pooling 3 x 12,845,056 bytes."""
    import bench

    parts, work = bench.layer_floors()
    assert work["triples"] == 649_076_736
    assert work["product_bytes"] == 6 * (19_668_992 + 12_845_056)
    assert work["pooling_bytes"] == 3 * 12_845_056
    assert abs(parts["distances_valu"] - 11 * 649_076_736 / 157.3e6) < 1e-9
    assert abs(parts["newton_mfma"] - 128 * 11 * 4 * 49 ** 3 / 157.3e6) < 1e-9
    assert abs(parts["products_hbm"] - 195_084_288 / 8e6) < 1e-9
    assert 78 < sum(parts.values()) < 80

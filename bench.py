"""Benchmark of the LaplaceSubtraction / NewtonInverse hot path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input already
resident in HBM: LaplaceSubtraction forward + backward (grad_query and grad_key)
at BASELINE config 2 (B=32 H=1 N=3136 M=49 d=64, fp16 storage, fp32 arithmetic).
``value`` is that step's throughput in G(i*j*d)/s (triples per second / 1e9).
NewtonInverse forward + backward at BASELINE config 3 (1024 x 64x64 fp32,
12 iterations) is timed the same way and reported under "newton"; the
attention layer (config 5) under "layer" and the large-landmark stress case
(config 4) under "config4".

Per-kernel durations come from HIP events recorded on the stream the kernels
run on (PyTorch's current stream). The CPU baseline is the C oracle
(oracle/laplace_oracle.c, OpenMP) on the same inputs, plus PyTorch's CPU
cdist / bmm Newton loop, both on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "L1-dist fwd+bwd G(i·j·d)/s + NS-inverse TFLOP/s, % of MI355X roofline"
PEAK_FP32_TFLOPS = 157.3  # MI355X fp32 vector and fp32 matrix peak (dense)
PEAK_HBM_GBS = 8000.0
L1_FLOPS_FWD, L1_FLOPS_BWD = 3, 8  # per (i,j,d) triple: |.|-add 3; dq 4 + dk 4


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU timing (approx)")
    p.add_argument("--only", choices=["laplace", "newton", "layer", "cfg4", "all"], default="all")
    p.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                   help="after timing, run one plain device copy of MIB MiB (HBM counter calibration)")
    return p.parse_args()


def gen(shape, seed, dtype, scale=1.0):
    import torch

    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


EVENT_EVERY = 8  # steps between event-bracketed samples inside the timed region


def time_steps(fns, steps, warmup):
    """Runs `fns` (a list of launch callables) once per step, `steps` times.

    Returns the wall-clock ms per step over the whole timed region (bracketed by
    device synchronisation) and the mean duration (ms) of each callable, taken
    from HIP events recorded on the current stream around every callable of
    every EVENT_EVERY-th step (each event record costs a few microseconds of GPU
    time, so recording them on every step would inflate the step time)."""
    import torch

    for _ in range(warmup):
        for f in fns:
            f()
    torch.cuda.synchronize()
    sampled = list(range(0, steps, EVENT_EVERY))
    evs = {s: [torch.cuda.Event(enable_timing=True) for _ in range(len(fns) + 1)] for s in sampled}
    t0 = time.perf_counter()
    for s in range(steps):
        e = evs.get(s)
        if e is None:
            for f in fns:
                f()
        else:
            e[0].record()
            for i, f in enumerate(fns):
                f()
                e[i + 1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    per = [sum(evs[s][i].elapsed_time(evs[s][i + 1]) for s in sampled) / len(sampled) for i in range(len(fns))]
    return wall, per


def bench_laplace(args, dev):
    import torch

    import laplacianformer_amd as lf

    B, H, N, M, C = 32, 1, 3136, 49, 64
    q = gen((B, H, N, C), 1002, torch.float16)
    kT = gen((B, H, M, C), 1003, torch.float16).transpose(-1, -2).contiguous()
    g = gen((B, H, N, M), 1004, torch.float16)
    qd, kd, gd = q.to(dev), kT.to(dev), g.to(dev)
    out = torch.empty((B, H, N, M), dtype=torch.float16, device=dev)
    dq = torch.empty_like(qd)
    dk = torch.empty_like(kd)
    L = lf.ext()
    fwd = lambda: L.LaplaceSubtraction_forward(qd, kd, out)  # noqa: E731
    bwd = lambda: L.LaplaceSubtraction_backward(gd, qd, kd, dq, dk)  # noqa: E731
    wall, (t_fwd, t_bwd) = time_steps([fwd, bwd], args.steps, args.warmup)
    # Reference-API backward (two separate entry points) for comparison.
    bq = lambda: L.LaplaceSubtraction_backward_query(gd, qd, kd, dq)  # noqa: E731
    bk = lambda: L.LaplaceSubtraction_backward_key(gd, qd, kd, dk)  # noqa: E731
    wall_ref, (t_f2, t_bq, t_bk) = time_steps([fwd, bq, bk], args.steps, args.warmup)

    T = B * H * N * M * C
    res = {
        "T": T, "wall_ms": wall, "fwd_ms": t_fwd, "bwd_ms": t_bwd,
        "ref_api_wall_ms": wall_ref, "ref_api_ms": {"forward": t_f2, "backward_query": t_bq, "backward_key": t_bk},
        "inputs": (q, kT, g),
    }
    return res


def bench_newton(args, dev):
    import torch

    import laplacianformer_amd as lf

    nm, n, iters = 1024, 64, 12
    kk = gen((nm, 1, n, 64), 1003, torch.float32)
    kd = kk.to(dev)
    dist = torch.empty((nm, 1, n, n), device=dev)
    lf.ext().LaplaceSubtraction_forward(kd, kd.transpose(-1, -2).contiguous(), dist)
    A = (torch.exp(-dist / 8.0) + 1e-3 * torch.eye(n, device=dev)).contiguous()
    G = gen((nm, 1, n, n), 1013, torch.float32).to(dev)
    V = torch.empty_like(A)
    dA = torch.empty_like(A)
    L = lf.ext()
    fwd = lambda: L.NewtonInverse_forward(A, V, iters)  # noqa: E731
    bwd = lambda: L.NewtonInverse_backward(G, V, dA)  # noqa: E731
    wall, (t_fwd, t_bwd) = time_steps([fwd, bwd], args.steps, args.warmup)
    flops_fwd = nm * iters * 4 * n ** 3
    flops_bwd = nm * 4 * n ** 3
    P = A.double() + 0.01 * torch.eye(n, device=dev, dtype=torch.float64)
    resid = torch.linalg.matrix_norm(P @ V.double() - torch.eye(n, device=dev, dtype=torch.float64)).mean().item()
    # The same op at the configuration-1 (ViT stage 1) landmark shape: B*H = 32 Gram matrices
    # exp(-L1(k, k) / sqrt(d)) + 1e-3 I of 49 landmarks, d = 64, 10 iterations. One workgroup per
    # matrix occupies 32 of the chip's CUs, so the whole-chip MFMA fraction is bounded by 32/CUs;
    # the per-occupied-CU fraction is reported beside it.
    nm1, n1, it1 = 32, 49, 10
    k1 = gen((nm1, 1, n1, 64), 1021, torch.float32).to(dev)
    d1 = torch.empty((nm1, 1, n1, n1), device=dev)
    L.LaplaceSubtraction_forward(k1, k1.transpose(-1, -2).contiguous(), d1)
    A1 = (torch.exp(-d1 / 8.0) + 1e-3 * torch.eye(n1, device=dev)).contiguous()
    G1 = gen((nm1, 1, n1, n1), 1031, torch.float32).to(dev)
    V1 = torch.empty_like(A1)
    dA1 = torch.empty_like(A1)
    wall1, (t1_fwd, t1_bwd) = time_steps([lambda: L.NewtonInverse_forward(A1, V1, it1),
                                          lambda: L.NewtonInverse_backward(G1, V1, dA1)], args.steps, args.warmup)
    P1 = A1.double() + 0.01 * torch.eye(n1, device=dev, dtype=torch.float64)
    resid1 = torch.linalg.matrix_norm(P1 @ V1.double() - torch.eye(n1, device=dev, dtype=torch.float64)).mean().item()
    stage1 = {"wall_ms": wall1, "fwd_ms": t1_fwd, "bwd_ms": t1_bwd, "flops_fwd": nm1 * it1 * 4 * n1 ** 3,
              "flops_bwd": nm1 * 4 * n1 ** 3, "n_mats": nm1, "n": n1, "iters": it1, "residual_fro_mean": resid1}
    return {"wall_ms": wall, "fwd_ms": t_fwd, "bwd_ms": t_bwd, "flops_fwd": flops_fwd, "flops_bwd": flops_bwd,
            "residual_fro_mean": resid, "A": A.cpu(), "G": G.cpu(), "n_mats": nm, "n": n, "iters": iters,
            "stage1": stage1}


def bench_layer(args, dev):
    """LaplacianFormer attention layer fwd+bwd (B=64 H=2 N=784 d=64 fp16,
    4x4-pooled landmarks M=49, NewtonInverse 10 it) through the autograd API."""
    import torch

    import laplacianformer_amd as lf

    B, H, N, d = 64, 2, 784, 64
    q, k, v, g = (gen((B, H, N, d), 1005 + i, torch.float16).to(dev) for i in range(4))
    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()

    def step():
        out = lf.laplacian_attention(q, k, v, grid=(28, 28), pool=4, iters=10)
        out.backward(g)

    steps = max(1, args.steps // 10)
    wall, _ = time_steps([step], steps, max(1, args.warmup // 10))
    # The same step captured once in a HIP graph (one launch per step instead of
    # ~40 host dispatches); gradients are overwritten, not accumulated, per replay.
    graphed = lf.GraphedStep(lambda a, b, c: lf.laplacian_attention(a, b, c, grid=(28, 28), pool=4, iters=10),
                             [q, k, v], g)
    wall_graph, _ = time_steps([graphed.replay], steps, max(1, args.warmup // 10))
    T = B * H * (2 * N * 49 + 49 * 49) * d
    return {"workload": "BASELINE config 5: LaplacianFormer attention fwd+bwd, B=64 H=2 N=784 (28x28) d=64 "
                        "fp16, M=49 (4x4 pooled K), NewtonInverse 10 it",
            "ms_per_step": wall, "ms_per_step_hip_graph": wall_graph, "l1_triples": T, "steps": steps}


def bench_cfg4(args, dev):
    """BASELINE config 4 (large-landmark stress): LaplaceSubtraction fwd + fused bwd at B=16 H=8
    N=4096 M=256 d=64, bf16 storage (q, k ~ N(0, 0.5)); NewtonInverse fwd (16 it) + bwd on 128
    matrices of 256 x 256 fp32 (the batched-GEMM path with its workspace)."""
    import torch

    import laplacianformer_amd as lf

    L = lf.ext()
    B, H, N, M, C = 16, 8, 4096, 256, 64
    q = gen((B, H, N, C), 1041, torch.bfloat16, 0.5).to(dev)
    kT = gen((B, H, C, M), 1042, torch.bfloat16, 0.5).to(dev)
    g = gen((B, H, N, M), 1043, torch.bfloat16).to(dev)
    out = torch.empty((B, H, N, M), dtype=torch.bfloat16, device=dev)
    dq, dk = torch.empty_like(q), torch.empty_like(kT)
    steps = max(1, args.steps // 20)
    wall, (t_f, t_b) = time_steps([lambda: L.LaplaceSubtraction_forward(q, kT, out),
                                   lambda: L.LaplaceSubtraction_backward(g, q, kT, dq, dk)],
                                  steps, max(1, args.warmup // 20))
    T = B * H * N * M * C
    n, nm, iters = 256, B * H, 16
    kk = gen((nm, n, 64), 1044, torch.float32)
    A = (torch.exp(-torch.cdist(kk, kk, p=1) / 8.0) + 1e-3 * torch.eye(n)).reshape(B, H, n, n).to(dev).contiguous()
    G = gen((B, H, n, n), 1045, torch.float32).to(dev)
    V, dA = torch.empty_like(A), torch.empty_like(A)
    wall_n, (tn_f, tn_b) = time_steps([lambda: L.NewtonInverse_forward(A, V, iters),
                                       lambda: L.NewtonInverse_backward(G, V, dA)], steps, max(1, args.warmup // 20))
    fl_f, fl_b = nm * iters * 4 * n ** 3, nm * 4 * n ** 3
    return {"workload": "BASELINE config 4: LaplaceSubtraction fwd+bwd B=16 H=8 N=4096 M=256 d=64 bf16; "
                        "NewtonInverse 128 x 256x256 fp32, 16 it, fwd+bwd",
            "l1": {"ms_per_step": wall, "value": T / (wall * 1e-3) / 1e9, "unit": "G(i*j*d)/s",
                   "fwd_ms": t_f, "bwd_ms": t_b,
                   "fwd_frac_fp32_peak": L1_FLOPS_FWD * T / (t_f * 1e-3) / 1e12 / PEAK_FP32_TFLOPS,
                   "bwd_frac_fp32_peak": L1_FLOPS_BWD * T / (t_b * 1e-3) / 1e12 / PEAK_FP32_TFLOPS},
            "newton": {"ms_per_step": wall_n, "fwd_ms": tn_f, "bwd_ms": tn_b,
                       "tflops": (fl_f + fl_b) / (wall_n * 1e-3) / 1e12,
                       "frac_fp32_mfma_peak": (fl_f + fl_b) / (wall_n * 1e-3) / 1e12 / PEAK_FP32_TFLOPS},
            "steps": steps}


def cpu_baseline(lap, ns, budget):
    """C oracle (OpenMP) on a slice sample of config 2, scaled to the full workload,
    plus PyTorch CPU cdist fwd+bwd (fp32) and the bmm Newton loop."""
    import numpy as np
    import torch

    import oracle

    torch.set_num_threads(os.cpu_count() or 1)
    q, kT, g = lap["inputs"]
    threads = oracle.max_threads()
    # Whole config-2 steps (fwd + dq + dk over all slices), repeated until ~budget/2 seconds.
    t_used, reps = 0.0, 0
    while t_used < budget / 2 or reps == 0:
        t0 = time.perf_counter()
        oracle.laplace_forward(q, kT, "f16")
        oracle.laplace_backward_query(g, q, kT, "f16")
        oracle.laplace_backward_key(g, q, kT, "f16")
        t_used += time.perf_counter() - t0
        reps += 1
    port_rate = lap["T"] * reps / t_used / 1e9

    # PyTorch CPU: cdist p=1 on [B,H,M,d] keys, fp32 (CPU cdist rejects fp16), forward + autograd backward.
    qf = q.float().requires_grad_()
    kf = kT.float().transpose(-1, -2).contiguous().requires_grad_()
    gf = g.float()
    t_cd, reps_cd = 0.0, 0
    while t_cd < budget / 4 or reps_cd == 0:
        t0 = time.perf_counter()
        d = torch.cdist(qf, kf, p=1)
        d.backward(gf)
        t_cd += time.perf_counter() - t0
        reps_cd += 1
    cd_rate = lap["T"] * reps_cd / t_cd / 1e9

    # Newton: bmm loop with the reference init on a sample of matrices.
    A = ns["A"].double()
    nmat = min(A.shape[0], 256)
    Ab = A[:nmat, 0].float()
    n = Ab.shape[-1]
    Gb = ns["G"][:nmat, 0]
    t_ns, reps_ns = 0.0, 0
    while t_ns < budget / 4 or reps_ns == 0:
        t0 = time.perf_counter()
        P = Ab + 0.01 * torch.eye(n)
        alpha = 1.8 / P.sum(-1).max(-1).values ** 2
        V = alpha[:, None, None] * P
        for _ in range(ns["iters"]):
            V = 2 * V - torch.bmm(V, torch.bmm(P, V))
        Vt = V.transpose(1, 2).contiguous()
        _ = -torch.bmm(torch.bmm(Vt, Gb), Vt)
        t_ns += time.perf_counter() - t0
        reps_ns += 1
    ns_flops = nmat * (ns["iters"] + 1) * 4 * n ** 3 * reps_ns
    return {
        "value": port_rate, "unit": "G(i*j*d)/s", "cores": threads, "kind": "port",
        "sample": f"C oracle (oracle/laplace_oracle.c) on the whole config-2 step (fwd + dq + dk, 32 (b,h) "
                  f"slices, fp32 accumulation in the reference's serial order) x {reps}, {t_used:.2f} s",
        "torch_cpu_cdist": {"value": cd_rate, "unit": "G(i*j*d)/s", "threads": torch.get_num_threads(),
                            "sample": f"torch.cdist(p=1) fp32 fwd+bwd on the config-2 step x {reps_cd}, {t_cd:.2f} s"},
        "torch_cpu_newton": {"value": ns_flops / t_ns / 1e12, "unit": "TFLOP/s", "threads": torch.get_num_threads(),
                             "sample": f"bmm Newton-Schulz fwd+bwd (12 it), {nmat} of 1024 config-3 matrices "
                                       f"x {reps_ns}, {t_ns:.2f} s"},
        "host": {"cpu_count": os.cpu_count(), "cpu_model": _cpu_model()},
    }


def _traffic(*kernels):
    """HBM bytes of one call made of the named kernel launches (exact names as rocprofv3 prints
    them, without the argument list), from the committed counter summary (profiles/hbm_traffic.json,
    FETCH_SIZE/WRITE_SIZE scaled by a plain-copy calibration); None if any is missing."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    table = data.get("kernels", {})
    if not all(k in table for k in kernels):
        return None
    rd = sum(table[k]["read_bytes"] for k in kernels)
    wr = sum(table[k]["write_bytes"] for k in kernels)
    return {"bytes": rd + wr, "read_bytes": rd, "write_bytes": wr, "kernels": list(kernels),
            "source": data.get("source")}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    lap = bench_laplace(args, dev) if args.only in ("laplace", "all") else None
    ns = bench_newton(args, dev) if args.only in ("newton", "all") else None
    layer = bench_layer(args, dev) if args.only in ("layer", "all") else None
    cfg4 = bench_cfg4(args, dev) if args.only in ("cfg4", "all") else None

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic"}
    if lap:
        T = lap["T"]
        B_, N_, M_, C_ = 32, 3136, 49, 64
        value = T / (lap["wall_ms"] * 1e-3) / 1e9
        bwd_tflops = L1_FLOPS_BWD * T / (lap["bwd_ms"] * 1e-3) / 1e12
        fwd_tflops = L1_FLOPS_FWD * T / (lap["fwd_ms"] * 1e-3) / 1e12
        step_tflops = (L1_FLOPS_FWD + L1_FLOPS_BWD) * T / (lap["wall_ms"] * 1e-3) / 1e12
        line.update({
            "value": value, "unit": "G(i*j*d)/s", "ms_per_step": lap["wall_ms"],
            "config": {"workload": "BASELINE config 2: LaplaceSubtraction forward + fused backward (dq, dk), "
                                   "B=32 H=1 N=3136 M=49 d=64", "storage": "f16", "accumulate": "f32",
                       "global_batch": 32, "seq_len": 3136, "landmarks": 49, "channels": 64},
            "roofline": {"bound": "valu",
                         "kernel": "LaplaceSubtraction_backward = laplace_bwd_bcast_kernel<49,dq,dk> + "
                                   "laplace_dk_reduce_cm_kernel (one call of the op, HIP events around both "
                                   "launches; fp32 vector peak)",
                         "achieved": bwd_tflops, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                         "frac": bwd_tflops / PEAK_FP32_TFLOPS,
                         "traffic": _traffic("lfamd::laplace_bwd_bcast_kernel<lfamd::f16s, 49, true, true, 0>",
                                             "lfamd::laplace_dk_reduce_cm_kernel<lfamd::f16s>"),
                         "algorithmic_bytes": 2 * (B_ * N_ * M_ + 2 * B_ * N_ * C_ + 2 * B_ * C_ * M_),
                         "work": f"{L1_FLOPS_BWD} flop per (i,j,d) triple x {T} triples per launch"},
            "kernels": {
                "forward (laplace_fwd_bcast_kernel<f16s,7,2>)": {
                    "ms": lap["fwd_ms"], "tflops": fwd_tflops, "frac_fp32_peak": fwd_tflops / PEAK_FP32_TFLOPS},
                "backward (laplace_bwd_bcast_kernel<49,dq,dk> + laplace_dk_reduce_cm_kernel)": {
                    "ms": lap["bwd_ms"], "tflops": bwd_tflops, "frac_fp32_peak": bwd_tflops / PEAK_FP32_TFLOPS},
                "step_fwd_bwd": {"ms": lap["wall_ms"], "tflops": step_tflops,
                                 "frac_fp32_peak": step_tflops / PEAK_FP32_TFLOPS},
                "reference_api_step": {"ms": lap["ref_api_wall_ms"], **{k: v for k, v in lap["ref_api_ms"].items()},
                                       "g_triples_per_s": T / (lap["ref_api_wall_ms"] * 1e-3) / 1e9},
            },
        })
    if ns:
        tf_f = ns["flops_fwd"] / (ns["fwd_ms"] * 1e-3) / 1e12
        tf_b = ns["flops_bwd"] / (ns["bwd_ms"] * 1e-3) / 1e12
        tf = (ns["flops_fwd"] + ns["flops_bwd"]) / (ns["wall_ms"] * 1e-3) / 1e12
        line["newton"] = {
            "workload": "BASELINE config 3: NewtonInverse fwd (12 it) + bwd, 1024 x 64x64 fp32",
            "tflops": tf, "ms_per_step": ns["wall_ms"], "frac_fp32_mfma_peak": tf / PEAK_FP32_TFLOPS,
            "fwd": {"ms": ns["fwd_ms"], "tflops": tf_f, "frac": tf_f / PEAK_FP32_TFLOPS},
            "bwd": {"ms": ns["bwd_ms"], "tflops": tf_b, "frac": tf_b / PEAK_FP32_TFLOPS},
            "residual_fro_mean": ns["residual_fro_mean"],
        }
        s1 = ns["stage1"]
        tf1 = (s1["flops_fwd"] + s1["flops_bwd"]) / (s1["wall_ms"] * 1e-3) / 1e12
        cus = props.multi_processor_count
        line["newton"]["stage1"] = {
            "workload": "BASELINE config 1 landmark shape: NewtonInverse fwd (10 it) + bwd, 32 x 49x49 fp32 "
                        "(one workgroup per matrix: 32 CUs occupied)",
            "ms_per_step": s1["wall_ms"], "fwd_ms": s1["fwd_ms"], "bwd_ms": s1["bwd_ms"], "tflops": tf1,
            "frac_fp32_mfma_peak": tf1 / PEAK_FP32_TFLOPS,
            "frac_per_occupied_cu": tf1 / (PEAK_FP32_TFLOPS * s1["n_mats"] / cus),
            "flops": "4 n^3 per iteration + 4 n^3 backward, n = 49 (algorithmic; the kernels pad to 64)",
            "residual_fro_mean": s1["residual_fro_mean"],
        }
        if not lap:
            line.update({"value": tf, "unit": "TFLOP/s", "ms_per_step": ns["wall_ms"],
                         "config": {"workload": line["newton"]["workload"]}})
    if layer:
        line["layer"] = layer
    if cfg4:
        line["config4"] = cfg4
    if args.calib_copy:
        src = torch.empty(args.calib_copy << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        line["calib_copy_bytes"] = args.calib_copy << 20
    line["device"] = {"name": props.name, "cus": props.multi_processor_count,
                      "arch": getattr(props, "gcnArchName", "")}
    if lap and ns and not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(lap, ns, args.cpu_budget)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the LaplaceSubtraction / NewtonInverse hot path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input already
resident in HBM: LaplaceSubtraction forward + backward (grad_query and grad_key)
at BASELINE config 2 (B=32 H=1 N=3136 M=49 d=64, fp16 storage, fp32 arithmetic).
``value`` is that step's throughput in G(i*j*d)/s (triples per second / 1e9).
NewtonInverse forward + backward at BASELINE config 3 (1024 x 64x64 fp32,
12 iterations) is timed the same way and reported under "newton".

Per-kernel durations come from HIP events recorded on the stream the kernels
run on (PyTorch's current stream). The CPU baseline is the C oracle
(oracle/laplace_oracle.c, OpenMP) on the same inputs, plus PyTorch's CPU
cdist / bmm Newton loop, both on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
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
    p.add_argument("--only", choices=["laplace", "newton", "all"], default="all")
    p.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                   help="after timing, run one plain device copy of MIB MiB (HBM counter calibration)")
    return p.parse_args()


def gen(shape, seed, dtype, scale=1.0):
    import torch

    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def time_steps(fns, steps, warmup):
    """Runs `fns` (a list of launch callables) per step. Returns wall ms/step and
    the mean duration (ms) of each callable from HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        for f in fns:
            f()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(fns) + 1)] for _ in range(steps)]
    t0 = time.perf_counter()
    for s in range(steps):
        e = evs[s]
        e[0].record()
        for i, f in enumerate(fns):
            f()
            e[i + 1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    per = [sum(evs[s][i].elapsed_time(evs[s][i + 1]) for s in range(steps)) / steps for i in range(len(fns))]
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
    return {"wall_ms": wall, "fwd_ms": t_fwd, "bwd_ms": t_bwd, "flops_fwd": flops_fwd, "flops_bwd": flops_bwd,
            "residual_fro_mean": resid, "A": A.cpu(), "G": G.cpu(), "n_mats": nm, "n": n, "iters": iters}


def cpu_baseline(lap, ns, budget):
    """C oracle (OpenMP) on a slice sample of config 2, scaled to the full workload,
    plus PyTorch CPU cdist fwd+bwd (fp32) and the bmm Newton loop."""
    import numpy as np
    import torch

    import oracle

    torch.set_num_threads(os.cpu_count() or 1)
    q, kT, g = lap["inputs"]
    B = q.shape[0]
    threads = oracle.max_threads()
    # Time slices until ~budget/2 seconds, at least one.
    t_used, nb, b = 0.0, 0, 0
    while b < B and (t_used < budget / 2 or nb == 0):
        qs, ks, gs = q[b:b + 1], kT[b:b + 1], g[b:b + 1]
        t0 = time.perf_counter()
        oracle.laplace_forward(qs, ks, "f16")
        oracle.laplace_backward_query(gs, qs, ks, "f16")
        oracle.laplace_backward_key(gs, qs, ks, "f16")
        t_used += time.perf_counter() - t0
        nb += 1
        b += 1
    trip = lap["T"] * nb / B
    port_rate = trip / t_used / 1e9

    # PyTorch CPU: cdist p=1 on [B,H,M,d] keys, fp32 (CPU cdist rejects fp16), forward + autograd backward.
    qf = q[:max(1, nb)].float().requires_grad_()
    kf = kT[:max(1, nb)].float().transpose(-1, -2).contiguous().requires_grad_()
    gf = g[:max(1, nb)].float()
    t0 = time.perf_counter()
    d = torch.cdist(qf, kf, p=1)
    d.backward(gf)
    t_cd = time.perf_counter() - t0
    cd_rate = lap["T"] * max(1, nb) / B / t_cd / 1e9

    # Newton: bmm loop with the reference init on a sample of matrices.
    A = ns["A"].double()
    nmat = min(A.shape[0], 256)
    Ab = A[:nmat, 0].float()
    n = Ab.shape[-1]
    t0 = time.perf_counter()
    P = Ab + 0.01 * torch.eye(n)
    alpha = 1.8 / P.sum(-1).max(-1).values ** 2
    V = alpha[:, None, None] * P
    for _ in range(ns["iters"]):
        V = 2 * V - torch.bmm(V, torch.bmm(P, V))
    Gb = ns["G"][:nmat, 0]
    Vt = V.transpose(1, 2).contiguous()
    _ = -torch.bmm(torch.bmm(Vt, Gb), Vt)
    t_ns = time.perf_counter() - t0
    ns_flops = nmat * (ns["iters"] + 1) * 4 * n ** 3
    return {
        "value": port_rate, "unit": "G(i*j*d)/s", "cores": threads, "kind": "port",
        "sample": f"C oracle (oracle/laplace_oracle.c) fwd + dq + dk on {nb} of {B} (b,h) slices of config 2, "
                  f"fp32 accumulation in the reference's serial order, {t_used:.2f} s",
        "torch_cpu_cdist": {"value": cd_rate, "unit": "G(i*j*d)/s", "threads": torch.get_num_threads(),
                            "sample": f"torch.cdist(p=1) fp32 fwd+bwd on {max(1, nb)} slice(s), {t_cd:.2f} s"},
        "torch_cpu_newton": {"value": ns_flops / t_ns / 1e12, "unit": "TFLOP/s", "threads": torch.get_num_threads(),
                             "sample": f"bmm Newton-Schulz fwd+bwd, {nmat} of 1024 matrices, {t_ns:.2f} s"},
        "host": {"cpu_count": os.cpu_count(), "cpu_model": platform.processor() or _cpu_model()},
    }


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

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic"}
    if lap:
        T = lap["T"]
        value = T / (lap["wall_ms"] * 1e-3) / 1e9
        bwd_tflops = L1_FLOPS_BWD * T / (lap["bwd_ms"] * 1e-3) / 1e12
        fwd_tflops = L1_FLOPS_FWD * T / (lap["fwd_ms"] * 1e-3) / 1e12
        step_tflops = (L1_FLOPS_FWD + L1_FLOPS_BWD) * T / (lap["wall_ms"] * 1e-3) / 1e12
        line.update({
            "value": value, "unit": "G(i*j*d)/s", "ms_per_step": lap["wall_ms"],
            "config": {"workload": "BASELINE config 2: LaplaceSubtraction forward + fused backward (dq, dk), "
                                   "B=32 H=1 N=3136 M=49 d=64", "storage": "f16", "accumulate": "f32",
                       "global_batch": 32, "seq_len": 3136, "landmarks": 49, "channels": 64},
            "roofline": {"bound": "valu", "kernel": "laplace_bwd_kernel<f16s,49,dq,dk>",
                         "achieved": bwd_tflops, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                         "frac": bwd_tflops / PEAK_FP32_TFLOPS, "traffic": None,
                         "work": f"{L1_FLOPS_BWD} flop per (i,j,d) triple x {T} triples per launch"},
            "kernels": {
                "laplace_fwd_kernel<f16s,7>": {"ms": lap["fwd_ms"], "tflops": fwd_tflops,
                                               "frac_fp32_peak": fwd_tflops / PEAK_FP32_TFLOPS},
                "laplace_bwd_kernel<f16s,49,dq,dk>": {"ms": lap["bwd_ms"], "tflops": bwd_tflops,
                                                      "frac_fp32_peak": bwd_tflops / PEAK_FP32_TFLOPS},
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
        if not lap:
            line.update({"value": tf, "unit": "TFLOP/s", "ms_per_step": ns["wall_ms"],
                         "config": {"workload": line["newton"]["workload"]}})
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

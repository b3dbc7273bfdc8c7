"""Benchmark of the LaplaceSubtraction / NewtonInverse hot path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input already
resident in HBM: LaplaceSubtraction forward + backward (grad_query and grad_key)
at BASELINE config 2 (B=32 H=1 N=3136 M=49 d=64, fp16 storage, fp32 arithmetic).
``value`` is that step's throughput in G(i*j*d)/s (triples per second / 1e9).
NewtonInverse forward + backward at BASELINE config 3 (1024 x 64x64 fp32,
12 iterations) is timed the same way and reported under "newton"; the
attention layer (config 5) under "layer" and the large-landmark stress case
(config 4) under "config4".

Every section warms up for at least --warmup steps and WARM_S seconds, then
times windows of exactly --steps steps (at least SECTION_REPS in the long
sections), each bracketed by a device synchronisation, and reports the median
with min and max. Per-op durations come from HIP events recorded on the stream
the kernels run on (PyTorch's current stream) around back-to-back calls. The
reference's own comparison (each op against eager PyTorch on the same GPU at
N = 16..128) is under "reference_figure". The CPU baseline is PyTorch's CPU
torch.cdist(p=1) on config 2, beside the C oracle (oracle/laplace_oracle.c,
OpenMP) and the bmm Newton loop, on this host's cores.
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
    p.add_argument("--only", choices=["laplace", "newton", "layer", "cfg4", "figure", "all"], default="all")
    p.add_argument("--profile-run", action="store_true",
                   help="one timed window per measurement and no time-based warm-up (for counter collection)")
    p.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                   help="after timing, run one plain device copy of MIB MiB (HBM counter calibration)")
    return p.parse_args()


def gen(shape, seed, dtype, scale=1.0):
    import torch

    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


WARM_S = 0.2      # seconds of untimed warm-up per section (after at least `warmup` steps)
TIMED_S = 0.15    # at least this many seconds of timed windows per measurement
MIN_WINDOWS = 5   # and at least this many windows
SECTION_REPS = 20  # floor on the timed steps of a window in the long sections


def _stats(xs):
    xs = sorted(xs)
    n = len(xs)
    med = xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])
    return {"median": med, "min": xs[0], "max": xs[-1], "windows": n}


def warm_up(fns, warmup):
    """At least `warmup` steps of `fns`, continued until WARM_S seconds have passed
    (clocks and caches reach steady state), then a device synchronisation."""
    import torch

    t0, n = time.perf_counter(), 0
    while n < warmup or time.perf_counter() - t0 < WARM_S:
        for f in fns:
            f()
        n += 1
        if n % 32 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_windows(fns, steps, warmup):
    """ms per step: windows of exactly `steps` steps of `fns`, each bracketed by a
    device synchronisation on both sides (wall clock), repeated until MIN_WINDOWS
    windows and TIMED_S seconds; median, min and max over the windows."""
    import torch

    warm_up(fns, warmup)
    per, t_all = [], 0.0
    while len(per) < MIN_WINDOWS or t_all < TIMED_S:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            for f in fns:
                f()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        t_all += dt
        per.append(dt * 1e3 / steps)
    return _stats(per)


def per_call(fn, calls, warmup=0):
    """ms per call of one op launched back to back: HIP events recorded on the
    current stream (the one the op launches on) around `calls` calls, over
    windows as in time_windows; median, min and max."""
    import torch

    warm_up([fn], warmup)
    per, t_all = [], 0.0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    while len(per) < MIN_WINDOWS or t_all < TIMED_S:
        e0.record()
        for _ in range(calls):
            fn()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1)
        t_all += ms * 1e-3
        per.append(ms / calls)
    return _stats(per)


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
    # Reference-API backward (two separate entry points) for comparison.
    bq = lambda: L.LaplaceSubtraction_backward_query(gd, qd, kd, dq)  # noqa: E731
    bk = lambda: L.LaplaceSubtraction_backward_key(gd, qd, kd, dk)  # noqa: E731
    step = time_windows([fwd, bwd], args.steps, args.warmup)
    calls = max(args.steps, 50)
    t_fwd, t_bwd = per_call(fwd, calls), per_call(bwd, calls)
    # The step itself by HIP events on its stream (the roofline's duration).
    t_step = per_call(lambda: (fwd(), bwd()), calls)
    ref_step = time_windows([fwd, bq, bk], args.steps, args.warmup)
    t_bq, t_bk = per_call(bq, calls), per_call(bk, calls)
    t_ref = per_call(lambda: (fwd(), bq(), bk()), calls)

    # Configuration 1's L1 part (q [2,2,196,32] fp32, key [2,2,32,49]): latency-bound, reported only.
    B1, H1, N1, M1, C1 = 2, 2, 196, 49, 32
    q1 = gen((B1, H1, N1, C1), 1001, torch.float32).to(dev)
    k1 = gen((B1, H1, M1, C1), 1011, torch.float32).transpose(-1, -2).contiguous().to(dev)
    g1 = gen((B1, H1, N1, M1), 1012, torch.float32).to(dev)
    o1, dq1, dk1 = torch.empty((B1, H1, N1, M1), device=dev), torch.empty_like(q1), torch.empty_like(k1)
    c1 = {"workload": "BASELINE config 1 L1: q [2,2,196,32] fp32, key [2,2,32,49]",
          "forward_ms": per_call(lambda: L.LaplaceSubtraction_forward(q1, k1, o1), calls, args.warmup),
          "backward_ms": per_call(lambda: L.LaplaceSubtraction_backward(g1, q1, k1, dq1, dk1), calls, args.warmup),
          "triples": B1 * H1 * N1 * M1 * C1}
    return {"T": B * H * N * M * C, "step": step, "fwd": t_fwd, "bwd": t_bwd, "step_ev": t_step,
            "ref_step": ref_step, "ref_step_ev": t_ref, "bq": t_bq, "bk": t_bk, "config1": c1,
            "inputs": (q, kT, g)}


def _newton_matrices(dev, nm, n, seed, scale):
    """exp(-L1(k_i, k_j) / scale) + 1e-3 I for nm sets of n points k ~ N(0,1), d = 64."""
    import torch

    import laplacianformer_amd as lf

    kk = gen((nm, 1, n, 64), seed, torch.float32).to(dev)
    dist = torch.empty((nm, 1, n, n), device=dev)
    lf.ext().LaplaceSubtraction_forward(kk, kk.transpose(-1, -2).contiguous(), dist)
    return (torch.exp(-dist / scale) + 1e-3 * torch.eye(n, device=dev)).contiguous()


def bench_newton(args, dev):
    import torch

    import laplacianformer_amd as lf

    L = lf.ext()
    nm, n, iters = 1024, 64, 12
    A = _newton_matrices(dev, nm, n, 1003, 8.0)
    G = gen((nm, 1, n, n), 1013, torch.float32).to(dev)
    V, dA = torch.empty_like(A), torch.empty_like(A)
    fwd = lambda: L.NewtonInverse_forward(A, V, iters)  # noqa: E731
    bwd = lambda: L.NewtonInverse_backward(G, V, dA)  # noqa: E731
    step = time_windows([fwd, bwd], args.steps, args.warmup)
    calls = max(args.steps, 50)
    t_fwd, t_bwd = per_call(fwd, calls), per_call(bwd, calls)
    P = A.double() + 0.01 * torch.eye(n, device=dev, dtype=torch.float64)
    resid = torch.linalg.matrix_norm(P @ V.double() - torch.eye(n, device=dev, dtype=torch.float64)).mean().item()
    # The same op at the configuration-1 (ViT stage 1) landmark shape: B*H = 32 Gram matrices
    # exp(-L1(k, k) / sqrt(d)) + 1e-3 I of 49 landmarks, d = 64, 10 iterations. One workgroup per
    # matrix occupies 32 of the chip's CUs, so the whole-chip MFMA fraction is bounded by 32/CUs;
    # the per-occupied-CU fraction is reported beside it.
    nm1, n1, it1 = 32, 49, 10
    A1 = _newton_matrices(dev, nm1, n1, 1021, 8.0)
    G1 = gen((nm1, 1, n1, n1), 1031, torch.float32).to(dev)
    V1, dA1 = torch.empty_like(A1), torch.empty_like(A1)
    f1 = lambda: L.NewtonInverse_forward(A1, V1, it1)  # noqa: E731
    b1 = lambda: L.NewtonInverse_backward(G1, V1, dA1)  # noqa: E731
    steps1 = max(args.steps, SECTION_REPS)
    step1 = time_windows([f1, b1], steps1, args.warmup)
    t1_fwd, t1_bwd = per_call(f1, max(calls, SECTION_REPS)), per_call(b1, max(calls, SECTION_REPS))
    P1 = A1.double() + 0.01 * torch.eye(n1, device=dev, dtype=torch.float64)
    resid1 = torch.linalg.matrix_norm(P1 @ V1.double() - torch.eye(n1, device=dev, dtype=torch.float64)).mean().item()
    stage1 = {"step": step1, "fwd": t1_fwd, "bwd": t1_bwd, "flops_fwd": nm1 * it1 * 4 * n1 ** 3,
              "flops_bwd": nm1 * 4 * n1 ** 3, "n_mats": nm1, "n": n1, "iters": it1, "residual_fro_mean": resid1,
              "steps": steps1}
    return {"step": step, "fwd": t_fwd, "bwd": t_bwd, "flops_fwd": nm * iters * 4 * n ** 3,
            "flops_bwd": nm * 4 * n ** 3, "residual_fro_mean": resid, "A": A.cpu(), "G": G.cpu(), "n_mats": nm,
            "n": n, "iters": iters, "stage1": stage1}


def layer_floors(B=64, H=2, N=784, M=49, d=64, iters=10):
    """Per-part lower bounds (us) of one config-5 layer step (fwd + bwd) on MI355X, from the
    algorithmic work at the published peaks: the three distances' VALU work (forward 3 and
    backward 8 flop per (row, landmark, channel) triple, fp32 vector 157.3 TFLOP/s);
    NewtonInverse (4 M^3 flop per iteration and 4 M^3 backward per matrix, fp32 MFMA 157.3
    TFLOP/s); the six N-row products and the pooling as HBM bytes at 8 TB/s (fp32 K_qm / K_km
    and their gradients [BH, N, M], fp16 q, k, v, out, grad [BH, N, d]). The products' flops
    (2 N M d each) run exactly on the bf16 matrix cores in well under their HBM time."""
    BH = B * H
    T = BH * (2 * N * M + M * M) * d
    kmat = BH * N * M * 4          # K_qm or K_km (or a gradient of one), fp32
    tok = BH * N * d * 2           # q, k, v, out or grad_out, fp16
    prod = 6 * (kmat + tok)        # K_km^T V, K_qm W; K_qm^T G, G W^T, K_km dkv, V dkv^T
    pool = 3 * tok                 # pooling reads k; its backward reads and writes grad_k
    parts = {
        "distances_valu": 11 * T / 157.3e12 * 1e6,
        "newton_mfma": BH * (iters + 1) * 4 * M ** 3 / 157.3e12 * 1e6,
        "products_hbm": prod / 8e12 * 1e6,
        "pooling_hbm": pool / 8e12 * 1e6,
    }
    return parts, {"triples": T, "product_bytes": prod, "pooling_bytes": pool}


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
        # Gradients set to None before each step (optimizer.zero_grad(set_to_none=True),
        # PyTorch's default), so that autograd writes them rather than adding to the last.
        q.grad = k.grad = v.grad = None
        out = lf.laplacian_attention(q, k, v, grid=(28, 28), pool=4, iters=10)
        out.backward(g)

    steps = max(SECTION_REPS, args.steps // 10)
    eager = time_windows([step], steps, args.warmup)
    # The same step captured once in a HIP graph (one launch per step instead of
    # ~40 host dispatches); gradients are overwritten, not accumulated, per replay.
    graphed = lf.GraphedStep(lambda a, b, c: lf.laplacian_attention(a, b, c, grid=(28, 28), pool=4, iters=10),
                             [q, k, v], g)
    graph = time_windows([graphed.replay], steps, args.warmup)
    T = B * H * (2 * N * 49 + 49 * 49) * d
    parts, work = layer_floors(B, H, N, 49, d, 10)
    floor_us = sum(parts.values())
    return {"workload": "BASELINE config 5: LaplacianFormer attention fwd+bwd, B=64 H=2 N=784 (28x28) d=64 "
                        "fp16, M=49 (4x4 pooled K), NewtonInverse 10 it",
            "ms_per_step": eager["median"], "ms_per_step_hip_graph": graph["median"], "eager": eager,
            "hip_graph": graph, "l1_triples": T, "steps_per_window": steps,
            "roofline": {"bound": "mixed (distances VALU, NewtonInverse MFMA, products and pooling HBM)",
                         "floor_us": floor_us, "parts_us": parts, "work": work,
                         "frac": floor_us / (eager["median"] * 1000.0),
                         "what": "sum of the parts' floors at MI355X peaks (157.3 TFLOP/s fp32 vector and "
                                 "MFMA, 8 TB/s) over the eager step"}}


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
    steps = max(SECTION_REPS, args.steps // 20)
    f = lambda: L.LaplaceSubtraction_forward(q, kT, out)  # noqa: E731
    b = lambda: L.LaplaceSubtraction_backward(g, q, kT, dq, dk)  # noqa: E731
    st = time_windows([f, b], steps, args.warmup)
    t_f, t_b = per_call(f, steps), per_call(b, steps)
    T = B * H * N * M * C
    n, nm, iters = 256, B * H, 16
    kk = gen((nm, n, 64), 1044, torch.float32)
    A = (torch.exp(-torch.cdist(kk, kk, p=1) / 8.0) + 1e-3 * torch.eye(n)).reshape(B, H, n, n).to(dev).contiguous()
    G = gen((B, H, n, n), 1045, torch.float32).to(dev)
    V, dA = torch.empty_like(A), torch.empty_like(A)
    nf = lambda: L.NewtonInverse_forward(A, V, iters)  # noqa: E731
    nb = lambda: L.NewtonInverse_backward(G, V, dA)  # noqa: E731
    st_n = time_windows([nf, nb], steps, args.warmup)
    tn_f, tn_b = per_call(nf, steps), per_call(nb, steps)
    fl_f, fl_b = nm * iters * 4 * n ** 3, nm * 4 * n ** 3
    wall, wall_n = st["median"], st_n["median"]
    return {"workload": "BASELINE config 4: LaplaceSubtraction fwd+bwd B=16 H=8 N=4096 M=256 d=64 bf16; "
                        "NewtonInverse 128 x 256x256 fp32, 16 it, fwd+bwd",
            "l1": {"ms_per_step": wall, "step": st, "value": T / (wall * 1e-3) / 1e9, "unit": "G(i*j*d)/s",
                   "fwd_ms": t_f, "bwd_ms": t_b,
                   "fwd_frac_fp32_peak": L1_FLOPS_FWD * T / (t_f["median"] * 1e-3) / 1e12 / PEAK_FP32_TFLOPS,
                   "bwd_frac_fp32_peak": L1_FLOPS_BWD * T / (t_b["median"] * 1e-3) / 1e12 / PEAK_FP32_TFLOPS},
            "newton": {"ms_per_step": wall_n, "step": st_n, "fwd_ms": tn_f, "bwd_ms": tn_b,
                       "tflops": (fl_f + fl_b) / (wall_n * 1e-3) / 1e12,
                       "frac_fp32_mfma_peak": (fl_f + fl_b) / (wall_n * 1e-3) / 1e12 / PEAK_FP32_TFLOPS},
            "steps_per_window": steps}


def bench_small_d(args, dev):
    """An output-write-bound small-d case: config 4's shape with d = 8 (B=16 H=8 N=4096 M=256,
    bf16): 2 flop-equivalents per triple against 2 bytes of output per (i, j), so HBM bytes,
    not VALU work, bound it. Reported as achieved GB/s against the 8 TB/s HBM peak."""
    import torch

    import laplacianformer_amd as lf

    L = lf.ext()
    B, H, N, M, C = 16, 8, 4096, 256, 8
    q = gen((B, H, N, C), 1051, torch.bfloat16).to(dev)
    k = gen((B, H, C, M), 1052, torch.bfloat16).to(dev)
    out = torch.empty((B, H, N, M), dtype=torch.bfloat16, device=dev)
    t = per_call(lambda: L.LaplaceSubtraction_forward(q, k, out), max(SECTION_REPS, args.steps // 10), args.warmup)
    nbytes = 2 * (q.numel() + k.numel() + out.numel())
    gbs = nbytes / (t["median"] * 1e-3) / 1e9
    return {"workload": "LaplaceSubtraction forward B=16 H=8 N=4096 M=256 d=8 bf16 (output-write-bound)",
            "ms": t, "bytes": nbytes, "gb_per_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS,
            "kernel": "laplace_fwd4_kernel<bf16s, 8, 4> (whole-line stores from registers)"}


def reference_figure(args, dev):
    """The reference's published comparison (README benchmark figure: each op against eager
    PyTorch on the same GPU at N = 16, 32, 64, 128, forward and backward), on this GPU.

    LaplaceSubtraction: B=32 H=1, N = M = n points, d = 64, fp32; eager equivalent
    torch.cdist(q, k, p=1) (k as [B,H,M,d]) and its autograd backward; ours the reference-API
    pair backward_query + backward_key and the fused backward. NewtonInverse: 1024 matrices
    n x n fp32 (the config-3 batch and construction), 12 iterations; eager equivalent the
    reference iteration as a torch.bmm loop (P = A + 0.01 I, V0 = 1.8 / max_i(sum_j P_ij)^2 P,
    V <- 2V - V(PV)); backward the reference's closed form -V^T G V^T as two bmm, and autograd
    through the loop. Times are medians of back-to-back calls (ms per call)."""
    import torch

    import laplacianformer_amd as lf

    L = lf.ext()
    calls = 20
    res = {"laplace": {}, "newton": {}}
    B, H, d = 32, 1, 64
    for n in (16, 32, 64, 128):
        q = gen((B, H, n, d), 1100 + n, torch.float32).to(dev)
        km = gen((B, H, n, d), 1200 + n, torch.float32).to(dev)     # [B,H,M,d] for cdist
        kT = km.transpose(-1, -2).contiguous()                       # [B,H,d,M] for the op
        g = gen((B, H, n, n), 1300 + n, torch.float32).to(dev)
        out, dq, dk = torch.empty((B, H, n, n), device=dev), torch.empty_like(q), torch.empty_like(kT)
        qa, ka = q.clone().requires_grad_(), km.clone().requires_grad_()
        dist = torch.cdist(qa, ka, p=1)
        L.LaplaceSubtraction_forward(q, kT, out)
        res["laplace"][str(n)] = {
            "ours_forward_ms": per_call(lambda: L.LaplaceSubtraction_forward(q, kT, out), calls)["median"],
            "ours_backward_ms": per_call(lambda: (L.LaplaceSubtraction_backward_query(g, q, kT, dq),
                                                  L.LaplaceSubtraction_backward_key(g, q, kT, dk)), calls)["median"],
            "ours_backward_fused_ms": per_call(lambda: L.LaplaceSubtraction_backward(g, q, kT, dq, dk),
                                               calls)["median"],
            "torch_forward_ms": per_call(lambda: torch.cdist(q, km, p=1), calls)["median"],
            "torch_backward_ms": per_call(lambda: dist.backward(g, retain_graph=True), calls)["median"],
            "max_abs_diff_forward": (out - dist.detach()).abs().max().item(),
        }
    nm, iters = 1024, 12
    for n in (16, 32, 64, 128):
        A = _newton_matrices(dev, nm, n, 1400 + n, 8.0)
        G = gen((nm, 1, n, n), 1500 + n, torch.float32).to(dev)
        V, dA = torch.empty_like(A), torch.empty_like(A)
        eye = torch.eye(n, device=dev)

        def torch_ns(Am):
            P = Am.reshape(nm, n, n) + 0.01 * eye
            alpha = 1.8 / P.sum(-1).max(-1).values ** 2
            X = alpha[:, None, None] * P
            for _ in range(iters):
                X = 2 * X - torch.bmm(X, torch.bmm(P, X))
            return X

        def torch_ns_bwd(X):
            Xt = X.transpose(1, 2).contiguous()
            return -torch.bmm(torch.bmm(Xt, G.reshape(nm, n, n)), Xt)

        Aa = A.clone().requires_grad_()
        Xa = torch_ns(Aa)
        X = Xa.detach()
        L.NewtonInverse_forward(A, V, iters)
        res["newton"][str(n)] = {
            "ours_forward_ms": per_call(lambda: L.NewtonInverse_forward(A, V, iters), calls)["median"],
            "ours_backward_ms": per_call(lambda: L.NewtonInverse_backward(G, V, dA), calls)["median"],
            "torch_forward_ms": per_call(lambda: torch_ns(A), calls)["median"],
            "torch_backward_closed_form_ms": per_call(lambda: torch_ns_bwd(X), calls)["median"],
            "torch_backward_autograd_ms": per_call(lambda: Xa.backward(G.reshape(nm, n, n), retain_graph=True),
                                                   calls)["median"],
            "max_abs_diff_forward": (V.reshape(nm, n, n) - X).abs().max().item(),
        }
    res["shapes"] = ("laplace: B=32 H=1 N=M=n d=64 fp32; newton: 1024 matrices n x n fp32 "
                     "(exp(-L1(k_i,k_j)/8) + 1e-3 I, k ~ N(0,1) d=64), 12 iterations")
    return res


def cpu_baseline(lap, ns, budget):
    """PyTorch CPU torch.cdist(p=1) fwd+bwd on a sample of config 2 (the north-star's pure-PyTorch
    equivalent; the headline value), plus the C oracle (OpenMP) and the bmm Newton loop."""
    import torch

    import oracle

    torch.set_num_threads(os.cpu_count() or 1)
    q, kT, g = lap["inputs"]
    threads = oracle.max_threads()
    # PyTorch CPU: cdist p=1 on [B,H,M,d] keys, fp32 (CPU cdist rejects fp16), forward + autograd backward.
    qf = q.float().requires_grad_()
    kf = kT.float().transpose(-1, -2).contiguous().requires_grad_()
    gf = g.float()
    t_cd, reps_cd = 0.0, 0
    while t_cd < budget / 3 or reps_cd == 0:
        t0 = time.perf_counter()
        d = torch.cdist(qf, kf, p=1)
        d.backward(gf)
        t_cd += time.perf_counter() - t0
        reps_cd += 1
    cd_rate = lap["T"] * reps_cd / t_cd / 1e9

    # C oracle: whole config-2 steps (fwd + dq + dk over all slices).
    t_used, reps = 0.0, 0
    while t_used < budget / 3 or reps == 0:
        t0 = time.perf_counter()
        oracle.laplace_forward(q, kT, "f16")
        oracle.laplace_backward_query(g, q, kT, "f16")
        oracle.laplace_backward_key(g, q, kT, "f16")
        t_used += time.perf_counter() - t0
        reps += 1
    port_rate = lap["T"] * reps / t_used / 1e9

    # Newton: bmm loop with the reference init on a sample of matrices.
    A = ns["A"].double()
    nmat = min(A.shape[0], 256)
    Ab = A[:nmat, 0].float()
    n = Ab.shape[-1]
    Gb = ns["G"][:nmat, 0]
    t_ns, reps_ns = 0.0, 0
    while t_ns < budget / 3 or reps_ns == 0:
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
        "value": cd_rate, "unit": "G(i*j*d)/s", "cores": torch.get_num_threads(), "kind": "port",
        "sample": f"torch.cdist(p=1) fp32 forward + autograd backward on the whole config-2 step "
                  f"(32 (b,h) slices, N=3136, M=49, d=64) x {reps_cd}, {t_cd:.2f} s, "
                  f"{torch.get_num_threads()} threads",
        "c_oracle": {"value": port_rate, "unit": "G(i*j*d)/s", "threads": threads,
                     "sample": f"C oracle (oracle/laplace_oracle.c) on the whole config-2 step (fwd + dq + dk, "
                               f"fp32 accumulation in the reference's serial order) x {reps}, {t_used:.2f} s"},
        "torch_cpu_newton": {"value": ns_flops / t_ns / 1e12, "unit": "TFLOP/s", "threads": torch.get_num_threads(),
                             "sample": f"bmm Newton-Schulz fwd (12 it) + closed-form bwd, {nmat} of 1024 config-3 "
                                       f"matrices x {reps_ns}, {t_ns:.2f} s"},
        "host": {"cpu_count": os.cpu_count(), "cpu_model": _cpu_model()},
    }


def _profile_table(name):
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def _traffic(*kernels):
    """HBM bytes of one call made of the named kernel launches (names as rocprofv3 prints them,
    without the argument list), from the committed counter summary (profiles/hbm_traffic.json,
    FETCH_SIZE/WRITE_SIZE scaled by a plain-copy calibration); None if any is missing."""
    data = _profile_table("hbm_traffic.json")
    if not data:
        return None
    table = data.get("kernels", {})
    if not all(k in table for k in kernels):
        return None
    rd = sum(table[k]["read_bytes"] for k in kernels)
    wr = sum(table[k]["write_bytes"] for k in kernels)
    return {"bytes": rd + wr, "read_bytes": rd, "write_bytes": wr, "kernels": list(kernels),
            "source": data.get("source")}


def _counters(*kernels):
    """Per-dispatch SQ/GRBM counter summaries of the named kernels (profiles/laplace_newton_counters.json)."""
    data = _profile_table("laplace_newton_counters.json")
    if not data:
        return None
    table = data.get("kernels", {})
    got = {k: table[k] for k in kernels if k in table}
    return {"kernels": got, "source": data.get("source")} if got else None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


K_FWD = "lfamd::(anonymous namespace)::laplace_fwd2_kernel<lfamd::f16s, 0, 16>"
K_BWD = "lfamd::(anonymous namespace)::laplace_bwd2_kernel<lfamd::f16s, 49, true, true, false>"
K_RED = "lfamd::(anonymous namespace)::laplace_dk_reduce_t_kernel<lfamd::f16s>"
K_NF = "lfamd::newton_fwd_kernel<float, 64, true, 2, 4>"
K_NB = "lfamd::newton_bwd_pipe_kernel<float, 64>"


def _ms(st):
    return {k: st[k] for k in ("median", "min", "max", "windows")}


def main():
    global WARM_S, TIMED_S, MIN_WINDOWS
    args = parse()
    if args.profile_run:
        WARM_S, TIMED_S, MIN_WINDOWS = 0.0, 0.0, 1
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
    fig = reference_figure(args, dev) if args.only in ("figure", "all") else None
    small_d = bench_small_d(args, dev) if args.only in ("figure", "all") else None

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic"}
    if lap:
        T = lap["T"]
        B_, N_, M_, C_ = 32, 3136, 49, 64
        wall = lap["step"]["median"]
        t_fwd, t_bwd = lap["fwd"]["median"], lap["bwd"]["median"]
        value = T / (wall * 1e-3) / 1e9
        bwd_tflops = L1_FLOPS_BWD * T / (t_bwd * 1e-3) / 1e12
        fwd_tflops = L1_FLOPS_FWD * T / (t_fwd * 1e-3) / 1e12
        step_tflops = (L1_FLOPS_FWD + L1_FLOPS_BWD) * T / (wall * 1e-3) / 1e12
        t_step = lap["step_ev"]["median"]
        step_ev_tflops = (L1_FLOPS_FWD + L1_FLOPS_BWD) * T / (t_step * 1e-3) / 1e12
        ref_wall = lap["ref_step"]["median"]
        t_ref = lap["ref_step_ev"]["median"]
        ref_tflops = (L1_FLOPS_FWD + L1_FLOPS_BWD) * T / (t_ref * 1e-3) / 1e12
        fwd_bytes = 2 * (B_ * N_ * C_ + B_ * C_ * M_ + B_ * N_ * M_)
        bwd_bytes = 2 * (B_ * N_ * M_ + 2 * B_ * N_ * C_ + 2 * B_ * C_ * M_)
        line.update({
            "value": value, "unit": "G(i*j*d)/s", "ms_per_step": wall,
            "timing": {"step_ms": _ms(lap["step"]),
                       "method": f"windows of exactly --steps steps, each bracketed by torch.cuda.synchronize(), "
                                 f"after >= --warmup steps and >= {WARM_S} s of warm-up; median (min, max) over "
                                 f">= {MIN_WINDOWS} windows and >= {TIMED_S} s"},
            "config": {"workload": "BASELINE config 2: LaplaceSubtraction forward + fused backward (dq, dk), "
                                   "B=32 H=1 N=3136 M=49 d=64", "storage": "f16", "accumulate": "f32",
                       "global_batch": 32, "seq_len": 3136, "landmarks": 49, "channels": 64},
            "roofline": {"bound": "valu",
                         "kernel": "the config-2 step: laplace_fwd2_kernel<f16s,0,16>, then "
                                   "laplace_bwd2_kernel<f16s,49,true,true,false> + laplace_dk_reduce_t_kernel<f16s> "
                                   "(HIP events on their stream around back-to-back steps; fp32 vector peak)",
                         "achieved": step_ev_tflops, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                         "frac": step_ev_tflops / PEAK_FP32_TFLOPS,
                         "ms": t_step, "ms_range": _ms(lap["step_ev"]),
                         "traffic": _traffic(K_FWD, K_BWD, K_RED),
                         "algorithmic_bytes": fwd_bytes + bwd_bytes,
                         "work": f"{L1_FLOPS_FWD + L1_FLOPS_BWD} flop per (i,j,d) triple (forward "
                                 f"{L1_FLOPS_FWD}, grad_query 4, grad_key 4) x {T} triples per step",
                         "parts": {
                             "forward": {"kernels": ["laplace_fwd2_kernel<f16s,0,16>"], "ms": t_fwd,
                                         "tflops": fwd_tflops, "frac": fwd_tflops / PEAK_FP32_TFLOPS,
                                         "traffic": _traffic(K_FWD), "algorithmic_bytes": fwd_bytes},
                             "backward_op": {"kernels": ["laplace_bwd2_kernel<f16s,49,true,true,false>",
                                                         "laplace_dk_reduce_t_kernel<f16s>"],
                                             "ms": t_bwd, "tflops": bwd_tflops, "frac": bwd_tflops / PEAK_FP32_TFLOPS,
                                             "traffic": _traffic(K_BWD, K_RED), "algorithmic_bytes": bwd_bytes},
                             "reference_api_step": {"entry_points": ["LaplaceSubtraction_forward",
                                                                     "LaplaceSubtraction_backward_query",
                                                                     "LaplaceSubtraction_backward_key"],
                                                    "ms": t_ref, "tflops": ref_tflops,
                                                    "frac": ref_tflops / PEAK_FP32_TFLOPS}},
                         "counters": _counters(K_BWD, K_RED, K_FWD)},
            "kernels": {
                "forward (laplace_fwd2_kernel<f16s,0,16>)": {
                    "ms": t_fwd, "ms_range": _ms(lap["fwd"]), "tflops": fwd_tflops,
                    "frac_fp32_peak": fwd_tflops / PEAK_FP32_TFLOPS, "traffic": _traffic(K_FWD)},
                "backward (laplace_bwd2_kernel<f16s,49,dq,dk> + laplace_dk_reduce_t_kernel)": {
                    "ms": t_bwd, "ms_range": _ms(lap["bwd"]), "tflops": bwd_tflops,
                    "frac_fp32_peak": bwd_tflops / PEAK_FP32_TFLOPS},
                # frac_fp32_peak is the roofline's figure (HIP events on the kernels' stream);
                # the wall-clock step (ms_per_step) gives frac_fp32_peak_wall.
                "step_fwd_bwd": {"ms": t_step, "tflops": step_ev_tflops,
                                 "frac_fp32_peak": step_ev_tflops / PEAK_FP32_TFLOPS,
                                 "ms_wall": wall, "frac_fp32_peak_wall": step_tflops / PEAK_FP32_TFLOPS},
                "reference_api_step": {"ms": ref_wall, "ms_range": _ms(lap["ref_step"]), "ms_hip_events": t_ref,
                                       "frac_fp32_peak_hip_events": ref_tflops / PEAK_FP32_TFLOPS,
                                       "backward_query_ms": lap["bq"]["median"],
                                       "backward_key_ms": lap["bk"]["median"],
                                       "g_triples_per_s": T / (ref_wall * 1e-3) / 1e9},
            },
            "config1_l1": {**lap["config1"], "forward_ms": _ms(lap["config1"]["forward_ms"]),
                           "backward_ms": _ms(lap["config1"]["backward_ms"])},
        })
    if ns:
        wall_n = ns["step"]["median"]
        tf_f = ns["flops_fwd"] / (ns["fwd"]["median"] * 1e-3) / 1e12
        tf_b = ns["flops_bwd"] / (ns["bwd"]["median"] * 1e-3) / 1e12
        tf = (ns["flops_fwd"] + ns["flops_bwd"]) / (wall_n * 1e-3) / 1e12
        line["newton"] = {
            "workload": "BASELINE config 3: NewtonInverse fwd (12 it) + bwd, 1024 x 64x64 fp32",
            "tflops": tf, "ms_per_step": wall_n, "step_ms": _ms(ns["step"]),
            "frac_fp32_mfma_peak": tf / PEAK_FP32_TFLOPS,
            "fwd": {"ms": ns["fwd"]["median"], "ms_range": _ms(ns["fwd"]), "tflops": tf_f,
                    "frac": tf_f / PEAK_FP32_TFLOPS, "traffic": _traffic(K_NF)},
            "bwd": {"ms": ns["bwd"]["median"], "ms_range": _ms(ns["bwd"]), "tflops": tf_b,
                    "frac": tf_b / PEAK_FP32_TFLOPS, "traffic": _traffic(K_NB)},
            "counters": _counters(K_NF, K_NB),
            "residual_fro_mean": ns["residual_fro_mean"],
        }
        s1 = ns["stage1"]
        w1 = s1["step"]["median"]
        tf1 = (s1["flops_fwd"] + s1["flops_bwd"]) / (w1 * 1e-3) / 1e12
        cus = props.multi_processor_count
        line["newton"]["stage1"] = {
            "workload": "BASELINE config 1 landmark shape: NewtonInverse fwd (10 it) + bwd, 32 x 49x49 fp32 "
                        "(one workgroup per matrix: 32 CUs occupied)",
            "ms_per_step": w1, "step_ms": _ms(s1["step"]), "fwd_ms": s1["fwd"]["median"],
            "bwd_ms": s1["bwd"]["median"], "tflops": tf1, "steps_per_window": s1["steps"],
            "frac_fp32_mfma_peak": tf1 / PEAK_FP32_TFLOPS,
            "frac_per_occupied_cu": tf1 / (PEAK_FP32_TFLOPS * s1["n_mats"] / cus),
            "flops": "4 n^3 per iteration + 4 n^3 backward, n = 49 (algorithmic; the kernels pad to 64)",
            "residual_fro_mean": s1["residual_fro_mean"],
        }
        if not lap:
            line.update({"value": tf, "unit": "TFLOP/s", "ms_per_step": wall_n,
                         "config": {"workload": line["newton"]["workload"]}})
    if layer:
        line["layer"] = layer
    if cfg4:
        line["config4"] = cfg4
    if fig:
        line["reference_figure"] = fig
    if small_d:
        line["small_d"] = small_d
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

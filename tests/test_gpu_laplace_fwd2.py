"""GPU parity of the row-staged M = 49 forward (laplace_fwd2.hip) across its work plans.

Each shape is chosen (for 256 CUs) to reach one plan of the kernel: 16 waves with
runs of 1-3 row sets and a tail wave, 16 waves with workgroups one row apart (the
tail length differs between them, 0 to 9 rows), and 8 waves with 7-set runs (full
and partial last set), at C from 8 to 64. The distance must be bit-identical to the
fp32 serial oracle (the kernel sums the channels in the reference's order); the
fused exp(-s * distance) variant is held to the fp32 rounding of s * d and expf.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from lfcheck import assert_bitwise, gen

pytestmark = pytest.mark.gpu

# (B, H, N, M, C, what)
SHAPES = [
    (1, 64, 272, 49, 64, "16 waves, 1 set + 4-row tail"),
    (1, 16, 2176, 49, 32, "16 waves, 2 sets + 8-row tail"),
    (1, 8, 5120, 49, 64, "16 waves, 3 sets (last partial)"),
    (4, 32, 784, 49, 64, "16 waves, 6 sets + 8-row tail (config-5 layer shape)"),
    (32, 1, 3141, 49, 64, "16 waves, 6 sets + 8/9-row tails (workgroups one row apart)"),
    (1, 8, 13440, 49, 40, "8 waves, 7 sets (last partial)"),
    (1, 8, 14336, 49, 8, "8 waves, 7 full sets"),
    (32, 1, 3073, 49, 64, "16 waves, 6 sets + 0/1-row tails"),
    (8, 5, 1200, 49, 16, "16 waves, 3 sets + 8-row tail, C = 16"),
    (1, 256, 420, 49, 64, "one workgroup per slice, 7 sets (last partial)"),
    (2, 3, 1000, 49, 64, "one partial set per workgroup"),
    (1, 16, 2176, 49, 64, "2 sets + 8-row tail, C = 64"),
]


def _ids(s):
    return "x".join(map(str, s[:5]))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_fwd2_plans(gpu, shape, dt):
    import laplacianformer_amd as lf

    B, H, N, M, C, what = shape
    print(f"fwd2 {shape[:5]} {dt}: {what}", flush=True)
    q = gen((B, H, N, C), 500 + N, dt)
    k = gen((B, H, C, M), 501 + N, dt)
    L = lf.ext()
    out = torch.empty((B, H, N, M), dtype=q.dtype, device=gpu)
    L.LaplaceSubtraction_forward(q.to(gpu), k.to(gpu), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.laplace_forward(q, k, dt), dt, f"forward bits ({what})")


# The wide-landmark forward (M in {128, 256}): whole and partial 192-row
# workgroups, one-row slices, C = 8 to 64, the config-4 shape on two slices; for
# C in {8, 16} the line-coalesced small-d kernel (whole and partial 256-row
# workgroups, both landmark counts, the small-d benchmark shape on two slices).
WIDE = [
    (1, 2, 700, 128, 64),
    (2, 1, 192, 256, 64),
    (1, 1, 1, 256, 8),
    (1, 3, 385, 256, 40),
    (1, 2, 4096, 256, 64),
    (2, 3, 500, 128, 16),
    (1, 4, 1000, 256, 8),
    (1, 2, 4096, 256, 8),
    (3, 1, 700, 128, 8),
    (1, 2, 513, 256, 16),
]


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", WIDE, ids=lambda s: "x".join(map(str, s)))
def test_fwd3_wide(gpu, shape, dt):
    import laplacianformer_amd as lf

    B, H, N, M, C = shape
    print(f"fwd3 {shape} {dt}", flush=True)
    q = gen((B, H, N, C), 700 + N, dt)
    k = gen((B, H, C, M), 701 + N, dt)
    out = torch.empty((B, H, N, M), dtype=q.dtype, device=gpu)
    lf.ext().LaplaceSubtraction_forward(q.to(gpu), k.to(gpu), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.laplace_forward(q, k, dt), dt, f"forward bits {shape}")


@pytest.mark.parametrize("shape", [SHAPES[1], SHAPES[4], SHAPES[5]], ids=_ids)
def test_fwd2_kernel_epilogue(gpu, shape):
    """The fused exp(-s * d) output of the same kernel, fp16 inputs."""
    import laplacianformer_amd as lf

    B, H, N, M, C, what = shape
    print(f"fwd2 exp {shape[:5]}: {what}", flush=True)
    q = gen((B, H, N, C), 600 + N, "f16")
    k = gen((B, H, C, M), 601 + N, "f16")
    s = 1.0 / math.sqrt(C)
    out = torch.empty((B, H, N, M), dtype=torch.float32, device=gpu)
    assert lf.ext().LaplaceKernel_forward(q.to(gpu), k.to(gpu), out, s) is True
    d32 = oracle.laplace_forward(q, k, "f32").astype(np.float64)
    ref = np.exp(-s * d32)
    got = out.cpu().double().numpy()
    lim = ref * (2.0 ** -21) * (1.0 + s * d32) + 1e-38
    assert not (np.abs(got - ref) > lim).any(), what


def test_fwd2_plan_cache_rotation(gpu):
    """Host plan cache (eight shapes per thread): ten shapes with different plans, called in
    turn three times (each call past the eighth evicts one), every result bit-identical to
    the oracle, so a stale or mismatched plan cannot go unnoticed."""
    import laplacianformer_amd as lf

    L = lf.ext()
    shapes = [(1, 4, n, 49, 64) for n in (1, 17, 64, 65, 130, 200, 272, 300, 392, 448)]
    data = []
    for i, (B, H, N, M, C) in enumerate(shapes):
        q = gen((B, H, N, C), 900 + i, "f16")
        k = gen((B, H, C, M), 950 + i, "f16")
        data.append((q, k, q.to(gpu), k.to(gpu), oracle.laplace_forward(q, k, "f16")))
    for rnd in range(3):
        print(f"fwd2 plan cache round {rnd}", flush=True)
        for (q, k, qd, kd, ref), shape in zip(data, shapes):
            out = torch.empty(shape[:3] + (shape[3],), dtype=torch.float16, device=gpu)
            L.LaplaceSubtraction_forward(qd, kd, out)
            torch.cuda.synchronize()
            assert_bitwise(out, ref, "f16", f"forward bits {shape} round {rnd}")


# The row-staged kernel copies each workgroup's span of outputs out of LDS in
# 16-byte vectors when the span is 16-byte aligned, in 4-byte words when it is
# 4-byte aligned, element by element otherwise, and reads the key element-wise;
# outputs and keys at odd element offsets must match the serial oracle bit for bit.
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("offset", [(1, 0), (0, 1), (3, 5)], ids=lambda o: f"out{o[0]}_key{o[1]}")
def test_fwd2_unaligned(gpu, dt, offset):
    import laplacianformer_amd as lf

    B, H, N, M, C = 32, 1, 3136, 49, 64
    oo, ko = offset
    print(f"fwd2 unaligned {dt} out+{oo} key+{ko}", flush=True)
    q = gen((B, H, N, C), 777, dt)
    k = gen((B, H, C, M), 778, dt)
    kbuf = torch.zeros(B * H * C * M + ko, dtype=k.dtype, device=gpu)
    kd = kbuf[ko:].view(B, H, C, M)
    kd.copy_(k.to(gpu))
    obuf = torch.zeros(B * H * N * M + oo, dtype=q.dtype, device=gpu)
    out = obuf[oo:].view(B, H, N, M)
    lf.ext().LaplaceSubtraction_forward(q.to(gpu), kd, out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.laplace_forward(q, k, dt), dt, f"forward bits (out +{oo}, key +{ko})")

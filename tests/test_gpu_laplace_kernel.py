"""Fused Laplacian kernel K = exp(-s * L1(q, key)) and its backward (the attention
layer's caller-side op, exp fused into the HIP distance kernels), against the
oracle composition: K = exp(-s * dist) with dist the fp32 serial oracle (which the
distance kernels match bit for bit), g = -s * gK * K, and dq / dk from the fp64 L1
oracle for that g."""
import math

import numpy as np
import pytest
import torch

import oracle
from lfcheck import assert_l1_close, gen

pytestmark = pytest.mark.gpu

# (B, H, N, M, C): fused-forward shapes (C % 8 == 0, M <= 256), incl. one-row and tail cases.
FWD_SHAPES = [
    (2, 2, 196, 49, 32),
    (1, 1, 1, 1, 8),
    (1, 3, 130, 64, 64),
    (2, 1, 65, 16, 16),
    (1, 2, 100, 100, 40),
    (1, 1, 129, 128, 64),
    (2, 1, 3136, 49, 64),
    (1, 1, 129, 256, 64),   # fp32 output tiles of all 256 columns exceed the LDS: two column groups
    (2, 1, 70, 240, 64),    # column groups of 128 and 112
]
# Fused-backward shapes: fp16, M in {16, 32, 49} (register-resident columns) and other
# 17 <= M <= 256 (column blocks, partial last block included); odd N * M and single rows.
BWD_SHAPES = [
    (2, 2, 196, 49, 32),
    (1, 1, 1, 49, 64),
    (1, 1, 7, 49, 64),
    (1, 2, 131, 16, 80),
    (2, 1, 200, 32, 64),
    (1, 1, 97, 32, 130),
    (2, 1, 3136, 49, 64),
    (32, 1, 4096, 49, 64),  # 512 rows per workgroup: the 12-wave kernel's largest wave row counts
    (1, 2, 150, 64, 64),
    (1, 1, 77, 81, 40),
    (2, 1, 130, 196, 64),
]


def _kernel_ref(q, k, dt, s):
    """fp64 exp(-s * dist32) with dist32 the fp32 serial-order oracle distance."""
    d32 = oracle.laplace_forward(q, k, "f64" if dt == "f64" else "f32").astype(np.float64)
    return np.exp(-s * d32), d32


def _check_kernel(got, ref, d32, s, what):
    """|K - exp(-s d)| <= K 2^-21 (1 + s d): fp32 s, the fp32 product s*d and expf, nothing else."""
    g = got.detach().cpu().double().numpy()
    assert np.isfinite(g).all(), what
    lim = ref * (2.0 ** -21) * (1.0 + s * d32) + 1e-38
    bad = np.abs(g - ref) > lim
    assert not bad.any(), (what, int(bad.sum()), float((np.abs(g - ref) / np.maximum(ref, 1e-300)).max()))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", FWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_kernel_forward(gpu, shape, dt):
    import laplacianformer_amd as lf

    B, H, N, M, C = shape
    print(f"laplace kernel forward {shape} {dt}", flush=True)
    q = gen((B, H, N, C), 300 + N + M, dt)
    k = gen((B, H, C, M), 301 + N + M, dt)
    s = 1.0 / math.sqrt(C)
    out = torch.empty((B, H, N, M), dtype=torch.float32, device=gpu)
    assert lf.ext().LaplaceKernel_forward(q.to(gpu), k.to(gpu), out, s) is True
    ref, d32 = _kernel_ref(q, k, dt, s)
    _check_kernel(out, ref, d32, s, "K")


@pytest.mark.parametrize("shape", BWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_kernel_backward_f16(gpu, shape):
    import laplacianformer_amd as lf

    B, H, N, M, C = shape
    print(f"laplace kernel backward {shape}", flush=True)
    q = gen((B, H, N, C), 400 + N + M, "f16")
    k = gen((B, H, C, M), 401 + N + M, "f16")
    gk = gen((B, H, N, M), 402 + N + M, "f32")
    s = 1.0 / math.sqrt(C)
    # K at the scale of the layer's kernels: exp of minus a few units (nonzero everywhere).
    kern = torch.exp(-torch.rand((B, H, N, M), generator=torch.Generator().manual_seed(N), dtype=torch.float32) * 4)
    qd, kd, gkd, kernd = q.to(gpu), k.to(gpu), gk.to(gpu), kern.to(gpu)
    L = lf.ext()
    dq, dk = torch.empty_like(qd), torch.empty_like(kd)
    assert L.LaplaceKernel_backward(gkd, kernd, qd, kd, dq, dk, s) is True
    dq1, dk1 = torch.empty_like(qd), torch.empty_like(kd)
    assert L.LaplaceKernel_backward(gkd, kernd, qd, kd, dq1, None, s) is True
    assert L.LaplaceKernel_backward(gkd, kernd, qd, kd, None, dk1, s) is True
    torch.cuda.synchronize()
    g64 = -s * gk.double().numpy() * kern.double().numpy()
    rq = oracle.laplace_backward_query(g64, q, k, "f64")
    rk = oracle.laplace_backward_key(g64, q, k, "f64")
    ga = np.abs(g64)
    assert_l1_close(dq, rq, "f16", "dq", np.broadcast_to(ga.sum(axis=3, keepdims=True), rq.shape))
    assert_l1_close(dk, rk, "f16", "dk", np.broadcast_to(ga.sum(axis=2, keepdims=True), rk.shape))
    assert torch.equal(dq.cpu(), dq1.cpu()), "grad_query differs between the fused and query-only calls"
    assert torch.equal(dk.cpu(), dk1.cpu()), "grad_key differs between the fused and key-only calls"


def test_kernel_unsupported_reports_false(gpu):
    """Outside the fused paths the exports return False and leave the outputs alone."""
    import laplacianformer_amd as lf

    L = lf.ext()
    q = gen((1, 1, 10, 12), 1, "f32").to(gpu)  # C % 8 != 0
    k = gen((1, 1, 12, 5), 2, "f32").to(gpu)
    out = torch.full((1, 1, 10, 5), 7.0, device=gpu)
    assert L.LaplaceKernel_forward(q, k, out, 0.5) is False
    assert bool((out == 7.0).all())
    q2 = gen((1, 1, 10, 16), 3, "f32").to(gpu)
    k2 = gen((1, 1, 16, 49), 4, "f32").to(gpu)
    kern = torch.rand((1, 1, 10, 49), device=gpu)
    dq = torch.full_like(q2, 7.0)
    assert L.LaplaceKernel_backward(kern, kern, q2, k2, dq, None, 0.5) is False  # fp32: no fused backward
    assert bool((dq == 7.0).all())
    # M = 8: below both fused backward paths.
    q5 = gen((1, 1, 10, 16), 9, "f16").to(gpu)
    k5 = gen((1, 1, 16, 8), 10, "f16").to(gpu)
    kern5 = torch.rand((1, 1, 10, 8), device=gpu)
    assert L.LaplaceKernel_backward(kern5, kern5, q5, k5, torch.empty_like(q5), None, 0.5) is False
    # M = 257: beyond the broadcast forward's 256 columns.
    q4 = gen((1, 1, 129, 64), 7, "f16").to(gpu)
    k4 = gen((1, 1, 64, 257), 8, "f16").to(gpu)
    assert L.LaplaceKernel_forward(q4, k4, torch.empty((1, 1, 129, 257), device=gpu), 0.5) is False
    with pytest.raises(RuntimeError):
        L.LaplaceKernel_forward(q2, k2, torch.empty((1, 1, 10, 49), dtype=torch.float16, device=gpu), 0.5)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_kernel_autograd(gpu, dt):
    """LaplaceKernelFunction through autograd (fused where it applies, composed
    elsewhere) against the oracle composition."""
    import laplacianformer_amd as lf

    B, H, N, M, C = 2, 1, 150, 49, 64
    print(f"laplace kernel autograd {dt}", flush=True)
    q = gen((B, H, N, C), 500, dt)
    k = gen((B, H, C, M), 501, dt)
    gk = gen((B, H, N, M), 502, "f32")
    s = 1.0 / math.sqrt(C)
    qd, kd = q.to(gpu).requires_grad_(), k.to(gpu).requires_grad_()
    K = lf.laplace_kernel(qd, kd, s)
    assert K.dtype == torch.float32
    K.backward(gk.to(gpu))
    ref, d32 = _kernel_ref(q, k, dt, s)
    _check_kernel(K, ref, d32, s, "K")
    g64 = -s * gk.double().numpy() * K.detach().cpu().double().numpy()
    rq = oracle.laplace_backward_query(g64, q, k, "f64")
    rk = oracle.laplace_backward_key(g64, q, k, "f64")
    ga = np.abs(g64)
    assert_l1_close(qd.grad, rq, dt, "dq", np.broadcast_to(ga.sum(axis=3, keepdims=True), rq.shape))
    assert_l1_close(kd.grad, rk, dt, "dk", np.broadcast_to(ga.sum(axis=2, keepdims=True), rk.shape))


def test_kernel_gradcheck_f64(gpu):
    """fp64 (the composed path): torch.autograd.gradcheck of exp(-s * L1)."""
    import laplacianformer_amd as lf

    torch.manual_seed(3)
    q = torch.randn(1, 2, 5, 3, dtype=torch.float64, device=gpu, requires_grad=True)
    k = torch.randn(1, 2, 3, 4, dtype=torch.float64, device=gpu, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: lf.laplace_kernel(a, b, 0.7), (q, k), eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("lens,bh", [((784, 784, 49), (2, 2)), ((65, 1, 200), (2, 2)), ((130, 7), (2, 2)),
                                     ((49, 784, 784), (16, 2)), ((65, 1, 200), (16, 2)), ((784, 784, 49), (16, 2))],
                         ids=lambda s: "-".join(map(str, s)))
def test_kernel_backward_multi(gpu, lens, bh):
    """lfamd_laplace_kernel_backward_multi: up to three row sources against one key in one launch.
    Each source's grad_query is bit-identical to its own lfamd_laplace_kernel_backward call (a
    row's grad_query does not depend on the workgroup or wave that takes it); grad_key, the sum
    over the sources, is held to the oracle's fp64 sum with the usual bound. With 4 slices each
    source takes workgroups of its own; with 32 slices (at most 8 workgroups per slice) the
    slice's rows are cut into equal workgroup ranges across the sources, waves keeping to one
    source (a 1-row source, a range starting inside K_mm's 49 rows, and sources in both orders)."""
    import ctypes

    import laplacianformer_amd as lf

    (B, H), M, C = bh, 49, 64
    print(f"laplace kernel backward multi {lens} B={B} H={H}", flush=True)
    lib = lf.capi()
    s = 1.0 / math.sqrt(C)
    k = gen((B, H, C, M), 831, "f16")
    srcs = []
    for i, n in enumerate(lens):
        q = gen((B, H, n, C), 840 + i, "f16")
        gk = gen((B, H, n, M), 850 + i, "f32")
        kern = torch.exp(-torch.rand((B, H, n, M), generator=torch.Generator().manual_seed(860 + i)) * 4)
        srcs.append((q, gk, kern))
    kd = k.to(gpu)
    qd = [q.to(gpu) for q, _, _ in srcs]
    gkd = [gk.to(gpu) for _, gk, _ in srcs]
    kvd = [kv.to(gpu) for _, _, kv in srcs]
    dqs = [torch.empty_like(q) for q in qd]
    dk = torch.empty_like(kd)
    ns = len(lens)
    nl = (ctypes.c_int64 * ns)(*lens)
    P = lambda ts: (ctypes.c_void_p * ns)(*[t.data_ptr() for t in ts])  # noqa: E731
    wsb = lib.lfamd_laplace_kernel_backward_multi_workspace_size(1, ns, nl, B, H, M, C)
    assert wsb > 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    lf.check(lib.lfamd_laplace_kernel_backward_multi(lf.dtype_code(kd), ns, P(gkd), P(kvd), P(qd), nl, kd.data_ptr(),
                                                      P(dqs), dk.data_ptr(), B, H, M, C, ctypes.c_float(s),
                                                      ws.data_ptr(), wsb, stream))
    L = lf.ext()
    rk = 0.0
    scale = 0.0
    for (q, gk, kern), q1, g1, kv1, dq in zip(srcs, qd, gkd, kvd, dqs):
        ref_dq = torch.empty_like(q1)
        assert L.LaplaceKernel_backward(g1, kv1, q1, kd, ref_dq, None, s) is True
        torch.cuda.synchronize()
        assert torch.equal(dq, ref_dq), "grad_query differs from the single-source call"
        g64 = -s * gk.double().numpy() * kern.double().numpy()
        rk = rk + oracle.laplace_backward_key(g64, q, k, "f64")
        scale = scale + np.abs(g64).sum(axis=2, keepdims=True)
    assert_l1_close(dk, rk, "f16", "dk (sum over the sources)", np.broadcast_to(scale, rk.shape))


def test_kernel_backward_multi_rejects(gpu):
    import ctypes

    import laplacianformer_amd as lf

    lib = lf.capi()
    null = ctypes.c_void_p(0)
    one = (ctypes.c_int64 * 1)(4)
    ptrs = (ctypes.c_void_p * 1)(16)
    call = lambda dt, ns, m, c: lib.lfamd_laplace_kernel_backward_multi(  # noqa: E731
        dt, ns, ptrs, ptrs, ptrs, one, ctypes.c_void_p(16), ptrs, ctypes.c_void_p(16), 1, 1, m, c, ctypes.c_float(1.0),
        null, 0, null)
    assert call(1, 0, 49, 64) == 1 and call(1, 4, 49, 64) == 1   # 1 to 3 sources
    assert call(1, 1, 48, 64) == 3                               # M != 49 (LFAMD_ERR_UNSUPPORTED)
    assert call(2, 1, 49, 64) == 3 and call(1, 1, 49, 40) == 3   # bf16; C % 64 != 0
    assert call(1, 1, 49, 64) == 1                               # no workspace
    assert lib.lfamd_laplace_kernel_backward_multi_workspace_size(1, 1, one, 1, 1, 48, 64) == 0
    assert lib.lfamd_laplace_kernel_backward_multi_workspace_size(2, 1, one, 1, 1, 49, 64) == 0  # bf16


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("lens", [(49, 784, 784), (1, 130, 49), (300, 5), (449,)], ids=lambda s: "-".join(map(str, s)))
def test_kernel_forward_multi(gpu, dt, lens):
    """lfamd_laplace_kernel_forward_multi: up to three row sources against one key in one launch
    (each with its own workgroup plan) give each source's lfamd_laplace_kernel_forward result,
    bit for bit."""
    import ctypes

    import laplacianformer_amd as lf

    B, H, M, C = 2, 2, 49, 64
    print(f"laplace kernel forward multi {lens} {dt}", flush=True)
    lib = lf.capi()
    k = gen((B, H, C, M), 811, dt).to(gpu)
    qs = [gen((B, H, n, C), 820 + i, dt).to(gpu) for i, n in enumerate(lens)]
    s = 1.0 / math.sqrt(C)
    outs = [torch.empty((B, H, n, M), dtype=torch.float32, device=gpu) for n in lens]
    ns = len(lens)
    P = lambda ts: (ctypes.c_void_p * ns)(*[t.data_ptr() for t in ts])  # noqa: E731
    nl = (ctypes.c_int64 * ns)(*lens)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    lf.check(lib.lfamd_laplace_kernel_forward_multi(lf.dtype_code(k), ns, P(qs), nl, k.data_ptr(), P(outs), B, H, M,
                                                     C, ctypes.c_float(s), stream))
    for q, o in zip(qs, outs):
        ref = torch.empty_like(o)
        assert lf.ext().LaplaceKernel_forward(q, k, ref, s) is True
        torch.cuda.synchronize()
        assert torch.equal(o, ref)


def test_kernel_forward_multi_rejects(gpu):
    import ctypes

    import laplacianformer_amd as lf

    lib = lf.capi()
    null = ctypes.c_void_p(0)
    one = (ctypes.c_int64 * 1)(4)
    ptrs = (ctypes.c_void_p * 1)(16)
    f = lambda dt, ns, m: lib.lfamd_laplace_kernel_forward_multi(dt, ns, ptrs, one, ctypes.c_void_p(16), ptrs, 1, 1,  # noqa: E731
                                                                 m, 64, ctypes.c_float(1.0), null)
    assert f(1, 0, 49) == 1 and f(1, 4, 49) == 1   # 1 to 3 sources
    assert f(1, 1, 48) == 3                        # M != 49 (LFAMD_ERR_UNSUPPORTED)
    assert f(3, 1, 49) == 3                        # fp64

"""LaplacianFormer attention layer through the HIP ops, against an
fp64 CPU composition built from torch.cdist (p=1) and the NewtonInverse oracle."""
import math

import numpy as np
import pytest
import torch

import oracle
from lfcheck import gen

pytestmark = pytest.mark.gpu


class _NewtonRef(torch.autograd.Function):
    """fp64 CPU NewtonInverse: the oracle's iteration forward, -V^T G V^T backward."""

    @staticmethod
    def forward(ctx, mat, iters):
        V = torch.from_numpy(oracle.newton_forward(mat.detach().numpy(), iters, "f64"))
        ctx.save_for_backward(V)
        return V

    @staticmethod
    def backward(ctx, g):
        (V,) = ctx.saved_tensors
        return torch.from_numpy(oracle.newton_backward(g.numpy(), V.numpy(), "f64")), None


def _ref_attention(q, k, v, grid, pool, iters, store_dtype=None):
    """fp64 composition. ``store_dtype``: the landmarks are pooled in fp32 and stored in
    that type first, as the layer stores them in its input type (fp16 landmarks tie
    with fp16 queries now and then, and a tie's subgradient is 0 on both sides)."""
    B, H, N, d = q.shape

    def pool2(x):
        x = torch.nn.functional.avg_pool2d(x.reshape(B * H, *grid, d).permute(0, 3, 1, 2), pool)
        return x.permute(0, 2, 3, 1).reshape(B, H, -1, d)

    km = pool2(k)
    if store_dtype is not None:  # stored value, fp64 gradient (straight through the rounding)
        km = km + (pool2(k.detach().float()).to(store_dtype).double() - km).detach()
    s = 1.0 / math.sqrt(d)
    k_qm = torch.exp(-torch.cdist(q, km, p=1) * s)
    k_mm = torch.exp(-torch.cdist(km, km, p=1) * s)
    k_mk = torch.exp(-torch.cdist(km, k, p=1) * s)
    inv = _NewtonRef.apply(k_mm, iters)
    return k_qm @ (inv @ (k_mk @ v))


def _norm_close(got, ref, tol, what):
    got = got.detach().cpu().double()
    err = (got - ref).abs().max().item()
    assert err <= tol * ref.abs().max().item(), (what, err, ref.abs().max().item())


def _run(gpu, B, H, grid, d, dtype, seed, pool=4, iters=10, slices=None):
    import laplacianformer_amd as lf

    N = grid[0] * grid[1]
    q, k, v = (gen((B, H, N, d), seed + i, dtype) for i in range(3))
    g = gen((B, H, N, d), seed + 3, dtype)
    qd, kd, vd = (t.to(gpu).requires_grad_() for t in (q, k, v))
    out = lf.laplacian_attention(qd, kd, vd, grid=grid, pool=pool, iters=iters)
    out.backward(g.to(gpu))
    assert out.dtype == q.dtype and out.shape == q.shape
    sl = slices if slices is not None else [slice(None)]
    tol = 2e-3 if dtype in ("f16", "bf16") else 1e-4
    if dtype == "bf16":
        # Two unit roundoffs: grad_k is the sum of two parts each rounded to bf16 (the
        # distance gradient and the pooled landmarks' share), and 2^-8 of the max is
        # only 0.5-1 ulp of it.
        tol = 2 ** -7
    for b in sl:
        qr, kr, vr = (t[b].double().requires_grad_() for t in (q, k, v))
        ref = _ref_attention(qr, kr, vr, grid, pool, iters, None if dtype == "f32" else q.dtype)
        ref.backward(g[b].double())
        _norm_close(out[b], ref.detach(), tol, "out")
        _norm_close(qd.grad[b], qr.grad, tol, "dq")
        _norm_close(kd.grad[b], kr.grad, tol, "dk")
        _norm_close(vd.grad[b], vr.grad, tol, "dv")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_attention_small(gpu, dtype):
    print(f"attention small {dtype}", flush=True)
    _run(gpu, 2, 2, (8, 8), 32, dtype, seed=50)


def test_attention_rect_grid(gpu):
    print("attention rectangular grid", flush=True)
    _run(gpu, 1, 3, (8, 12), 16, "f32", seed=60, pool=2)


def test_attention_config5(gpu):
    """B=64 H=2 N=784 (28x28) d=64 fp16, 4x4 pooled landmarks (M=49), 10 iterations;
    one GPU run of the whole batch, the CPU fp64 reference on every batch entry (each with
    its own norm)."""
    print("attention config 5", flush=True)
    _run(gpu, 64, 2, (28, 28), 64, "f16", seed=1005, slices=[slice(b, b + 1) for b in range(64)])


@pytest.mark.parametrize("dtype,d", [("bf16", 64), ("f32", 64), ("f16", 32)])
def test_attention_config5_grid_types(gpu, dtype, d):
    """The single-node layer entry at config 5's grid (28x28 pooled 4x4: M = 49) in the other
    element types and at d = 32: bf16 and fp32 take the fused forward and the per-source
    backward fallback inside the entry (the one-launch backward is fp16 only), fp16 at d = 32
    the per-source fallback for C % 64 != 0."""
    print(f"attention 28x28 {dtype} d={d}", flush=True)
    _run(gpu, 2, 2, (28, 28), d, dtype, seed=80 + d, slices=[slice(0, 1), slice(1, 2)])


@pytest.mark.parametrize("grid,dtype", [((28, 32), "f16"), ((32, 32), "f32")], ids=["m56-f16", "m64-f32"])
def test_attention_landmark_buckets(gpu, grid, dtype):
    """Landmark counts 56 and 64 (a partial and a full 64 bucket): the fused landmark
    kernels on their general instantiation (every k block whole)."""
    print(f"attention grid {grid} {dtype}", flush=True)
    _run(gpu, 2, 2, grid, 64, dtype, seed=90 + grid[1], slices=[slice(0, 1), slice(1, 2)])


def test_attention_many_slices(gpu):
    """512 (batch, head) slices: the fused landmark forward with two waves per strip (more
    than two matrices per CU); every token a landmark (pool 1, M = 49)."""
    print("attention 512 slices", flush=True)
    _run(gpu, 128, 4, (7, 7), 16, "f32", seed=95, pool=1, slices=[slice(0, 1), slice(127, 128)])


def test_attention_gradcheck(gpu):
    """fp64 end to end on the GPU: torch.autograd.gradcheck of the layer (Newton run to
    convergence, where -V^T G V^T is the exact derivative)."""
    import laplacianformer_amd as lf

    print("attention gradcheck", flush=True)
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 1, 16, 4, dtype=torch.float64, device=gpu, requires_grad=True) for _ in range(3))
    f = lambda a, b, c: lf.laplacian_attention(a, b, c, grid=(4, 4), pool=2, iters=60)  # noqa: E731
    assert torch.autograd.gradcheck(f, (q, k, v), eps=1e-6, atol=1e-5, rtol=1e-4)


def test_attention_module(gpu):
    import laplacianformer_amd as lf

    torch.manual_seed(1)
    m = lf.LaplacianAttention(64, 2).to(gpu)
    x = torch.randn(2, 64, 64, device=gpu, requires_grad=True)
    y = m(x)
    y.sum().backward()
    assert y.shape == x.shape and torch.isfinite(x.grad).all()
    with pytest.raises(ValueError):
        lf.LaplacianAttention(63, 2)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_attention_first_stage_grid(gpu, dtype):
    """A first-stage grid: 56x56 tokens pooled 4x4 -> M = 196 landmarks (fused forward with
    column groups, composed backward on the column-block kernel with a partial last block,
    NewtonInverse on the batched-GEMM path at n = 196, library products for widths > 64)."""
    print(f"attention 56x56 grid {dtype}", flush=True)
    _run(gpu, 2, 1, (56, 56), 32, dtype, seed=70, iters=12)


def test_attention_host_entry_rejects(gpu):
    """The layer's two host calls check their arguments before any launch."""
    import laplacianformer_amd as lf

    L = lf.ext()
    q = torch.randn(1, 2, 64, 16, device=gpu, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="token grid"):
        L.LaplacianAttention_forward(q, q, q, 8, 6, 4, 10)            # 8 x 6 != 64
    with pytest.raises(RuntimeError, match="token grid"):
        L.LaplacianAttention_forward(q, q, q, 8, 8, 3, 10)            # 8 % 3 != 0
    with pytest.raises(RuntimeError, match="one shape"):
        L.LaplacianAttention_forward(q, q[:, :, :32], q, 8, 8, 4, 10)
    with pytest.raises(RuntimeError, match="one type"):
        L.LaplacianAttention_forward(q, q.float(), q, 8, 8, 4, 10)
    wide = torch.randn(1, 1, 16, 80, device=gpu, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="<= 64"):
        L.LaplacianAttention_forward(wide, wide, wide, 4, 4, 2, 10)   # d = 80
    with pytest.raises(RuntimeError, match="11 saved"):
        L.LaplacianAttention_backward(q, [q, q], 8, 8, 4)
    # Device checks come before any launch: a CPU tensor among the inputs, or a CPU
    # grad_output / saved tensor in the backward, is rejected.
    qc = q.cpu()
    with pytest.raises(RuntimeError, match="one GPU"):
        L.LaplacianAttention_forward(q, qc, q, 8, 8, 4, 10)
    with pytest.raises(RuntimeError, match="one GPU"):
        L.LaplacianAttention_forward(qc, qc, qc, 8, 8, 4, 10)
    out, *saved = L.LaplacianAttention_forward(q, q, q, 8, 8, 4, 10)
    with pytest.raises(RuntimeError, match="grad_output"):
        L.LaplacianAttention_backward(out.cpu(), [q, q, q] + saved, 8, 8, 4)
    with pytest.raises(RuntimeError, match="saved tensors"):
        L.LaplacianAttention_backward(out, [q, q, q] + saved[:-1] + [saved[-1].cpu()], 8, 8, 4)

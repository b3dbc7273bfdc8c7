"""GPU parity of NewtonInverse against the CPU oracle and closed forms."""
import numpy as np
import pytest
import torch

import oracle
from lfcheck import TORCH_DT, assert_newton_close, gen

pytestmark = pytest.mark.gpu


def gram(bh, n, d, seed, shift=1e-3, scale=1.0):
    """A = exp(-L1(k_i, k_j) / sqrt(d)) + shift*I from k ~ N(0, scale^2) (BASELINE config recipe)."""
    k = gen((1, bh, n, d), seed, "f64", scale=scale)
    D = oracle.laplace_forward(k, k.transpose(-1, -2).contiguous(), "f64")[0]
    return np.exp(-D / np.sqrt(d)) + shift * np.eye(n)


NS = [1, 5, 16, 17, 32, 48, 49, 64, 65, 80, 96, 100, 112, 113, 128]


@pytest.mark.parametrize("n", NS)
@pytest.mark.parametrize("iters", [0, 1, 10])
def test_newton_forward_f32(gpu, n, iters):
    import laplacianformer_amd as lf

    print(f"newton forward n={n} iters={iters}", flush=True)
    A = torch.from_numpy(gram(6, n, 32, seed=n)).float().reshape(2, 3, n, n)
    out = torch.empty_like(A, device=gpu)
    lf.ext().NewtonInverse_forward(A.to(gpu), out, iters)
    ref = oracle.newton_forward(A, iters, "f32")
    assert_newton_close(out, ref, "f32", f"n={n} it={iters}")


@pytest.mark.parametrize("dt", ["f16", "bf16", "f64"])
@pytest.mark.parametrize("n", [16, 49, 64, 96])
def test_newton_forward_dtypes(gpu, dt, n):
    import laplacianformer_amd as lf

    print(f"newton forward {dt} n={n}", flush=True)
    A = torch.from_numpy(gram(4, n, 64, seed=100 + n)).reshape(2, 2, n, n).to(TORCH_DT[dt])
    out = torch.empty_like(A, device=gpu)
    lf.ext().NewtonInverse_forward(A.to(gpu), out, 10)
    ref = oracle.newton_forward(A, 10, dt)
    assert_newton_close(out, ref, dt, f"{dt} n={n}", rtol=1e-4 if dt != "f64" else 1e-10)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16", "f64"])
@pytest.mark.parametrize("n", [1, 16, 17, 49, 64, 65, 96, 128])
def test_newton_backward(gpu, dt, n):
    import laplacianformer_amd as lf

    print(f"newton backward {dt} n={n}", flush=True)
    V = gen((2, 2, n, n), 7 + n, dt, scale=0.3)
    G = gen((2, 2, n, n), 8 + n, dt)
    out = torch.empty_like(V, device=gpu)
    if dt == "f64" and n > 96:
        # Outside the fp64 envelope (two fp64 n x n buffers per workgroup in LDS):
        # the documented rejection, before any launch.
        with pytest.raises(RuntimeError, match="fp64"):
            lf.ext().NewtonInverse_backward(G.to(gpu), V.to(gpu), out)
        return
    lf.ext().NewtonInverse_backward(G.to(gpu), V.to(gpu), out)
    ref = oracle.newton_backward(G, V, dt)
    assert_newton_close(out, ref, dt, f"bwd {dt} n={n}", rtol=1e-5 if dt != "f64" else 1e-12)


def test_newton_backward_not_square(gpu):
    """A non-square inverse is rejected before any launch (the kernels would read
    and write B*H*N*N elements of [B, H, N, K] tensors)."""
    import laplacianformer_amd as lf

    V = torch.zeros((1, 2, 8, 5), device=gpu)
    G = torch.zeros((1, 2, 8, 5), device=gpu)
    out = torch.empty((1, 2, 8, 5), device=gpu)
    with pytest.raises(RuntimeError, match="last two dims of inverse must be equal"):
        lf.ext().NewtonInverse_backward(G, V, out)


def test_newton_config3(gpu):
    """1024 matrices 64x64 fp32, 12 iterations, forward + backward."""
    import laplacianformer_amd as lf

    print("newton config 3", flush=True)
    A = torch.from_numpy(gram(1024, 64, 64, seed=1003)).float().reshape(1024, 1, 64, 64)
    G = gen((1024, 1, 64, 64), 1013, "f32")
    Ad, Gd = A.to(gpu), G.to(gpu)
    V = torch.empty_like(Ad)
    dA = torch.empty_like(Ad)
    lf.ext().NewtonInverse_forward(Ad, V, 12)
    lf.ext().NewtonInverse_backward(Gd, V, dA)
    ref = oracle.newton_forward(A, 12, "f32")
    assert_newton_close(V, ref, "f32", "cfg3 fwd")
    assert_newton_close(dA, oracle.newton_backward(G, V.cpu(), "f32"), "f32", "cfg3 bwd", rtol=1e-5)
    # Residual ||P X - I||_F matches the oracle's within 1e-4 * sqrt(n).
    P = A.double() + 0.01 * torch.eye(64, dtype=torch.float64)
    r_gpu = torch.linalg.matrix_norm(P @ V.cpu().double() - torch.eye(64, dtype=torch.float64))
    r_ref = torch.linalg.matrix_norm(P @ torch.from_numpy(ref).double() - torch.eye(64, dtype=torch.float64))
    assert (r_gpu - r_ref).abs().max().item() <= 1e-4 * 8


@pytest.mark.parametrize("bh", [257, 600, 1000, 2048])
def test_newton_backward_persistent(gpu, bh):
    """Full 64 x 64 fp32 matrices at 2 to 8 per CU take the persistent backward (one
    workgroup per CU, its matrices through four LDS slots in turn); counts that leave
    the last workgroup short, against the oracle."""
    import laplacianformer_amd as lf

    print(f"newton backward persistent bh={bh}", flush=True)
    V = gen((bh, 1, 64, 64), 40 + bh, "f32", scale=0.3)
    G = gen((bh, 1, 64, 64), 41 + bh, "f32")
    out = torch.empty_like(V, device=gpu)
    lf.ext().NewtonInverse_backward(G.to(gpu), V.to(gpu), out)
    assert_newton_close(out, oracle.newton_backward(G, V, "f32"), "f32", f"bwd persistent bh={bh}", rtol=1e-5)


@pytest.mark.parametrize("case", ["symmetric", "one_pair", "general"])
@pytest.mark.parametrize("bh", [3, 600])
def test_newton_forward_n49_symmetry(gpu, case, bh):
    """fp32 n = 49 runs the symmetric iteration (upper tiles, mirrored) when P is exactly
    symmetric and the general one otherwise, decided per matrix in the kernel. Both against
    the oracle; the symmetric path's result is exactly symmetric, a matrix with a single
    asymmetric pair and a general matrix take the general path. 600 matrices: two waves per
    strip (the 8-wave variant of the symmetric body)."""
    import laplacianformer_amd as lf

    print(f"newton forward n=49 {case} bh={bh}", flush=True)
    n = 49
    A = gram(bh, n, 64, seed=300 + bh)
    if case == "one_pair":
        A[:, 3, 40] += 1e-3  # every matrix asymmetric in one element pair
    elif case == "general":
        A = A + 1e-4 * np.random.default_rng(7).standard_normal(A.shape)
    At = torch.from_numpy(A).float().reshape(bh, 1, n, n)
    out = torch.empty_like(At, device=gpu)
    lf.ext().NewtonInverse_forward(At.to(gpu), out, 10)
    ref = oracle.newton_forward(At, 10, "f32")
    assert_newton_close(out, ref, "f32", f"n=49 {case}", rtol=1e-4)
    o = out.cpu()
    if case == "symmetric":
        assert torch.equal(o, o.transpose(-1, -2)), "symmetric path result not exactly symmetric"


def test_newton_closed_forms(gpu):
    """Diagonal A = c I: X_k = (1 - (-0.8)^(2^k)) / mu * I with mu = c + 0.01; and iter = 0 gives alpha P."""
    import laplacianformer_amd as lf

    for n, c in ((16, 0.5), (49, 2.0), (128, 0.09)):
        mu = c + 0.01
        A = (c * torch.eye(n)).reshape(1, 1, n, n).repeat(2, 1, 1, 1)
        for k in (0, 1, 3, 6):
            out = torch.empty_like(A, device=gpu)
            lf.ext().NewtonInverse_forward(A.to(gpu), out, k)
            expect = (1 - (-0.8) ** (2 ** k)) / mu
            d = torch.diagonal(out.cpu().double(), dim1=-2, dim2=-1)
            assert torch.allclose(d, torch.full_like(d, expect), rtol=2e-6), (n, c, k)
            off = out.cpu().double() - torch.diag_embed(d)
            assert off.abs().max().item() == 0.0


def test_newton_errors(gpu):
    import laplacianformer_amd as lf

    L = lf.ext()
    A = torch.zeros((1, 1, 257, 257), device=gpu)
    with pytest.raises(RuntimeError, match="N=257 is not supported"):
        L.NewtonInverse_forward(A, torch.empty_like(A), 3)
    with pytest.raises(RuntimeError, match="must be 4D"):
        L.NewtonInverse_forward(torch.zeros((3, 4, 4), device=gpu), torch.empty((3, 4, 4), device=gpu), 3)
    with pytest.raises(RuntimeError, match="same shape"):
        L.NewtonInverse_forward(torch.zeros((1, 1, 4, 4), device=gpu), torch.empty((1, 1, 5, 5), device=gpu), 3)
    assert L.NewtonInverse_is_supported(256) and not L.NewtonInverse_is_supported(257)
    assert not L.NewtonInverse_is_supported(0)


def test_newton_autograd(gpu):
    import laplacianformer_amd as lf

    A = torch.from_numpy(gram(2, 49, 32, seed=4)).float().reshape(1, 2, 49, 49)
    Ad = A.to(gpu).requires_grad_()
    V = lf.newton_inverse(Ad, 10)
    G = gen((1, 2, 49, 49), 5, "f32")
    V.backward(G.to(gpu))
    assert_newton_close(V, oracle.newton_forward(A, 10), "f32")
    assert_newton_close(Ad.grad, oracle.newton_backward(G, V.detach().cpu()), "f32", rtol=1e-5)


def test_newton_golden_closed_form(gpu):
    """tests/golden/newton_closed.npz: eigen closed form of the iteration with the reference init."""
    import os

    import laplacianformer_amd as lf

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "newton_closed.npz"))
    for n in (5, 49, 64, 136):
        A = torch.from_numpy(z[f"A_{n}"]).float().reshape(1, 1, n, n)
        for it in (0, 1, 4, 10):
            out = torch.empty_like(A, device=gpu)
            lf.ext().NewtonInverse_forward(A.to(gpu), out, it)
            assert_newton_close(out, z[f"X_{n}_{it}"][None, None], "f32", f"closed n={n} it={it}")


# ---- 128 < n <= 256: batched-GEMM path (beyond the reference's n <= 128) ----

@pytest.mark.parametrize("n", [129, 130, 192, 200, 256])
@pytest.mark.parametrize("iters", [0, 1, 10])
def test_newton_large_forward_f32(gpu, n, iters):
    import laplacianformer_amd as lf

    print(f"newton large forward n={n} iters={iters}", flush=True)
    A = torch.from_numpy(gram(3, n, 32, seed=n)).float().reshape(3, 1, n, n)
    out = torch.empty_like(A, device=gpu)
    lf.ext().NewtonInverse_forward(A.to(gpu), out, iters)
    assert_newton_close(out, oracle.newton_forward(A, iters, "f32"), "f32", f"n={n} it={iters}")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_newton_large_forward_dtypes(gpu, dt):
    import laplacianformer_amd as lf

    n = 200
    print(f"newton large forward {dt} n={n}", flush=True)
    A = torch.from_numpy(gram(2, n, 64, seed=300)).reshape(1, 2, n, n).to(TORCH_DT[dt])
    out = torch.empty_like(A, device=gpu)
    lf.ext().NewtonInverse_forward(A.to(gpu), out, 10)
    assert_newton_close(out, oracle.newton_forward(A, 10, dt), dt, f"{dt} n={n}")


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n", [129, 200, 256])
def test_newton_large_backward(gpu, dt, n):
    import laplacianformer_amd as lf

    print(f"newton large backward {dt} n={n}", flush=True)
    V = gen((2, 1, n, n), 17 + n, dt, scale=0.1)
    G = gen((2, 1, n, n), 18 + n, dt)
    out = torch.empty_like(V, device=gpu)
    lf.ext().NewtonInverse_backward(G.to(gpu), V.to(gpu), out)
    assert_newton_close(out, oracle.newton_backward(G, V, dt), dt, f"bwd {dt} n={n}", rtol=1e-5)


def test_newton_large_backward_in_place_and_unaligned(gpu):
    """fp32 n = 256 reads and writes the caller's tensors directly unless the output
    overlaps the inverse or a pointer is not 16-byte aligned; every route gives the
    same bits."""
    import laplacianformer_amd as lf

    n = 256
    print("newton large backward aliasing / alignment", flush=True)
    V = gen((2, 1, n, n), 41, "f32", scale=0.1).to(gpu)
    G = gen((2, 1, n, n), 42, "f32").to(gpu)
    L = lf.ext()
    want = torch.empty_like(V)
    L.NewtonInverse_backward(G, V, want)
    got = V.clone()
    L.NewtonInverse_backward(G, got, got)  # output written over the inverse
    assert torch.equal(got, want)
    buf = torch.empty(3 * V.numel() + 1, device=gpu)
    Vu = buf[1:1 + V.numel()].view_as(V).copy_(V)  # 4-byte offset: not 16-byte aligned
    Gu = buf[1 + V.numel():1 + 2 * V.numel()].view_as(G).copy_(G)
    Ou = buf[1 + 2 * V.numel():].view_as(V)
    L.NewtonInverse_backward(Gu, Vu, Ou)
    assert torch.equal(Ou, want)
    A = torch.from_numpy(gram(1, n, 32, seed=5)).float().reshape(1, 1, n, n).to(gpu)
    fa = torch.empty_like(A)
    L.NewtonInverse_forward(A, fa, 3)
    fb = torch.empty(A.numel() + 1, device=gpu)[1:].view_as(A)
    L.NewtonInverse_forward(A, fb, 3)
    assert torch.equal(fa, fb)


def test_newton_large_closed_form(gpu):
    """Diagonal A = c I at n = 256: X_k = (1 - (-0.8)^(2^k)) / (c + 0.01) * I, off-diagonal exactly 0."""
    import laplacianformer_amd as lf

    n, c = 256, 0.3
    mu = c + 0.01
    A = (c * torch.eye(n)).reshape(1, 1, n, n)
    for k in (0, 2, 5):
        out = torch.empty_like(A, device=gpu)
        lf.ext().NewtonInverse_forward(A.to(gpu), out, k)
        d = torch.diagonal(out.cpu().double(), dim1=-2, dim2=-1)
        assert torch.allclose(d, torch.full_like(d, (1 - (-0.8) ** (2 ** k)) / mu), rtol=2e-6), k
        assert (out.cpu().double() - torch.diag_embed(d)).abs().max().item() == 0.0


def test_newton_config4(gpu):
    """BASELINE config 4 (Newton part): 128 Gram matrices 256x256 fp32, 16 iterations, fwd + bwd."""
    import laplacianformer_amd as lf

    print("newton config 4", flush=True)
    A = torch.from_numpy(gram(128, 256, 64, seed=1004, scale=0.5)).float().reshape(16, 8, 256, 256)
    G = gen((16, 8, 256, 256), 1014, "f32")
    Ad, Gd = A.to(gpu), G.to(gpu)
    V = torch.empty_like(Ad)
    dA = torch.empty_like(Ad)
    lf.ext().NewtonInverse_forward(Ad, V, 16)
    lf.ext().NewtonInverse_backward(Gd, V, dA)
    ref = oracle.newton_forward(A, 16, "f32")
    assert_newton_close(V, ref, "f32", "cfg4 fwd")
    assert_newton_close(dA, oracle.newton_backward(G, V.cpu(), "f32"), "f32", "cfg4 bwd", rtol=1e-5)

"""The attention layer's row products on the HIP row-product kernel
(lfamd_mix_rows, torch export MixRows): c[..., n, q] = sum_p a[..., n, p] * b[..., q, p]
against an fp64 CPU product, |err| <= 1e-5 * sum_p |a| |b| (fp32 sums of <= 64
products), plus the autograd Functions the layer uses against fp64 CPU
autograd of the same products."""
import pytest
import torch

from lfcheck import gen

pytestmark = pytest.mark.gpu

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _check(c, a, b_qp, what):
    a64, b64 = a.detach().cpu().double(), b_qp.detach().cpu().double()
    ref = torch.matmul(a64, b64.transpose(-1, -2))
    bound = torch.matmul(a64.abs(), b64.abs().transpose(-1, -2))
    err = (c.detach().cpu().double() - ref).abs()
    assert torch.isfinite(c).all(), what
    assert bool((err <= 1e-5 * bound + 1e-30).all()), (what, float((err / (bound + 1e-30)).max()))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 64, 784, 49, 64), (2, 64, 784, 64, 49), (1, 3, 100, 7, 64),
                                   (1, 1, 1, 1, 1), (3, 2, 65, 64, 64), (1, 5, 129, 33, 17)],
                         ids=lambda s: "x".join(map(str, s)))
def test_mix_rows(gpu, dt, shape):
    import laplacianformer_amd as lf

    B, H, N, P, Q = shape
    print(f"mix rows {shape} {dt}", flush=True)
    a = gen((B, H, N, P), 11 + N + P, dt)
    w = gen((B, H, P, Q), 12 + N + Q, "f32")
    ad, wd = a.to(gpu), w.to(gpu)
    c = lf.mix_rows(ad, wd.transpose(-1, -2))        # a @ w, b read transposed in place
    _check(c, a, w.transpose(-1, -2), "a @ w")
    wq = gen((B, H, Q, P), 13 + N, "f32")
    c2 = lf.mix_rows(ad, wq.to(gpu))                  # a @ wq^T, b contiguous
    _check(c2, a, wq, "a @ wq^T")


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("out", [torch.float16, torch.bfloat16])
def test_mix_rows_output_type(gpu, dt, out):
    """A 16-bit output is the fp32 result rounded once (bit-identical to casting it)."""
    import laplacianformer_amd as lf

    print(f"mix rows output {dt} -> {out}", flush=True)
    a = gen((2, 3, 333, 49), 21, dt).to(gpu)
    w = gen((2, 3, 64, 49), 22, "f32").to(gpu)
    c = lf.mix_rows(a, w, out)
    assert c.dtype == out
    assert torch.equal(c, lf.mix_rows(a, w).to(out))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 8, 784, 49, 64), (2, 8, 784, 64, 49), (1, 3, 100, 7, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_mix_rows_wide_range(gpu, dt, shape):
    """Entries spread over many binades (the bf16 pieces of every operand carry
    their own exponents): still within 1e-5 of sum |a| |b| of the fp64 product."""
    import laplacianformer_amd as lf

    B, H, N, P, Q = shape
    print(f"mix rows wide range {shape} {dt}", flush=True)
    g = torch.Generator().manual_seed(41 + P)
    span = 12 if dt == "f16" else 40
    a = (gen((B, H, N, P), 42 + N, "f32") * torch.exp2(torch.randint(-span, span + 1, (B, H, N, P), generator=g)))
    a = a.to(TORCH_DT[dt])
    w = gen((B, H, Q, P), 43 + Q, "f32") * torch.exp2(torch.randint(-40, 41, (B, H, Q, P), generator=g).float())
    c = lf.mix_rows(a.to(gpu), w.to(gpu))
    _check(c, a, w, "wide range")


def test_mix_rows_nonfinite(gpu):
    """An infinity or NaN in a row of A, or in a column of B, makes exactly the
    outputs it takes part in non-finite (for the products through the bf16
    pieces an infinity may come out as NaN)."""
    import laplacianformer_amd as lf

    for (N, P, Q) in ((784, 49, 64), (784, 64, 49), (100, 7, 64)):
        print(f"mix rows nonfinite {N}x{P}x{Q}", flush=True)
        a = gen((1, 2, N, P), 51, "f32")
        w = gen((1, 2, Q, P), 52, "f32")
        a[0, 0, 5, 3] = float("inf")
        a[0, 1, N - 1, P - 1] = float("nan")
        w[0, 1, 2, 1] = float("-inf")
        c = lf.mix_rows(a.to(gpu), w.to(gpu)).cpu()
        ref = torch.matmul(a.double(), w.double().transpose(-1, -2))
        assert torch.equal(torch.isfinite(c), torch.isfinite(ref))


def test_mix_rows_rejects(gpu):
    import laplacianformer_amd as lf

    a = torch.randn(1, 1, 10, 65, device=gpu)
    with pytest.raises(RuntimeError):
        lf.mix_rows(a, torch.randn(1, 1, 8, 65, device=gpu))  # inner width 65 > 64
    b = torch.randn(2, 3, 8, 5, device=gpu)[:, :2]           # batch dims that do not collapse
    with pytest.raises(RuntimeError):
        lf.mix_rows(torch.randn(2, 2, 10, 5, device=gpu), b.transpose(0, 1))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 64, 784, 49, 64), (1, 3, 100, 7, 64), (1, 1, 1, 1, 1), (3, 2, 65, 64, 64),
                                   (1, 5, 129, 33, 17), (1, 2, 3000, 49, 64), (2, 1, 0, 49, 64),
                                   (1, 2, 96, 49, 6)],
                         ids=lambda s: "x".join(map(str, s)))
def test_tall_t(gpu, dt, shape):
    """c = a^T b over the rows (lfamd_tall_t, torch export TallT) against an fp64 CPU product,
    |err| <= 1e-5 * sum_n |a| |b|; deterministic (two calls give the same bits)."""
    import laplacianformer_amd as lf

    B, H, N, P, Q = shape
    print(f"tall_t {shape} {dt}", flush=True)
    a = gen((B, H, N, P), 31 + N + P, "f32")
    b = gen((B, H, N, Q), 32 + N + Q, dt)
    c = lf.tall_t(a.to(gpu), b.to(gpu))
    assert c.shape == (B, H, P, Q) and c.dtype == torch.float32
    _check(c, a.transpose(-1, -2), b.transpose(-1, -2), "a^T b")
    assert torch.equal(c, lf.tall_t(a.to(gpu), b.to(gpu)))


def test_tall_t_rejects(gpu):
    import laplacianformer_amd as lf

    L = lf.ext()
    a = torch.randn(1, 1, 10, 65, device=gpu)
    with pytest.raises(RuntimeError):
        L.TallT(a, torch.randn(1, 1, 10, 8, device=gpu), torch.empty(1, 1, 65, 8, device=gpu))  # P = 65 > 64
    with pytest.raises(RuntimeError):
        L.TallT(a[..., :8].half(), torch.randn(1, 1, 10, 8, device=gpu), torch.empty(1, 1, 8, 8, device=gpu))


@pytest.mark.parametrize("vdt", ["f32", "f16"])
def test_tall_functions_autograd(gpu, vdt):
    """K_qm . W and K_km^T V with their gradients (the layer's use), against fp64 CPU autograd."""
    import laplacianformer_amd as lf

    B, H, N, M, d = 2, 2, 300, 49, 64
    print(f"tall functions autograd {vdt}", flush=True)
    k = torch.rand(B, H, N, M, generator=torch.Generator().manual_seed(1))
    v = gen((B, H, N, d), 2, vdt)
    w = gen((B, H, M, d), 3, "f32")
    g1 = gen((B, H, N, d), 4, "f32")
    g2 = gen((B, H, M, d), 5, "f32")
    kd = k.to(gpu).requires_grad_()
    vd = v.to(gpu).requires_grad_()
    wd = w.to(gpu).requires_grad_()
    out = lf.tall_mix(kd, wd)
    kv = lf.tall_product(kd, vd)
    torch.autograd.backward([out, kv], [g1.to(gpu), g2.to(gpu)])
    k64 = k.double().requires_grad_()
    v64 = v.double().requires_grad_()
    w64 = w.double().requires_grad_()
    torch.autograd.backward([k64 @ w64, k64.transpose(-1, -2) @ v64], [g1.double(), g2.double()])
    for got, ref, name in ((out, (k64 @ w64), "out"), (kv, k64.transpose(-1, -2) @ v64, "kv"),
                           (kd.grad, k64.grad, "grad K"), (wd.grad, w64.grad, "grad W"),
                           (vd.grad, v64.grad, "grad V")):
        r = ref.detach()
        tol = (1e-3 if (name == "grad V" and vdt == "f16") else 2e-5) * r.abs().max().item()
        err = (got.detach().cpu().double() - r).abs().max().item()
        assert err <= tol, (name, err, tol)

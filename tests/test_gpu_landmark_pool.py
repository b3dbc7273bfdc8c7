"""The attention layer's landmark pooling kernels (lfamd_landmark_pool,
lfamd_landmark_pool_backward) through the C ABI against the tensor-op
compositions they replace: the pool x pool mean in fp32 (summed in another
order: within the fp32 summation bound and one rounding to the element type,
and bit-identical for integer-valued inputs, whose sums are exact) and, bit for
bit, the backward's elementwise chain (each step rounded to the element type)."""
import ctypes

import pytest
import torch

from lfcheck import gen

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
# (B, H, gh, gw, pool, d); the last one's landmark row (64 x 64) exceeds the staged backward's LDS
SHAPES = [(64, 2, 28, 28, 4, 64), (2, 3, 8, 12, 4, 32), (1, 2, 9, 6, 3, 8), (2, 1, 4, 4, 1, 5), (1, 1, 56, 56, 8, 16),
          (1, 1, 4, 128, 2, 64)]


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _pool_ref(k, gh, gw, p):
    B, H, N, d = k.shape
    return k.reshape(B, H, gh // p, p, gw // p, p, d).mean(dim=(3, 5), dtype=torch.float32).reshape(B, H, -1, d)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("integer", [False, True])
def test_landmark_pool(gpu, dt, shape, integer):
    import laplacianformer_amd as lf

    B, H, gh, gw, p, d = shape
    print(f"landmark pool {shape} {dt} integer={integer}", flush=True)
    lib = lf.capi()
    k = gen((B, H, gh * gw, d), 61 + d, dt, integer=8 if integer else None).to(gpu)
    M = (gh // p) * (gw // p)
    km = torch.empty((B, H, M, d), dtype=DT[dt], device=gpu)
    km_cm = torch.empty((B, H, d, M), dtype=DT[dt], device=gpu)
    lf.check(lib.lfamd_landmark_pool(lf.dtype_code(k), k.data_ptr(), km.data_ptr(), km_cm.data_ptr(), B, H, gh, gw,
                                     p, d, _stream()))
    ref32 = _pool_ref(k, gh, gw, p)
    ref = ref32.to(DT[dt])
    assert torch.equal(km_cm, km.transpose(-1, -2).contiguous())
    if integer and p * p in (1, 4, 16, 64):  # exact sums, exact division: the same bits
        assert torch.equal(km, ref)
    else:
        # fp32 sums in another order (each within eps * sum |k| of the exact one), then
        # one rounding to the element type
        ulp = {"f32": 2.0 ** -23, "f16": 2.0 ** -10, "bf16": 2.0 ** -7}[dt]
        acc = 2.0 ** -22 * p * p * _pool_ref(k.abs(), gh, gw, p)
        tol = ulp * ref32.abs() + acc + 2.0 ** -24
        assert bool(((km.float() - ref32).abs() <= tol).all())


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_landmark_pool_backward(gpu, dt, shape):
    import laplacianformer_amd as lf

    B, H, gh, gw, p, d = shape
    print(f"landmark pool backward {shape} {dt}", flush=True)
    lib = lf.capi()
    M = (gh // p) * (gw // p)
    dk = gen((B, H, gh * gw, d), 71, dt).to(gpu)
    dkm = gen((B, H, M, d), 72, dt).to(gpu)
    dcm = [gen((B, H, d, M), 73 + i, dt).to(gpu) for i in range(3)]
    # the composition the kernel replaces, each op rounded to the element type
    t = dcm[0].clone()
    t += dcm[1]
    t += dcm[2]
    u = dkm.clone()
    u += t.transpose(-1, -2)
    gs = (u.float() / (p * p)).to(dk.dtype)
    ref = dk.clone()
    ref.view(B, H, gh // p, p, gw // p, p, d).add_(gs.view(B, H, gh // p, 1, gw // p, 1, d))
    out = dk.clone()
    lf.check(lib.lfamd_landmark_pool_backward(lf.dtype_code(dk), out.data_ptr(), dkm.data_ptr(), dcm[0].data_ptr(),
                                              dcm[1].data_ptr(), dcm[2].data_ptr(), B, H, gh, gw, p, d, _stream()))
    assert torch.equal(out, ref)


def test_landmark_pool_rejects(gpu):
    import laplacianformer_amd as lf

    lib = lf.capi()
    null = ctypes.c_void_p(0)
    assert lib.lfamd_landmark_pool(0, null, null, null, 1, 1, 6, 8, 4, 64, null) == 1       # 6 % 4 != 0
    assert lib.lfamd_landmark_pool(3, null, null, null, 1, 1, 8, 8, 4, 64, null) == 2       # fp64
    assert lib.lfamd_landmark_pool(0, null, null, null, 1, 1, 8, 8, 4, 64, null) == 1       # null pointers
    assert lib.lfamd_landmark_pool(0, null, null, null, 0, 1, 8, 8, 4, 64, null) == 0       # nothing to do
    assert lib.lfamd_landmark_pool_backward(0, null, null, null, null, null, 1, 1, 8, 8, 0, 64, null) == 1

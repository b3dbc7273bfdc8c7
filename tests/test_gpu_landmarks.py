"""The attention layer's fused landmark kernels (lfamd_attention_landmarks_forward /
_backward) through the C ABI, against the unfused C-ABI operations they replace and an
fp64 torch composition.

The inverse is the same kernel body as lfamd_newton_forward (same variant for the same
matrix count and size) and the tall product's partials are summed in the same workgroup
order as lfamd_tall_t's reduction, so inv and kv must match those bit for bit; w, dkv and
the inverse's gradient are fp32 products checked against fp64 within 1e-5 of
sum |a| |b|."""
import pytest
import torch

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
UNSUPPORTED = 3  # LFAMD_ERR_UNSUPPORTED


def _inputs(slices, rows, m, d, vdt, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand((slices, m, m), generator=g, dtype=torch.float64)
    kmm = (torch.exp(-3.0 * a) + torch.eye(m, dtype=torch.float64)).float()  # well conditioned, positive
    kkm = torch.rand((slices, rows, m), generator=g).float()
    v = torch.randn((slices, rows, d), generator=g).to(TD[vdt])
    return kmm.to(gpu), kkm.to(gpu), v.to(gpu)


def _close(got, ref, scale, what):
    err = (got.double() - ref).abs()
    lim = 1e-5 * scale + 1e-30
    assert not (err > lim).any(), (what, (err / lim).max().item())


@pytest.mark.parametrize("slices,rows,m,d,vdt", [
    (3, 784, 49, 64, "f16"),      # the layer's shape: one live row in the last strip (KL = 1)
    (5, 200, 64, 64, "f32"),      # a full 64 bucket
    (4, 96, 56, 16, "bf16"),      # a partial bucket, narrow d
    (600, 32, 49, 32, "f16"),     # more than two matrices per CU: two waves per strip
])
def test_landmarks_forward(gpu, slices, rows, m, d, vdt):
    import laplacianformer_amd as lf

    print(f"landmarks forward {slices}x{rows} m={m} d={d} {vdt}", flush=True)
    lib = lf.capi()
    kmm, kkm, v = _inputs(slices, rows, m, d, vdt, 11 + m + d, gpu)
    iters = 10
    wsb = lib.lfamd_tall_t_workspace_size(slices, rows)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    inv = torch.empty_like(kmm)
    kv = torch.empty((slices, m, d), device=gpu)
    w = torch.empty_like(kv)
    vt = lf.dtype_code(v.dtype)
    lf.check(lib.lfamd_attention_landmarks_forward(kmm.data_ptr(), kkm.data_ptr(), vt, v.data_ptr(), inv.data_ptr(),
                                                   kv.data_ptr(), w.data_ptr(), slices, rows, m, d, iters,
                                                   ws.data_ptr(), wsb, None))
    # The unfused operations.
    inv_u = torch.empty_like(kmm)
    kv_u = torch.empty_like(kv)
    lf.check(lib.lfamd_newton_forward(0, kmm.data_ptr(), inv_u.data_ptr(), slices, m, iters, None, 0, None))
    lf.check(lib.lfamd_tall_t(vt, kkm.data_ptr(), v.data_ptr(), kv_u.data_ptr(), slices, rows, m, d, ws.data_ptr(),
                              wsb, None))
    torch.cuda.synchronize()
    assert torch.equal(inv, inv_u), "inverse differs from lfamd_newton_forward"
    assert torch.equal(kv, kv_u), "kv differs from lfamd_tall_t"
    i64, k64 = inv.double(), kv.double()
    _close(w, i64 @ k64, i64.abs() @ k64.abs(), "w = inv kv")


@pytest.mark.parametrize("slices,rows,m,d,dt", [
    (3, 784, 49, 64, "f16"),
    (5, 200, 64, 64, "f32"),
    (4, 96, 56, 16, "bf16"),
    (600, 32, 49, 32, "f16"),
])
def test_landmarks_backward(gpu, slices, rows, m, d, dt):
    import laplacianformer_amd as lf

    print(f"landmarks backward {slices}x{rows} m={m} d={d} {dt}", flush=True)
    lib = lf.capi()
    kmm, kqm, g = _inputs(slices, rows, m, d, dt, 21 + m + d, gpu)
    _, kkm, v = _inputs(slices, rows, m, d, dt, 31 + m + d, gpu)
    inv = torch.empty_like(kmm)
    lf.check(lib.lfamd_newton_forward(0, kmm.data_ptr(), inv.data_ptr(), slices, m, 10, None, 0, None))
    gen = torch.Generator().manual_seed(5)
    kv = torch.randn((slices, m, d), generator=gen).to(gpu)
    w = torch.randn((slices, m, d), generator=gen).to(gpu)
    wsb = lib.lfamd_tall_t_workspace_size(slices, rows)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    dkqm = torch.empty((slices, rows, m), device=gpu)
    dkkm = torch.empty_like(dkqm)
    dv = torch.empty_like(v)
    dkv = torch.empty_like(kv)
    dkmm = torch.empty_like(kmm)
    code = lf.dtype_code(g.dtype)
    lf.check(lib.lfamd_attention_landmarks_backward(
        kqm.data_ptr(), code, g.data_ptr(), v.data_ptr(), kkm.data_ptr(), w.data_ptr(), kv.data_ptr(), inv.data_ptr(),
        dkqm.data_ptr(), dkkm.data_ptr(), dv.data_ptr(), dkv.data_ptr(), dkmm.data_ptr(), slices, rows, m, d,
        ws.data_ptr(), wsb, None))
    # The unfused operations: the tall product (dw) and the row products one call each.
    dw = torch.empty_like(kv)
    lf.check(lib.lfamd_tall_t(code, kqm.data_ptr(), g.data_ptr(), dw.data_ptr(), slices, rows, m, d, ws.data_ptr(), wsb,
                              None))
    md = m * d
    r_kqm, r_kkm, r_dv = torch.empty_like(dkqm), torch.empty_like(dkkm), torch.empty_like(dv)
    lf.check(lib.lfamd_mix_rows(code, g.data_ptr(), w.data_ptr(), 0, r_kqm.data_ptr(), slices, rows, d, m, d, 1, md,
                                None))
    lf.check(lib.lfamd_mix_rows(code, v.data_ptr(), dkv.data_ptr(), 0, r_kkm.data_ptr(), slices, rows, d, m, d, 1, md,
                                None))
    lf.check(lib.lfamd_mix_rows(0, kkm.data_ptr(), dkv.data_ptr(), code, r_dv.data_ptr(), slices, rows, m, d, 1, d, md,
                                None))
    torch.cuda.synchronize()
    # The one launch of the three products runs the same per-row arithmetic as one call each.
    assert torch.equal(dkqm, r_kqm), "g w^T differs from lfamd_mix_rows"
    assert torch.equal(dkkm, r_kkm), "v dkv^T differs from lfamd_mix_rows"
    assert torch.equal(dv, r_dv), "k_km dkv differs from lfamd_mix_rows"
    i64, k64, w64 = inv.double(), kv.double(), dw.double()
    wabs = kqm.double().abs().transpose(1, 2) @ g.double().abs()
    _close(dkv, i64.transpose(1, 2) @ w64, i64.abs().transpose(1, 2) @ wabs, "dkv = inv^T dw")
    dinv = w64 @ k64.transpose(1, 2)
    dinv_abs = wabs @ k64.abs().transpose(1, 2)
    ref = -(i64.transpose(1, 2) @ dinv) @ i64.transpose(1, 2)
    scale = (i64.abs().transpose(1, 2) @ dinv_abs) @ i64.abs().transpose(1, 2)
    _close(dkmm, ref, scale, "dkmm = -(inv^T dinv) inv^T")


def test_landmarks_unsupported(gpu):
    """Shapes outside the fused kernels return LFAMD_ERR_UNSUPPORTED (the layer then takes
    the unfused operations) before anything is launched."""
    import laplacianformer_amd as lf

    lib = lf.capi()
    slices, rows, d = 2, 64, 16
    kmm, kkm, v = _inputs(slices, rows, 49, d, "f32", 3, gpu)
    wsb = lib.lfamd_tall_t_workspace_size(slices, rows)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    out = torch.empty((slices, 64, 64), device=gpu)
    p = out.data_ptr()
    for m, dd, vptr in ((48, d, v.data_ptr()), (65, d, v.data_ptr()), (49, 65, v.data_ptr()),
                        (49, d, v.data_ptr() + 4)):  # last: v not 16-byte aligned
        rc = lib.lfamd_attention_landmarks_forward(kmm.data_ptr(), kkm.data_ptr(), 0, vptr, p, p, p, slices, rows, m,
                                                   dd, 10, ws.data_ptr(), wsb, None)
        assert rc == UNSUPPORTED, (m, dd, rc)
        rc = lib.lfamd_attention_landmarks_backward(kkm.data_ptr(), 0, vptr, vptr, kkm.data_ptr(), p, p, p, p, p, p, p,
                                                    p, slices, rows, m, dd, ws.data_ptr(), wsb, None)
        assert rc == UNSUPPORTED, (m, dd, rc)
    torch.cuda.synchronize()

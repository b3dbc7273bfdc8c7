"""GPU parity of LaplaceSubtraction against the CPU oracle (drop-in module and C ABI)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from lfcheck import TORCH_DT, assert_bitwise, assert_l1_close, check_l1, gen, l1_refs

pytestmark = pytest.mark.gpu

# (B, H, N, M, C): reference-config shapes, tile tails, one-element and channel-split cases.
SHAPES = [
    (2, 2, 196, 49, 32),
    (1, 1, 1, 1, 1),
    (1, 1, 63, 7, 5),
    (2, 1, 65, 17, 64),
    (1, 3, 130, 64, 65),
    (1, 1, 64, 65, 16),
    (1, 2, 100, 100, 33),
    (1, 1, 129, 256, 64),
    (2, 1, 96, 48, 130),
    # M a multiple of 32 (column blocks of 32 per wave): M = 32, 96, 128 with odd N and
    # partial channel blocks.
    (2, 1, 77, 32, 64),
    (1, 2, 200, 96, 48),
    (1, 1, 33, 128, 130),
    # Register-resident columns (M = 16, 49) for every type: odd N * M (fp32 only there),
    # several channel blocks, a single row.
    (2, 1, 131, 16, 80),
    (1, 1, 7, 49, 64),
    (1, 2, 1, 49, 128),
    # Column-split backward (16-bit, M in {16, 32, 49}, C % 64 = 0) either side of one
    # workgroup per slice (up to 64 rows: grad_key written without partials).
    (1, 2, 64, 32, 128),
    (2, 1, 65, 49, 64),
    # Odd M beyond the register-resident set: column blocks with 16-bit rows of odd length.
    (1, 2, 77, 81, 64),
    (2, 1, 50, 225, 40),
    # M > 256: the multi-block backward (16-bit grad staging, dq over several column
    # blocks), with full and partial channel blocks.
    (1, 1, 70, 300, 64),
    (1, 2, 33, 260, 40),
]
DTYPES = ["f32", "f16", "bf16", "f64"]


def _inputs(B, H, N, M, C, dt, seed, integer=None, scale=1.0):
    q = gen((B, H, N, C), seed, dt, scale, integer)
    k = gen((B, H, C, M), seed + 1, dt, scale, integer)
    g = gen((B, H, N, M), seed + 2, dt, 1.0, 4 if integer else None)
    return q, k, g


def _run(dev, q, k, g):
    import laplacianformer_amd as lf

    L = lf.ext()
    qd, kd, gd = q.to(dev), k.to(dev), g.to(dev)
    B, H, N, C = q.shape
    M = k.shape[3]
    out = torch.empty((B, H, N, M), dtype=q.dtype, device=dev)
    dq = torch.empty_like(qd)
    dk = torch.empty_like(kd)
    dq2 = torch.empty_like(qd)
    dk2 = torch.empty_like(kd)
    L.LaplaceSubtraction_forward(qd, kd, out)
    L.LaplaceSubtraction_backward_query(gd, qd, kd, dq)
    L.LaplaceSubtraction_backward_key(gd, qd, kd, dk)
    L.LaplaceSubtraction_backward(gd, qd, kd, dq2, dk2)
    torch.cuda.synchronize()
    return out, dq, dk, dq2, dk2


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_laplace_parity(gpu, shape, dt):
    B, H, N, M, C = shape
    print(f"laplace parity {shape} {dt}", flush=True)
    q, k, g = _inputs(B, H, N, M, C, dt, seed=1000 + sum(shape))
    out, dq, dk, dq2, dk2 = _run(gpu, q, k, g)
    refs = l1_refs(q, k, g, dt)
    check_l1(out, dq, dk, refs, dt, "separate ")
    check_l1(out, dq2, dk2, refs, dt, "fused ")
    # The forward follows the reference's serial channel order exactly: bit-identical
    # to the fp32 (fp64 for double) serial oracle. The gradients are held to the
    # tolerance only (the fp16 backward sums 2g*step - g instead of g*sgn).
    assert_bitwise(out, oracle.laplace_forward(q, k, dt), dt, "forward bits")
    assert torch.equal(dq.cpu(), dq2.cpu()), "grad_query differs between the separate and fused entry points"


@pytest.mark.parametrize("M", [49, 64, 196, 256])
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_laplace_integer_ties(gpu, dt, M):
    """Integer inputs: every sum is exact and ties (sgn(0) = 0) are frequent."""
    B, H, N, C = 2, 2, 150, 64
    print(f"laplace integer ties {dt} M={M}", flush=True)
    q, k, g = _inputs(B, H, N, M, C, dt, seed=77, integer=3)
    out, dq, dk, dq2, dk2 = _run(gpu, q, k, g)
    ties = (q.float()[..., :, None, :] == k.float().transpose(-1, -2)[..., None, :, :]).sum().item()
    assert ties > 1000
    for got, ref in ((out, oracle.laplace_forward(q, k, dt)), (dq, oracle.laplace_backward_query(g, q, k, dt)),
                     (dk, oracle.laplace_backward_key(g, q, k, dt)), (dq2, oracle.laplace_backward_query(g, q, k, dt)),
                     (dk2, oracle.laplace_backward_key(g, q, k, dt))):
        assert_bitwise(got, ref, dt, "integer exact")


def test_laplace_full_workgroups(gpu):
    """fp16, M = 49, 512 rows per workgroup (B=32, N=4096: eight workgroups per slice): the
    column-split backward's waves take their largest row counts (up to 46 rows for the two older
    waves of a SIMD); every slice against the oracle."""
    B, H, N, M, C = 32, 1, 4096, 49, 64
    print("laplace 512-row workgroups", flush=True)
    q = gen((B, H, N, C), 1101, "f16")
    k = gen((B, H, M, C), 1102, "f16").transpose(-1, -2).contiguous()
    g = gen((B, H, N, M), 1103, "f16")
    out, dq, dk, dq2, dk2 = (t.cpu() for t in _run(gpu, q, k, g))
    assert torch.equal(dq, dq2)
    refs = l1_refs(q, k, g, "f16")
    check_l1(out, dq, dk, refs, "f16", "separate ")
    check_l1(out, dq2, dk2, refs, "f16", "fused ")


def test_laplace_config2_full(gpu):
    """B=32 H=1 N=3136 M=49 d=64 fp16, fwd + bwd."""
    B, H, N, M, C = 32, 1, 3136, 49, 64
    print("laplace config 2 full", flush=True)
    q = gen((B, H, N, C), 1002, "f16")
    k = gen((B, H, M, C), 1003, "f16").transpose(-1, -2).contiguous()
    g = gen((B, H, N, M), 1004, "f16")
    out, dq, dk, dq2, dk2 = _run(gpu, q, k, g)
    refs = l1_refs(q, k, g, "f16")
    check_l1(out, dq, dk, refs, "f16", "separate ")
    check_l1(out, dq2, dk2, refs, "f16", "fused ")
    assert_bitwise(out, oracle.laplace_forward(q, k, "f16"), "f16", "forward bits")
    assert torch.equal(dq.cpu(), dq2.cpu())
    # Size-independent identity: sum_i dq[i,c] + sum_j dk[c,j] = 0 (exactly, in real arithmetic).
    s = dq2.double().sum(dim=2) + dk2.double().sum(dim=3)
    assert s.abs().max().item() < 0.05 * dq2.double().abs().sum(dim=2).max().item() + 1.0


def test_laplace_config4_full(gpu):
    """BASELINE config 4 (bf16, B=16 H=8 N=4096 M=256 d=64): one GPU run of the
    whole batch, every (b, h) slice checked against the oracle (fp64 bounds and
    forward bits), one batch entry at a time."""
    B, H, N, M, C = 16, 8, 4096, 256, 64
    print("laplace config 4 full", flush=True)
    q = gen((B, H, N, C), 1004, "bf16", scale=0.5)
    k = gen((B, H, M, C), 1005, "bf16", scale=0.5).transpose(-1, -2).contiguous()
    g = gen((B, H, N, M), 1006, "bf16")
    out, dq, dk, dq2, dk2 = (t.cpu() for t in _run(gpu, q, k, g))
    assert torch.equal(dq, dq2)
    for b in range(B):
        sl = slice(b, b + 1)
        qs, ks, gs = q[sl], k[sl], g[sl]
        refs = l1_refs(qs, ks, gs, "bf16")
        check_l1(out[sl], dq[sl], dk[sl], refs, "bf16", f"batch {b} separate ")
        check_l1(out[sl], dq2[sl], dk2[sl], refs, "bf16", f"batch {b} fused ")
        assert_bitwise(out[sl], oracle.laplace_forward(qs, ks, "bf16"), "bf16", f"batch {b} forward bits")
        print(f"  batch {b} ok", flush=True)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16", "f64"])
def test_reduce_forward(gpu, dt):
    import laplacianformer_amd as lf

    for (B, H, N, M, C) in ((1, 2, 33, 9, 64), (1, 1, 10, 5, 3), (1, 1, 7, 3, 300)):
        print(f"reduce forward {dt} {(B, H, N, M, C)}", flush=True)
        q, k, _ = _inputs(B, H, N, M, C, dt, seed=5 + C)
        out = torch.empty((B, H, N, M), dtype=q.dtype, device=gpu)
        lf.ext().LaplaceSubtraction_reduce_forward(q.to(gpu), k.to(gpu), out)
        ref = oracle.laplace_reduce_forward(q, k, dt)
        got = out.cpu().to(torch.float64).numpy()
        assert np.array_equal(got, np.asarray(ref, dtype=np.float64)), (dt, C)


# Non-finite inputs in the backward (C = 64; M = 49: the 16-bit column-split
# kernel for fp16 / bf16, the clamped-step kernel for fp32; M = 64: the
# column-block kernel, with the same steps). Rows 0-7 of channel 3
# and rows 8-15 of channel 5 hold +inf / -inf, as do key columns 0-4 of channel 3
# and 10-14 of channel 5, so those pairs are infinite ties; rows 20 / 21 of
# channels 7 / 9 hold NaN of either sign.
#  * 16-bit: the order-preserving image of the patterns makes an infinite tie an
#    exact tie (sgn 0, as the reference's sign of inf - inf = NaN), and orders a
#    NaN pattern beyond the infinity of its sign (sgn +-1 against every key; the
#    reference gives 0) -- the oracle is run with the NaN replaced by a finite
#    value beyond every key of its channel.
#  * fp32: sgn of a NaN difference (a NaN input or an infinite tie) is -1 (the
#    clamp of NaN is 0); the reference gives 0 -- the oracle is run with each
#    infinity replaced by a finite value that keeps every comparison but makes the
#    ties q < k, and the NaN by a value below every key.
@pytest.mark.parametrize("M", [49, 64])
@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_laplace_nonfinite_backward(gpu, dt, M):
    import laplacianformer_amd as lf

    B, H, N, C = 1, 1, 64, 64
    print(f"laplace non-finite backward {dt} M={M}", flush=True)
    q, k, g = _inputs(B, H, N, M, C, dt, seed=91)
    q = q.float()
    k = k.float()
    q[..., 0:8, 3] = float("inf")
    q[..., 8:16, 5] = float("-inf")
    k[..., 3, 0:5] = float("inf")
    k[..., 5, 10:15] = float("-inf")
    q[..., 20, 7] = float("nan")
    q[..., 21, 9] = -float("nan") if dt != "f32" else float("nan")
    qd, kd = q.to(TORCH_DT[dt]), k.to(TORCH_DT[dt])
    L = lf.ext()
    dq = torch.empty_like(qd, device=gpu)
    dk = torch.empty_like(kd, device=gpu)
    L.LaplaceSubtraction_backward(g.to(gpu), qd.to(gpu), kd.to(gpu), dq, dk)
    torch.cuda.synchronize()
    qr, kr = q.double().clone(), k.double().clone()
    big = 1.0e30
    if dt != "f32":
        # The NaN's sign is that of its 16-bit pattern (the cast may not keep the
        # fp32 sign: torch rounds fp32 NaN to bf16 0xffff).
        for i, c in ((20, 7), (21, 9)):
            neg = qd[0, 0, i, c].view(torch.int16).item() < 0
            qr[..., i, c] = -big if neg else big
    else:
        qr[qr == float("inf")] = big
        qr[qr == float("-inf")] = -2 * big
        kr[kr == float("inf")] = 2 * big
        kr[kr == float("-inf")] = -big
        qr[torch.isnan(qr)] = -4 * big
    refs = l1_refs(qr, kr, g.double(), "f64")
    assert_l1_close(dq, refs["dq"][0], dt, f"{dt} dq non-finite", refs["dq"][1])
    assert_l1_close(dk, refs["dk"][0], dt, f"{dt} dk non-finite", refs["dk"][1])


# fp32 denormals (pinned, IEEE): every fp32 kernel keeps denormal operands and results, so a
# query/key pair whose difference is an fp32 denormal has sgn +-1 and adds that exact
# difference to the forward sum, as IEEE arithmetic and the fp32 oracle give. The
# reference's fast-math build (setup.py:29, -ftz) flushes them and gives sgn 0 and no
# contribution: the oracle's ftz mode restates that build, and the test checks that
# ours departs from it exactly at those pairs (by sum_j g over them in grad_query).
@pytest.mark.parametrize("M,C", [(49, 64), (64, 64), (5, 3)], ids=["m49", "m64", "m5c3"])
def test_laplace_f32_denormal_differences(gpu, M, C):
    import laplacianformer_amd as lf

    B, H, N = 1, 2, 64
    print(f"laplace fp32 denormal differences M={M} C={C}", flush=True)
    q, k, g = _inputs(B, H, N, M, C, "f32", seed=95)
    a, b = np.float32(1.5e-38), np.float32(1.2e-38)          # a - b is an exact fp32 denormal
    q[..., :, 0] = float(a)
    k[..., 0, 0::2] = float(b)                                # even columns: denormal difference
    k[..., 0, 1::4] = float(a)                                # ties
    q[..., 0:N:3, C - 1] = 1e-40                              # denormal query values
    k[..., C - 1, 0:M:3] = 0.0
    L = lf.ext()
    qd, kd, gd = q.to(gpu), k.to(gpu), g.to(gpu)
    out = torch.empty((B, H, N, M), device=gpu)
    dq, dk = torch.empty_like(qd), torch.empty_like(kd)
    L.LaplaceSubtraction_forward(qd, kd, out)
    L.LaplaceSubtraction_backward(gd, qd, kd, dq, dk)
    dq1, dk1 = torch.empty_like(qd), torch.empty_like(kd)
    L.LaplaceSubtraction_backward_query(gd, qd, kd, dq1)
    L.LaplaceSubtraction_backward_key(gd, qd, kd, dk1)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.laplace_forward(q, k, "f32"), "f32", "forward (IEEE, denormals kept)")
    refs = l1_refs(q, k, g, "f32")
    for got, key in ((dq, "dq"), (dk, "dk"), (dq1, "dq"), (dk1, "dk")):
        assert_l1_close(got, refs[key][0], "f32", f"{key} (IEEE signs of denormal differences)", refs[key][1])
    # Where the flushing build differs: channel 0 of every row loses sum over the even
    # columns of g (sgn +1 there, 0 when flushed).
    rq_z = oracle.laplace_backward_query(g, q, k, "f32", ftz=True)
    gap = (dq.cpu().double()[..., 0] - torch.from_numpy(rq_z[..., 0]).double())
    want = g.double()[..., 0::2].sum(-1)
    assert torch.allclose(gap, want, rtol=1e-5, atol=1e-5 * g.abs().double().sum(-1).max().item())


@pytest.mark.parametrize("M", [49, 300])
def test_laplace_misaligned_grad(gpu, M):
    """fp16 grad_output that is a contiguous view at an odd element offset (its
    data is 2-byte but not 4-byte aligned): the backward kernels that read
    grad rows as 4-byte words must not be chosen; results match the oracle."""
    import laplacianformer_amd as lf

    B, H, N, C = 1, 2, 90, 64
    print(f"laplace misaligned grad M={M}", flush=True)
    q, k, g = _inputs(B, H, N, M, C, "f16", seed=17 + M)
    buf = torch.empty(g.numel() + 1, dtype=torch.float16, device=gpu)
    buf[1:] = g.reshape(-1).to(gpu)
    gd = buf[1:].view(g.shape)
    assert gd.is_contiguous() and gd.storage_offset() == 1
    L = lf.ext()
    qd, kd = q.to(gpu), k.to(gpu)
    dq, dk = torch.empty_like(qd), torch.empty_like(kd)
    dq1, dk1 = torch.empty_like(qd), torch.empty_like(kd)
    L.LaplaceSubtraction_backward(gd, qd, kd, dq, dk)
    L.LaplaceSubtraction_backward_query(gd, qd, kd, dq1)
    L.LaplaceSubtraction_backward_key(gd, qd, kd, dk1)
    torch.cuda.synchronize()
    refs = l1_refs(q, k, g, "f16")
    for tag, a, b in (("fused", dq, dk), ("separate", dq1, dk1)):
        assert_l1_close(a, refs["dq"][0], "f16", f"{tag} dq", refs["dq"][1])
        assert_l1_close(b, refs["dk"][0], "f16", f"{tag} dk", refs["dk"][1])


def test_empty_and_errors(gpu):
    import laplacianformer_amd as lf

    L = lf.ext()
    q = torch.zeros((1, 1, 0, 8), device=gpu)
    k = torch.zeros((1, 1, 8, 5), device=gpu)
    out = torch.empty((1, 1, 0, 5), device=gpu)
    L.LaplaceSubtraction_forward(q, k, out)
    # Reduction length zero: gradients are zero.
    q = torch.randn((1, 1, 4, 8), device=gpu)
    k0 = torch.zeros((1, 1, 8, 0), device=gpu)
    g0 = torch.zeros((1, 1, 4, 0), device=gpu)
    dq = torch.full((1, 1, 4, 8), 7.0, device=gpu)
    L.LaplaceSubtraction_backward_query(g0, q, k0, dq)
    assert dq.abs().max().item() == 0
    with pytest.raises(RuntimeError, match="query and key must match"):
        L.LaplaceSubtraction_forward(q, torch.zeros((1, 1, 7, 5), device=gpu), torch.empty((1, 1, 4, 5), device=gpu))
    with pytest.raises(RuntimeError, match="contiguous"):
        L.LaplaceSubtraction_forward(q.transpose(2, 3), k, torch.empty((1, 1, 8, 5), device=gpu))
    with pytest.raises(RuntimeError, match="not implemented for 'Int'"):
        L.LaplaceSubtraction_forward(q.int(), k.int(), torch.empty((1, 1, 4, 5), device=gpu, dtype=torch.int32))


def test_capi_direct(gpu):
    """The C ABI called with raw pointers and an explicit stream matches the oracle."""
    import laplacianformer_amd as lf

    lib = lf.capi()
    B, H, N, M, C = 2, 1, 200, 49, 64
    print("capi direct", flush=True)
    q, k, g = _inputs(B, H, N, M, C, "f16", seed=31)
    qd, kd, gd = q.to(gpu), k.to(gpu), g.to(gpu)
    out = torch.empty((B, H, N, M), dtype=torch.float16, device=gpu)
    dq = torch.empty_like(qd)
    dk = torch.empty_like(kd)
    st = torch.cuda.Stream()
    dt = lf.dtype_code(torch.float16)
    ws_bytes = lib.lfamd_laplace_backward_workspace_size(dt, B, H, N, M, C)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=gpu)
    torch.cuda.synchronize()
    s = ctypes.c_void_p(st.cuda_stream)
    lf.check(lib.lfamd_laplace_forward(dt, qd.data_ptr(), kd.data_ptr(), out.data_ptr(), B, H, N, M, C, s))
    lf.check(lib.lfamd_laplace_backward(dt, gd.data_ptr(), qd.data_ptr(), kd.data_ptr(), dq.data_ptr(),
                                        dk.data_ptr(), B, H, N, M, C, ws.data_ptr(), ws_bytes, s))
    st.synchronize()
    assert_bitwise(out, oracle.laplace_forward(q, k, "f16"), "f16")
    check_l1(out, dq, dk, l1_refs(q, k, g, "f16"), "f16", "capi ")
    # Too small a workspace is rejected before anything is launched.
    rc = lib.lfamd_laplace_backward_key(dt, gd.data_ptr(), qd.data_ptr(), kd.data_ptr(), dk.data_ptr(),
                                        B, H, N, M, C, ws.data_ptr(), 1, s)
    assert rc == 1 and b"workspace" in lib.lfamd_last_error()
    # A workspace off the partials' 4-byte alignment is rejected too.
    rc = lib.lfamd_laplace_backward_key(dt, gd.data_ptr(), qd.data_ptr(), kd.data_ptr(), dk.data_ptr(),
                                        B, H, N, M, C, ws.data_ptr() + 2, ws_bytes, s)
    assert rc == 1 and b"aligned" in lib.lfamd_last_error()


@pytest.mark.parametrize("dt,M", [("f32", 49), ("bf16", 256), ("f16", 49)])
def test_repeat_deterministic(gpu, dt, M):
    """Repeated backward calls on one stream give identical bits (every sum in a fixed order)."""
    import laplacianformer_amd as lf

    B, H, N, C = 4, 2, 700, 64
    q, k, g = _inputs(B, H, N, M, C, dt, seed=9)
    qd, kd, gd = q.to(gpu), k.to(gpu), g.to(gpu)
    res = []
    for _ in range(3):
        dq = torch.empty_like(qd)
        dk = torch.empty_like(kd)
        lf.ext().LaplaceSubtraction_backward(gd, qd, kd, dq, dk)
        res.append((dq.cpu(), dk.cpu()))
    torch.cuda.synchronize()
    for a, b in res[1:]:
        assert torch.equal(a, res[0][0]) and torch.equal(b, res[0][1])


def test_autograd_function(gpu):
    import laplacianformer_amd as lf

    q, k, g = _inputs(1, 2, 90, 49, 32, "f32", seed=3)
    qd = q.to(gpu).requires_grad_()
    kd = k.to(gpu).requires_grad_()
    out = lf.laplace_subtraction(qd, kd)
    out.backward(g.to(gpu))
    check_l1(out, qd.grad, kd.grad, l1_refs(q, k, g, "f32"), "f32", "autograd ")


def test_key_layout_mc(gpu):
    """key_layout="mc" takes the key as [B,H,M,d] (BASELINE config 1 fixture holds that layout and
    its fp64 gradient from torch.cdist)."""
    import os

    import laplacianformer_amd as lf

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "config1_l1.npz"))
    qd = torch.from_numpy(z["q"]).to(gpu).requires_grad_()
    kd = torch.from_numpy(z["k_mc"]).to(gpu).requires_grad_()
    out = lf.laplace_subtraction(qd, kd, key_layout="mc")
    out.backward(torch.from_numpy(z["g"]).to(gpu))
    ga = np.abs(z["g"].astype(np.float64))
    assert_l1_close(out, z["out"], "f32", "mc forward")
    assert_l1_close(qd.grad, z["dq"], "f32", "mc dq", np.broadcast_to(ga.sum(3, keepdims=True), qd.shape))
    assert_l1_close(kd.grad, z["dk_mc"], "f32", "mc dk",
                    np.broadcast_to(np.swapaxes(ga.sum(2, keepdims=True), -1, -2), kd.shape))
    with pytest.raises(ValueError):
        lf.laplace_subtraction(qd, kd, key_layout="xy")


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16", "f64"])
def test_golden_kat(gpu, dt):
    """Integer known-answer fixture (tests/golden/kat_l1.npz): exact in every type."""
    import os

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "kat_l1.npz"))
    q, k, g = (torch.from_numpy(z[n]).to(TORCH_DT[dt]) for n in ("q", "k", "g"))
    out, dq, dk, dq2, dk2 = _run(gpu, q, k, g)
    for got, name in ((out, "out"), (dq, "dq"), (dk, "dk"), (dq2, "dq"), (dk2, "dk")):
        assert np.array_equal(got.cpu().double().numpy(), z[name]), (dt, name)


def test_golden_config1(gpu):
    """BASELINE config 1 fixture (fp64 torch.cdist results) against the fp32 kernels."""
    import os

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "config1_l1.npz"))
    q = torch.from_numpy(z["q"])
    kT = torch.from_numpy(z["k_mc"]).transpose(-1, -2).contiguous()
    g = torch.from_numpy(z["g"])
    out, dq, dk, dq2, dk2 = _run(gpu, q, kT, g)
    ga = np.abs(z["g"].astype(np.float64))
    assert_l1_close(out, z["out"], "f32", "fixture forward")
    assert_l1_close(dq2, z["dq"], "f32", "fixture dq", np.broadcast_to(ga.sum(3, keepdims=True), dq2.shape))
    assert_l1_close(dk2, np.swapaxes(z["dk_mc"], -1, -2), "f32", "fixture dk",
                    np.broadcast_to(ga.sum(2, keepdims=True), dk2.shape))


def test_laplace_beyond_2pow31_elements(gpu):
    """Output and grad_output with more than 2^31 elements (fp16, N = 2^23 + 128, M = 256,
    C = 8): 64-bit indexing everywhere. grad_output is zero except for sampled rows at the
    start, middle and end, so grad_key depends on those rows only and every gradient is
    checked exactly against the oracle; forward rows at the same places bit for bit."""
    import laplacianformer_amd as lf

    L = lf.ext()
    N, M, C = (1 << 23) + 128, 256, 8
    assert N * M > 2 ** 31
    print("laplace beyond 2^31 elements", flush=True)
    q = gen((1, 1, N, C), 2031, "f16")
    k = gen((1, 1, C, M), 2032, "f16")
    rows = [0, 1, 63, N // 2, N // 2 + 5, N - 129, N - 2, N - 1]
    gs = gen((1, 1, len(rows), M), 2033, "f16")
    qd, kd = q.to(gpu), k.to(gpu)
    gd = torch.zeros((1, 1, N, M), dtype=torch.float16, device=gpu)
    gd[0, 0, rows] = gs[0, 0].to(gpu)
    out = torch.empty((1, 1, N, M), dtype=torch.float16, device=gpu)
    dq = torch.empty_like(qd)
    dk = torch.empty_like(kd)
    L.LaplaceSubtraction_forward(qd, kd, out)
    L.LaplaceSubtraction_backward(gd, qd, kd, dq, dk)
    torch.cuda.synchronize()
    qs = q[:, :, rows]
    assert_bitwise(out[:, :, rows], oracle.laplace_forward(qs, k, "f16"), "f16", "forward rows")
    refs = l1_refs(qs, k, gs, "f16")
    check_l1(out[:, :, rows], dq[:, :, rows], dk, refs, "f16", "sampled rows ")
    zero_rows = torch.ones(N, dtype=torch.bool)
    zero_rows[rows] = False
    assert not dq[0, 0][zero_rows.to(gpu)].any(), "grad_query of rows with zero grad_output"

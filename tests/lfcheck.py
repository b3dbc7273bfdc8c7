"""Shared helpers of the test suite: seeded inputs and the comparison rules.

Comparison rules (fixed up front, per the operator contract):
* L1 ops are compared with the fp64 oracle (exact up to ~1e-16 of the sum).
  Elementwise |x - ref| <= ulp_out + 1e-5 * sum|terms| (fp32 accumulation;
  1e-12 for fp64), ulp_out = one output ulp for fp16/bf16 outputs, 0 otherwise.
  For the all-positive forward sum sum|terms| = |ref|, i.e. plain 1e-5 relative;
  for dq/dk (sums of +-g with cancellation) it is sum|g| over the reduced index.
  Norm-relative max|x - ref| / max|ref| <= 1e-5 (fp32), 1e-12 (fp64), 2e-3
  (fp16) and 2^-8 (bf16, whose rounding unit alone exceeds 2e-3).
* Forward and dq additionally match the fp32 serial-order oracle bit for bit
  (same association order as the reference).
* NewtonInverse: elementwise |x - ref| <= 1e-4 * max|ref| at the same iteration
  count (fp32 math; fp16/bf16 outputs add one output ulp).
"""
from __future__ import annotations

import numpy as np
import torch

import oracle

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}


def gen(shape, seed, dtype="f32", scale=1.0, integer=None):
    """Seeded CPU normal (or integer-valued) tensor cast to the element type."""
    g = torch.Generator().manual_seed(seed)
    if integer is not None:
        x = torch.randint(-integer, integer + 1, shape, generator=g).to(torch.float32)
    else:
        x = torch.randn(shape, generator=g, dtype=torch.float32) * scale
    return x.to(TORCH_DT[dtype])


def _ulp(ref: torch.Tensor) -> torch.Tensor:
    """Spacing of the element type at |ref| (ref already in that type)."""
    a = ref.abs().to(torch.float32)
    if ref.dtype == torch.float16:
        tiny, mant = 2.0 ** -24, 10
    else:  # bfloat16
        tiny, mant = 2.0 ** -133, 7
    e = torch.floor(torch.log2(torch.clamp(a, min=np.finfo(np.float32).tiny)))
    return torch.clamp(torch.exp2(e - mant), min=tiny)


def l1_refs(q, k, g, dtype):
    """fp64 oracle results of the three L1 ops plus the per-element scale
    sum|terms| of each sum (forward: the result itself; dq: sum_j |g_ij|;
    dk: sum_i |g_ij|)."""
    rf = oracle.laplace_forward(q, k, "f64")
    rq = oracle.laplace_backward_query(g, q, k, "f64")
    rk = oracle.laplace_backward_key(g, q, k, "f64")
    ga = np.abs(oracle.widen(g, "f64"))
    sq = np.broadcast_to(ga.sum(axis=3, keepdims=True), rq.shape)
    sk = np.broadcast_to(ga.sum(axis=2, keepdims=True), rk.shape)
    return {"fwd": (rf, None), "dq": (rq, sq), "dk": (rk, sk)}


NORM_TOL = {"f32": 1e-5, "f64": 1e-12, "f16": 2e-3, "bf16": 2.0 ** -8}


def assert_l1_close(got: torch.Tensor, ref64: np.ndarray, dtype: str, what: str = "", scale=None):
    """Checks an L1-op result against the fp64 oracle.

    Elementwise: |x - ref| <= ulp_out(ref) + acc * scale, where scale is
    sum|terms| of that output's sum (|ref| for the all-positive forward sum),
    acc = 1e-5 (fp32 accumulation; 1e-12 for fp64) and ulp_out is one unit in the
    last place of the fp16/bf16 output type (0 for fp32/fp64 outputs).
    Norm-relative: max|x - ref| / max|ref| <= 1e-5 (fp32), 1e-12 (fp64),
    2e-3 (fp16), 2^-8 (bf16: its own rounding unit exceeds 2e-3).
    """
    got_c = got.detach().cpu()
    ref = torch.from_numpy(np.ascontiguousarray(ref64, dtype=np.float64))
    g64 = got_c.to(torch.float64)
    assert g64.shape == ref.shape, (what, g64.shape, ref.shape)
    if ref.numel() == 0:
        return
    assert torch.isfinite(g64).all(), what
    err = (g64 - ref).abs()
    mx = ref.abs().max().item()
    if mx > 0:
        assert err.max().item() / mx <= NORM_TOL[dtype], (what, "norm-relative", err.max().item() / mx)
    sc = ref.abs() if scale is None else torch.from_numpy(np.ascontiguousarray(scale, dtype=np.float64))
    acc = 1e-12 if dtype == "f64" else 1e-5
    lim = acc * sc
    if dtype in ("f16", "bf16"):
        lim = lim + _ulp(ref.to(TORCH_DT[dtype])).to(torch.float64)
    bad = err > lim
    assert not bool(bad.any()), (what, "elementwise", int(bad.sum()), (err - lim).max().item())


def check_l1(out, dq, dk, refs, dtype, tag=""):
    assert_l1_close(out, refs["fwd"][0], dtype, tag + "forward")
    assert_l1_close(dq, refs["dq"][0], dtype, tag + "dq", refs["dq"][1])
    assert_l1_close(dk, refs["dk"][0], dtype, tag + "dk", refs["dk"][1])


def assert_bitwise(got: torch.Tensor, acc_ref: np.ndarray, dtype: str, what: str = ""):
    rref = oracle.round_to(acc_ref, dtype)
    rref = torch.as_tensor(rref) if not isinstance(rref, torch.Tensor) else rref
    got_c = got.detach().cpu()
    eq = got_c.to(TORCH_DT[dtype]).view(-1).view(torch.int16 if dtype in ("f16", "bf16") else (torch.int32 if dtype == "f32" else torch.int64)) == \
        rref.to(TORCH_DT[dtype]).contiguous().view(-1).view(torch.int16 if dtype in ("f16", "bf16") else (torch.int32 if dtype == "f32" else torch.int64))
    assert bool(eq.all()), (what, int((~eq).sum()), eq.numel())


def assert_newton_close(got: torch.Tensor, ref: np.ndarray, dtype: str, what: str = "", rtol=1e-4):
    g = got.detach().cpu().to(torch.float64)
    r = torch.from_numpy(np.ascontiguousarray(ref)).to(torch.float64)
    assert torch.isfinite(g).all(), what
    mx = r.abs().max().item()
    tol = rtol * mx
    if dtype in ("f16", "bf16"):
        tol = tol + _ulp(r.to(TORCH_DT[dtype])).to(torch.float64)
    err = (g - r).abs()
    bad = err > tol
    assert not bool(bad.any()), (what, (err / max(mx, 1e-300)).max().item())

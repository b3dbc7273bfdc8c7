"""Autograd wrappers over the drop-in extension.

The reference ships the raw out-parameter ops only (its autograd glue is not in
the repository); these Functions pair forward with backward the way a model
uses them: LaplaceSubtraction forward (reference src/wrapper.cpp:81-82) with
the fused dq+dk backward (one pass; equal to backward_query + backward_key,
src/wrapper.cpp:84-88), and NewtonInverse forward with its -V^T G V^T backward
(src/wrapper.cpp:93-96). LaplaceKernelFunction is the caller-side
exp(-scale * dist) of the LaplacianFormer layer with the exp fused into the
HIP kernels where the fused path covers the sizes.
"""
from __future__ import annotations

import torch

from ._lib import ext


class LaplaceSubtractionFunction(torch.autograd.Function):
    """dist[b,h,i,j] = sum_c |query[b,h,i,c] - key[b,h,c,j]| with key channel-major."""

    @staticmethod
    def forward(ctx, query: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
        query = query.contiguous()
        key = key.contiguous()
        B, H, N, _ = query.shape
        M = key.shape[3]
        out = torch.empty((B, H, N, M), dtype=query.dtype, device=query.device)
        ext().LaplaceSubtraction_forward(query, key, out)
        ctx.save_for_backward(query, key)
        return out

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        query, key = ctx.saved_tensors
        grad = grad.contiguous()
        need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dq = torch.empty_like(query) if need_q else None
        dk = torch.empty_like(key) if need_k else None
        if need_q and need_k:
            ext().LaplaceSubtraction_backward(grad, query, key, dq, dk)
        elif need_q:
            ext().LaplaceSubtraction_backward_query(grad, query, key, dq)
        elif need_k:
            ext().LaplaceSubtraction_backward_key(grad, query, key, dk)
        return dq, dk


def _acc_type(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


class LaplaceKernelFunction(torch.autograd.Function):
    """K[b,h,i,j] = exp(-scale * sum_c |query[b,h,i,c] - key[b,h,c,j]|), key channel-major.

    K is fp32 (fp64 for fp64 inputs); the distance is never rounded to the input
    type. Where the fused HIP path applies, the exp runs in the forward's epilogue
    and the backward forms g = -scale * dK * K while staging its batches; elsewhere
    both sides compose the plain ops on inputs upcast to the accumulation type,
    which is the same arithmetic (fp32 accumulation of exact differences).
    """

    @staticmethod
    def forward(ctx, query: torch.Tensor, key: torch.Tensor, scale: float) -> torch.Tensor:
        query = query.contiguous()
        key = key.contiguous()
        B, H, N, _ = query.shape
        M = key.shape[3]
        scale = float(scale)
        acc = _acc_type(query.dtype)
        out = torch.empty((B, H, N, M), dtype=acc, device=query.device)
        if not (acc == torch.float32 and ext().LaplaceKernel_forward(query, key, out, scale)):
            dist = torch.empty_like(out)
            ext().LaplaceSubtraction_forward(query.to(acc), key.to(acc), dist)
            out = torch.exp(dist * -scale)
        ctx.scale = scale
        ctx.save_for_backward(query, key, out)
        return out

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        query, key, kern = ctx.saved_tensors
        need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_q or need_k):
            return None, None, None
        grad = grad.contiguous().to(kern.dtype)
        dq = torch.empty_like(query) if need_q else None
        dk = torch.empty_like(key) if need_k else None
        if kern.dtype == torch.float32 and ext().LaplaceKernel_backward(grad, kern, query, key, dq, dk, ctx.scale):
            return dq, dk, None
        acc = kern.dtype
        g = grad * kern * -ctx.scale
        qa, ka = query.to(acc), key.to(acc)
        dqa = torch.empty_like(qa) if need_q else None
        dka = torch.empty_like(ka) if need_k else None
        if need_q and need_k:
            ext().LaplaceSubtraction_backward(g, qa, ka, dqa, dka)
        elif need_q:
            ext().LaplaceSubtraction_backward_query(g, qa, ka, dqa)
        else:
            ext().LaplaceSubtraction_backward_key(g, qa, ka, dka)
        return (dqa.to(query.dtype) if need_q else None), (dka.to(key.dtype) if need_k else None), None


class NewtonInverseFunction(torch.autograd.Function):
    """Newton-Schulz approximate inverse of mat + 0.01 I; backward -V^T G V^T."""

    @staticmethod
    def forward(ctx, mat: torch.Tensor, iters: int) -> torch.Tensor:
        mat = mat.contiguous()
        out = torch.empty_like(mat)
        ext().NewtonInverse_forward(mat, out, int(iters))
        ctx.save_for_backward(out)
        return out

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        (inv,) = ctx.saved_tensors
        dmat = torch.empty_like(inv)
        ext().NewtonInverse_backward(grad.contiguous(), inv, dmat)
        return dmat, None


_MIX_MAX = 64  # widest inner / output dimension of the HIP row-product kernel


def _mixable(*widths: int) -> bool:
    return all(0 < w <= _MIX_MAX for w in widths)


def mix_rows(a: torch.Tensor, b_qp: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """c[..., n, q] = sum_p a[..., n, p] * b_qp[..., q, p], summed in float32 on the
    HIP row-product kernel and returned in ``out_dtype`` (fp32/fp16/bf16, one
    rounding); a contiguous fp32/fp16/bf16, b_qp an fp32 view of any strides whose
    batch dims collapse to one stride; widths <= 64."""
    c = torch.empty(a.shape[:-1] + (b_qp.shape[-2],), dtype=out_dtype, device=a.device)
    ext().MixRows(a.contiguous(), b_qp.float(), c)
    return c


def tall_t(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T @ b -> fp32 [..., P, Q] for a tall fp32 a [..., N, P] and b [..., N, Q]
    (fp32/fp16/bf16, used as fp32): the HIP split-row reduction where P, Q <= 64,
    torch.matmul elsewhere."""
    if a.dtype == torch.float32 and b.dtype in (torch.float32, torch.float16, torch.bfloat16) \
            and _mixable(a.shape[-1], b.shape[-1]):
        a, b = a.contiguous(), b.contiguous()
        c = torch.empty(a.shape[:-2] + (a.shape[-1], b.shape[-1]), dtype=torch.float32, device=a.device)
        ext().TallT(a, b, c)
        return c
    return torch.matmul(a.transpose(-1, -2).float(), b.float())


class TallMixFunction(torch.autograd.Function):
    """C = A @ W for a tall A [..., N, P] and a small fp32 W [..., P, Q] (the
    attention layer's K_qm . (V^-1 . kv)); grad_A = G W^T on the row-product
    kernel, grad_W = A^T G on the split-row reduction (tall_t)."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, w: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
        ctx.save_for_backward(a, w)
        return mix_rows(a, w.transpose(-1, -2), out_dtype)

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        a, w = ctx.saved_tensors
        g = g.contiguous()
        ga = mix_rows(g, w, a.dtype) if ctx.needs_input_grad[0] else None
        gw = tall_t(a.float(), g).to(w.dtype) if ctx.needs_input_grad[1] else None
        return ga, gw, None


class TallProductFunction(torch.autograd.Function):
    """C = A^T @ B for tall A [..., N, P] (fp32) and B [..., N, Q] (any float
    type, used as fp32) -> [..., P, Q] (the layer's K_km^T V); forward on the
    split-row reduction (tall_t), both row-streaming backward products on the
    row-product kernel: grad_A = B G^T, grad_B = A G."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        ctx.save_for_backward(a, b)
        return tall_t(a, b)

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        a, b = ctx.saved_tensors
        g = g.float().contiguous()
        ga = mix_rows(b, g, a.dtype) if ctx.needs_input_grad[0] else None
        gb = mix_rows(a, g.transpose(-1, -2), b.dtype) if ctx.needs_input_grad[1] else None
        return ga, gb


def tall_mix(a: torch.Tensor, w: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """a @ w for tall a [..., N, P] and small fp32 w [..., P, Q], returned in ``out_dtype``
    (default w's type); the HIP row-product kernel where P, Q <= 64, a is fp32/fp16/bf16
    and out_dtype is one of those, torch.matmul elsewhere."""
    out_dtype = out_dtype or w.dtype
    if (a.dtype != torch.float64 and out_dtype != torch.float64 and w.dtype != torch.float64
            and _mixable(a.shape[-1], w.shape[-1])):
        return TallMixFunction.apply(a, w, out_dtype)
    return torch.matmul(a, w).to(out_dtype)


def tall_product(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T @ b for tall a [..., N, P] and b [..., N, Q] (b used in a's type)."""
    if a.dtype != torch.float64 and _mixable(a.shape[-1], b.shape[-1]):
        return TallProductFunction.apply(a, b)
    return torch.matmul(a.transpose(-1, -2), b.to(a.dtype))


def laplace_subtraction(query: torch.Tensor, key: torch.Tensor, key_layout: str = "cm") -> torch.Tensor:
    """Pairwise L1 distance with autograd.

    ``key_layout="cm"`` takes the reference's channel-major key ``[B,H,C,M]``;
    ``"mc"`` takes ``[B,H,M,C]`` and transposes it (one copy).
    """
    if key_layout == "mc":
        key = key.transpose(-1, -2)
    elif key_layout != "cm":
        raise ValueError("key_layout must be 'cm' or 'mc'")
    return LaplaceSubtractionFunction.apply(query, key)


def laplace_kernel(query: torch.Tensor, key: torch.Tensor, scale: float) -> torch.Tensor:
    """exp(-scale * L1(query, key)) with autograd, key channel-major ``[B,H,C,M]``;
    fp32 result (fp64 for fp64 inputs)."""
    return LaplaceKernelFunction.apply(query, key, scale)


def newton_inverse(mat: torch.Tensor, iters: int) -> torch.Tensor:
    """Newton-Schulz inverse with autograd; mat is ``[B,H,n,n]``, 1 <= n <= 256."""
    return NewtonInverseFunction.apply(mat, iters)

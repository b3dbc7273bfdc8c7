"""LaplacianFormer attention layer: the immediate caller of LaplaceSubtraction
and NewtonInverse (no counterpart in the reference, which ships the two ops
only; the composition follows BASELINE config 5 of this build).

For each (batch, head), with tokens on a grid of gh x gw:
  Km   = pool x pool average pooling of K over the grid        (M landmarks)
  Kxy  = exp(-L1(x, y) / sqrt(d))                              (Laplacian kernel)
  out  = K_qm . NewtonInverse(K_mm, iters) . (K_mk . V)
The landmark-to-token kernel K_mk is taken as the transpose of K_km
(L1 is symmetric), so every distance uses the landmarks as the channel-major
key and no [B,H,d,N] copy of K is made. q, k and the landmarks (pooled in
fp32, stored in the input type) enter the distances in the input type; the
distances accumulate in fp32 and are never rounded to it (an fp16 distance,
~70 at d = 64, would move exp(-dist/8) by ~0.4 %): the Laplacian kernels come
out of the fused distance+exp op in fp32 (fp64 for fp64 inputs), and the
products from there on run in that type. The result is returned in the input
type. The products that stream the N-row matrices (K_qm . W with
W = NewtonInverse(K_mm) . K_km^T V, and in the backward G . W^T, V . grad_kv^T,
K_km . grad_kv) run on the HIP row-product kernel (inner and output widths
<= 64), K_km^T V and K_qm^T G on the HIP split-row reduction, the M x M
products on the library GEMM.
"""
from __future__ import annotations

import math

import torch

from ._lib import ext
from .functional import _acc_type, laplace_kernel, mix_rows, newton_inverse, tall_mix, tall_product, tall_t


def landmarks(k: torch.Tensor, grid: tuple[int, int], pool: int, dtype: torch.dtype | None = None) -> torch.Tensor:
    """pool x pool average pooling of k [B,H,N,d] over its gh x gw token grid -> [B,H,M,d],
    accumulated and returned in ``dtype`` (default: k's type) without a converted copy of k."""
    B, H, N, d = k.shape
    gh, gw = grid
    if gh * gw != N or gh % pool or gw % pool:
        raise ValueError(f"token grid {gh}x{gw} does not match N={N} or pool={pool}")
    # A mean over the two in-window axes of a view: its backward is a broadcast,
    # cheaper than avg_pool2d's on this channel-last layout.
    x = k.reshape(B, H, gh // pool, pool, gw // pool, pool, d)
    return x.mean(dim=(3, 5), dtype=dtype).reshape(B, H, -1, d)


class _PooledLandmarks(torch.autograd.Function):
    """landmarks(k, grid, pool, acc) rounded to k's type, with a backward that forms
    grad_k = (grad_km / pool^2) broadcast over each pool x pool patch in k's type in
    one copy (autograd's mean backward would expand in the accumulation type, divide,
    then cast: two passes over an fp32 [B,H,N,d] tensor). Same values: the
    division is done in the accumulation type and rounded once to k's type."""

    @staticmethod
    def forward(ctx, k: torch.Tensor, grid: tuple[int, int], pool: int, acc: torch.dtype) -> torch.Tensor:
        ctx.shape, ctx.grid, ctx.pool, ctx.acc = k.shape, grid, pool, acc
        return landmarks(k, grid, pool, dtype=acc).to(k.dtype)

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        B, H, N, d = ctx.shape
        gh, gw = ctx.grid
        p = ctx.pool
        gs = (g.to(ctx.acc) / (p * p)).to(g.dtype).reshape(B, H, gh // p, 1, gw // p, 1, d)
        return gs.expand(B, H, gh // p, p, gw // p, p, d).reshape(B, H, N, d), None, None, None


def _kernel_fwd(query: torch.Tensor, key_cm: torch.Tensor, scale: float) -> torch.Tensor:
    """exp(-scale * L1(query, key)) in fp32: the fused HIP op, or the composition
    LaplaceKernelFunction falls back to (same arithmetic)."""
    B, H, N, _ = query.shape
    out = torch.empty((B, H, N, key_cm.shape[3]), dtype=torch.float32, device=query.device)
    if ext().LaplaceKernel_forward(query, key_cm, out, scale):
        return out
    dist = torch.empty_like(out)
    ext().LaplaceSubtraction_forward(query.float(), key_cm.float(), dist)
    return torch.exp(dist * -scale)


def _kernel_bwd(grad: torch.Tensor, kern: torch.Tensor, query: torch.Tensor, key_cm: torch.Tensor, scale: float):
    """(grad_query, grad_key) of exp(-scale * L1(query, key_cm)) for fp32 dL/dK = grad."""
    dq, dk = torch.empty_like(query), torch.empty_like(key_cm)
    if ext().LaplaceKernel_backward(grad, kern, query, key_cm, dq, dk, scale):
        return dq, dk
    qa, ka = query.float(), key_cm.float()
    dqa, dka = torch.empty_like(qa), torch.empty_like(ka)
    ext().LaplaceSubtraction_backward(grad * kern * -scale, qa, ka, dqa, dka)
    return dqa.to(query.dtype), dka.to(key_cm.dtype)


class _AttentionFunction(torch.autograd.Function):
    """The whole layer as one autograd node for 16-bit / fp32 inputs whose widths the
    row-product kernel takes (d, M <= 64): the same operations as the composition in
    laplacian_attention, issued directly on both sides (one node instead of about ten,
    so an eager step is not bound by the host's autograd bookkeeping)."""

    @staticmethod
    def forward(ctx, q, k, v, grid, pool, iters):
        in_dtype = q.dtype
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        d = q.shape[-1]
        s = 1.0 / math.sqrt(d)
        km = landmarks(k, grid, pool, dtype=torch.float32).to(in_dtype)   # [B,H,M,d]
        km_cm = km.transpose(-1, -2).contiguous()                          # [B,H,d,M]
        k_qm = _kernel_fwd(q, km_cm, s)
        k_mm = _kernel_fwd(km, km_cm, s)
        k_km = _kernel_fwd(k, km_cm, s)
        inv = torch.empty_like(k_mm)
        ext().NewtonInverse_forward(k_mm, inv, int(iters))
        kv = tall_t(k_km, v)                                               # K_km^T V  [B,H,M,d]
        w = torch.matmul(inv, kv)                                         # [B,H,M,d]
        out = mix_rows(k_qm, w.transpose(-1, -2), in_dtype)              # K_qm W, rounded once
        ctx.grid, ctx.pool, ctx.s = grid, pool, s
        ctx.save_for_backward(q, k, v, km, km_cm, k_qm, k_mm, k_km, inv, kv, w)
        return out

    @staticmethod
    def backward(ctx, g):
        q, k, v, km, km_cm, k_qm, k_mm, k_km, inv, kv, w = ctx.saved_tensors
        s, p = ctx.s, ctx.pool
        g = g.contiguous()
        d_kqm = mix_rows(g, w, torch.float32)                             # G W^T       [B,H,N,M]
        d_w = tall_t(k_qm, g)                                             # K_qm^T G    [B,H,M,d]
        d_inv = torch.matmul(d_w, kv.transpose(-1, -2))                   # [B,H,M,M]
        d_kv = torch.matmul(inv.transpose(-1, -2), d_w)                   # [B,H,M,d]
        d_kkm = mix_rows(v, d_kv, torch.float32)                          # V dkv^T     [B,H,N,M]
        d_v = mix_rows(k_km, d_kv.transpose(-1, -2), v.dtype)             # K_km dkv    [B,H,N,d]
        d_kmm = torch.empty_like(k_mm)
        ext().NewtonInverse_backward(d_inv.contiguous(), inv, d_kmm)
        d_q, d_cm = _kernel_bwd(d_kqm, k_qm, q, km_cm, s)
        d_km, d_cm2 = _kernel_bwd(d_kmm, k_mm, km, km_cm, s)
        d_k, d_cm3 = _kernel_bwd(d_kkm, k_km, k, km_cm, s)
        d_cm += d_cm2
        d_cm += d_cm3
        d_km += d_cm.transpose(-1, -2)
        # Pooling's backward: each landmark's gradient / pool^2 on its pool x pool patch
        # (divided in fp32, rounded once), added to the distance gradient of k in place.
        B, H, N, dd = k.shape
        gh, gw = ctx.grid
        gs = (d_km.float() / (p * p)).to(d_k.dtype)
        d_k.view(B, H, gh // p, p, gw // p, p, dd).add_(gs.view(B, H, gh // p, 1, gw // p, 1, dd))
        return d_q, d_k, d_v, None, None, None


def laplacian_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, grid: tuple[int, int] | None = None,
                        pool: int = 4, iters: int = 10) -> torch.Tensor:
    """LaplacianFormer attention of q, k, v [B,H,N,d] (autograd through the HIP ops).

    ``grid`` is the token grid (default square); landmarks are ``pool x pool`` averages of k.
    Returns [B,H,N,d] in the input type.
    """
    in_dtype = q.dtype
    B, H, N, d = q.shape
    if grid is None:
        side = math.isqrt(N)
        grid = (side, side)
    gh, gw = grid
    if gh * gw != N or gh % pool or gw % pool:
        raise ValueError(f"token grid {gh}x{gw} does not match N={N} or pool={pool}")
    M = (gh // pool) * (gw // pool)
    if in_dtype in (torch.float16, torch.bfloat16, torch.float32) and d <= 64 and M <= 64:
        return _AttentionFunction.apply(q, k, v, (gh, gw), pool, iters)
    ct = _acc_type(q.dtype)
    km = _PooledLandmarks.apply(k, grid, pool, ct)
    km_cm = km.transpose(-1, -2).contiguous()  # [B,H,d,M]: the reference's key layout
    s = 1.0 / math.sqrt(d)
    k_qm = laplace_kernel(q, km_cm, s)         # [B,H,N,M]
    k_mm = laplace_kernel(km, km_cm, s)        # [B,H,M,M]
    k_km = laplace_kernel(k, km_cm, s)         # [B,H,N,M] = K_mk^T
    inv = newton_inverse(k_mm, iters)          # [B,H,M,M]
    kv = tall_product(k_km, v)                 # [B,H,M,d] = K_km^T V
    out = tall_mix(k_qm, torch.matmul(inv, kv), in_dtype)  # [B,H,N,d]
    return out.to(in_dtype)


class LaplacianAttention(torch.nn.Module):
    """Multi-head LaplacianFormer attention on a token grid: qkv projection, the
    Laplacian-kernel Nystrom attention above, output projection."""

    def __init__(self, dim: int, heads: int, pool: int = 4, iters: int = 10):
        super().__init__()
        if dim % heads:
            raise ValueError("dim must be divisible by heads")
        self.heads, self.pool, self.iters = heads, pool, iters
        self.qkv = torch.nn.Linear(dim, 3 * dim)
        self.proj = torch.nn.Linear(dim, dim)

    def forward(self, x: torch.Tensor, grid: tuple[int, int] | None = None) -> torch.Tensor:
        B, N, C = x.shape
        qkv = self.qkv(x).reshape(B, N, 3, self.heads, C // self.heads).permute(2, 0, 3, 1, 4)
        q, k, v = (t.contiguous() for t in qkv)
        o = laplacian_attention(q, k, v, grid=grid, pool=self.pool, iters=self.iters)
        return self.proj(o.transpose(1, 2).reshape(B, N, C))

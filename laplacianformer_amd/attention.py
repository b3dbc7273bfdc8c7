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
from .functional import _acc_type, laplace_kernel, newton_inverse, tall_mix, tall_product


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


class _AttentionFunction(torch.autograd.Function):
    """The whole layer as one autograd node for 16-bit / fp32 inputs whose widths the
    row-product kernel takes (d, M <= 64): the same operations as the composition in
    laplacian_attention, issued by the extension's LaplacianAttention_forward /
    LaplacianAttention_backward (csrc/torch/LaplacianAttention_hip.cpp), so that an
    eager step makes one host call per direction instead of about forty."""

    @staticmethod
    def forward(ctx, q, k, v, grid, pool, iters):
        gh, gw = grid
        out, *saved = ext().LaplacianAttention_forward(q, k, v, gh, gw, pool, int(iters))
        ctx.grid, ctx.pool = grid, pool
        # saved = km, km_cm, k_qm, k_mm, k_km, inv, kv, w (q, k, v as made contiguous there)
        ctx.save_for_backward(q.contiguous(), k.contiguous(), v.contiguous(), *saved)
        return out

    @staticmethod
    def backward(ctx, g):
        gh, gw = ctx.grid
        d_q, d_k, d_v = ext().LaplacianAttention_backward(g, list(ctx.saved_tensors), gh, gw, ctx.pool)
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
    if q.is_cuda and in_dtype in (torch.float16, torch.bfloat16, torch.float32) and d <= 64 and M <= 64:
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

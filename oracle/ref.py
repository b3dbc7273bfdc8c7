"""CPU restatement of the reference's LaplaceSubtraction and NewtonInverse.

TEST INFRASTRUCTURE ONLY (see the package docstring). Every function cites the
reference lines it restates. The L1 loops call the C file ``laplace_oracle.c``
(fp32 accumulation in the reference's serial order); Newton-Schulz and the
legacy reduce tree are numpy.

Conventions: arrays are numpy; ``q`` is ``[B,H,N,C]``, ``k`` is channel-major
``[B,H,C,M]`` (reference src/LaplaceSubtraction_cuda.cu:25-27,62), ``g`` is
``[B,H,N,M]``. ``dtype`` names the element type of the operator call:
"f32", "f16", "bf16" or "f64". Laplace results are returned as unrounded fp32
(fp64 for "f64") accumulators; ``round_to`` applies the single rounding the
reference does at its store.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liblforacle.so")
_lib = None

__all__ = [
    "build", "max_threads", "widen", "round_to", "laplace_forward", "laplace_backward_query",
    "laplace_backward_key", "laplace_reduce_forward", "newton_alpha", "newton_forward",
    "newton_backward", "newton_variant",
]


def build(force: bool = False) -> str:
    """Compiles laplace_oracle.c with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        build()
        lib = ctypes.CDLL(_LIB_PATH)
        for suf in ("f32", "f32ftz", "f64"):
            for name, nptr in (("forward", 3), ("backward_query", 4), ("backward_key", 4)):
                fn = getattr(lib, f"lf_oracle_{name}_{suf}")
                fn.argtypes = [ctypes.c_void_p] * nptr + [ctypes.c_int64] * 4
                fn.restype = None
        lib.lf_oracle_max_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def max_threads() -> int:
    """OpenMP threads the C oracle uses."""
    return int(_load().lf_oracle_max_threads())


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------
def widen(x, dtype: str) -> np.ndarray:
    """Exact widening of an operator input to the accumulation type.

    ``x`` is a numpy array or a CPU torch tensor. fp16/bf16/fp32 widen to fp32
    (reference to_acc, src/LaplaceSubtraction_cuda_kernel.cu:21-24), fp64 stays.
    """
    if hasattr(x, "detach"):
        import torch

        x = x.detach().cpu()
        x = x.to(torch.float64 if dtype == "f64" else torch.float32).numpy()
    return np.ascontiguousarray(x, dtype=np.float64 if dtype == "f64" else np.float32)


def round_to(acc: np.ndarray, dtype: str):
    """Single round-to-nearest-even to the element type (reference from_acc, :26-29).

    Returns a numpy array for f16/f32/f64 and a torch bfloat16 tensor for bf16
    (numpy has no bfloat16).
    """
    if dtype == "f16":
        return acc.astype(np.float32).astype(np.float16)
    if dtype == "f32":
        return acc.astype(np.float32)
    if dtype == "f64":
        return acc.astype(np.float64)
    if dtype == "bf16":
        import torch

        return torch.from_numpy(np.ascontiguousarray(acc, dtype=np.float32)).to(torch.bfloat16)
    raise ValueError(dtype)


def _call(name, dtype, arrays, out_shape, dims, ftz=False):
    lib = _load()
    suf = "f64" if dtype == "f64" else ("f32ftz" if ftz else "f32")
    arrs = [widen(a, dtype) for a in arrays]
    out = np.empty(out_shape, dtype=arrs[0].dtype)
    getattr(lib, f"lf_oracle_{name}_{suf}")(*[a.ctypes.data for a in arrs], out.ctypes.data, *dims)
    return out


# ---------------------------------------------------------------------------
# LaplaceSubtraction
# ---------------------------------------------------------------------------
def laplace_forward(q, k, dtype: str = "f32", ftz: bool = False) -> np.ndarray:
    """out[b,h,i,j] = sum_c |q[b,h,i,c] - k[b,h,c,j]|, c ascending, fp32 accumulator.

    Reference src/LaplaceSubtraction_cuda_kernel.cu:84-125 (loop order), :137 (store).
    ``ftz``: the reference's fast-math build (setup.py:29: fp32 denormal operands and
    results flushed to zero); fp32 accumulation only.
    """
    B, H, N, C = q.shape
    M = k.shape[3]
    return _call("forward", dtype, [q, k], (B, H, N, M), (B * H, N, M, C), ftz)


def laplace_backward_query(g, q, k, dtype: str = "f32", ftz: bool = False) -> np.ndarray:
    """dq[b,h,i,c] = sum_j g[b,h,i,j] * sgn(q[b,h,i,c] - k[b,h,c,j]), j ascending.

    Reference src/LaplaceSubtraction_cuda_kernel.cu:206-249 (unsplit order), sgn :34-38.
    ``ftz`` as in laplace_forward.
    """
    B, H, N, C = q.shape
    M = k.shape[3]
    return _call("backward_query", dtype, [g, q, k], (B, H, N, C), (B * H, N, M, C), ftz)


def laplace_backward_key(g, q, k, dtype: str = "f32", ftz: bool = False) -> np.ndarray:
    """dk[b,h,c,j] = -sum_i g[b,h,i,j] * sgn(q[b,h,i,c] - k[b,h,c,j]), i ascending.

    Reference src/LaplaceSubtraction_cuda_kernel.cu:332-375 (unsplit order).
    ``ftz`` as in laplace_forward.
    """
    B, H, N, C = q.shape
    M = k.shape[3]
    return _call("backward_key", dtype, [g, q, k], (B, H, C, M), (B * H, N, M, C), ftz)


def _native(x, dtype):
    """Element-type arithmetic for the legacy reduce kernel: numpy f16/f32/f64, or
    fp32 values re-rounded to bf16 after every operation."""
    if dtype == "f16":
        return widen(x, "f32").astype(np.float16)
    if dtype == "f64":
        return widen(x, "f64")
    return widen(x, "f32")


def _rb(x, dtype):
    if dtype != "bf16":
        return x
    import torch

    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def laplace_reduce_forward(q, k, dtype: str):
    """Legacy reduce forward (reference src/LaplaceSubtraction_cuda_kernel.cu:399-447, 611-647).

    bd = min(C, 256) partial sums s_t = sum_{c = t, t+bd, ...} |q_c - k_c| in the
    element type, then the halving tree ``for stride = bd/2; stride > 0; stride >>= 1:
    s[t] += s[t + stride] (t < stride)``; the result is s[0]. When bd is not a power
    of two the tree skips some partials, exactly like the reference. Returns values
    already in the element type (numpy f16/f32/f64; fp32 array holding bf16 values).
    """
    B, H, N, C = q.shape
    M = k.shape[3]
    qn = _native(q, dtype)[..., :, None, :]                     # [B,H,N,1,C]
    kn = np.swapaxes(_native(k, dtype), -1, -2)[..., None, :, :]  # [B,H,1,M,C]
    bd = min(C, 256)
    parts = []
    for t in range(bd):
        s = np.zeros((B, H, N, M), dtype=qn.dtype)
        for c in range(t, C, bd):
            diff = _rb(qn[..., c] - kn[..., c], dtype)
            s = _rb(s + np.abs(diff), dtype)
        parts.append(s)
    stride = bd // 2
    while stride > 0:
        for t in range(stride):
            parts[t] = _rb(parts[t] + parts[t + stride], dtype)
        stride //= 2
    return parts[0]


# ---------------------------------------------------------------------------
# NewtonInverse
# ---------------------------------------------------------------------------
def newton_variant(n: int) -> str:
    """Association order the reference picks for size n (src/NewtonInverse_cuda_kernel.cu:693-728):
    3-buffer V(PV) below N_MAX=128 (96/112 fit in 160 KB of LDS), 2-buffer (VP)V at 128.
    n > 128 is outside the reference's envelope; this build computes it in the V(PV) order."""
    nmax = ((n + 15) // 16) * 16
    return "2buf" if nmax == 128 else "3buf"


def newton_alpha(P: np.ndarray) -> np.ndarray:
    """alpha = 1.8 / (max_i sum_j P_ij)^2 with signed row sums in ascending j
    (reference src/NewtonInverse_cuda_kernel.cu:91-99, :116). P is [..., n, n]."""
    s = np.zeros(P.shape[:-1], dtype=P.dtype)
    for j in range(P.shape[-1]):
        s = s + P[..., j]
    m = s.max(axis=-1)
    return (P.dtype.type(1.8) / (m * m)).astype(P.dtype)


def newton_forward(mat, iters: int, dtype: str = "f32", variant: str | None = None) -> np.ndarray:
    """Newton-Schulz inverse restated (reference src/NewtonInverse_cuda_kernel.cu:125-255, 277-464).

    P = mat + 0.01 I (:169), alpha from newton_alpha, V0 = alpha P (:176-178),
    iters x V <- 2V - V(PV) [3buf] or 2V - (VP)V [2buf]. fp32 arithmetic
    (fp64 for "f64"); returns the unrounded result in that type.
    """
    A = widen(mat, dtype)
    n = A.shape[-1]
    variant = variant or newton_variant(n)
    P = A + A.dtype.type(0.01) * np.eye(n, dtype=A.dtype)
    alpha = newton_alpha(P)
    V = alpha[..., None, None] * P
    for _ in range(max(int(iters), 0)):
        if variant == "3buf":
            V = A.dtype.type(2) * V - V @ (P @ V)
        else:
            V = A.dtype.type(2) * V - (V @ P) @ V
    return V


def newton_backward(grad, inverse, dtype: str = "f32") -> np.ndarray:
    """grad_mat = -(V^T G) V^T (reference src/NewtonInverse_cuda_kernel.cu:520-570)."""
    G = widen(grad, dtype)
    V = widen(inverse, dtype)
    Vt = np.swapaxes(V, -1, -2)
    return -((Vt @ G) @ Vt)

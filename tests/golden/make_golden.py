"""Writes the committed golden fixtures of tests/golden/.

The reference ships no tests or vectors, so every expected value here comes
from an implementation independent of the C oracle under test:

* kat_l1.npz      - small integer-valued q, key, g (every sum exact in fp16/fp32)
                    with forward / dq / dk from straightforward pure-Python loops
                    over the definitions (reference src/LaplaceSubtraction_cuda_kernel.cu
                    :121-122, :243-244, :369-370; sgn(0) = 0 per :34-38).
* config1_l1.npz  - BASELINE config 1 inputs (seed 1001) and fp64 results from
                    torch.cdist(p=1) and its autograd backward (independent code).
* newton_closed.npz - NewtonInverse closed forms in fp64: symmetric P = U diag(l) U^T
                    gives X_k = U diag((1 - (1 - alpha l^2)^(2^k)) / l) U^T with the
                    reference init (P = A + 0.01 I, alpha = 1.8 / (max row sum)^2,
                    src/NewtonInverse_cuda_kernel.cu:91-116, :169, :176-178).

Run: python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def sgn(v):
    return int(v > 0) - int(v < 0)


def kat_l1():
    rng = np.random.default_rng(20240601)
    B, H, N, M, C = 1, 2, 5, 4, 3
    q = rng.integers(-3, 4, (B, H, N, C)).astype(np.float64)
    k = rng.integers(-3, 4, (B, H, C, M)).astype(np.float64)
    g = rng.integers(-4, 5, (B, H, N, M)).astype(np.float64)
    out = np.zeros((B, H, N, M))
    dq = np.zeros((B, H, N, C))
    dk = np.zeros((B, H, C, M))
    for b in range(B):
        for h in range(H):
            for i in range(N):
                for j in range(M):
                    s = 0.0
                    for c in range(C):
                        s += abs(q[b, h, i, c] - k[b, h, c, j])
                    out[b, h, i, j] = s
            for i in range(N):
                for c in range(C):
                    s = 0.0
                    for j in range(M):
                        s += g[b, h, i, j] * sgn(q[b, h, i, c] - k[b, h, c, j])
                    dq[b, h, i, c] = s
            for c in range(C):
                for j in range(M):
                    s = 0.0
                    for i in range(N):
                        s -= g[b, h, i, j] * sgn(q[b, h, i, c] - k[b, h, c, j])
                    dk[b, h, c, j] = s
    ties = int(sum(q[0, h, i, c] == k[0, h, c, j] for h in range(H) for i in range(N) for c in range(C)
                   for j in range(M)))
    np.savez_compressed(os.path.join(HERE, "kat_l1.npz"), q=q, k=k, g=g, out=out, dq=dq, dk=dk, ties=ties)


def config1():
    gen = torch.Generator().manual_seed(1001)
    q = torch.randn((2, 2, 196, 32), generator=gen)
    k = torch.randn((2, 2, 49, 32), generator=gen)
    g = torch.randn((2, 2, 196, 49), generator=gen)
    qd = q.double().requires_grad_()
    kd = k.double().requires_grad_()
    d = torch.cdist(qd, kd, p=1)
    d.backward(g.double())
    np.savez_compressed(os.path.join(HERE, "config1_l1.npz"), q=q.numpy(), k_mc=k.numpy(), g=g.numpy(),
                        out=d.detach().numpy(), dq=qd.grad.numpy(), dk_mc=kd.grad.numpy())


def newton_closed():
    rng = np.random.default_rng(7)
    cases = {}
    for n in (5, 49, 64, 136):
        # Landmark Gram matrix of the BASELINE recipe: exp(-L1(k_i, k_j) / sqrt(d)) + 1e-3 I.
        # Non-negative and symmetric, so lambda_max <= max row sum and alpha*lambda^2 <= 1.8.
        d = 16
        kk = rng.standard_normal((n, d))
        D = np.abs(kk[:, None, :] - kk[None, :, :]).sum(-1)
        A = np.exp(-D / np.sqrt(d)) + 1e-3 * np.eye(n)
        # n > 128 (the batched-GEMM path) is stored in fp32 to keep the fixture small; its
        # closed form is computed from exactly the stored fp32 matrix.
        store = np.float32 if n > 128 else np.float64
        A = A.astype(store).astype(np.float64)
        P = A + 0.01 * np.eye(n)
        w, U = np.linalg.eigh(P)
        alpha = 1.8 / P.sum(axis=1).max() ** 2
        for it in (0, 1, 4, 10):
            x = (1.0 - (1.0 - alpha * w * w) ** (2 ** it)) / w
            cases[f"A_{n}"] = A.astype(store)
            cases[f"X_{n}_{it}"] = ((U * x) @ U.T).astype(store)
    np.savez_compressed(os.path.join(HERE, "newton_closed.npz"), **cases)


if __name__ == "__main__":
    kat_l1()
    config1()
    newton_closed()
    print("golden fixtures written to", HERE)

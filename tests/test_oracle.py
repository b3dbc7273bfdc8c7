"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked against something that does not share its
code: closed forms (torch.cdist and its autograd, eigen-decomposition closed
forms of Newton-Schulz, torch.linalg.inv and its autograd), brute-force
pure-Python loops, integer known-answer fixtures and invariants. The mutation
tests at the end plant plausible mistakes in a copy of the oracle and show that
these checks catch them.
"""
import os

import numpy as np
import pytest
import torch

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rand(shape, seed, integer=None):
    g = torch.Generator().manual_seed(seed)
    if integer:
        return torch.randint(-integer, integer + 1, shape, generator=g).double()
    return torch.randn(shape, generator=g, dtype=torch.float64)


# ---------------------------------------------------------------------------
# LaplaceSubtraction
# ---------------------------------------------------------------------------
def cdist_ref(q, kT, g):
    """fp64 torch.cdist(p=1) forward and autograd backward on the channel-major key."""
    qd = q.clone().requires_grad_()
    kd = kT.transpose(-1, -2).contiguous().requires_grad_()
    d = torch.cdist(qd, kd, p=1)
    d.backward(g)
    return d.detach().numpy(), qd.grad.numpy(), kd.grad.transpose(-1, -2).numpy()


@pytest.mark.parametrize("shape", [(1, 1, 1, 1, 1), (2, 3, 17, 9, 5), (1, 2, 64, 49, 32), (2, 1, 33, 70, 65)])
@pytest.mark.parametrize("integer", [None, 2])
def test_laplace_f64_vs_cdist(shape, integer):
    B, H, N, M, C = shape
    q = rand((B, H, N, C), 1, integer)
    kT = rand((B, H, C, M), 2, integer)
    g = rand((B, H, N, M), 3, integer)
    out, dq, dk = cdist_ref(q, kT, g)
    np.testing.assert_allclose(oracle.laplace_forward(q, kT, "f64"), out, rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(oracle.laplace_backward_query(g, q, kT, "f64"), dq, rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(oracle.laplace_backward_key(g, q, kT, "f64"), dk, rtol=1e-13, atol=1e-12)


def _brute_f32(q, kT, g):
    """Serial fp32 loops in the reference's order, one numpy float32 operation at a time."""
    q = q.numpy().astype(np.float32)
    kT = kT.numpy().astype(np.float32)
    g = g.numpy().astype(np.float32)
    B, H, N, C = q.shape
    M = kT.shape[3]
    out = np.zeros((B, H, N, M), np.float32)
    dq = np.zeros((B, H, N, C), np.float32)
    dk = np.zeros((B, H, C, M), np.float32)
    one = np.float32(1)
    for b in range(B):
        for h in range(H):
            for i in range(N):
                for j in range(M):
                    acc = np.float32(0)
                    for c in range(C):
                        acc = np.float32(acc + abs(np.float32(q[b, h, i, c] - kT[b, h, c, j])))
                    out[b, h, i, j] = acc
                for c in range(C):
                    acc = np.float32(0)
                    for j in range(M):
                        d = np.float32(q[b, h, i, c] - kT[b, h, c, j])
                        s = one if d > 0 else (-one if d < 0 else np.float32(0))
                        acc = np.float32(acc + g[b, h, i, j] * s)
                    dq[b, h, i, c] = acc
            for c in range(C):
                for j in range(M):
                    acc = np.float32(0)
                    for i in range(N):
                        d = np.float32(q[b, h, i, c] - kT[b, h, c, j])
                        s = one if d > 0 else (-one if d < 0 else np.float32(0))
                        acc = np.float32(acc - g[b, h, i, j] * s)
                    dk[b, h, c, j] = acc
    return out, dq, dk


def test_laplace_f32_serial_bitexact():
    q = rand((1, 2, 9, 7), 11).float()
    kT = rand((1, 2, 7, 6), 12).float()
    g = rand((1, 2, 9, 6), 13).float()
    out, dq, dk = _brute_f32(q, kT, g)
    assert np.array_equal(oracle.laplace_forward(q, kT, "f32"), out)
    assert np.array_equal(oracle.laplace_backward_query(g, q, kT, "f32"), dq)
    assert np.array_equal(oracle.laplace_backward_key(g, q, kT, "f32"), dk)


def test_laplace_golden_kat():
    z = np.load(os.path.join(GOLD, "kat_l1.npz"))
    assert int(z["ties"]) > 0
    for dt in ("f64", "f32", "f16"):
        q, k, g = (torch.from_numpy(z[n]) for n in ("q", "k", "g"))
        if dt == "f16":
            q, k, g = q.half(), k.half(), g.half()
        assert np.array_equal(oracle.laplace_forward(q, k, dt), z["out"])
        assert np.array_equal(oracle.laplace_backward_query(g, q, k, dt), z["dq"])
        assert np.array_equal(oracle.laplace_backward_key(g, q, k, dt), z["dk"])


def test_laplace_golden_config1():
    z = np.load(os.path.join(GOLD, "config1_l1.npz"))
    q = torch.from_numpy(z["q"])
    kT = torch.from_numpy(z["k_mc"]).transpose(-1, -2).contiguous()
    g = torch.from_numpy(z["g"])
    np.testing.assert_allclose(oracle.laplace_forward(q, kT, "f64"), z["out"], rtol=1e-12)
    np.testing.assert_allclose(oracle.laplace_backward_query(g, q, kT, "f64"), z["dq"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.laplace_backward_key(g, q, kT, "f64"), np.swapaxes(z["dk_mc"], -1, -2),
                               rtol=1e-12, atol=1e-12)
    # fp32 serial accumulation stays within 1e-5 of the exact result.
    np.testing.assert_allclose(oracle.laplace_forward(q, kT, "f32"), z["out"], rtol=1e-5)


def test_laplace_invariants():
    k = rand((2, 2, 30, 16), 21)  # [B,H,M,d]
    kT = k.transpose(-1, -2).contiguous()
    gram = oracle.laplace_forward(k, kT, "f64")
    assert np.all(gram >= 0)
    assert np.array_equal(np.diagonal(gram, axis1=-2, axis2=-1), np.zeros((2, 2, 30)))
    np.testing.assert_allclose(gram, np.swapaxes(gram, -1, -2), rtol=0, atol=0)
    q = rand((2, 2, 11, 16), 22)
    base = oracle.laplace_forward(q, kT, "f64")
    np.testing.assert_allclose(oracle.laplace_forward(q + 0.375, kT + 0.375, "f64"), base, rtol=1e-12)
    np.testing.assert_allclose(oracle.laplace_forward(-2.5 * q, -2.5 * kT, "f64"), 2.5 * base, rtol=1e-12)
    # sum_i dq[i,c] + sum_j dk[c,j] = 0, exactly for integer data.
    qi = rand((1, 2, 40, 8), 23, integer=3)
    ki = rand((1, 2, 8, 12), 24, integer=3)
    gi = rand((1, 2, 40, 12), 25, integer=4)
    dq = oracle.laplace_backward_query(gi, qi, ki, "f64")
    dk = oracle.laplace_backward_key(gi, qi, ki, "f64")
    assert np.array_equal(dq.sum(axis=2) + dk.sum(axis=3), np.zeros((1, 2, 8)))


def test_laplace_ftz_mode_known_answers():
    """The f32ftz restatement of the reference's fast-math build (setup.py:29, -ftz=true):
    hand-computed cases. Sterbenz: 1.5e-38 - 1.2e-38 is exact in fp32, a denormal, so the
    IEEE oracle keeps it (sgn +1, forward = the difference) and the flushing one gives 0;
    a denormal operand (1e-40) counts as 0 only in the flushing one; normal values agree."""
    f = np.float32
    a, b, tiny = f(1.5e-38), f(1.2e-38), f(1e-40)
    assert 0 < a - b < np.finfo(np.float32).tiny and tiny < np.finfo(np.float32).tiny
    q = np.array([[[[a, tiny, f(2.0)]]]], dtype=np.float32)          # [1,1,1,3]
    k = np.array([[[[b, a], [f(0.0), f(0.0)], [f(1.0), f(3.0)]]]], dtype=np.float32)  # [1,1,3,2]
    g = np.array([[[[f(1.0), f(1.0)]]]], dtype=np.float32)
    fwd = oracle.laplace_forward(q, k, "f32")
    fwd_z = oracle.laplace_forward(q, k, "f32", ftz=True)
    # column 0: |a-b| + |tiny| + 1; column 1: 0 + |tiny| + 1
    assert fwd[0, 0, 0, 0] == f(f(f(a - b) + tiny) + f(1.0)) and fwd_z[0, 0, 0, 0] == f(1.0)
    assert fwd_z[0, 0, 0, 1] == f(1.0)
    dq = oracle.laplace_backward_query(g, q, k, "f32")[0, 0, 0]
    dq_z = oracle.laplace_backward_query(g, q, k, "f32", ftz=True)[0, 0, 0]
    assert dq.tolist() == [1.0, 2.0, 0.0] and dq_z.tolist() == [0.0, 0.0, 0.0]
    dk = oracle.laplace_backward_key(g, q, k, "f32")[0, 0]
    dk_z = oracle.laplace_backward_key(g, q, k, "f32", ftz=True)[0, 0]
    assert dk.tolist() == [[-1.0, 0.0], [-1.0, -1.0], [-1.0, 1.0]]
    assert dk_z.tolist() == [[0.0, 0.0], [0.0, 0.0], [-1.0, 1.0]]
    # Away from the denormal range both modes are the same function.
    qn, kn, gn = (np.random.default_rng(5).standard_normal(s).astype(np.float32)
                  for s in ((1, 2, 7, 5), (1, 2, 5, 4), (1, 2, 7, 4)))
    assert np.array_equal(oracle.laplace_forward(qn, kn, "f32"), oracle.laplace_forward(qn, kn, "f32", ftz=True))
    assert np.array_equal(oracle.laplace_backward_key(gn, qn, kn, "f32"),
                          oracle.laplace_backward_key(gn, qn, kn, "f32", ftz=True))


def test_round_to():
    x = np.array([1.0, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 65504.0, 1e-8], dtype=np.float64)
    assert oracle.round_to(x, "f16").tolist() == [1.0, 1.0, 1.0 + 2 ** -9, 65504.0, 0.0]
    b = oracle.round_to(np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8]), "bf16").float().tolist()
    assert b == [1.0, 1.0 + 2 ** -6]


# ---------------------------------------------------------------------------
# Legacy reduce forward
# ---------------------------------------------------------------------------
def test_reduce_forward_power_of_two_equals_forward():
    q = rand((1, 2, 13, 64), 31)
    kT = rand((1, 2, 64, 7), 32)
    np.testing.assert_allclose(oracle.laplace_reduce_forward(q, kT, "f64"),
                               oracle.laplace_forward(q, kT, "f64"), rtol=1e-13)


def test_reduce_forward_tree_closed_forms():
    """bd = C = 3: stride 1 folds s1 into s0 and drops s2. bd = 6: strides 3 then 1
    give d0+d3+d1+d4 and drop d2, d5 (the reference's tree, :437-442)."""
    q = rand((1, 1, 5, 6), 41, integer=4)
    kT = rand((1, 1, 6, 4), 42, integer=4)
    d = (q[..., :, None, :] - kT.transpose(-1, -2)[..., None, :, :]).abs().numpy()  # [1,1,N,M,C]
    np.testing.assert_array_equal(oracle.laplace_reduce_forward(q, kT, "f64"),
                                  d[..., 0] + d[..., 3] + d[..., 1] + d[..., 4])
    q3, k3 = q[..., :3].contiguous(), kT[..., :3, :].contiguous()
    np.testing.assert_array_equal(oracle.laplace_reduce_forward(q3, k3, "f64"), d[..., 0] + d[..., 1])
    # C > 256: thread t first sums c = t, t+256 in order.
    q = rand((1, 1, 3, 300), 43, integer=2)
    kT = rand((1, 1, 300, 2), 44, integer=2)
    np.testing.assert_array_equal(oracle.laplace_reduce_forward(q, kT, "f64"),
                                  oracle.laplace_forward(q, kT, "f64"))


def test_reduce_forward_half_accumulates_in_half():
    """fp16 partial sums round at every step; 2048 + 1 + 1 in fp16 stays 2048."""
    q = torch.zeros((1, 1, 1, 3), dtype=torch.float16)
    q[..., 0] = 2048
    q[..., 1] = 1
    q[..., 2] = 1
    kT = torch.zeros((1, 1, 3, 1), dtype=torch.float16)
    # bd = 3 drops c = 2; 2048 + 1 = 2049 rounds to 2048 in fp16.
    assert oracle.laplace_reduce_forward(q, kT, "f16").item() == 2048.0


# ---------------------------------------------------------------------------
# NewtonInverse
# ---------------------------------------------------------------------------
def test_newton_closed_form_fixture():
    z = np.load(os.path.join(GOLD, "newton_closed.npz"))
    for n in (5, 49, 64, 136):
        A = z[f"A_{n}"].astype(np.float64)[None, None]
        # n = 136 is stored in fp32 (its closed form rounded once to fp32).
        tol = 1e-9 if z[f"X_{n}_0"].dtype == np.float64 else 2e-6
        for it in (0, 1, 4, 10):
            X = oracle.newton_forward(A, it, "f64")[0, 0]
            np.testing.assert_allclose(X, z[f"X_{n}_{it}"], rtol=tol, atol=tol * np.abs(X).max())
            Xf = oracle.newton_forward(A.astype(np.float32), it, "f32")[0, 0]
            assert np.abs(Xf - z[f"X_{n}_{it}"]).max() <= 1e-4 * np.abs(X).max()


def test_newton_diagonal_and_iter0():
    for c in (0.5, 2.0, 0.09):
        mu = c + 0.01
        A = (c * np.eye(7))[None, None]
        for it in range(6):
            X = oracle.newton_forward(A, it, "f64")
            np.testing.assert_allclose(X[0, 0], (1 - (-0.8) ** (2 ** it)) / mu * np.eye(7), rtol=1e-12, atol=1e-15)
    A = rand((2, 2, 9, 9), 51).numpy()
    P = A + 0.01 * np.eye(9)
    alpha = 1.8 / P.sum(-1).max(-1) ** 2  # signed row sums
    np.testing.assert_allclose(oracle.newton_forward(A, 0, "f64"), alpha[..., None, None] * P, rtol=1e-14)


def test_newton_converges_to_inverse_and_variants_agree():
    A = np.load(os.path.join(GOLD, "newton_closed.npz"))["A_49"][None, None]
    P = A + 0.01 * np.eye(49)
    X = oracle.newton_forward(A, 40, "f64")
    np.testing.assert_allclose(X[0, 0], np.linalg.inv(P[0, 0]), rtol=1e-8, atol=1e-8)
    X2 = oracle.newton_forward(A, 10, "f64", variant="2buf")
    X3 = oracle.newton_forward(A, 10, "f64", variant="3buf")
    np.testing.assert_allclose(X2, X3, rtol=1e-10, atol=1e-12)
    assert oracle.newton_variant(49) == "3buf" and oracle.newton_variant(112) == "3buf"
    assert oracle.newton_variant(113) == "2buf" and oracle.newton_variant(128) == "2buf"
    # Beyond the reference's envelope (n > 128) this build uses the V(PV) order.
    assert oracle.newton_variant(129) == "3buf" and oracle.newton_variant(256) == "3buf"


def test_newton_backward():
    """-V^T G V^T is the derivative of the exact inverse: compare with autograd of
    torch.linalg.inv at a converged V; G = I gives -(V^2)^T."""
    A = np.load(os.path.join(GOLD, "newton_closed.npz"))["A_64"]
    P = torch.from_numpy(A + 0.01 * np.eye(64)).requires_grad_()
    inv = torch.linalg.inv(P)
    G = rand((64, 64), 61)
    inv.backward(G)
    V = oracle.newton_forward(A[None, None], 60, "f64")
    got = oracle.newton_backward(G.numpy()[None, None], V, "f64")[0, 0]
    np.testing.assert_allclose(got, P.grad.numpy(), rtol=1e-7, atol=1e-7 * np.abs(got).max())
    Vs = rand((1, 1, 10, 10), 62).numpy()
    np.testing.assert_allclose(oracle.newton_backward(np.eye(10)[None, None], Vs, "f64")[0, 0],
                               -(Vs[0, 0] @ Vs[0, 0]).T, rtol=1e-14)


# ---------------------------------------------------------------------------
# The checks above catch planted mistakes (mutation tests on the CPU oracle).
# ---------------------------------------------------------------------------
def test_mutations_are_caught():
    q = rand((1, 2, 12, 6), 71, integer=2)
    kT = rand((1, 2, 6, 5), 72, integer=2)
    g = rand((1, 2, 12, 5), 73, integer=3)
    out, dq, dk = cdist_ref(q, kT, g)
    # dk with the sign flipped.
    assert not np.allclose(-oracle.laplace_backward_key(g, q, kT, "f64"), dk)
    # key read row-major [M, C] instead of channel-major [C, M].
    kbad = kT.reshape(1, 2, 5, 6).transpose(-1, -2).contiguous()
    assert not np.allclose(oracle.laplace_forward(q, kbad, "f64"), out)
    # sgn(0) taken as +1 (ties are present in integer data).
    dq_pos = (g.numpy()[..., :, None, :] *
              np.where(q.numpy()[..., :, :, None] - kT.numpy()[..., None, :, :] >= 0, 1.0, -1.0)).sum(-1)
    assert not np.allclose(dq_pos, dq)
    # Newton init from unshifted A, or alpha from |row sums|, moves the result off the closed form.
    z = np.load(os.path.join(GOLD, "newton_closed.npz"))
    A = z["A_49"][None, None]
    assert not np.allclose(oracle.newton_forward(A - 0.01 * np.eye(49), 4, "f64")[0, 0], z["X_49_4"], rtol=1e-6)
    # alpha from absolute row sums instead of signed ones fails the iter-0 check on a
    # matrix with negative entries.
    R = rand((1, 1, 9, 9), 51).numpy()
    P = R + 0.01 * np.eye(9)
    alpha_abs = 1.8 / np.abs(P).sum(-1).max(-1) ** 2
    assert not np.allclose(alpha_abs[..., None, None] * P, oracle.newton_forward(R, 0, "f64"))

"""The attention layer's forward + backward captured in a HIP graph: every
replay, with eager work and synchronisations between replays, must give the
eager step's output and gradients bit for bit (every kernel on the path is
deterministic), also after the static inputs are refilled with new values."""
import pytest
import torch

from lfcheck import gen

pytestmark = pytest.mark.gpu


def test_graphed_layer_step_matches_eager(gpu):
    import laplacianformer_amd as lf

    B, H, N, d = 4, 2, 784, 64
    print("graphed attention step", flush=True)
    q, k, v, g = (gen((B, H, N, d), 70 + i, "f16").to(gpu) for i in range(4))
    for t in (q, k, v):
        t.requires_grad_()
    fn = lambda a, b, c: lf.laplacian_attention(a, b, c, grid=(28, 28), pool=4, iters=10)

    def eager():
        qe, ke, ve = (t.detach().clone().requires_grad_() for t in (q, k, v))
        out = fn(qe, ke, ve)
        out.backward(g)
        return out.detach().clone(), [t.grad.clone() for t in (qe, ke, ve)]

    step = lf.GraphedStep(fn, [q, k, v], g)
    for rep in range(3):
        ref_out, ref_grads = eager()  # eager work between replays
        torch.cuda.synchronize()
        step.replay()
        torch.cuda.synchronize()
        assert torch.equal(step.out, ref_out), rep
        for got, want, name in zip(step.grads, ref_grads, "qkv"):
            assert torch.equal(got, want), (rep, name)
        if rep == 1:  # new values in the static inputs
            with torch.no_grad():
                for i, t in enumerate((q, k, v)):
                    t.copy_(gen((B, H, N, d), 90 + i, "f16").to(gpu))


def test_graphed_operators_match_eager(gpu):
    """The raw operators in one captured graph: LaplaceSubtraction forward + fused
    backward (with its grad_key workspace and reduction kernel), backward_query /
    backward_key, and NewtonInverse forward + backward at n = 256 (batched-GEMM
    path with its workspace). Three replays, eager work between them, bit for bit."""
    import laplacianformer_amd as lf

    L = lf.ext()
    print("graphed operators", flush=True)
    q = gen((2, 1, 3136, 64), 81, "f16").to(gpu)
    k = gen((2, 1, 64, 49), 82, "f16").to(gpu)
    go = gen((2, 1, 3136, 49), 83, "f16").to(gpu)
    A = (torch.rand(4, 1, 256, 256, generator=torch.Generator().manual_seed(84)) / 256).to(gpu)
    A = A + A.transpose(-1, -2) + torch.eye(256, device=gpu)
    G = gen((4, 1, 256, 256), 85, "f32").to(gpu)
    outs = [torch.empty_like(go), torch.empty_like(q), torch.empty_like(k), torch.empty_like(q),
            torch.empty_like(k), torch.empty_like(A), torch.empty_like(A)]

    def run(o):
        L.LaplaceSubtraction_forward(q, k, o[0])
        L.LaplaceSubtraction_backward(go, q, k, o[1], o[2])
        L.LaplaceSubtraction_backward_query(go, q, k, o[3])
        L.LaplaceSubtraction_backward_key(go, q, k, o[4])
        L.NewtonInverse_forward(A, o[5], 16)
        L.NewtonInverse_backward(G, o[5], o[6])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(outs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(outs)
    for rep in range(3):
        ref = [torch.empty_like(t) for t in outs]
        run(ref)  # eager work between replays
        torch.cuda.synchronize()
        for t in outs:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(outs, ref)):
            assert torch.equal(got, want), (rep, i)


def test_operators_on_concurrent_streams(gpu):
    """Two problems launched on two streams at once (each operator takes the calling
    stream and a workspace of its own) give the same bits as one after the other."""
    import laplacianformer_amd as lf

    L = lf.ext()
    print("operators on two streams", flush=True)
    probs = []
    for i in range(2):
        q = gen((8, 1, 3136, 64), 300 + i, "f16").to(gpu)
        k = gen((8, 1, 64, 49), 310 + i, "f16").to(gpu)
        go = gen((8, 1, 3136, 49), 320 + i, "f16").to(gpu)
        A = (torch.rand(16, 1, 256, 256, generator=torch.Generator().manual_seed(330 + i)) / 256).to(gpu)
        A = A + A.transpose(-1, -2) + torch.eye(256, device=gpu)
        probs.append((q, k, go, A))

    def run(p):
        q, k, go, A = p
        o = [torch.empty_like(go), torch.empty_like(q), torch.empty_like(k), torch.empty_like(A)]
        L.LaplaceSubtraction_forward(q, k, o[0])
        L.LaplaceSubtraction_backward(go, q, k, o[1], o[2])
        L.NewtonInverse_forward(A, o[3], 16)
        return o

    ref = [run(p) for p in probs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got = [None, None]
    for rep in range(3):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                got[i] = run(probs[i])
        torch.cuda.synchronize()
        for i in range(2):
            for j, (a, b) in enumerate(zip(got[i], ref[i])):
                assert torch.equal(a, b), (rep, i, j)

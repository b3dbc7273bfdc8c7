"""The attention layer's pooled-landmark op: forward and gradient identical to the
plain composition landmarks(k, ..., dtype=acc).to(k.dtype) under autograd (CPU)."""
import pytest
import torch

from laplacianformer_amd.attention import _PooledLandmarks, landmarks


@pytest.mark.parametrize("dt,acc", [(torch.float16, torch.float32), (torch.bfloat16, torch.float32),
                                    (torch.float32, torch.float32), (torch.float64, torch.float64)])
@pytest.mark.parametrize("grid,pool", [((8, 8), 4), ((12, 8), 2)])
def test_pooled_landmarks_match_autograd_composition(dt, acc, grid, pool):
    g = torch.Generator().manual_seed(7)
    n = grid[0] * grid[1]
    k = torch.randn(2, 3, n, 8, generator=g).to(dt).requires_grad_(True)
    k2 = k.detach().clone().requires_grad_(True)
    a = _PooledLandmarks.apply(k, grid, pool, acc)
    b = landmarks(k2, grid, pool, dtype=acc).to(dt)
    assert a.dtype == dt and torch.equal(a, b)
    go = torch.randn(a.shape, generator=g).to(dt)
    a.backward(go)
    b.backward(go)
    assert torch.equal(k.grad, k2.grad)

"""HIP-graph capture of a whole forward + backward step (torch.cuda.CUDAGraph
on ROCm records a hipGraph): one launch per replay instead of one host dispatch
per kernel, for steps whose kernels are short enough that dispatch dominates
(the LaplacianFormer attention layer runs ~40 kernels per step).

The HIP operators of this package record cleanly: every launch goes to the
current stream, workspaces come from PyTorch's allocator (the graph's private
pool during capture), and no operator issues a memset or a host synchronisation.
"""
from __future__ import annotations

from typing import Callable, Sequence

import torch


class GraphedStep:
    """``fn(*inputs).backward(grad_out)`` captured once on static tensors.

    After construction ``out`` is the captured forward result and ``grads`` the
    inputs' gradients; ``replay()`` re-runs the step on whatever the static
    ``inputs`` and ``grad_out`` tensors hold at that time and overwrites ``out``
    and ``grads`` in place (gradients are not accumulated across replays).
    """

    def __init__(self, fn: Callable[..., torch.Tensor], inputs: Sequence[torch.Tensor], grad_out: torch.Tensor,
                 warmup: int = 3):
        self.inputs = list(inputs)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # allocations and lazy set-up happen outside the capture
            for _ in range(max(1, warmup)):
                for t in self.inputs:
                    t.grad = None
                fn(*self.inputs).backward(grad_out)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for t in self.inputs:
            t.grad = None
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = fn(*self.inputs)
            self.out.backward(grad_out)
        self.grads = [t.grad for t in self.inputs]

    def replay(self) -> None:
        self.graph.replay()

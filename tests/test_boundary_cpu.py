"""The drop-in module on the CPU: same name and exports as the reference
module (src/wrapper.cpp:73-99) and the reference's CPU-tensor errors
(include/LaplaceSubtraction.h:50, include/NewtonInverse.h:26-28,40-41)."""
import pytest
import torch

REFERENCE_EXPORTS = [
    "get_compiler_version", "get_cuda_version", "has_cuda", "LaplaceSubtraction_forward",
    "LaplaceSubtraction_backward_query", "LaplaceSubtraction_backward_key", "LaplaceSubtraction_reduce_forward",
    "NewtonInverse_forward", "NewtonInverse_backward", "NewtonInverse_is_supported",
]


@pytest.fixture(scope="module")
def L():
    import laplacianformer_amd as lf

    return lf.ext()


def test_module_identity(L):
    assert L.__name__ == "Laplace_subtraction_cuda"
    import Laplace_subtraction_cuda  # registered by the package

    assert Laplace_subtraction_cuda is L
    for name in REFERENCE_EXPORTS + ["LaplaceSubtraction_backward"]:
        assert callable(getattr(L, name)), name


def test_version_probes(L):
    assert L.has_cuda() is False
    assert L.get_cuda_version().startswith("HIP ")
    assert L.get_compiler_version()
    assert L.NewtonInverse_is_supported(256) and not L.NewtonInverse_is_supported(257)


def test_cpu_tensors_raise_reference_errors(L):
    q = torch.randn(1, 1, 4, 8)
    k = torch.randn(1, 1, 8, 3)
    g = torch.randn(1, 1, 4, 3)
    for fn, args in ((L.LaplaceSubtraction_forward, (q, k, torch.empty(1, 1, 4, 3))),
                     (L.LaplaceSubtraction_backward_query, (g, q, k, torch.empty_like(q))),
                     (L.LaplaceSubtraction_backward_key, (g, q, k, torch.empty_like(k))),
                     (L.LaplaceSubtraction_reduce_forward, (q, k, torch.empty(1, 1, 4, 3))),
                     (L.LaplaceSubtraction_backward, (g, q, k, torch.empty_like(q), torch.empty_like(k)))):
        with pytest.raises(RuntimeError, match="Not implemented on the CPU"):
            fn(*args)
    m = torch.randn(1, 1, 4, 4)
    with pytest.raises(RuntimeError, match="mat must be on GPU"):
        L.NewtonInverse_forward(m, torch.empty_like(m), 3)
    with pytest.raises(RuntimeError, match="tensors must be on GPU"):
        L.NewtonInverse_backward(m, m, torch.empty_like(m))


def test_no_cpu_fallback_in_functional():
    import laplacianformer_amd as lf

    q = torch.randn(1, 1, 4, 8, requires_grad=True)
    k = torch.randn(1, 1, 8, 3, requires_grad=True)
    with pytest.raises(RuntimeError, match="Not implemented on the CPU"):
        lf.laplace_subtraction(q, k)
    with pytest.raises(RuntimeError, match="mat must be on GPU"):
        lf.newton_inverse(torch.randn(1, 1, 4, 4), 3)
    # The attention layer: CPU inputs take the per-op composition, whose first distance
    # raises; the single-node entry rejects them before any launch.
    x = torch.randn(1, 1, 64, 16)
    with pytest.raises(RuntimeError, match="Not implemented on the CPU"):
        lf.laplacian_attention(x, x, x, grid=(8, 8), pool=4)
    with pytest.raises(RuntimeError, match="one GPU"):
        lf.ext().LaplacianAttention_forward(x, x, x, 8, 8, 4, 10)


def test_product_never_imports_the_oracle():
    """The product package does not import, load or call the test oracle."""
    import glob
    import os
    import re

    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "laplacianformer_amd")
    for path in glob.glob(os.path.join(pkg, "**", "*.*"), recursive=True):
        if path.endswith((".py", ".hip", ".cpp", ".h")):
            text = open(path).read()
            assert not re.search(r"^\s*(import|from)\s+oracle\b", text, re.M), path
            assert "liblforacle" not in text and "laplace_oracle" not in text, path

"""MI355X-native LaplaceSubtraction and NewtonInverse for LaplacianFormer.

Drop-in for the reference's ``Laplace_subtraction_cuda`` extension: ``ext()``
returns a module with the same name and exports, backed by hand-written gfx950
HIP kernels behind the C ABI of ``include/laplacianformer_amd.h``.
"""
from ._lib import EXT_PATH, LIB_PATH, capi, check, dtype_code, ext
from .attention import LaplacianAttention, laplacian_attention
from .graphs import GraphedStep
from .functional import (LaplaceKernelFunction, LaplaceSubtractionFunction, NewtonInverseFunction,
                         TallMixFunction, TallProductFunction, laplace_kernel, laplace_subtraction, mix_rows,
                         newton_inverse, tall_mix, tall_product, tall_t)

__all__ = [
    "EXT_PATH", "LIB_PATH", "capi", "check", "dtype_code", "ext", "LaplaceKernelFunction",
    "LaplaceSubtractionFunction", "NewtonInverseFunction", "LaplacianAttention", "laplace_kernel",
    "laplace_subtraction", "laplacian_attention", "newton_inverse", "TallMixFunction", "TallProductFunction",
    "mix_rows", "tall_mix", "tall_product", "tall_t", "GraphedStep",
]

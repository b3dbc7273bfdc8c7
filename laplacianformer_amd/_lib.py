"""Loaders for the two in-tree native libraries.

``ext()`` returns the drop-in PyTorch module ``Laplace_subtraction_cuda`` (the
reference's module name; it is also registered in ``sys.modules`` under that
name so ``import Laplace_subtraction_cuda`` works once this package is
imported). ``capi()`` returns ``liblfamd.so`` through ctypes with the prototypes
of ``include/laplacianformer_amd.h``. Both raise if the library is missing:
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "liblfamd.so")
EXT_NAME = "Laplace_subtraction_cuda"
EXT_PATH = os.path.join(PKG_DIR, EXT_NAME + ".so")

_ext = None
_capi = None

# (name, restype, argtypes) for every symbol of include/laplacianformer_amd.h.
_P, _I, _I64, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
_DIMS = [_I64] * 5
CAPI_PROTOTYPES = [
    ("lfamd_laplace_forward", _I, [_I, _P, _P, _P] + _DIMS + [_P]),
    ("lfamd_laplace_backward_query", _I, [_I, _P, _P, _P, _P] + _DIMS + [_P]),
    ("lfamd_laplace_backward_workspace_size", _SZ, [_I] + _DIMS),
    ("lfamd_laplace_backward_key", _I, [_I, _P, _P, _P, _P] + _DIMS + [_P, _SZ, _P]),
    ("lfamd_laplace_backward", _I, [_I, _P, _P, _P, _P, _P] + _DIMS + [_P, _SZ, _P]),
    ("lfamd_laplace_reduce_forward", _I, [_I, _P, _P, _P] + _DIMS + [_P]),
    ("lfamd_laplace_backward_noalloc", _I, [_I, _P, _P, _P, _P, _P] + _DIMS + [_P]),
    ("lfamd_laplace_backward_noalloc_limit", _SZ, []),
    ("lfamd_laplace_kernel_forward", _I, [_I, _P, _P, _P] + _DIMS + [ctypes.c_float, _P]),
    ("lfamd_laplace_kernel_backward", _I, [_I, _P, _P, _P, _P, _P, _P] + _DIMS + [ctypes.c_float, _P, _SZ, _P]),
    ("lfamd_laplace_kernel_forward_multi", _I, [_I, _I, _P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_float, _P]),
    ("lfamd_laplace_kernel_backward_multi_workspace_size", _SZ, [_I, _I, _P, _I64, _I64, _I64, _I64]),
    ("lfamd_laplace_kernel_backward_multi", _I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                                  ctypes.c_float, _P, _SZ, _P]),
    ("lfamd_newton_workspace_size", _SZ, [_I, _I64, _I64]),
    ("lfamd_newton_forward", _I, [_I, _P, _P, _I64, _I64, _I, _P, _SZ, _P]),
    ("lfamd_newton_backward", _I, [_I, _P, _P, _P, _I64, _I64, _P, _SZ, _P]),
    ("lfamd_newton_is_supported", _I, [_I64]),
    ("lfamd_mix_rows", _I, [_I, _P, _P, _I, _P, _I64, _I64, _I, _I, _I64, _I64, _I64, _P]),
    ("lfamd_tall_t_workspace_size", _SZ, [_I64, _I64]),
    ("lfamd_tall_t", _I, [_I, _P, _P, _P, _I64, _I64, _I, _I, _P, _SZ, _P]),
    ("lfamd_attention_landmarks_forward", _I, [_P, _P, _I, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _P, _SZ, _P]),
    ("lfamd_attention_landmarks_backward", _I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I,
                                                _I, _P, _SZ, _P]),
    ("lfamd_landmark_pool", _I, [_I, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _P]),
    ("lfamd_landmark_pool_backward", _I, [_I, _P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _P]),
    ("lfamd_runtime_version", _I, []),
    ("lfamd_status_string", ctypes.c_char_p, [_I]),
    ("lfamd_last_error", ctypes.c_char_p, []),
]

# Element type codes (LFAMD_F32, ...).
DTYPE_CODES = {"float32": 0, "float16": 1, "bfloat16": 2, "float64": 3}


def _require(path: str) -> None:
    if not os.path.exists(path):
        raise ImportError(
            f"{os.path.basename(path)} is not built; run `python -m laplacianformer_amd._build` "
            "(laplacianformer_amd has no CPU fallback)")


def ext():
    """The drop-in extension module (reference module name and exports)."""
    global _ext
    if _ext is None:
        import torch  # noqa: F401  (loads PyTorch's HIP runtime first)

        _require(LIB_PATH)
        _require(EXT_PATH)
        spec = importlib.util.spec_from_file_location(EXT_NAME, EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        sys.modules.setdefault(EXT_NAME, mod)
        _ext = mod
    return _ext


def capi():
    """ctypes handle on liblfamd.so with the C prototypes applied."""
    global _capi
    if _capi is None:
        import torch  # noqa: F401  (share PyTorch's HIP runtime)

        _require(LIB_PATH)
        lib = ctypes.CDLL(LIB_PATH)
        for name, res, args in CAPI_PROTOTYPES:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _capi = lib
    return _capi


def dtype_code(t) -> int:
    """C-ABI element type code of a torch dtype or tensor."""
    name = str(getattr(t, "dtype", t)).replace("torch.", "")
    if name not in DTYPE_CODES:
        raise TypeError(f"unsupported element type {name}")
    return DTYPE_CODES[name]


def check(status: int) -> None:
    """Raises RuntimeError carrying lfamd_last_error() for a non-zero status."""
    if status != 0:
        lib = capi()
        msg = lib.lfamd_last_error().decode() or lib.lfamd_status_string(status).decode()
        raise RuntimeError(msg)

"""C ABI checks that need no GPU: the library loads, exports every symbol that
include/*.h declares, and rejects bad arguments before touching the device."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(lfamd_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    import laplacianformer_amd as lf

    return lf.capi()


def test_exports_every_declared_symbol(lib):
    names = declared_symbols()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    import laplacianformer_amd._lib as L

    assert sorted(n for n, _, _ in L.CAPI_PROTOTYPES) == names


def test_status_strings_and_version(lib):
    assert lib.lfamd_status_string(0) == b"ok"
    assert lib.lfamd_status_string(3) == b"size outside the supported envelope"
    assert lib.lfamd_status_string(99) == b"unknown status"
    v = lib.lfamd_runtime_version()
    assert v >= 600, v  # HIP >= 6.0 as major*100 + minor


def test_newton_envelope(lib):
    table = {0: 0, 1: 1, 16: 1, 49: 1, 64: 1, 100: 1, 128: 1, 129: 1, 256: 1, 257: 0, -3: 0}
    for n, want in table.items():
        assert lib.lfamd_newton_is_supported(n) == want, n


def test_argument_errors_without_device(lib):
    null = ctypes.c_void_p(0)
    assert lib.lfamd_laplace_forward(7, null, null, null, 1, 1, 1, 1, 1, null) == 2
    assert b"dtype" in lib.lfamd_last_error()
    assert lib.lfamd_laplace_forward(0, null, null, null, -1, 1, 1, 1, 1, null) == 1
    # Empty problems succeed without launching anything.
    assert lib.lfamd_laplace_forward(0, null, null, null, 0, 4, 5, 6, 7, null) == 0
    assert lib.lfamd_laplace_backward(1, null, null, null, null, null, 2, 2, 0, 3, 4, null, 0, null) in (0, 4)
    assert lib.lfamd_newton_forward(0, null, null, 4, 257, 3, null, 0, null) == 3
    assert b"N=257" in lib.lfamd_last_error()
    assert lib.lfamd_newton_forward(3, null, null, 4, 100, 3, null, 0, null) == 3  # fp64 envelope is n <= 96
    assert lib.lfamd_newton_backward(9, null, null, null, 4, 16, null, 0, null) == 2
    # 128 < n <= 256 needs the fp32 workspace; without one the call is rejected before any launch.
    ws = lib.lfamd_newton_workspace_size(0, 4, 200)
    assert ws == 4 * (4 * 256 * 256 + 256) * 4  # per matrix: four padded fp32 copies + the row sums
    assert lib.lfamd_newton_workspace_size(0, 4, 128) == 0
    assert lib.lfamd_newton_workspace_size(3, 4, 90) == 0
    # Row products: dtype, width and pointer checks happen before any launch.
    assert lib.lfamd_mix_rows(3, null, null, 0, null, 2, 10, 49, 64, 1, 64, 3136, null) == 2  # no fp64
    assert lib.lfamd_mix_rows(0, null, null, 0, null, 2, 10, 65, 64, 1, 64, 4160, null) == 3  # inner > 64
    assert lib.lfamd_mix_rows(0, null, null, 0, null, 2, 10, 49, 64, 1, 64, 3136, null) == 1  # null pointers
    assert lib.lfamd_mix_rows(0, null, null, 0, null, 0, 10, 49, 64, 1, 64, 3136, null) == 0  # nothing to do
    assert lib.lfamd_mix_rows(0, null, null, 3, null, 2, 10, 49, 64, 1, 64, 3136, null) == 2  # fp64 output
    dummy = ctypes.c_void_p(16)
    assert lib.lfamd_newton_forward(0, dummy, dummy, 4, 200, 3, null, 0, null) == 1
    assert b"workspace" in lib.lfamd_last_error()
    assert lib.lfamd_newton_backward(0, dummy, dummy, dummy, 4, 200, null, ws - 1, null) == 1
    # Fused Laplacian-kernel pair: dtype and envelope checks come before any pointer use.
    assert lib.lfamd_laplace_kernel_forward(7, null, null, null, 1, 1, 4, 4, 8, 0.5, null) == 2
    assert lib.lfamd_laplace_kernel_forward(3, null, null, null, 1, 1, 4, 4, 8, 0.5, null) == 3  # fp64
    assert lib.lfamd_laplace_kernel_forward(0, null, null, null, 1, 1, 4, 4, 12, 0.5, null) == 3  # C % 8
    assert lib.lfamd_laplace_kernel_forward(0, null, null, null, 1, 1, 4, 300, 8, 0.5, null) == 3  # M > 256
    assert lib.lfamd_laplace_kernel_forward(1, null, null, null, 1, 1, 4, 49, 64, 0.5, null) == 1  # null
    assert lib.lfamd_laplace_kernel_forward(1, null, null, null, 0, 1, 4, 49, 64, 0.5, null) == 0  # empty
    kb = lib.lfamd_laplace_kernel_backward
    assert kb(0, null, null, null, null, dummy, null, 1, 1, 8, 49, 64, 0.5, null, 0, null) == 3  # fp32
    assert kb(1, null, null, null, null, dummy, null, 1, 1, 8, 8, 64, 0.5, null, 0, null) == 3  # M = 8
    assert kb(1, null, null, null, null, dummy, null, 1, 1, 8, 257, 64, 0.5, null, 0, null) == 3  # M = 257
    assert kb(1, null, null, null, null, dummy, null, 1, 1, 8, 50, 64, 0.5, null, 0, null) == 1  # M = 50: null
    assert kb(1, null, null, null, null, dummy, null, 1, 1, 8, 49, 64, 0.5, null, 0, null) == 1  # null
    assert kb(1, null, null, null, null, null, dummy, 1, 1, 8, 49, 64, 0.5, null, 0, null) == 1  # ws
    assert b"workspace" in lib.lfamd_last_error() or b"null" in lib.lfamd_last_error()
    assert kb(1, null, null, null, null, null, null, 1, 1, 8, 49, 64, 0.5, null, 0, null) == 0  # nothing asked
    assert lib.lfamd_laplace_backward_workspace_size(1, 32, 1, 3136, 49, 64) > 0
    assert lib.lfamd_laplace_backward_workspace_size(1, 0, 1, 3136, 49, 64) == 0


def test_multi_backward_bounds_without_device(lib):
    """The segmented fused-kernel backward keeps row counts and its linear workgroup id in
    32-bit ints: a source longer than INT32_MAX / 2 rows, or a dtype the path does not take,
    gives no workspace size and an LFAMD_ERR_UNSUPPORTED call, before any device query."""
    n = (ctypes.c_int64 * 3)(49, 2 ** 31, 784)
    ws = lib.lfamd_laplace_kernel_backward_multi_workspace_size
    assert ws(1, 3, n, 64, 2, 49, 64) == 0
    assert ws(1, 3, (ctypes.c_int64 * 3)(49, 2 ** 30, 784), 64, 2, 49, 64) == 0
    assert ws(0, 1, (ctypes.c_int64 * 1)(784), 64, 2, 49, 64) == 0   # fp32: the path is fp16 only
    assert ws(2, 1, (ctypes.c_int64 * 1)(784), 64, 2, 49, 64) == 0   # bf16
    dummy = ctypes.c_void_p(16)
    ptrs = (ctypes.c_void_p * 3)(16, 16, 16)
    st = lib.lfamd_laplace_kernel_backward_multi(1, 3, ptrs, ptrs, ptrs, n, dummy, ptrs, dummy, 64, 2, 49, 64,
                                                 ctypes.c_float(0.125), dummy, 1 << 20, ctypes.c_void_p(0))
    assert st == 3
    assert b"rows" in lib.lfamd_last_error()

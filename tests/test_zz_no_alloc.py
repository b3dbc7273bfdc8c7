"""lfamd_laplace_backward_noalloc (static-scratch backward, no allocation) against
lfamd_laplace_backward with a caller workspace: identical bits, on two calls in a
row with the second smaller, plus the size limit rejected before any launch."""
import ctypes

import pytest
import torch

from lfcheck import gen

pytestmark = pytest.mark.gpu


def _pair(gpu, lib, lf, dt_name, B, H, N, M, C, seed):
    dt = lf.dtype_code(getattr(torch, {"f16": "float16", "bf16": "bfloat16", "f32": "float32"}[dt_name]))
    q = gen((B, H, N, C), seed, dt_name).to(gpu)
    k = gen((B, H, C, M), seed + 1, dt_name).to(gpu)
    g = gen((B, H, N, M), seed + 2, dt_name).to(gpu)
    dq_a, dk_a = torch.empty_like(q), torch.empty_like(k)
    dq_b, dk_b = torch.full_like(q, 7.0), torch.full_like(k, 7.0)
    ws_bytes = lib.lfamd_laplace_backward_workspace_size(dt, B, H, N, M, C)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=gpu)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    lf.check(lib.lfamd_laplace_backward(dt, g.data_ptr(), q.data_ptr(), k.data_ptr(), dq_a.data_ptr(),
                                        dk_a.data_ptr(), B, H, N, M, C, ws.data_ptr(), ws_bytes, s))
    lf.check(lib.lfamd_laplace_backward_noalloc(dt, g.data_ptr(), q.data_ptr(), k.data_ptr(), dq_b.data_ptr(),
                                                dk_b.data_ptr(), B, H, N, M, C, s))
    torch.cuda.synchronize()
    assert torch.equal(dq_a.cpu(), dq_b.cpu()), (dt_name, B, H, N, M, C, "grad_query")
    assert torch.equal(dk_a.cpu(), dk_b.cpu()), (dt_name, B, H, N, M, C, "grad_key")


@pytest.mark.parametrize("dt_name", ["f16", "f32"])
def test_noalloc_matches_workspace_entry(gpu, dt_name):
    import laplacianformer_amd as lf

    lib = lf.capi()
    print(f"no-alloc backward {dt_name}", flush=True)
    _pair(gpu, lib, lf, dt_name, 4, 2, 1000, 49, 64, 41)   # first call: the larger one
    _pair(gpu, lib, lf, dt_name, 1, 1, 300, 49, 64, 51)    # second call, smaller, same scratch


def test_noalloc_limit(gpu):
    import laplacianformer_amd as lf

    lib = lf.capi()
    assert lib.lfamd_laplace_backward_noalloc_limit() == 8 << 20
    # BASELINE config 4 sizes need far more workspace: rejected before touching any pointer.
    rc = lib.lfamd_laplace_backward_noalloc(2, None, None, None, None, None, 16, 8, 4096, 256, 64, None)
    assert rc == 3 and b"static scratch" in lib.lfamd_last_error()

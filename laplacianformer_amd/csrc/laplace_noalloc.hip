// Allocation-free variant of the fused LaplaceSubtraction backward.
//
// lfamd_laplace_backward takes its grad_key partial sums in a caller-provided
// workspace. Callers that cannot allocate device memory at all (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc) call
// lfamd_laplace_backward_noalloc instead: the partials live in `scratch`, a
// file-scope device array of kNoAllocScratchBytes that every GPU the library
// runs on holds until the process ends. Requests needing more are rejected.
//
// The array's name is a host-side stand-in, not a device address: its address
// on the current device comes from hipGetSymbolAddress, taken once per device
// (with that device current) and kept. Every call on a GPU shares that GPU's
// array: calls that overlap on one GPU (different streams, or host threads)
// race on it. The kernels overwrite every partial they read, so nothing has to
// start at zero.
#include <mutex>

#include "lf_common.h"
#include "lf_internal.h"

namespace lfamd {

constexpr size_t kNoAllocScratchBytes = 8u << 20;  // 8 MiB: configs 1, 2 and 5 need <= 3.1 MiB
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kNoAllocMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LFAMD_ERR_HIP, "laplace backward (no-alloc): hipGetDevice failed");
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return fail(LFAMD_ERR_UNSUPPORTED, "laplace backward (no-alloc): device %d beyond %d", dev, kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LFAMD_ERR_HIP, "laplace backward (no-alloc): hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ok();
}

}  // namespace
}  // namespace lfamd

using namespace lfamd;

extern "C" {

size_t lfamd_laplace_backward_noalloc_limit(void) { return kNoAllocScratchBytes; }

int lfamd_laplace_backward_noalloc(int dtype, const void* grad_output, const void* query, const void* key,
                                   void* grad_query, void* grad_key, int64_t batch, int64_t heads, int64_t q_len,
                                   int64_t k_len, int64_t channels, void* stream) {
  const size_t need = lfamd_laplace_backward_workspace_size(dtype, batch, heads, q_len, k_len, channels);
  if (need > kNoAllocScratchBytes)
    return fail(LFAMD_ERR_UNSUPPORTED,
                "laplace backward (no-alloc): these sizes need %zu bytes of workspace, the static scratch holds %zu",
                need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int s = scratch_address(&ws);
    if (s) return s;
  }
  return lfamd_laplace_backward(dtype, grad_output, query, key, grad_query, grad_key, batch, heads, q_len, k_len,
                                channels, ws, need > 0 ? kNoAllocScratchBytes : 0, stream);
}

}  // extern "C"

// Runtime plumbing of the C ABI: status strings, per-thread error text, cached
// device limits and the HIP runtime version probe.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>

#include "lf_internal.h"

namespace lfamd {

static thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_last_error[0] = '\0';
  return LFAMD_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LFAMD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

int max_lds_bytes() {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  // The opt-in limit (what hipFuncSetAttribute may raise a kernel to) if the
  // runtime reports one, else the default per-workgroup limit.
  int v = 0, optin = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
    v = 65536;
  if (hipDeviceGetAttribute(&optin, hipDeviceAttributeSharedMemPerBlockOptin, dev) == hipSuccess && optin > v)
    v = optin;
  cache[dev] = v;
  return v;
}

int set_dyn_lds(const void* fn, size_t bytes, const char* what) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> done;
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lk(mu);
  size_t& have = done[{fn, dev}];
  if (have >= bytes) return LFAMD_OK;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess)
    return fail(LFAMD_ERR_HIP, "%s: hipFuncSetAttribute failed", what);
  have = bytes;
  return LFAMD_OK;
}

int check_fit(const void* fn, unsigned threads, size_t dynLds, const char* what) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, hipFuncAttributes> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  hipFuncAttributes a{};
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find({fn, dev});
    if (it != cache.end()) {
      a = it->second;
    } else {
      if (hipFuncGetAttributes(&a, fn) != hipSuccess)
        return fail(LFAMD_ERR_HIP, "%s: hipFuncGetAttributes failed", what);
      cache[{fn, dev}] = a;
    }
  }
  // A workgroup of W waves puts ceil(W / 4) of them on each of the CU's four
  // SIMDs at once, and a SIMD holds 512 VGPRs per lane, allocated in granules
  // of 8. Inline asm that names registers above what the launch bounds allow
  // only draws a compiler warning, and a dispatch that cannot fit aborts the
  // queue (HSA_STATUS_ERROR_INVALID_ISA), so the fit is checked before it.
  const int waves = (int)((threads + 63) / 64), perSimd = (waves + 3) / 4;
  const int regs = (a.numRegs + 7) / 8 * 8;
  if ((int)threads > a.maxThreadsPerBlock || regs * perSimd > 512 ||
      a.sharedSizeBytes + dynLds > (size_t)max_lds_bytes())
    return fail(LFAMD_ERR_HIP,
                "%s: the kernel (%d VGPRs, %zu + %zu bytes of LDS, at most %d threads) does not fit a %u-thread "
                "workgroup on one CU",
                what, a.numRegs, (size_t)a.sharedSizeBytes, dynLds, a.maxThreadsPerBlock, threads);
  return LFAMD_OK;
}

int num_cus() {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  cache[dev] = v;
  return v;
}

}  // namespace lfamd

extern "C" {

int lfamd_runtime_version(void) {
  int v = 0;
  if (hipRuntimeGetVersion(&v) != hipSuccess) return 0;
  // hipRuntimeGetVersion encodes major*10000000 + minor*100000 + patch.
  int major = v / 10000000, minor = (v / 100000) % 100;
  return major * 100 + minor;
}

const char* lfamd_status_string(int status) {
  switch (status) {
    case LFAMD_OK: return "ok";
    case LFAMD_ERR_ARG: return "invalid argument";
    case LFAMD_ERR_DTYPE: return "unsupported element type";
    case LFAMD_ERR_UNSUPPORTED: return "size outside the supported envelope";
    case LFAMD_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

const char* lfamd_last_error(void) { return lfamd::g_last_error; }

}  // extern "C"

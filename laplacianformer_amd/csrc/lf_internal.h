// Host-side internals shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/laplacianformer_amd.h"

namespace lfamd {

// Records a message for lfamd_last_error() on the calling thread and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the calling thread's error message and returns LFAMD_OK.
int ok();

// Turns a pending launch error into LFAMD_ERR_HIP.
int check_launch(const char* what);

// Max dynamic LDS bytes per workgroup on the current device (cached per device).
int max_lds_bytes();

// Checks, once per kernel and device (cached), that kernel `fn` fits a
// workgroup of `threads` threads with `dynLds` bytes of dynamic LDS on one CU:
// its VGPRs times the waves each SIMD must hold, its LDS and its launch bound.
// LFAMD_OK, or LFAMD_ERR_HIP with `what` before anything is dispatched.
int check_fit(const void* fn, unsigned threads, size_t dynLds, const char* what);

// Compute units of the current device (cached per device; 256 if unknown).
int num_cus();

// Raises kernel `fn`'s dynamic LDS limit on the current device to at least
// `bytes` (hipFuncSetAttribute once per kernel, device and size; later calls
// with no larger size are a lookup). LFAMD_OK or LFAMD_ERR_HIP with `what`.
int set_dyn_lds(const void* fn, size_t bytes, const char* what);

// Column-split fused backward of 16-bit LaplaceSubtraction (laplace_bwd2.hip).
// With B2Grad::gk set, the gradient is that of the fused kernel exp(-scale * distance):
// fp32 gk = dL/dK and kv = K replace g (fp16 only).
struct B2Grad {
  const float* gk = nullptr;
  const float* kv = nullptr;
  float scale = 0.0f;
};
bool b2_ok(int dtype, int64_t BH, int64_t N, int64_t M, int64_t C);
size_t b2_workspace_elems(int64_t BH, int64_t N, int64_t M, int64_t C);
int b2_launch(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, size_t wsBytes,
              int64_t BH, int64_t N, int64_t M, int64_t C, hipStream_t st, const char* who,
              const B2Grad& kg = B2Grad{});
// The fused-kernel gradient (fp16, M = 49, C % 64 == 0) of up to three row
// sources sharing one key in one launch: per source n[i] rows, gk[i], kv[i],
// query q[i] (4-byte aligned) and grad_query dq[i]; grad_key dk sums them all.
size_t b2_workspace_elems_multi(int nsrc, const int64_t* n, int64_t BH, int64_t C);
// Workgroups of that launch (its linear workgroup id must fit an int).
int64_t b2_multi_workgroups(int nsrc, const int64_t* n, int64_t BH, int64_t C);
int b2_launch_multi(int nsrc, const float* const* gk, const float* const* kv, const void* const* q, void* const* dq,
                    const int64_t* n, const void* k, void* dk, void* ws, size_t wsBytes, int64_t BH, int64_t C,
                    float scale, hipStream_t st, const char* who);

// Row-staged forward of LaplaceSubtraction at M = 49 (laplace_fwd2.hip); kernelEpi:
// exp(-scale * distance) in fp32 instead of the distance in the element type.
bool f2_ok(int dtype, int64_t BH, int64_t N, int64_t M, int64_t C, const void* q);
// Wide-landmark forward, M in {128, 256} (laplace_fwd2.hip).
bool f3_ok(int dtype, int64_t BH, int64_t N, int64_t M, int64_t C, const void* q, const void* out);
int f3_launch(int dtype, const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t M, int64_t C,
              hipStream_t st);
int f2_launch(int dtype, bool kernelEpi, const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t C,
              float scale, hipStream_t st);
// exp(-scale * distance) over up to three row sources (n[i] rows per slice,
// query q[i], fp32 output o[i]) sharing one key, in one launch.
int f2_launch_multi(int dtype, int nsrc, const void* const* q, const int64_t* n, const void* k, float* const* o,
                    int64_t BH, int64_t C, float scale, hipStream_t st);

// The bf16 tall product's per-workgroup partials (mix_kernels.hip): [slices][per][64][64]
// fp32, entry [p][q] = sum over a workgroup's rows of a[n][p] * b[n][q]; *perOut = per.
// Checks a tall product's partial launch (tall_t_partials) and gives its workgroups per slice.
int tall_t_check(int b_dtype, const float* A, const void* B, size_t wsBytes, int64_t slices, int64_t N, int P, int Q,
                 int* perOut);
int tall_t_partials(int b_dtype, const float* A, const void* B, float* ws, size_t wsBytes, int64_t slices,
                    int64_t N, int P, int Q, hipStream_t st, int* perOut);

// Three row products c[i][s][n][q] = sum_p a[i][s][n][p] * b[i][s](q, p) in one
// launch (mix_kernels.hip): i = 0, 1 with A of element type dtype [N][P[0]],
// fp32 C [N][Q[0]], B strides sq[0], sp[0], bStride[0]; i = 2 with fp32 A
// [N][P[1]] and C of element type dtype [N][Q[1]] (strides [1]).
// LFAMD_ERR_UNSUPPORTED where the bf16 row kernel does not take them. Only
// products first..2 run (first = 0: all three).
int mix_rows_trio(int dtype, const void* const* A, const float* const* B, void* const* C, int64_t slices, int64_t N,
                  const int* P, const int* Q, const int64_t* sq, const int64_t* sp, const int64_t* bStride,
                  hipStream_t st, int first = 0);

inline bool valid_dtype(int dt) {
  return dt == LFAMD_F32 || dt == LFAMD_F16 || dt == LFAMD_BF16 || dt == LFAMD_F64;
}
inline size_t dtype_size(int dt) { return dt == LFAMD_F64 ? 8 : (dt == LFAMD_F32 ? 4 : 2); }

}  // namespace lfamd

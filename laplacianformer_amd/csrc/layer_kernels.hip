// layer_kernels.hip - the LaplacianFormer attention layer's landmark pooling
// on gfx950 (no reference counterpart: the reference ships the two operators
// only; the layer around them is its caller's).
//
// Landmarks are pool x pool means of K over its gh x gw token grid:
//   km[b,h,m,c] = cast(sum_{patch} f32(k[b,h,n,c]) * f32(1 / pool^2)),  m = (gy, gx) of n
// written both as km [B,H,M,d] and channel-major as km_cm [B,H,d,M] (the key
// layout of the distance kernels), in one pass over K.
//
// Their backward adds each landmark's gradient / pool^2 to the pool x pool
// patch of K's gradient. The landmark gradient is the sum of the distance
// backward's grad_query of the landmark rows, dkm [B,H,M,d], and the three
// channel-major grad_keys dcm0..2 [B,H,d,M]; with every operation rounded to
// the element type as the composition of elementwise tensor ops it replaces:
//   t   = cast(cast(dcm0 + dcm1) + dcm2)
//   u   = cast(dkm + t^T)
//   dk += cast(f32(u) * f32(1 / pool^2))   (dk += : cast(f32(dk) + f32(.)))
// (a tensor divided by a scalar is multiplied by the scalar's fp32 reciprocal)
// A workgroup per landmark row stages the row's share in LDS, then adds it to
// the pool token rows under it (one contiguous strip of K's gradient).
#include <algorithm>

#include "lf_common.h"
#include "lf_internal.h"

namespace lfamd {

namespace {

constexpr int kPoolLds = 2048;  // floats of one staged landmark row (mw * d) in the backward

// Grid (gh / pool landmark rows, B*H), 256 threads over the row's (landmark
// column, channel) pairs, channels fastest. For pool = 4 the 16 patch values
// of a thread are all loaded before the sum (row-major patch order either way).
template <typename T>
__global__ void __launch_bounds__(256)
landmark_pool_kernel(const T* __restrict__ k, T* __restrict__ km, T* __restrict__ kmcm, int gh, int gw, int pool,
                     int d) {
  const int my = blockIdx.x, mw = gw / pool, M = (gh / pool) * mw;
  const int64_t bh = blockIdx.y;
  const float inv = 1.0f / (float)(pool * pool);
  const int total = mw * d;
  for (int e = threadIdx.x; e < total; e += 256) {
    const int mx = e / d, c = e - mx * d;
    const T* src = k + (bh * gh * gw + (int64_t)my * pool * gw + (int64_t)mx * pool) * d + c;
    float s = 0.0f;
    if (pool == 4) {
      T v[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) v[t] = src[((t >> 2) * gw + (t & 3)) * d];
#pragma unroll
      for (int t = 0; t < 16; ++t) s += to_acc(v[t]);
    } else {
      for (int i = 0; i < pool; ++i)
        for (int j = 0; j < pool; ++j) s += to_acc(src[(i * gw + j) * d]);
    }
    const T r = from_acc<T>(s * inv);
    km[(bh * M + (int64_t)my * mw + mx) * d + c] = r;
    kmcm[(bh * d + c) * M + (int64_t)my * mw + mx] = r;
  }
}

// The landmark row's gradient share gs[mx][c] = cast(f32(u) * f32(1 / pool^2)),
// u = cast(dkm + t^T), t = cast(cast(dcm0 + dcm1) + dcm2), into LDS (the
// channel-major parts read landmark-fastest, dkm channel-fastest).
template <typename T>
__device__ __forceinline__ void pool_bwd_stage(float* __restrict__ tt, float* __restrict__ gsm,
                                               const T* __restrict__ dkm, const T* __restrict__ dcm0,
                                               const T* __restrict__ dcm1, const T* __restrict__ dcm2, int64_t bh,
                                               int my, int mw, int M, int d, float inv) {
#pragma clang fp contract(off)  // the product is rounded before it is used, as the tensor ops do
  const int total = mw * d;
  for (int e = threadIdx.x; e < total; e += 256) {
    const int c = e / mw, mx = e - c * mw;
    const int64_t cm = (bh * d + c) * M + (int64_t)my * mw + mx;
    tt[c * mw + mx] = to_acc(from_acc<T>(to_acc(from_acc<T>(to_acc(dcm0[cm]) + (dcm1 ? to_acc(dcm1[cm]) : 0.0f))) +
                                         (dcm2 ? to_acc(dcm2[cm]) : 0.0f)));
  }
  __syncthreads();
  for (int e = threadIdx.x; e < total; e += 256) {
    const int mx = e / d, c = e - mx * d;
    const T u = from_acc<T>(to_acc(dkm[(bh * M + (int64_t)my * mw + mx) * d + c]) + tt[c * mw + mx]);
    gsm[e] = to_acc(from_acc<T>(to_acc(u) * inv));
  }
  __syncthreads();
}

// Grid (gh / pool landmark rows, B*H), 256 threads: the landmark row's
// gradient share staged in LDS once (mw * d <= kPoolLds) and spread to a token
// row's gw * d elements (<= 8 * 256), then added to the pool token rows of K's
// gradient under it (one contiguous strip), the next row's loads in flight.
template <typename T>
__global__ void __launch_bounds__(256)
landmark_pool_bwd_kernel(T* __restrict__ dk, const T* __restrict__ dkm, const T* __restrict__ dcm0,
                         const T* __restrict__ dcm1, const T* __restrict__ dcm2, int gh, int gw, int pool, int d) {
  __shared__ float tt[kPoolLds], gsm[kPoolLds], gsx[8 * 256];
  const int my = blockIdx.x, mw = gw / pool, M = (gh / pool) * mw;
  const int64_t bh = blockIdx.y;
  const int R = gw * d;  // elements of one token row
  T* strip = dk + (bh * gh + (int64_t)my * pool) * R;
  T v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = strip[min((int)threadIdx.x + 256 * k, R - 1)];  // row 0, during the staging
  pool_bwd_stage<T>(tt, gsm, dkm, dcm0, dcm1, dcm2, bh, my, mw, M, d, 1.0f / (float)(pool * pool));
  for (int e = threadIdx.x; e < R; e += 256) {
    const int x = e / d, c = e - x * d;
    gsx[e] = gsm[(x / pool) * d + c];
  }
  __syncthreads();
  for (int i = 0; i < pool; ++i) {
    T w[8];
    const int in = min(i + 1, pool - 1);  // (the last row reloads itself)
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = strip[(int64_t)in * R + min((int)threadIdx.x + 256 * k, R - 1)];
#pragma unroll
    for (int k = 0; k < 8; ++k) asm volatile("" : "+v"(w[k]));  // (issued before this row's stores)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = threadIdx.x + 256 * k;
      if (e < R) strip[(int64_t)i * R + e] = from_acc<T>(to_acc(v[k]) + gsx[e]);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = w[k];
  }
}

// Any size: a thread per element of K's gradient, every part read from global.
template <typename T>
__global__ void __launch_bounds__(256)
landmark_pool_bwd_any_kernel(T* __restrict__ dk, const T* __restrict__ dkm, const T* __restrict__ dcm0,
                             const T* __restrict__ dcm1, const T* __restrict__ dcm2, int gh, int gw, int pool, int d) {
#pragma clang fp contract(off)
  const int y = blockIdx.x, mw = gw / pool, M = (gh / pool) * mw;
  const int64_t bh = blockIdx.y;
  const float inv = 1.0f / (float)(pool * pool);
  T* row = dk + (bh * gh + y) * (int64_t)gw * d;
  for (int e = threadIdx.x; e < gw * d; e += 256) {
    const int x = e / d, c = e - x * d;
    const int m = (y / pool) * mw + x / pool;
    const int64_t cm = (bh * d + c) * M + m;
    const T t = from_acc<T>(to_acc(from_acc<T>(to_acc(dcm0[cm]) + (dcm1 ? to_acc(dcm1[cm]) : 0.0f))) +
                            (dcm2 ? to_acc(dcm2[cm]) : 0.0f));
    const T u = from_acc<T>(to_acc(dkm[(bh * M + m) * d + c]) + to_acc(t));
    const T gs = from_acc<T>(to_acc(u) * inv);
    row[e] = from_acc<T>(to_acc(row[e]) + to_acc(gs));
  }
}

template <typename T>
void launch_pool_bwd(void* dk, const void* dkm, const void* dcm0, const void* dcm1, const void* dcm2, int64_t BH,
                     int gh, int gw, int pool, int d, hipStream_t st) {
  if ((int64_t)(gw / pool) * d <= kPoolLds && (int64_t)gw * d <= 8 * 256)
    hipLaunchKernelGGL(landmark_pool_bwd_kernel<T>, dim3((unsigned)(gh / pool), (unsigned)BH), dim3(256), 0, st,
                       static_cast<T*>(dk), static_cast<const T*>(dkm), static_cast<const T*>(dcm0),
                       static_cast<const T*>(dcm1), static_cast<const T*>(dcm2), gh, gw, pool, d);
  else
    hipLaunchKernelGGL(landmark_pool_bwd_any_kernel<T>, dim3((unsigned)gh, (unsigned)BH), dim3(256), 0, st,
                       static_cast<T*>(dk), static_cast<const T*>(dkm), static_cast<const T*>(dcm0),
                       static_cast<const T*>(dcm1), static_cast<const T*>(dcm2), gh, gw, pool, d);
}

int check_pool(int dtype, int64_t B, int64_t H, int gh, int gw, int pool, int d, const char* what) {
  if (dtype != LFAMD_F32 && dtype != LFAMD_F16 && dtype != LFAMD_BF16)
    return fail(LFAMD_ERR_DTYPE, "%s: unsupported dtype %d", what, dtype);
  if (B < 0 || H < 0 || gh < 1 || gw < 1 || pool < 1 || d < 1 || gh % pool || gw % pool || B * H > 65535 ||
      (int64_t)gh * gw * d > ((int64_t)1 << 30))
    return fail(LFAMD_ERR_ARG, "%s: bad sizes (B=%lld H=%lld grid=%dx%d pool=%d d=%d)", what, (long long)B,
                (long long)H, gh, gw, pool, d);
  return LFAMD_OK;
}

}  // namespace

}  // namespace lfamd

using namespace lfamd;

extern "C" int lfamd_landmark_pool(int dtype, const void* k, void* km, void* km_cm, int64_t B, int64_t H, int gh,
                                   int gw, int pool, int d, void* stream) {
  if (int s = check_pool(dtype, B, H, gh, gw, pool, d, "landmark pool")) return s;
  if (B * H == 0) return ok();
  if (!k || !km || !km_cm) return fail(LFAMD_ERR_ARG, "landmark pool: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(gh / pool), (unsigned)(B * H)), block(256);
  switch (dtype) {
    case LFAMD_F32:
      hipLaunchKernelGGL(landmark_pool_kernel<float>, grid, block, 0, st, static_cast<const float*>(k),
                         static_cast<float*>(km), static_cast<float*>(km_cm), gh, gw, pool, d);
      break;
    case LFAMD_F16:
      hipLaunchKernelGGL(landmark_pool_kernel<f16s>, grid, block, 0, st, static_cast<const f16s*>(k),
                         static_cast<f16s*>(km), static_cast<f16s*>(km_cm), gh, gw, pool, d);
      break;
    default:
      hipLaunchKernelGGL(landmark_pool_kernel<bf16s>, grid, block, 0, st, static_cast<const bf16s*>(k),
                         static_cast<bf16s*>(km), static_cast<bf16s*>(km_cm), gh, gw, pool, d);
  }
  return check_launch("landmark pool");
}

extern "C" int lfamd_landmark_pool_backward(int dtype, void* dk, const void* dkm, const void* dcm0, const void* dcm1,
                                            const void* dcm2, int64_t B, int64_t H, int gh, int gw, int pool, int d,
                                            void* stream) {
  if (int s = check_pool(dtype, B, H, gh, gw, pool, d, "landmark pool backward")) return s;
  if (B * H == 0) return ok();
  if (!dk || !dkm || !dcm0) return fail(LFAMD_ERR_ARG, "landmark pool backward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LFAMD_F32: launch_pool_bwd<float>(dk, dkm, dcm0, dcm1, dcm2, B * H, gh, gw, pool, d, st); break;
    case LFAMD_F16: launch_pool_bwd<f16s>(dk, dkm, dcm0, dcm1, dcm2, B * H, gh, gw, pool, d, st); break;
    default: launch_pool_bwd<bf16s>(dk, dkm, dcm0, dcm1, dcm2, B * H, gh, gw, pool, d, st);
  }
  return check_launch("landmark pool backward");
}

// mix_kernels.hip - the LaplacianFormer attention layer's output-heavy products
// on gfx950 (no reference counterpart: the reference ships the two operators
// only; these are the caller's matrix products around them).
//
//   C[s][n][q] = sum_{p < P} A[s][n][p] * B[s](q, p),   q < Q,  P, Q <= 64
//
// with A a tall [N, P] matrix per slice s (N in the thousands) and B a small
// Q x P matrix addressed through element strides (so that both W and W^T are
// read in place), and the tall transposed product C[s][p][q] = sum_n
// A[s][n][p] * B[s][n][q]. The layer's K_qm . W, grad_out . W^T, V . grad_kv^T
// and K_km . grad_kv are of the first form, K_km^T V and K_qm^T grad_out of the
// second. With inner and output widths of at most 64 they move ~32 MB per
// product at config 5, and their fp32 products, padded to 64 x 64 tiles, take
// about as long on the fp32 matrix cores as that HBM traffic. The main kernels
// (mix_rows_bf16_kernel, tall_t_bf16_kernel) therefore run them on the bf16
// matrix cores with fp32 operands split exactly into bf16 pieces, to fp32
// accuracy; operands without 16-byte aligned rows take the fp32 MFMA kernels
// (mix_rows_kernel, tall_t_kernel). C is written in fp32, fp16 or bf16 (one
// rounding of the fp32 sum); tests compare against an fp64 product within 1e-5
// of sum |a| |b|.
#include <algorithm>

#include "lf_common.h"
#include "lf_internal.h"
#include "mix_common.h"

namespace lfamd {


// B (4096 slots, 16 per thread) into Bs[q][p] (pitch kMixLS), zero outside
// Q x P; consecutive threads along B's smaller stride (coalesced for W and for
// W^T). The caller synchronizes.
__device__ __forceinline__ void stage_b(float* Bs, const float* __restrict__ Bm, int P, int Q, int64_t sq,
                                        int64_t sp) {
  const bool qFast = sq < sp;
  float v[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int e = threadIdx.x + 256 * u;
    const int q = qFast ? (e & 63) : (e >> 6), p = qFast ? (e >> 6) : (e & 63);
    v[u] = Bm[min(q, Q - 1) * sq + min(p, P - 1) * sp];
  }
  // (The empty asm uses every loaded value, so the compiler cannot sink the
  // loads into per-slot branches that would wait on each in turn.)
#pragma unroll
  for (int u = 0; u < 16; ++u) asm volatile("" : "+v"(v[u]));
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int e = threadIdx.x + 256 * u;
    const int q = qFast ? (e & 63) : (e >> 6), p = qFast ? (e >> 6) : (e & 63);
    Bs[q * kMixLS + p] = (q < Q && p < P) ? v[u] : 0.0f;
  }
}

// The fp32-MFMA row product for any alignment: a workgroup (4 waves) stages B
// once in LDS (pitch 68 floats); after that single barrier each wave works
// alone on 16-row groups g, g + 4 * gridDim.x, ... of its slice: the group's
// rows (loaded one group ahead, unconditionally at clamped indices) go to the
// wave's own 16 LDS rows, four 16 x 16 v_mfma_f32_16x16x4_f32 accumulators
// compute its 16 x Q outputs with k permuted per lane (k = 16 kb + 4 (lane / 16)
// + step) so that both operands are read as float4, and the outputs go back
// through the same LDS rows to be stored as one contiguous run of 16 * Q
// elements (64 consecutive per store).
template <typename TA, typename TC>
__global__ void __launch_bounds__(256)
mix_rows_kernel(const TA* __restrict__ A, const float* __restrict__ B, TC* __restrict__ C, int N, int P,
                int Q, int64_t sq, int64_t sp, int64_t bStride) {
  __shared__ __align__(16) float Bs[kMixPMax * kMixLS];      // Bs[q][p], zero outside Q x P
  __shared__ __align__(16) float Ws[4][kMixGroup * kMixLS];  // per wave: its A rows, then its C rows
  const int s = blockIdx.y;
  const int groups = (N + kMixGroup - 1) / kMixGroup;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const float* Bm = B + (size_t)s * bStride;
  const TA* A0 = A + (size_t)s * N * P;
  TC* C0 = C + (size_t)s * N * Q;
  float* W = Ws[wave];

  // Group g's rows into registers, raw: xa[u] = A[16 g + u][lane] at clamped
  // indices, zeroed outside the rows and P only when stored to LDS, so that the
  // loads are unconditional and stay in flight across the current group's work.
  TA xa[kMixGroup];
  auto loadA = [&](int g) {
    const int r0 = kMixGroup * g, last = min(kMixGroup, N - r0) - 1, pc = min(lane, P - 1);
#pragma unroll
    for (int u = 0; u < kMixGroup; ++u) xa[u] = A0[(size_t)(r0 + min(u, last)) * P + pc];
  };
  int g = blockIdx.x * 4 + wave;
  const int gstep = gridDim.x * 4;
  loadA(min(g, groups - 1));  // in flight while B is staged

  stage_b(Bs, Bm, P, Q, sq, sp);
  __syncthreads();  // the only workgroup barrier: from here on each wave works alone

  const float invQ = 1.0f / (float)Q;
  for (; g < groups; g += gstep) {
    const int r0 = kMixGroup * g, rows = min(kMixGroup, N - r0);
#pragma unroll
    for (int u = 0; u < kMixGroup; ++u) W[u * kMixLS + lane] = (u < rows && lane < P) ? to_acc(xa[u]) : 0.0f;
    wave_lds_sync();
    loadA(min(g + gstep, groups - 1));  // the last group reloads itself (cached)
    v4f acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 av = *reinterpret_cast<const float4*>(&W[li * kMixLS + 16 * kb + 4 * lg]);
      const float a[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 bv = *reinterpret_cast<const float4*>(&Bs[(16 * c + li) * kMixLS + 16 * kb + 4 * lg]);
        const float b[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int st = 0; st < 4; ++st) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], b[st], acc[c], 0, 0, 0);
      }
    }
    // C rows of the group through the wave's LDS rows (its A rows are read), then
    // written as one contiguous run of rows * Q elements, 64 consecutive per store.
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) W[(4 * lg + r) * kMixLS + 16 * c + li] = acc[c][r];
    wave_lds_sync();
    const int total = rows * Q;
    TC* Cg = C0 + (size_t)r0 * Q;
    float ov[kMixGroup];
#pragma unroll
    for (int j = 0; j < kMixGroup; ++j) {
      const int f = min(lane + 64 * j, total - 1);
      const int r = (int)(((float)f + 0.5f) * invQ), col = f - r * Q;
      ov[j] = W[r * kMixLS + col];
    }
    // (Every LDS read is issued before the stores, which are masked per lane.)
#pragma unroll
    for (int j = 0; j < kMixGroup; ++j) asm volatile("" : "+v"(ov[j]));
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < kMixGroup; ++j)
      if (lane + 64 * j < total) Cg[lane + 64 * j] = from_acc<TC>(ov[j]);
  }
}


// Grid (workgroups per slice, slices).
template <typename TA, typename TC, bool DIRECT>
__global__ void __launch_bounds__(64 * kMixWaves)
mix_rows_bf16_kernel(const TA* __restrict__ A, const float* __restrict__ B, TC* __restrict__ C, int N, int P,
                     int Q, int64_t sq, int64_t sp, int64_t bStride) {
  mix_rows_bf16_body<TA, TC, DIRECT>(A, B, C, N, P, Q, sq, sp, bStride, blockIdx.y, blockIdx.x, gridDim.x);
}

// Three row products in one launch (grid (workgroups per slice, 3 * slices),
// each product's workgroups after the previous one's; or products first..2 only): products 0 and 1 of one
// shape, A of element type TA [N][P0] and fp32 C [N][Q0]; product 2 with fp32 A
// [N][P1] and C of element type TA [N][Q1] (the attention layer's g w^T,
// v dkv^T and K_km dkv).
struct MixTrio {
  const void* A[3];
  const float* B[3];
  void* C[3];
  int P[2], Q[2];
  int64_t sq[2], sp[2], bStride[2];
};
template <typename TA, bool DIRECT01>
__global__ void __launch_bounds__(64 * kMixWaves)
mix_rows_bf16_trio_kernel(MixTrio t, int slices, int N, int first) {
  const int src = first + (int)blockIdx.y / slices, s = (int)blockIdx.y % slices;
  if (src < 2)
    mix_rows_bf16_body<TA, float, DIRECT01>(static_cast<const TA*>(t.A[src]), t.B[src], static_cast<float*>(t.C[src]),
                                            N, t.P[0], t.Q[0], t.sq[0], t.sp[0], t.bStride[0], s, blockIdx.x,
                                            gridDim.x);
  else
    mix_rows_bf16_body<float, TA, false>(static_cast<const float*>(t.A[2]), t.B[2], static_cast<TA*>(t.C[2]), N,
                                         t.P[1], t.Q[1], t.sq[1], t.sp[1], t.bStride[1], s, blockIdx.x, gridDim.x);
}

// Workgroups per slice. The bf16 kernel: one kMixWaves-wave workgroup per CU
// over the grid, at most one 16-row group per wave (measured at config 5,
// 128 slices of 784 rows, per call: 9.0 / 9.8 us for the two layouts with 12
// waves and two workgroups per slice, against 9.5 / 10.1 with 8 waves, 10.2 /
// 11.4 with 16, and 10.9 / 11.9 us with four 4-wave workgroups per slice: B is
// split once per CU, and three waves per SIMD overlap one another's loads,
// splits and MFMAs). The fp32 kernel (4 waves): about two workgroups per CU.
// A 16-byte aligned A with P = 64, or with 16-byte aligned slices, takes the
// bf16 kernel; anything else the fp32 LDS-staged kernel.
template <typename TA, typename TC>
int launch_mix(const void* A, const float* B, void* C, int64_t slices, int64_t N, int P, int Q, int64_t sq,
               int64_t sp, int64_t bStride, hipStream_t st) {
  const int64_t groups = (N + kMixGroup - 1) / kMixGroup;
  const int64_t cus = num_cus();
  const bool aligned = (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  const bool direct = aligned && P == kMixPMax;
  if (direct || (aligned && (N * P * (int64_t)sizeof(TA)) % 16 == 0)) {
    const int64_t per = std::max<int64_t>(
        1, std::min<int64_t>((groups + kMixWaves - 1) / kMixWaves, (cus + slices - 1) / slices));
    const dim3 grid((unsigned)per, (unsigned)slices), block(64 * kMixWaves);
    if (direct)
      hipLaunchKernelGGL((mix_rows_bf16_kernel<TA, TC, true>), grid, block, 0, st, static_cast<const TA*>(A), B,
                         static_cast<TC*>(C), (int)N, P, Q, sq, sp, bStride);
    else
      hipLaunchKernelGGL((mix_rows_bf16_kernel<TA, TC, false>), grid, block, 0, st, static_cast<const TA*>(A), B,
                         static_cast<TC*>(C), (int)N, P, Q, sq, sp, bStride);
  } else {
    const int64_t per =
        std::max<int64_t>(1, std::min<int64_t>((groups + 3) / 4, (2 * cus + slices - 1) / slices));
    hipLaunchKernelGGL((mix_rows_kernel<TA, TC>), dim3((unsigned)per, (unsigned)slices), dim3(256), 0, st,
                       static_cast<const TA*>(A), B, static_cast<TC*>(C), (int)N, P, Q, sq, sp, bStride);
  }
  return check_launch("mix rows");
}

// ---------------------------------------------------------------------------
// Tall transposed product C[s][p][q] = sum_n A[s][n][p] * B[s][n][q], A fp32
// [N][P], B [N][Q] (fp32 / fp16 / bf16, widened at load), P, Q <= 64: the
// layer's K_km^T V and K_qm^T grad_out, a long reduction over the N rows into a
// small output. The rows are split over `per` workgroups per slice, each
// leaving its [64][64] fp32 partial in the workspace; tall_t_reduce_kernel sums
// the partials in workgroup order (so the result is deterministic). Slices with
// 16-byte aligned rows take tall_t_bf16_kernel below; the others this fp32
// kernel: each workgroup takes 64-row tiles t, t + per, ... (the next tile's
// loads in flight during the current one's products), wave w computes output
// rows [16w, 16w + 16) x all Q columns as four v_mfma_f32_16x16x4_f32
// accumulators, k = row of the tile. (Config 5, 128 slices x 784 rows x 49 x
// 64, fp16 B: 17.8 us for this kernel, 13.6 us for the bf16 one, 31 us for
// torch.matmul on a converted fp32 copy of B.)
constexpr int kTallLS = 80;  // LDS pitch (floats): lanes 16 apart in k land 16 banks apart

template <typename TB>
__global__ void __launch_bounds__(256)
tall_t_kernel(const float* __restrict__ A, const TB* __restrict__ B, float* __restrict__ part, int N, int P, int Q) {
  __shared__ __align__(16) float As[kMixRows * kTallLS];  // As[r][p]
  __shared__ __align__(16) float Bs[kMixRows * kTallLS];  // Bs[r][q]
  const int s = blockIdx.y, per = gridDim.x;
  const int tiles = (N + kMixRows - 1) / kMixRows;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const float* A0 = A + (size_t)s * N * P;
  const TB* B0 = B + (size_t)s * N * Q;
  // Unconditional loads at clamped indices (rows >= 1), zeroed outside by a
  // select, so that all 32 are in flight at once.
  float va[16], vb[16];
  auto load = [&](int t) {
    const int n0 = t * kMixRows, rows = min(kMixRows, N - n0);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = threadIdx.x + 256 * u, r = e >> 6, c = e & 63;
      const size_t row = (size_t)(n0 + min(r, rows - 1));
      const float x = A0[row * P + min(c, P - 1)];
      const float y = to_acc(B0[row * Q + min(c, Q - 1)]);
      va[u] = (r < rows && c < P) ? x : 0.0f;
      vb[u] = (r < rows && c < Q) ? y : 0.0f;
    }
  };
  v4f acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
  int t = blockIdx.x;
  if (t < tiles) load(t);
  for (; t < tiles; t += per) {
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = threadIdx.x + 256 * u;
      As[(e >> 6) * kTallLS + (e & 63)] = va[u];
      Bs[(e >> 6) * kTallLS + (e & 63)] = vb[u];
    }
    __syncthreads();
    if (t + per < tiles) load(t + per);
#pragma unroll
    for (int kb = 0; kb < kMixRows / 4; ++kb) {
      const int r = 4 * kb + lg;
      const float a = As[r * kTallLS + 16 * wave + li];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Bs[r * kTallLS + 16 * c + li], acc[c], 0, 0, 0);
    }
    __syncthreads();  // every wave's reads of this tile are done before the next is stored
  }
  float* out = part + ((size_t)s * per + blockIdx.x) * 64 * 64;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) out[(16 * wave + 4 * lg + rr) * 64 + 16 * c + li] = acc[c][rr];
}



template <typename TB>
__global__ void __launch_bounds__(64 * kTallWaves)
tall_t_bf16_kernel(const float* __restrict__ A, const TB* __restrict__ B, float* __restrict__ part, int N, int P,
                   int Q) {
  __shared__ __align__(16) float Ws[tall_lds_floats()];
  tall_t_bf16_body<TB>(A, B, part, N, P, Q, Ws, blockIdx.y, blockIdx.x, gridDim.x);
}

__global__ void __launch_bounds__(256)
tall_t_reduce_kernel(const float* __restrict__ part, float* __restrict__ C, int per, int P, int Q) {
  const int s = blockIdx.y, e = blockIdx.x * 256 + threadIdx.x;
  if (e >= P * Q) return;
  const int p = e / Q, q = e - p * Q;
  const float* src = part + (size_t)s * per * 64 * 64 + p * 64 + q;
  float sum = 0.0f;
  int i = 0;
  for (; i + 4 <= per; i += 4) {  // four loads in flight, summed in order
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = src[(size_t)(i + k) * 64 * 64];
#pragma unroll
    for (int k = 0; k < 4; ++k) sum += v[k];
  }
  for (; i < per; ++i) sum += src[(size_t)i * 64 * 64];
  C[(size_t)s * P * Q + e] = sum;
}

__global__ void __launch_bounds__(256) tall_t_zero_kernel(float* __restrict__ C, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    C[i] = 0.0f;
}

// Workgroups per slice: about one per CU over the grid for the bf16 kernel
// (kTallWaves waves each), two for the fp32 kernel (4 waves each).
int tall_t_per(int64_t slices, int64_t N) {
  const int64_t tiles = (N + kMixRows - 1) / kMixRows;
  return (int)std::max<int64_t>(1, std::min<int64_t>(tiles, (2 * (int64_t)num_cus() + slices - 1) / slices));
}
int tall_t_bf16_per(int64_t slices, int64_t N) {
  const int64_t blocks = (N + kTallKB - 1) / kTallKB;
  return (int)std::max<int64_t>(
      1, std::min<int64_t>((blocks + kTallWaves - 1) / kTallWaves, ((int64_t)num_cus() + slices - 1) / slices));
}

template <typename TB>
int launch_tall_t(const float* A, const void* B, float* C, float* ws, int64_t slices, int64_t N, int P, int Q,
                  hipStream_t st) {
  const bool rowsAligned = (reinterpret_cast<uintptr_t>(A) & 15) == 0 && (reinterpret_cast<uintptr_t>(B) & 15) == 0 &&
                           (N * P * 4) % 16 == 0 && (N * Q * (int64_t)sizeof(TB)) % 16 == 0;
  const int per = rowsAligned ? tall_t_bf16_per(slices, N) : tall_t_per(slices, N);
  if (rowsAligned)
    hipLaunchKernelGGL(tall_t_bf16_kernel<TB>, dim3((unsigned)per, (unsigned)slices), dim3(64 * kTallWaves), 0, st,
                       A, static_cast<const TB*>(B), ws, (int)N, P, Q);
  else
    hipLaunchKernelGGL(tall_t_kernel<TB>, dim3((unsigned)per, (unsigned)slices), dim3(256), 0, st, A,
                       static_cast<const TB*>(B), ws, (int)N, P, Q);
  int s = check_launch("tall product");
  if (s) return s;
  hipLaunchKernelGGL(tall_t_reduce_kernel, dim3((unsigned)((P * Q + 255) / 256), (unsigned)slices), dim3(256), 0,
                     st, ws, C, per, P, Q);
  return check_launch("tall product reduction");
}

// The three row products of MixTrio in one launch of the bf16 kernel (about one
// workgroup per CU per product). LFAMD_ERR_UNSUPPORTED where the bf16 kernel
// does not take an operand (the caller then makes one call per product).
int mix_rows_trio(int dtype, const void* const* A, const float* const* B, void* const* C, int64_t slices, int64_t N,
                  const int* P, const int* Q, const int64_t* sq, const int64_t* sp, const int64_t* bStride,
                  hipStream_t st, int first) {
  const int64_t es = dtype == LFAMD_F32 ? 4 : 2;
  bool direct = P[0] == kMixPMax, rows16 = (N * P[0] * es) % 16 == 0;
  for (int i = first; i < 2; ++i)
    if ((reinterpret_cast<uintptr_t>(A[i]) & 15) != 0) direct = rows16 = false;
  const bool two16 = (reinterpret_cast<uintptr_t>(A[2]) & 15) == 0 && (N * P[1] * 4) % 16 == 0;
  if (!(direct || rows16) || !two16 || slices < 1 || N < 1 || 3 * slices > 65535 || first < 0 || first > 2)
    return fail(LFAMD_ERR_UNSUPPORTED, "row product trio: operands the bf16 kernel does not take");
  for (int i = 0; i < 2; ++i)
    if (P[i] > kMixPMax || Q[i] > kMixPMax || P[i] < 1 || Q[i] < 1)
      return fail(LFAMD_ERR_UNSUPPORTED, "row product trio: widths above %d", kMixPMax);
  const MixTrio t{{A[0], A[1], A[2]}, {B[0], B[1], B[2]}, {C[0], C[1], C[2]}, {P[0], P[1]}, {Q[0], Q[1]},
                  {sq[0], sq[1]}, {sp[0], sp[1]}, {bStride[0], bStride[1]}};
  const int64_t groups = (N + kMixGroup - 1) / kMixGroup;
  const int64_t nsrc = 3 - first;
  const int64_t per = std::max<int64_t>(1, std::min<int64_t>((groups + kMixWaves - 1) / kMixWaves,
                                                             ((int64_t)num_cus() + nsrc * slices - 1) / (nsrc * slices)));
  const dim3 grid((unsigned)per, (unsigned)(nsrc * slices)), block(64 * kMixWaves);
#define LFAMD_TRIO(TA)                                                                                             \
  do {                                                                                                             \
    if (direct)                                                                                                    \
      hipLaunchKernelGGL((mix_rows_bf16_trio_kernel<TA, true>), grid, block, 0, st, t, (int)slices, (int)N, first); \
    else                                                                                                           \
      hipLaunchKernelGGL((mix_rows_bf16_trio_kernel<TA, false>), grid, block, 0, st, t, (int)slices, (int)N, first); \
  } while (0)
  switch (dtype) {
    case LFAMD_F32: LFAMD_TRIO(float); break;
    case LFAMD_F16: LFAMD_TRIO(f16s); break;
    case LFAMD_BF16: LFAMD_TRIO(bf16s); break;
    default: return fail(LFAMD_ERR_DTYPE, "row product trio: unsupported dtype %d", dtype);
  }
#undef LFAMD_TRIO
  return check_launch("row product trio");
}

// The bf16 tall product's per-workgroup partials only ([slices][per][64][64]
// fp32, entry [p][q]; the caller sums them): b_dtype F32 / F16 / BF16, inner and
// cols <= 64, 16-byte aligned slices (else LFAMD_ERR_UNSUPPORTED).
int tall_t_check(int b_dtype, const float* A, const void* B, size_t wsBytes, int64_t slices, int64_t N, int P, int Q,
                 int* perOut) {
  if (b_dtype != LFAMD_F32 && b_dtype != LFAMD_F16 && b_dtype != LFAMD_BF16)
    return fail(LFAMD_ERR_DTYPE, "tall product partials: unsupported dtype %d", b_dtype);
  const size_t elems = b_dtype == LFAMD_F32 ? 4 : 2;
  const bool rowsAligned = (reinterpret_cast<uintptr_t>(A) & 15) == 0 && (reinterpret_cast<uintptr_t>(B) & 15) == 0 &&
                           (N * P * 4) % 16 == 0 && (N * Q * (int64_t)elems) % 16 == 0;
  if (!rowsAligned || P > kMixPMax || Q > kMixPMax || N < 1 || slices < 1)
    return fail(LFAMD_ERR_UNSUPPORTED, "tall product partials: unaligned or unsupported sizes");
  const int per = tall_t_bf16_per(slices, N);
  if (wsBytes < (size_t)slices * per * 64 * 64 * sizeof(float))
    return fail(LFAMD_ERR_ARG, "tall product partials: workspace too small");
  *perOut = per;
  return LFAMD_OK;
}

int tall_t_partials(int b_dtype, const float* A, const void* B, float* ws, size_t wsBytes, int64_t slices,
                    int64_t N, int P, int Q, hipStream_t st, int* perOut) {
  if (int s = tall_t_check(b_dtype, A, B, wsBytes, slices, N, P, Q, perOut)) return s;
  const int per = *perOut;
  const dim3 grid((unsigned)per, (unsigned)slices), block(64 * kTallWaves);
  switch (b_dtype) {
    case LFAMD_F32:
      hipLaunchKernelGGL(tall_t_bf16_kernel<float>, grid, block, 0, st, A, static_cast<const float*>(B), ws, (int)N, P, Q);
      break;
    case LFAMD_F16:
      hipLaunchKernelGGL(tall_t_bf16_kernel<f16s>, grid, block, 0, st, A, static_cast<const f16s*>(B), ws, (int)N, P, Q);
      break;
    case LFAMD_BF16:
      hipLaunchKernelGGL(tall_t_bf16_kernel<bf16s>, grid, block, 0, st, A, static_cast<const bf16s*>(B), ws, (int)N, P, Q);
      break;
    default: return fail(LFAMD_ERR_DTYPE, "tall product partials: unsupported dtype %d", b_dtype);
  }
  return check_launch("tall product partials");
}

}  // namespace lfamd

using namespace lfamd;

extern "C" size_t lfamd_tall_t_workspace_size(int64_t slices, int64_t rows) {
  if (slices <= 0 || rows <= 0) return 0;
  return (size_t)slices * std::max(tall_t_per(slices, rows), tall_t_bf16_per(slices, rows)) * 64 * 64 * sizeof(float);
}

extern "C" int lfamd_tall_t(int b_dtype, const float* a, const void* b, float* c, int64_t slices, int64_t rows,
                            int inner, int cols, void* workspace, size_t workspace_bytes, void* stream) {
  if (b_dtype != LFAMD_F32 && b_dtype != LFAMD_F16 && b_dtype != LFAMD_BF16)
    return fail(LFAMD_ERR_DTYPE, "tall product: unsupported dtype %d", b_dtype);
  if (slices < 0 || rows < 0 || inner < 1 || cols < 1 || slices > 65535 || rows > (int64_t)1 << 30)
    return fail(LFAMD_ERR_ARG, "tall product: bad sizes (slices=%lld rows=%lld inner=%d cols=%d)",
                (long long)slices, (long long)rows, inner, cols);
  if (inner > kMixPMax || cols > kMixPMax)
    return fail(LFAMD_ERR_UNSUPPORTED, "tall product: inner=%d, cols=%d exceed %d", inner, cols, kMixPMax);
  if (slices == 0) return ok();
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0) {  // an empty sum (no memset: the call may be captured in a graph)
    if (!c) return fail(LFAMD_ERR_ARG, "tall product: null pointer");
    const int64_t n = slices * inner * cols;
    hipLaunchKernelGGL(tall_t_zero_kernel, dim3((unsigned)std::min<int64_t>(1024, (n + 255) / 256)), dim3(256), 0, st,
                       c, n);
    return check_launch("tall product (empty)");
  }
  if (!a || !b || !c) return fail(LFAMD_ERR_ARG, "tall product: null pointer");
  const size_t need = lfamd_tall_t_workspace_size(slices, rows);
  if (!workspace || workspace_bytes < need)
    return fail(LFAMD_ERR_ARG, "tall product: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  float* ws = static_cast<float*>(workspace);
  switch (b_dtype) {
    case LFAMD_F32: return launch_tall_t<float>(a, b, c, ws, slices, rows, inner, cols, st);
    case LFAMD_F16: return launch_tall_t<f16s>(a, b, c, ws, slices, rows, inner, cols, st);
    default: return launch_tall_t<bf16s>(a, b, c, ws, slices, rows, inner, cols, st);
  }
}

template <typename TA>
int launch_mix_c(int c_dtype, const void* a, const float* b, void* c, int64_t slices, int64_t rows, int inner,
                 int cols, int64_t sq, int64_t sp, int64_t bStride, hipStream_t st) {
  switch (c_dtype) {
    case LFAMD_F32: return launch_mix<TA, float>(a, b, c, slices, rows, inner, cols, sq, sp, bStride, st);
    case LFAMD_F16: return launch_mix<TA, f16s>(a, b, c, slices, rows, inner, cols, sq, sp, bStride, st);
    default: return launch_mix<TA, bf16s>(a, b, c, slices, rows, inner, cols, sq, sp, bStride, st);
  }
}

extern "C" int lfamd_mix_rows(int dtype, const void* a, const float* b, int c_dtype, void* c, int64_t slices,
                              int64_t rows, int inner, int cols, int64_t b_col_stride, int64_t b_inner_stride,
                              int64_t b_slice_stride, void* stream) {
  if (dtype != LFAMD_F32 && dtype != LFAMD_F16 && dtype != LFAMD_BF16)
    return fail(LFAMD_ERR_DTYPE, "mix rows: unsupported dtype %d", dtype);
  if (c_dtype != LFAMD_F32 && c_dtype != LFAMD_F16 && c_dtype != LFAMD_BF16)
    return fail(LFAMD_ERR_DTYPE, "mix rows: unsupported output dtype %d", c_dtype);
  if (slices < 0 || rows < 0 || inner < 1 || cols < 1 || slices > 65535 || rows > (int64_t)1 << 30)
    return fail(LFAMD_ERR_ARG, "mix rows: bad sizes (slices=%lld rows=%lld inner=%d cols=%d)", (long long)slices,
                (long long)rows, inner, cols);
  if (inner > kMixPMax || cols > kMixPMax)
    return fail(LFAMD_ERR_UNSUPPORTED, "mix rows: inner=%d, cols=%d exceed %d", inner, cols, kMixPMax);
  if (slices == 0 || rows == 0) return ok();
  if (!a || !b || !c) return fail(LFAMD_ERR_ARG, "mix rows: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LFAMD_F32: return launch_mix_c<float>(c_dtype, a, b, c, slices, rows, inner, cols, b_col_stride, b_inner_stride, b_slice_stride, st);
    case LFAMD_F16: return launch_mix_c<f16s>(c_dtype, a, b, c, slices, rows, inner, cols, b_col_stride, b_inner_stride, b_slice_stride, st);
    default: return launch_mix_c<bf16s>(c_dtype, a, b, c, slices, rows, inner, cols, b_col_stride, b_inner_stride, b_slice_stride, st);
  }
}

// Column-split backward of LaplaceSubtraction for 16-bit element types on gfx950.
//
// Reference semantics (src/LaplaceSubtraction_cuda_kernel.cu):
//   dq[i,c] = sum_j g[i,j] * sgn(q[i,c] - k[c,j])          (:183-266)
//   dk[c,j] = -sum_i g[i,j] * sgn(q[i,c] - k[c,j])         (:309-392)
//   sgn(0) = 0 (:34-38), fp32 accumulation (:17-19).
//
// Per triple this kernel issues three full-rate VALU instructions:
//   y  = clamp(T(q) + (0.5 - T(k)))    one v_add_f32 with the clamp modifier
//   dq += 2g * y,   dk += 2g * y        two v_fmac_f32
// where T maps a 16-bit float pattern onto 2^22 + 2^14 + t/2 with t the signed
// magnitude of the pattern (+0 and -0 both give t = 0). T is strictly increasing
// in the value for every non-NaN fp16 / bf16 (infinities included), the sums are
// exact in fp32, so y is exactly 0 (q < k), 1/2 (q == k) or 1 (q > k), i.e.
// (sgn(q - k) + 1) / 2, and sgn = 2y - 1:
//   dq[i,c] = sum_j 2g y - sum_j g        dk[c,j] = sum_i g - sum_i 2g y.
// (A NaN pattern orders beyond the infinities, so its sign is +-1 where the
// reference's sign of a NaN difference is 0.)
//
// Mapping. A workgroup is 8 waves (2 per SIMD: the register file holds two of
// these waves, and the SIMD issues two VALU instructions per 4 cycles only from
// an even number of waves). One channel block of 64 channels per workgroup;
// lane (h, p), h = lane / 32, p = lane % 32, owns channels 2p and 2p + 1 and the
// key columns [h * JC, h * JC + JC), JC = ceil(M / 2). Its key terms and grad_key
// sums stay in registers; the grad rows are staged in LDS (2g as fp32, the two
// halves of a row 16-byte aligned, the row sum in slot JC of each half) and read
// back as 16-byte wave-wide reads with two addresses, each feeding 24 VALU
// instructions (two channels x four columns x three). The row loop itself is the
// generated asm block of l1_asm_gen.h (register map chosen to avoid VGPR bank
// clashes, grad rows of the next batch loaded during the current one).
//
// grad_key: each wave's partial (column sums of g minus the accumulated 2g y) is
// summed over the workgroup's waves in LDS in a fixed order and written per
// workgroup channel-major; laplace_dk_reduce_t_kernel sums the workgroups of a
// slice in workgroup order. Results are deterministic.
#include <algorithm>

#include "lf_common.h"
#include "lf_internal.h"
#include "l1_asm_gen.h"

namespace lfamd {

namespace {

constexpr int kB2Waves = 8;   // waves per workgroup (2 per SIMD)
constexpr int kB2RB = 8;      // grad rows per staged batch (the asm block's RB)
constexpr int kB2Bufs = 4;    // LDS accumulators of the workgroup grad_key reduction

template <typename T> struct B2Traits;
template <> struct B2Traits<f16s> { static constexpr bool bf16 = false; };
template <> struct B2Traits<bf16s> { static constexpr bool bf16 = true; };

// Layout constants shared by the kernel and the host plan.
struct B2Shape {
  int M, JC, EPL, XV, HP, PITCH, NKK;
  __host__ __device__ constexpr B2Shape(int m)
      : M(m), JC((m + 1) / 2), EPL((m + 7) / 8), XV(m / ((m + 7) / 8)), HP((((m + 1) / 2) + 1 + 3) / 4 * 4),
        PITCH(2 * ((((m + 1) / 2) + 1 + 3) / 4 * 4)), NKK((2 * ((m + 1) / 2) + 3) / 4) {}
  // Per-wave staging slot: RB rows plus one row the read-ahead may touch, plus a
  // 64-byte scratch area for the writes of lanes without a real destination.
  __host__ __device__ constexpr int slot_bytes() const { return ((kB2RB + 1) * PITCH) * 4 + 64; }
  __host__ __device__ constexpr int kk_bytes() const { return NKK * 64 * 16; }
  __host__ __device__ constexpr int red_bytes() const { return kB2Bufs * M * 65 * 4; }
  __host__ __device__ constexpr int lds_bytes() const {
    return kk_bytes() + kB2Waves * slot_bytes() > red_bytes() ? kk_bytes() + kB2Waves * slot_bytes() : red_bytes();
  }
};

// T(pattern) = 2^22 + 2^14 + t / 2 (see the file comment), as the fp32 bit pattern 0x4a808000 + t.
__device__ __forceinline__ float tmap16(uint16_t bits) {
  const int t = (bits & 0x8000) ? -(int)(bits & 0x7fff) : (int)bits;
  return __builtin_bit_cast(float, (uint32_t)(0x4a808000 + t));
}

// Dispatch to the generated row loops (grad_query and grad_key together or alone).
template <typename T, int M, bool DQ, bool DK> struct B2Rows;
#define LFAMD_B2ROWS(TY, MM, DQ_, DK_, FN)                                                            \
  template <> struct B2Rows<TY, MM, DQ_, DK_> {                                                        \
    static constexpr B2Shape S{MM};                                                                    \
    __device__ static void run(float (&dk)[2 * S.JC], float (&cs)[S.EPL], const void* g, const void* q,    \
                               void* dq, unsigned qs, int nfull, int tail, const void* gt, const void* qt, \
                               unsigned rda, unsigned vq, unsigned goff, unsigned gofft, unsigned rs,       \
                               float vx, float vrt, unsigned kka, const unsigned (&st)[S.EPL],              \
                               unsigned wpar, const unsigned (&g0)[S.EPL], const unsigned (&q0)[kB2RB]) {   \
      FN;                                                                                              \
    }                                                                                                  \
  };
#define LFAMD_B2ARGS dk, cs, g, q, dq, qs, nfull, tail, gt, qt, rda, vq, goff, gofft, rs, vx, vrt, kka, st, wpar, g0, q0
#define LFAMD_B2ALL(TY, TN, MM)                                                \
  LFAMD_B2ROWS(TY, MM, true, true, bwd2_rows_##TN##_m##MM##_qk(LFAMD_B2ARGS))   \
  LFAMD_B2ROWS(TY, MM, true, false, bwd2_rows_##TN##_m##MM##_q(LFAMD_B2ARGS))   \
  LFAMD_B2ROWS(TY, MM, false, true, bwd2_rows_##TN##_m##MM##_k(LFAMD_B2ARGS))
LFAMD_B2ALL(f16s, f16, 49)
LFAMD_B2ALL(bf16s, bf16, 49)
LFAMD_B2ALL(f16s, f16, 32)
LFAMD_B2ALL(bf16s, bf16, 32)
LFAMD_B2ALL(f16s, f16, 16)
LFAMD_B2ALL(bf16s, bf16, 16)
#undef LFAMD_B2ALL
#undef LFAMD_B2ARGS
#undef LFAMD_B2ROWS

// Grid: (nx workgroups per slice, channel blocks, B*H). The slice's N rows are
// split evenly over its nx * 8 waves.
template <typename T, int M, bool DQ, bool DK>
__global__ void __launch_bounds__(64 * kB2Waves, 1)
laplace_bwd2_kernel(const T* __restrict__ gout, const T* __restrict__ query, const T* __restrict__ key,
                    T* __restrict__ dq, float* __restrict__ partial, int N, int C) {
  constexpr B2Shape S{M};
  constexpr int JC = S.JC, EPL = S.EPL, XV = S.XV, HP = S.HP, PITCH = S.PITCH;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int x = blockIdx.x, nx = gridDim.x, cb = blockIdx.y, bh = blockIdx.z;
  const int ncb = gridDim.y;

  extern __shared__ __align__(16) unsigned char smem[];
  const unsigned ldsBase = (unsigned)(uintptr_t)smem;
  float* kkt = reinterpret_cast<float*>(smem);                                   // [NKK][64][4]
  unsigned char* slot = smem + S.kk_bytes() + wave * S.slot_bytes();             // this wave's staging slot
  const unsigned slotA = ldsBase + S.kk_bytes() + wave * S.slot_bytes();
  const unsigned scratchA = slotA + (kB2RB + 1) * PITCH * 4;

  // This wave's rows.
  const int gw = x * kB2Waves + wave, nw = nx * kB2Waves;
  const int r0 = uniform((int)((int64_t)gw * N / nw)), r1 = uniform((int)((int64_t)(gw + 1) * N / nw));
  const int rows = r1 - r0;
  // The first batch's raw grad elements and query patterns are loaded before the
  // key table is built, so that their memory latency overlaps it.
  const int nfull0 = rows / kB2RB, tail0 = rows - nfull0 * kB2RB;
  const int rl = lane >> 3, xsl = lane & 7;
  unsigned g0[EPL], q0[kB2RB];
  {
    const uint16_t* gsrc = reinterpret_cast<const uint16_t*>(gout) + ((size_t)bh * N + r0) * M;
    const uint16_t* qsrc = reinterpret_cast<const uint16_t*>(query) + ((size_t)bh * N + r0) * C + cb * 64 +
                           2 * (lane & 31) + (lane >> 5);
    const int nr = nfull0 > 0 ? kB2RB : tail0;
    const int rr0 = nfull0 > 0 ? rl : min(rl, max(nr - 1, 0));
    const int eoff = rr0 * M + (xsl < XV ? xsl * EPL : 0);
#pragma unroll
    for (int e = 0; e < EPL; ++e) g0[e] = rows > 0 ? gsrc[eoff + e] : 0u;
#pragma unroll
    for (int rr = 0; rr < kB2RB; ++rr) q0[rr] = rr < nr ? qsrc[(size_t)rr * C] : 0u;
  }

  // Key terms 0.5 - T(k[c][col]) for lane (h, p): [c][j] = channel 2p + c, column h*JC + j.
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(key) + (size_t)bh * C * M;
  for (int t = threadIdx.x; t < 64 * S.NKK * 4; t += blockDim.x) {
    const int l = (t >> 2) & 63, grp = t >> 8, e = grp * 4 + (t & 3);
    float v = 0.0f;
    if (e < 2 * JC) {
      const int c = e / JC, j = e - c * JC;
      const int col = (l >> 5) * JC + j;
      const int ch = cb * 64 + 2 * (l & 31) + c;
      if (col < M) v = 0.5f - tmap16(kb[(size_t)ch * M + col]);
    }
    kkt[t] = v;
  }
  // The staging slot starts zeroed (half 1's pad column of an odd M is never written).
  for (int t = lane; t * 4 < S.slot_bytes(); t += 64) reinterpret_cast<float*>(slot)[t] = 0.0f;
  __syncthreads();

  float dk[2 * JC], cs[EPL];
  if (rows > 0) {
    const int nfull = rows / kB2RB, tail = rows - nfull * kB2RB;
    const T* gw0 = gout + ((size_t)bh * N + r0) * M;
    const T* qw0 = query + ((size_t)bh * N + r0) * C + cb * 64;
    T* dqw0 = dq + ((size_t)bh * N + r0) * C + cb * 64;
    const T* gt = gw0 + (size_t)nfull * kB2RB * M;
    const T* qt = qw0 + (size_t)nfull * kB2RB * C;
    // Staging lane (r, xs): row r of the batch, elements [xs*EPL, xs*EPL + EPL).
    const int r = lane >> 3, xs = lane & 7;
    const bool xv = xs < XV;
    unsigned st[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int col = xs * EPL + e;
      const int h = col >= JC ? 1 : 0;
      st[e] = xv ? slotA + (unsigned)(r * PITCH + h * HP + (col - h * JC)) * 4 : scratchA + lane % 16 * 4;
    }
    const unsigned rs = xs < 4 ? slotA + (unsigned)(r * PITCH + (xs & 1) * HP + JC) * 4 : scratchA + lane % 16 * 4;
    const unsigned goff = (unsigned)(r * M + (xv ? xs * EPL : 0)) * 2;
    const int rt = tail > 0 ? min(r, tail - 1) : 0;
    const unsigned gofft = (unsigned)(rt * M + (xv ? xs * EPL : 0)) * 2;
    const unsigned rda = slotA + (unsigned)((lane >> 5) * HP) * 4;
    const unsigned vq = (unsigned)(2 * (lane & 31) + (lane >> 5)) * 2;
    const unsigned kka = ldsBase + (unsigned)lane * 16;
    B2Rows<T, M, DQ, DK>::run(dk, cs, gw0, qw0, dqw0, (unsigned)C * 2, nfull, tail, gt, qt, rda, vq, goff, gofft, rs,
                      xv ? 1.0f : 0.0f, r < tail ? 1.0f : 0.0f, kka, st, (unsigned)uniform(wave >= 4 ? 1 : 0), g0, q0);
  } else {
#pragma unroll
    for (int j = 0; j < 2 * JC; ++j) dk[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) cs[e] = 0.0f;
  }

  if constexpr (!DK) return;
  // Column sums of 2g over this wave's rows: column col = xs*EPL + e collects the
  // staging lanes (r, xs) of the 8 batch rows r, summed in r order.
  float* csw = reinterpret_cast<float*>(slot);            // [64][EPL]
  float* colsum = csw + 64 * EPL;                          // [M] sum_i g (half of the 2g sum)
  wave_sync();
#pragma unroll
  for (int e = 0; e < EPL; ++e) csw[lane * EPL + e] = cs[e];
  wave_sync();
  if (lane < M) {
    const int xs = lane / EPL, e = lane - xs * EPL;
    float s = 0.0f;
#pragma unroll
    for (int rr = 0; rr < kB2RB; ++rr) s += csw[(rr * 8 + xs) * EPL + e];
    colsum[lane] = 0.5f * s;
  }
  wave_sync();
  // Partial grad_key of this wave: column sum minus the accumulated 2g y.
  const int h = lane >> 5, p = lane & 31;
#pragma unroll
  for (int j = 0; j < JC; ++j) {
    const int col = h * JC + j;
    const float cv = colsum[col < M ? col : 0];
    dk[j] = cv - dk[j];
    dk[JC + j] = cv - dk[JC + j];
  }

  // Workgroup sum over the waves in a fixed order: wave w adds into accumulator
  // w % kB2Bufs in rounds of increasing w / kB2Bufs; accumulators are [M][65]
  // (channel fastest, padded), summed 0..3 and written channel-major.
  float* red = reinterpret_cast<float*>(smem);
  float* buf = red + (wave % kB2Bufs) * M * 65;
  __syncthreads();
  for (int round = 0; round * kB2Bufs < kB2Waves; ++round) {
    if (wave / kB2Bufs == round) {
#pragma unroll
      for (int j = 0; j < JC; ++j) {
        const int col = h * JC + j;
        if (col < M) {
          float* a = buf + col * 65 + 2 * p;
          if (round == 0) {
            a[0] = dk[j];
            a[1] = dk[JC + j];
          } else {
            a[0] += dk[j];
            a[1] += dk[JC + j];
          }
        }
      }
    }
    __syncthreads();
  }
  float* out = partial + (((size_t)bh * ncb + cb) * nx + x) * 64 * M;   // [64][M] channel-major
  for (int t = threadIdx.x; t < 64 * M; t += blockDim.x) {
    const int c = t / M, col = t - c * M;
    float s = red[col * 65 + c];
#pragma unroll
    for (int b = 1; b < kB2Bufs; ++b) s += red[b * M * 65 + col * 65 + c];
    out[t] = s;
  }
}

// grad_key[c][j] = sum over the slice's nx workgroup partials (workgroup order),
// rounded once. Partials and grad_key are both channel-major [C][M], so reads
// and writes are contiguous.
template <typename T>
__global__ void __launch_bounds__(256)
laplace_dk_reduce_t_kernel(const float* __restrict__ partial, T* __restrict__ dk, int nx, int M, int C) {
  const int ncb = gridDim.y, cb = blockIdx.y, bh = blockIdx.z;
  const int n = 64 * M;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const int c = t / M, col = t - c * M;
  if (cb * 64 + c >= C) return;
  const float* p = partial + ((size_t)bh * ncb + cb) * nx * n + t;
  float s = 0.0f;
  for (int i = 0; i < nx; ++i) s += p[(size_t)i * n];
  dk[((size_t)bh * C + cb * 64 + c) * M + col] = from_acc<T>(s);
}

struct B2Plan {
  int nx, ncb;
  size_t lds, partialElems;
};

B2Plan plan_b2(int64_t BH, int64_t N, int64_t M, int64_t C) {
  B2Plan p{};
  p.ncb = (int)(C / 64);
  const int64_t slices = BH * p.ncb;
  p.nx = (int)std::max<int64_t>(1, std::min<int64_t>(num_cus() / std::max<int64_t>(slices, 1),
                                                      (N + kB2Waves - 1) / kB2Waves));
  p.lds = (size_t)B2Shape((int)M).lds_bytes();
  p.partialElems = (size_t)slices * p.nx * 64 * (size_t)M;
  return p;
}

template <typename T, int M, bool DQ, bool DK>
int launch_b2_m(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, int64_t BH, int64_t N,
                int64_t C, const B2Plan& p, hipStream_t st) {
  dim3 grid(p.nx, p.ncb, (unsigned)BH);
  hipLaunchKernelGGL((laplace_bwd2_kernel<T, M, DQ, DK>), grid, dim3(64 * kB2Waves), p.lds, st, static_cast<const T*>(g),
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<T*>(dq),
                     static_cast<float*>(ws), (int)N, (int)C);
  int s = check_launch("laplace backward (column-split)");
  if (s || !DK) return s;
  dim3 rgrid((64 * M + 255) / 256, p.ncb, (unsigned)BH);
  hipLaunchKernelGGL(laplace_dk_reduce_t_kernel<T>, rgrid, dim3(256), 0, st, static_cast<const float*>(ws),
                     static_cast<T*>(dk), p.nx, M, (int)C);
  return check_launch("laplace backward_key reduction");
}

template <typename T, bool DQ, bool DK>
int launch_b2_t(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, int64_t BH, int64_t N,
                int64_t M, int64_t C, const B2Plan& p, hipStream_t st) {
  switch (M) {
    case 16: return launch_b2_m<T, 16, DQ, DK>(g, q, k, dq, dk, ws, BH, N, C, p, st);
    case 32: return launch_b2_m<T, 32, DQ, DK>(g, q, k, dq, dk, ws, BH, N, C, p, st);
    default: return launch_b2_m<T, 49, DQ, DK>(g, q, k, dq, dk, ws, BH, N, C, p, st);
  }
}

template <bool DQ, bool DK>
int launch_b2(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, int64_t BH,
              int64_t N, int64_t M, int64_t C, const B2Plan& p, hipStream_t st) {
  if (dtype == LFAMD_BF16) return launch_b2_t<bf16s, DQ, DK>(g, q, k, dq, dk, ws, BH, N, M, C, p, st);
  return launch_b2_t<f16s, DQ, DK>(g, q, k, dq, dk, ws, BH, N, M, C, p, st);
}

}  // namespace

// grad_query and / or grad_key on the column-split kernel (null dq or dk: that
// half is skipped): fp16 / bf16, M in {16, 32, 49}, C a multiple of 64 (one
// channel block per 64 channels), N >= 1.
bool b2_ok(int dtype, int64_t BH, int64_t N, int64_t M, int64_t C) {
  if (!(dtype == LFAMD_F16 || dtype == LFAMD_BF16)) return false;
  if (!(M == 16 || M == 32 || M == 49)) return false;
  if (C <= 0 || C % 64 != 0 || N <= 0 || BH <= 0) return false;
  return C / 64 <= 65535 && N <= INT32_MAX / 2;
}

size_t b2_workspace_elems(int64_t BH, int64_t N, int64_t M, int64_t C) {
  return plan_b2(BH, N, M, C).partialElems;
}

int b2_launch(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, size_t wsBytes,
              int64_t BH, int64_t N, int64_t M, int64_t C, hipStream_t st, const char* who) {
  const B2Plan p = plan_b2(BH, N, M, C);
  if (dk && (!ws || wsBytes < p.partialElems * 4))
    return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, p.partialElems * 4, wsBytes);
  if (dq && dk) return launch_b2<true, true>(dtype, g, q, k, dq, dk, ws, BH, N, M, C, p, st);
  if (dq) return launch_b2<true, false>(dtype, g, q, k, dq, dk, ws, BH, N, M, C, p, st);
  return launch_b2<false, true>(dtype, g, q, k, dq, dk, ws, BH, N, M, C, p, st);
}

}  // namespace lfamd

// Device helpers of the fp32-exact products on the bf16 matrix cores, and the
// tall transposed product's workgroup body, shared by the row / tall product
// kernels and the attention layer's fused landmark kernels.
#pragma once

#include "lf_common.h"

namespace lfamd {

typedef float v4f __attribute__((ext_vector_type(4)));  // one 16 x 16 MFMA accumulator per lane

constexpr int kMixPMax = 64;   // largest inner / output width
constexpr int kMixRows = 64;   // rows of A per tile of the tall transposed product
constexpr int kMixLS = 68;     // LDS pitch (floats): lane-varying 16-byte reads without conflicts
constexpr int kMixGroup = 16;  // rows of A per wave and step

// Orders one wave's LDS stores before its lanes read each other's values (a wave's
// LDS operations run in issue order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Values of one 16-byte vector of A as fp32.
template <typename T> __device__ __forceinline__ void unpack16(const uint4& v, float* f);
template <> __device__ __forceinline__ void unpack16<float>(const uint4& v, float* f) {
  f[0] = __builtin_bit_cast(float, v.x);
  f[1] = __builtin_bit_cast(float, v.y);
  f[2] = __builtin_bit_cast(float, v.z);
  f[3] = __builtin_bit_cast(float, v.w);
}
template <> __device__ __forceinline__ void unpack16<f16s>(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
}
template <> __device__ __forceinline__ void unpack16<bf16s>(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = __builtin_bit_cast(float, (e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// x = p1 + p2 + p3 exactly for fp32 x (bf16 truncations: p1 the top 8
// significant bits, p2 the next 8, p3 the last 8; an infinity is all in p1),
// for two values at once, returned as three packed bf16 pairs (x0 low half).
__device__ __forceinline__ void split3_pair(float x0, float x1, uint32_t& h1, uint32_t& h2, uint32_t& h3) {
  const uint32_t u0 = __builtin_bit_cast(uint32_t, x0), u1 = __builtin_bit_cast(uint32_t, x1);
  const float t0 = __builtin_bit_cast(float, u0 & 0xffff0000u), t1 = __builtin_bit_cast(float, u1 & 0xffff0000u);
  const float r0 = t0 == x0 ? 0.0f : x0 - t0;  // (an infinity gives 0, not inf - inf)
  const float r1 = t1 == x1 ? 0.0f : x1 - t1;
  const uint32_t v0 = __builtin_bit_cast(uint32_t, r0), v1 = __builtin_bit_cast(uint32_t, r1);
  const float q0 = r0 - __builtin_bit_cast(float, v0 & 0xffff0000u);
  const float q1 = r1 - __builtin_bit_cast(float, v1 & 0xffff0000u);
  h1 = __builtin_amdgcn_perm(u1, u0, 0x07060302u);
  h2 = __builtin_amdgcn_perm(v1, v0, 0x07060302u);
  h3 = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, q1), __builtin_bit_cast(uint32_t, q0), 0x07060302u);
}

// Pieces of A per element type: fp32 needs three, fp16 two (11 significant
// bits), bf16 one.
template <typename T> struct APieces { static constexpr int n = 3; };
template <> struct APieces<f16s> { static constexpr int n = 2; };
template <> struct APieces<bf16s> { static constexpr int n = 1; };

// x[0..7] = p1 + ... + pNP (bf16 pieces of split3_pair), each piece as 8 packed
// bf16 (one MFMA operand).
template <int NP>
__device__ __forceinline__ void split8(const float (&x)[8], uint4 (&out)[NP]) {
  uint32_t h[3][4];
#pragma unroll
  for (int e = 0; e < 4; ++e) split3_pair(x[2 * e], x[2 * e + 1], h[0][e], h[1][e], h[2][e]);
#pragma unroll
  for (int pc = 0; pc < NP; ++pc) out[pc] = make_uint4(h[pc][0], h[pc][1], h[pc][2], h[pc][3]);
}

// The tall transposed product on the bf16 matrix cores (A fp32 in three exact
// bf16 pieces, B in APieces<TB> pieces; the pieces' products of weight at least
// 2^-16 of the leading one, accumulated in fp32; what is left out is below
// 2^-22 |a| |b|). For 16-byte aligned slices (N * P * 4 and N * Q *
// sizeof(TB) multiples of 16). A workgroup is kTallWaves waves (one workgroup
// per CU); each works alone on 32-row blocks kb, kb + kTallWaves * per, ... of
// its slice (the next block's 16-byte loads in flight):
// the block's A rows, one contiguous run, go to the wave's LDS as they are
// (pitch P) and its B rows as fp32 with pitch 80 where Q is a multiple of the
// vector width (else pitch Q), and the wave accumulates the whole 64 x 64
// output over its blocks (16 tiles of v_mfma_f32_16x16x32_bf16, k = row: lane
// (i, h) = (lane % 16, lane / 16) holds rows h + 4 e, e < 8, of column i of a
// tile, so that the four lane groups read distinct banks for P = 49 and pitch
// 80). Rows past the end of a last partial block are zero in LDS; columns past
// P or Q only reach outputs that are never read. At the end the waves' sums
// are added in wave order and the workgroup's partial goes to the workspace,
// as for tall_t_kernel. (Config 5, 128 slices of 784 rows, per call: 11.2 us
// with 8 waves and two workgroups per slice, against 11.7 us with four 4-wave
// workgroups per slice.)
constexpr int kTallKB = 32;    // rows per block: one k-step of the bf16 MFMA
constexpr int kTallBP = 80;    // padded B pitch (floats)
constexpr int kTallWaves = 8;  // waves per workgroup (two per SIMD)

template <typename TB>
__device__ __forceinline__ void tall_t_bf16_body(const float* __restrict__ A, const TB* __restrict__ B,
                                                 float* __restrict__ part, int N, int P, int Q, float* Wsb, int s,
                                                 int bx, int per) {
  constexpr int EB = 16 / (int)sizeof(TB);   // B elements per 16-byte vector
  constexpr int NB = APieces<TB>::n;
  constexpr int CHA = kTallKB * kMixPMax;    // floats of one staged A block
  constexpr int CHB = kTallKB * kTallBP;     // floats of one staged B block
  constexpr int LVA = CHA / 4 / 64, LVB = CHA / EB / 64;
  // Wsb: per wave, A rows | B rows; then its 64 x 64 sums (kTallWaves * (CHA + CHB) floats).
  const int kblocks = (N + kTallKB - 1) / kTallKB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  if (wave < kTallWaves) {  // waves past kTallWaves (a larger block) only meet the barrier below
    const float* A0 = A + (size_t)s * N * P;
    const TB* B0 = B + (size_t)s * N * Q;
    float* WA = Wsb + wave * (CHA + CHB);
    float* WB = WA + CHA;
    const bool padB = Q % EB == 0;
    const int BPq = padB ? kTallBP : Q;
    const float invQ = 1.0f / (float)Q;

    uint4 xa[LVA], xb[LVB];
    auto load = [&](int kb) {
      const int r0 = kTallKB * kb, rows = min(kTallKB, N - r0);
      const uint4* sa = reinterpret_cast<const uint4*>(A0 + (size_t)r0 * P);
      const uint4* sb = reinterpret_cast<const uint4*>(B0 + (size_t)r0 * Q);
      const int na = (rows * P + 3) / 4, nb = (rows * Q + EB - 1) / EB;
#pragma unroll
      for (int v = 0; v < LVA; ++v) xa[v] = sa[min(lane + 64 * v, na - 1)];
#pragma unroll
      for (int v = 0; v < LVB; ++v) xb[v] = sb[min(lane + 64 * v, nb - 1)];
    };
    v4f acc[4][4];
#pragma unroll
    for (int tp = 0; tp < 4; ++tp)
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) acc[tp][tq] = v4f{0.f, 0.f, 0.f, 0.f};
    int kb = bx * kTallWaves + wave;
    const int kstep = per * kTallWaves;
    load(min(kb, kblocks - 1));
    for (; kb < kblocks; kb += kstep) {
      const int rows = min(kTallKB, N - kTallKB * kb);
      const int na = (rows * P + 3) / 4, nb = (rows * Q + EB - 1) / EB;
#pragma unroll
      for (int v = 0; v < LVA; ++v) {
        float f[4];
        unpack16<float>(xa[v], f);
        *reinterpret_cast<float4*>(WA + 4 * min(lane + 64 * v, na - 1)) = make_float4(f[0], f[1], f[2], f[3]);
      }
#pragma unroll
      for (int v = 0; v < LVB; ++v) {
        float f[EB];
        unpack16<TB>(xb[v], f);
        const int e0 = EB * min(lane + 64 * v, nb - 1);
        int pos = e0;
        if (padB) {  // the vector's EB elements lie in one row
          const int r = (int)(((float)e0 + 0.5f) * invQ);
          pos = r * kTallBP + (e0 - r * Q);
        }
        float4* dst = reinterpret_cast<float4*>(WB + pos);
#pragma unroll
        for (int e = 0; e < EB / 4; ++e) dst[e] = make_float4(f[4 * e], f[4 * e + 1], f[4 * e + 2], f[4 * e + 3]);
      }
      if (rows < kTallKB) {  // zero rows [rows, 32) of both blocks (wave-uniform)
        for (int i = rows * P + lane; i < CHA; i += 64) WA[i] = 0.0f;
        for (int i = rows * BPq + lane; i < CHB; i += 64) WB[i] = 0.0f;
      }
      wave_lds_sync();
      load(min(kb + kstep, kblocks - 1));  // the last block reloads itself (cached)
      uint4 bp[4][NB];
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = WB[(lg + 4 * e) * BPq + 16 * tq + li];
        split8<NB>(x, bp[tq]);
      }
#pragma unroll
      for (int tp = 0; tp < 4; ++tp) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = WA[(lg + 4 * e) * P + 16 * tp + li];
        uint4 ap[3];
        split8<3>(x, ap);
#pragma unroll
        for (int tq = 0; tq < 4; ++tq)
#pragma unroll
          for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j)
              if (i + j <= 2)
                acc[tp][tq] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ap[i]),
                                                                      __builtin_bit_cast(bf16x8, bp[tq][j]),
                                                                      acc[tp][tq], 0, 0, 0);
      }
      wave_lds_sync();
    }
    // The wave's sums into its own LDS area ([p][q], 64 x 64), then the areas
    // added in wave order.
#pragma unroll
    for (int tp = 0; tp < 4; ++tp)
#pragma unroll
      for (int tq = 0; tq < 4; ++tq)
#pragma unroll
        for (int r = 0; r < 4; ++r) WA[(16 * tp + 4 * lg + r) * 64 + 16 * tq + li] = acc[tp][tq][r];
  }
  __syncthreads();
  if (threadIdx.x < 64 * kTallWaves) {
    float* out = part + ((size_t)s * per + bx) * 64 * 64;
#pragma unroll
    for (int u = 0; u < 64 * 64 / (64 * kTallWaves); ++u) {
      const int e = threadIdx.x + 64 * kTallWaves * u;
      float sum = Wsb[e];
#pragma unroll
      for (int w = 1; w < kTallWaves; ++w) sum += Wsb[w * (CHA + CHB) + e];
      out[e] = sum;
    }
  }
}

// Floats of LDS tall_t_bf16_body needs.
constexpr int tall_lds_floats() { return kTallWaves * kTallKB * (kMixPMax + kTallBP); }

// The row product on the bf16 matrix cores, exact to fp32 rounding: A and B are
// split into bf16 pieces (A exactly; B = b1 + b2 + b3 exactly) and the products
// of the pieces whose weight is at least 2^-16 of the leading one
// (a1 b1, a1 b2, a2 b1, a1 b3, a2 b2, a3 b1) are accumulated in fp32 by
// v_mfma_f32_16x16x32_bf16; the terms left out are below 2^-22 |a| |b|.
// A workgroup is WAVES waves (kMixWaves by default); each works alone on 16-row groups g,
// g + W * per, ... of its slice (one group's loads ahead). Lane (i, h) = (lane % 16, lane / 16) holds the A
// operand of row i, k = 16 h + 8 kb + e (kb < 2, e < 8), i.e. elements
// [16 h, 16 h + 16) of the row:
//  * DIRECT (P = 64): loaded as 16-byte vectors straight from the row;
//  * otherwise (N * P * sizeof(TA) a multiple of 16): the group's rows * P
//    elements are one contiguous run of 16-byte vectors, written to the wave's
//    LDS rows as fp32 with pitch P and read back per lane.
// The workgroup splits B once into LDS in operand order (piece, column tile,
// kb, lane). Outputs go straight from the accumulators to C.
constexpr int kMixWaves = 12;  // one workgroup per CU, three waves per SIMD
template <typename TA, typename TC, bool DIRECT, int WAVES = kMixWaves>
__device__ __forceinline__ void mix_rows_bf16_body(const TA* __restrict__ A, const float* __restrict__ B,
                                                   TC* __restrict__ C, int N, int P, int Q, int64_t sq, int64_t sp,
                                                   int64_t bStride, int s, int xb, int per) {
  constexpr int EV = 16 / (int)sizeof(TA);  // elements per 16-byte vector
  constexpr int LV = 16 / EV;               // vectors per lane and group
  constexpr int NA = APieces<TA>::n;
  __shared__ __align__(16) uint4 Bp[3 * 4 * 2 * 64];                     // [piece][c][kb][lane]
  __shared__ __align__(16) float Ws[DIRECT ? 1 : WAVES][kMixGroup * kMixPMax];  // per wave: its rows (fp32)
  const int groups = (N + kMixGroup - 1) / kMixGroup;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const TA* A0 = A + (size_t)s * N * P;
  TC* C0 = C + (size_t)s * N * Q;

  uint4 xv[LV];
  auto load = [&](int g) {
    const int r0 = kMixGroup * g, rows = min(kMixGroup, N - r0);
    if constexpr (DIRECT) {
      const uint4* src = reinterpret_cast<const uint4*>(A0 + (size_t)(r0 + min(li, rows - 1)) * kMixPMax + 16 * lg);
#pragma unroll
      for (int v = 0; v < LV; ++v) xv[v] = src[v];
    } else {
      const uint4* src = reinterpret_cast<const uint4*>(A0 + (size_t)r0 * P);
      const int nv = (rows * P + EV - 1) / EV;
#pragma unroll
      for (int v = 0; v < LV; ++v) xv[v] = src[min(lane + 64 * v, nv - 1)];
    }
  };
  int g = xb * WAVES + wave;
  const int gstep = per * WAVES;
  load(min(g, groups - 1));  // in flight while B is split

  // B's pieces: thread t < 256 takes (c, kb, lane) = (t / 128, (t / 64) % 2,
  // t % 64) and t + 256: B[k][16 c + i] for k = 16 h + 8 kb + e, zero outside Q x P.
  if (threadIdx.x < 256) {  // (the first four waves)
    const float* Bm = B + (size_t)s * bStride;
    float bv[2][8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int cmb = threadIdx.x + 256 * t, ln = cmb & 63, kb = (cmb >> 6) & 1, c = cmb >> 7;
      const int q = 16 * c + (ln & 15), p0 = 16 * (ln >> 4) + 8 * kb;
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[t][e] = Bm[min(q, Q - 1) * sq + min(p0 + e, P - 1) * sp];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(bv[t][e]));
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int cmb = threadIdx.x + 256 * t, ln = cmb & 63, kb = (cmb >> 6) & 1, c = cmb >> 7;
      const int q = 16 * c + (ln & 15), p0 = 16 * (ln >> 4) + 8 * kb;
      uint32_t h[3][4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = (q < Q && p0 + 2 * e < P) ? bv[t][2 * e] : 0.0f;
        const float x1 = (q < Q && p0 + 2 * e + 1 < P) ? bv[t][2 * e + 1] : 0.0f;
        split3_pair(x0, x1, h[0][e], h[1][e], h[2][e]);
      }
#pragma unroll
      for (int pc = 0; pc < 3; ++pc) Bp[((pc * 4 + c) * 2 + kb) * 64 + ln] = make_uint4(h[pc][0], h[pc][1], h[pc][2], h[pc][3]);
    }
  }
  __syncthreads();  // the only workgroup barrier
  float* W = Ws[DIRECT ? 0 : wave];

  for (; g < groups; g += gstep) {
    const int r0 = kMixGroup * g, rows = min(kMixGroup, N - r0);
    float a[16];  // the lane's A operand, k = 16 lg + j
    if constexpr (DIRECT) {
#pragma unroll
      for (int v = 0; v < LV; ++v) unpack16<TA>(xv[v], &a[v * EV]);
    } else {
      const int nv = (rows * P + EV - 1) / EV;
#pragma unroll
      for (int v = 0; v < LV; ++v) {
        float f[EV];
        unpack16<TA>(xv[v], f);
        float4* dst = reinterpret_cast<float4*>(W + min(lane + 64 * v, nv - 1) * EV);
#pragma unroll
        for (int e = 0; e < EV / 4; ++e) dst[e] = make_float4(f[4 * e], f[4 * e + 1], f[4 * e + 2], f[4 * e + 3]);
      }
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < 16; ++j) a[j] = W[min(li * P + 16 * lg + j, kMixGroup * kMixPMax - 1)];
#pragma unroll
      for (int j = 0; j < 16; ++j) asm volatile("" : "+v"(a[j]));  // (keeps the reads unconditional)
#pragma unroll
      for (int j = 0; j < 16; ++j) a[j] = 16 * lg + j < P ? a[j] : 0.0f;  // k >= P: the next row's value
      wave_lds_sync();
    }
    load(min(g + gstep, groups - 1));  // the last group reloads itself (cached)
    asm volatile("" ::: "memory");  // B's pieces are read from LDS per group, not held in registers
    uint4 ap[3][2];  // [piece][kb]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      uint32_t h[3][4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split3_pair(a[8 * kb + 2 * e], a[8 * kb + 2 * e + 1], h[0][e], h[1][e], h[2][e]);
#pragma unroll
      for (int pc = 0; pc < 3; ++pc) ap[pc][kb] = make_uint4(h[pc][0], h[pc][1], h[pc][2], h[pc][3]);
    }
    v4f acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 b1 = __builtin_bit_cast(bf16x8, Bp[((0 * 4 + c) * 2 + kb) * 64 + lane]);
        const bf16x8 b2 = __builtin_bit_cast(bf16x8, Bp[((1 * 4 + c) * 2 + kb) * 64 + lane]);
        const bf16x8 b3 = __builtin_bit_cast(bf16x8, Bp[((2 * 4 + c) * 2 + kb) * 64 + lane]);
        const bf16x8 a1 = __builtin_bit_cast(bf16x8, ap[0][kb]);
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc[c], 0, 0, 0);
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2, acc[c], 0, 0, 0);
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b3, acc[c], 0, 0, 0);
        if constexpr (NA >= 2) {
          const bf16x8 a2 = __builtin_bit_cast(bf16x8, ap[1][kb]);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b1, acc[c], 0, 0, 0);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b2, acc[c], 0, 0, 0);
        }
        if constexpr (NA >= 3) {
          const bf16x8 a3 = __builtin_bit_cast(bf16x8, ap[2][kb]);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b1, acc[c], 0, 0, 0);
        }
      }
    }
    TC* Cg = C0 + (size_t)r0 * Q;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * lg + r, col = 16 * c + li;
        if (row < rows && col < Q) Cg[(size_t)row * Q + col] = from_acc<TC>(acc[c][r]);
      }
  }
}


}  // namespace lfamd

// NewtonInverse on gfx950: batched Newton-Schulz inverse with the matrices kept
// in LDS for all iterations, products on the fp32 matrix cores.
//
// Reference semantics (src/NewtonInverse_cuda_kernel.cu):
//   P = f32(mat) + 0.01 I                                       (:169, :320)
//   alpha = 1.8 / (max_i sum_j P_ij)^2, signed row sums          (:82-120)
//   V0 = alpha P; iters x V <- 2V - V(PV)   [n <= 112]            (:181-248)
//                          V <- 2V - (VP)V  [n = 128]             (:381-457)
//   grad_mat = -(V^T G) V^T                                     (:469-573)
// Matrices are zero-padded to NP = 16*ceil(n/16) (the reference's N_MAX
// buckets, :677-688); the padding stays exactly zero through the iteration.
//
// Mapping: one workgroup per matrix, WPR waves per 16-row strip; a wave owns
// the strip's rows and NP/16/WPR column tiles, one v_mfma_f32_16x16x4_f32
// accumulator (4 VGPRs) per 16x16 tile. MFMA 16x16x4 operand layout (wave64):
//   A[i][k]: lane = i + 16k     B[k][j]: lane = j + 16k
//   D[i][j]: lane = j + 16*(i/4), register i%4.
#include <algorithm>
#include <cstdint>
#include <initializer_list>
#include <type_traits>

#include "lf_common.h"
#include "lf_internal.h"
#include "mix_common.h"

namespace lfamd {

typedef float v4f __attribute__((ext_vector_type(4)));

// WPR waves per 16-row strip: wave w owns strip w / WPR and the column tiles
// [(w % WPR) * TW, (w % WPR + 1) * TW). WPR = 2 doubles the waves of a matrix
// (more latency hiding when there are few matrices per CU).
template <int NP, int WPR = 1> struct NsLayout {
  static constexpr int NT = NP / 16;       // tiles per dimension
  static constexpr int TW = NT / WPR;      // column tiles per wave
  static constexpr int NW = NT * WPR;      // waves per workgroup
  static constexpr int LS = NP + 4;        // LDS row stride (floats)
  static constexpr int ELEMS = NP * LS;
  static constexpr int THREADS = NW * 64;
  static_assert(NT % WPR == 0, "whole tiles per wave");
};

// acc[t] = X(rows of this wave) * Y(:, tile t), X and Y row-major in LDS.
// TRANS_X: X is read transposed (X[i][k] := Xs[k][i]); TRANS_Y likewise.
//
// The k index is walked in blocks of 16 with k = k0 + 4*lk + s for MFMA step s
// (lane group lk = lane/16 supplies the MFMA's inner index lk): every k of the
// block is used once, by the same inner index in A and B. With the row stride
// LS = NP + 4 this makes every operand read free of LDS bank conflicts: a
// row-major A operand and a transposed B operand are one 16-byte read per lane
// for four steps (lanes of one lk group on distinct 16-byte bank groups), a
// row-major B operand and a transposed A operand one 4-byte read per step on
// 64 distinct banks (the step-order k = k0 + lk puts 4 lanes on one bank).
//
// KL < 4: the inner dimension n has n - (NP - 16) = KL < 4 live k in the last
// block (n = 16 m + KL); there the MFMA steps s >= KL, whose four k are all
// zero padding, are left out (every skipped term is 0 * 0).
template <int NP, int WPR, bool TRANS_X, bool TRANS_Y, int KL = 4>
__device__ __forceinline__ void mfma_rowstrip(const float* __restrict__ Xs, const float* __restrict__ Ys,
                                              int wave, int lane, v4f (&acc)[NP / 16 / WPR]) {
  using L = NsLayout<NP, WPR>;
  const int strip = wave / WPR, t0 = (wave % WPR) * L::TW;
  static_assert(L::LS % 64 == 4 || L::LS % 64 == 20 || L::LS % 64 == 36 || L::LS % 64 == 52,
                "row stride 4 (mod 16) floats");
  const int li = lane & 15, lk = lane >> 4;
  const int i = 16 * strip + li;
#pragma unroll
  for (int t = 0; t < L::TW; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  constexpr int KEND = KL < 4 ? NP - 16 : NP;
  // The wide layouts (4 waves per strip, few matrices per CU) are latency-bound:
  // with at most 4 k blocks every operand read goes out before the first MFMA.
  // Elsewhere one block at a time keeps the register count (and occupancy) low.
  constexpr int kUnroll = WPR == 4 && L::NT <= 4 ? L::NT : 1;
#pragma unroll kUnroll
  for (int k0 = 0; k0 < KEND; k0 += 16) {  // (a trimmed last block follows the loop)
    const int kb = k0 + 4 * lk;  // this lane's 4 consecutive k
    float a[4];
    if constexpr (TRANS_X) {
#pragma unroll
      for (int s = 0; s < 4; ++s) a[s] = Xs[(kb + s) * L::LS + i];
    } else {
      const float4 v = *reinterpret_cast<const float4*>(&Xs[i * L::LS + kb]);
      a[0] = v.x; a[1] = v.y; a[2] = v.z; a[3] = v.w;
    }
    float b[L::TW][4];
#pragma unroll
    for (int t = 0; t < L::TW; ++t) {
      const int j = 16 * (t0 + t) + li;
      if constexpr (TRANS_Y) {
        const float4 v = *reinterpret_cast<const float4*>(&Ys[j * L::LS + kb]);
        b[t][0] = v.x; b[t][1] = v.y; b[t][2] = v.z; b[t][3] = v.w;
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) b[t][s] = Ys[(kb + s) * L::LS + j];
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < L::TW; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[t][s], acc[t], 0, 0, 0);
  }
  if constexpr (KL < 4) {
    const int kb = KEND + 4 * lk;
    float a[KL];
#pragma unroll
    for (int s = 0; s < KL; ++s) a[s] = TRANS_X ? Xs[(kb + s) * L::LS + i] : Xs[i * L::LS + kb + s];
    float b[L::TW][KL];
#pragma unroll
    for (int t = 0; t < L::TW; ++t) {
      const int j = 16 * (t0 + t) + li;
#pragma unroll
      for (int s = 0; s < KL; ++s) b[t][s] = TRANS_Y ? Ys[j * L::LS + kb + s] : Ys[(kb + s) * L::LS + j];
    }
#pragma unroll
    for (int s = 0; s < KL; ++s)
#pragma unroll
      for (int t = 0; t < L::TW; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[t][s], acc[t], 0, 0, 0);
  }
}

// As mfma_rowstrip with X held in registers: pa[b][s] = X[16*strip + lane%16][16b + 4*(lane/16) + s],
// the row-major A operand of k block b, step s; Y in LDS, row-major or (TRANS_Y) transposed.
template <int NP, int WPR, int KL = 4, bool TRANS_Y = false>
__device__ __forceinline__ void mfma_rowstrip_areg(const float (&pa)[NP / 16][4], const float* __restrict__ Ys,
                                                   int wave, int lane, v4f (&acc)[NP / 16 / WPR]) {
  using L = NsLayout<NP, WPR>;
  const int t0 = (wave % WPR) * L::TW;
  const int li = lane & 15, lk = lane >> 4;
#pragma unroll
  for (int t = 0; t < L::TW; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < L::NT; ++kb) {
    const int k = 16 * kb + 4 * lk;
    float b[L::TW][4];
#pragma unroll
    for (int t = 0; t < L::TW; ++t) {
      const int j = 16 * (t0 + t) + li;
      if constexpr (TRANS_Y) {
        if (kb + 1 < L::NT || KL == 4) {
          const float4 v = *reinterpret_cast<const float4*>(&Ys[j * L::LS + k]);
          b[t][0] = v.x; b[t][1] = v.y; b[t][2] = v.z; b[t][3] = v.w;
        } else {
#pragma unroll
          for (int s = 0; s < KL; ++s) b[t][s] = Ys[j * L::LS + k + s];
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (kb + 1 < L::NT || s < KL) b[t][s] = Ys[(k + s) * L::LS + j];
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (kb + 1 < L::NT || s < KL)  // folded at compile time (kb unrolled)
#pragma unroll
        for (int t = 0; t < L::TW; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[kb][s], b[t][s], acc[t], 0, 0, 0);
  }
}

// Element (r) of this wave's tile t: row 16*strip + 4*(lane/16) + r, col 16*(t0 + t) + lane%16.
template <int NP, int WPR>
__device__ __forceinline__ void store_strip(float* __restrict__ Ds, int wave, int lane,
                                            const v4f (&acc)[NP / 16 / WPR]) {
  using L = NsLayout<NP, WPR>;
  const int strip = wave / WPR, t0 = (wave % WPR) * L::TW;
#pragma unroll
  for (int t = 0; t < L::TW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      Ds[(16 * strip + 4 * (lane >> 4) + r) * L::LS + 16 * (t0 + t) + (lane & 15)] = acc[t][r];
}

// Transposed store: Ds[j][i] = D[i][j] for this wave's tiles. A lane's 4 rows
// are consecutive in the transposed row: one 16-byte write per tile (16 lanes of
// a lane group on distinct bank groups, LS = 4 mod 16).
template <int NP, int WPR>
__device__ __forceinline__ void store_strip_t(float* __restrict__ Ds, int wave, int lane,
                                              const v4f (&acc)[NP / 16 / WPR]) {
  using L = NsLayout<NP, WPR>;
  const int strip = wave / WPR, t0 = (wave % WPR) * L::TW;
#pragma unroll
  for (int t = 0; t < L::TW; ++t)
    *reinterpret_cast<v4f*>(&Ds[(16 * (t0 + t) + (lane & 15)) * L::LS + 16 * strip + 4 * (lane >> 4)]) = acc[t];
}

// V <- 2V - U on this wave's strip.
template <int NP, int WPR>
__device__ __forceinline__ void update_strip(float* __restrict__ Vs, int wave, int lane,
                                             const v4f (&acc)[NP / 16 / WPR]) {
  using L = NsLayout<NP, WPR>;
  const int strip = wave / WPR, t0 = (wave % WPR) * L::TW;
#pragma unroll
  for (int t = 0; t < L::TW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* p = &Vs[(16 * strip + 4 * (lane >> 4) + r) * L::LS + 16 * (t0 + t) + (lane & 15)];
      *p = 2.0f * (*p) - acc[t][r];
    }
}

// Sum of x over the four 16-lane rows of the wave, in every lane, as
// (row 0 + row 1) + (row 2 + row 3). v_permlane16_swap on two copies of x
// leaves rows (0, 0, 2, 2) in one and (1, 1, 3, 3) in the other, whose sum is
// each row pair's total; v_permlane32_swap does the same for the halves. The
// swaps are written as asm on two distinct registers: the builtin, given the
// same value twice, was folded to one result. s_nop 1 covers the VALU write
// of an operand just before the swap.
__device__ __forceinline__ float sum_rows4(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  const float y = a + b;
  float c = y, d = y;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
  return c + d;
}

// P = f32(mat) + 0.01 I on the live n x n block (the slot's padding is left as is).
template <typename T, int NP, int WPR>
__device__ __forceinline__ void load_P(float* __restrict__ Ps, const T* __restrict__ M, int n) {
  using L = NsLayout<NP, WPR>;
  for (int e = threadIdx.x; e < n * n; e += L::THREADS) {
    const int i = e / n, j = e - i * n;
    Ps[i * L::LS + j] = to_acc(M[e]) + (i == j ? 0.01f : 0.f);
  }
}

// P = f32(mat) + 0.01 I on the live n x n block and zero on the rest of the
// NP x NP slot, in one pass (each slot element written once, no zero fill
// and barrier ahead of it).
template <typename T, int NP, int WPR>
__device__ __forceinline__ void load_P_padded(float* __restrict__ Ps, const T* __restrict__ M, int n) {
  using L = NsLayout<NP, WPR>;
  for (int e = threadIdx.x; e < NP * NP; e += L::THREADS) {
    const int i = e / NP, j = e - i * NP;
    float v = 0.f;
    if (i < n && j < n) v = to_acc(M[i * n + j]) + (i == j ? 0.01f : 0.f);
    Ps[i * L::LS + j] = v;
  }
}

// alpha = 1.8 / (max_i sum_j P_ij)^2; row sums in ascending j, one thread per row.
template <int NP, int WPR>
__device__ __forceinline__ float compute_alpha(const float* __restrict__ Ps, int n, float* __restrict__ red) {
  using L = NsLayout<NP, WPR>;
  const int tid = threadIdx.x;
  float row = -1e30f;
  if (tid < n) {
    // The whole padded row as 16-byte reads, four at a time ahead of their sums:
    // columns past n are zero (the slot is zero-filled whenever n < NP), so
    // summing all NP in ascending j adds exact zeros after the reference's n terms.
    float s = 0.f;
#pragma unroll
    for (int q0 = 0; q0 < NP / 4; q0 += 4) {
      float4 v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const float4*>(&Ps[tid * L::LS + 4 * (q0 + q)]);
#pragma unroll
      for (int q = 0; q < 4; ++q) s = (((s + v[q].x) + v[q].y) + v[q].z) + v[q].w;
    }
    row = s;
  }
  for (int off = 32; off > 0; off >>= 1) row = fmaxf(row, __shfl_xor(row, off));
  if ((tid & 63) == 0) red[tid >> 6] = row;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < L::NW; ++w) m = fmaxf(m, red[w]);
  return 1.8f / (m * m);
}

// The forward variant whose U = V T reads V from registers (see the loop): the
// one-live-row path with two or four waves per strip.
template <int NP, int WPR, int KL> constexpr bool fwd_va() { return KL == 1 && WPR >= 2; }

// PV_FIRST: V <- 2V - V(PV) (the reference's order for n <= 112), P held in
// registers as this wave's A operand after the set-up, so the LDS holds V and
// T = PV only. Otherwise V <- 2V - (VP)V (its order for n = 128): LDS holds V
// and P, P is overwritten by W = VP and reloaded each iteration.
template <typename T, int NP, bool PV_FIRST, int WPR, int KL>
__device__ __forceinline__ void newton_fwd_body(const T* __restrict__ mat, T* __restrict__ out, int n, int iters) {
  using L = NsLayout<NP, WPR>;
  extern __shared__ __align__(16) float nsm[];
  __shared__ float red[16];
  float* Ps = nsm;                 // P; then T = PV (PV_FIRST) or W = VP
  float* Vs = nsm + L::ELEMS;      // V
  // With KL = 1 the last strip's waves (one live row, on the VALU) are the
  // workgroup's first hardware waves: a SIMD issues its oldest waves first, and
  // that row is the longest chain of each product.
  const int hw = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wave = KL == 1 ? (hw + (L::NT - 1) * WPR) % L::NW : hw;
  const T* Mg = mat + (size_t)blockIdx.x * n * n;
  T* Og = out + (size_t)blockIdx.x * n * n;

  // P = f32(mat) + 0.01 I on the live block, zero on the rest of the NP x NP
  // slot, in one pass; with few elements per thread (PER) each thread keeps its
  // own and writes V = alpha P from them below.
  constexpr int PER = NP * NP / L::THREADS;
  static_assert(PER * L::THREADS == NP * NP, "whole slot rows per pass");
  constexpr bool KEEP = PER <= 8;
  float pv[KEEP ? PER : 1];
  if constexpr (KEEP) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = threadIdx.x + q * L::THREADS, i = e / NP, j = e - i * NP;
      float v = 0.f;
      if (i < n && j < n) v = to_acc(Mg[i * n + j]) + (i == j ? 0.01f : 0.f);
      Ps[i * L::LS + j] = v;
      pv[q] = v;
    }
  } else {
    load_P_padded<T, NP, WPR>(Ps, Mg, n);
  }
  __syncthreads();

  // n = NP - 15 (KL = 1): the last strip holds one live row, r1 = NP - 16. Its
  // waves compute that row on the VALU (lane (li, lk): column 16 (t0 + t) + li
  // of each of its tiles, partial sums over its own k = 16 kb + 4 lk + s,
  // added over lk by two exchanges) and leave the matrix core to the other
  // strips; rows and columns past it stay zero padding. pa holds, for li = 0,
  // row r1 of P: every lane takes its k set of that row.
  constexpr int r1 = NP - 16;
  const bool rowv = KL == 1 && wave / WPR == L::NT - 1;
  float pa[PV_FIRST ? L::NT : 1][4];
  auto load_pa = [&]() {  // A operand of T = P V
    const int i = rowv ? r1 : 16 * (wave / WPR) + (lane & 15), kq = 4 * (lane >> 4);
#pragma unroll
    for (int kb = 0; kb < L::NT; ++kb) {
      const float4 v = *reinterpret_cast<const float4*>(&Ps[i * L::LS + 16 * kb + kq]);
      pa[kb][0] = v.x; pa[kb][1] = v.y; pa[kb][2] = v.z; pa[kb][3] = v.w;
    }
  };
  // Small slots: read ahead of alpha's reduction (larger ones would hold more
  // registers across it than their occupancy allows).
  if constexpr (PV_FIRST && KEEP) load_pa();
  const float alpha = compute_alpha<NP, WPR>(Ps, n, red);
  if constexpr (KEEP) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = threadIdx.x + q * L::THREADS, i = e / NP, j = e - i * NP;
      Vs[i * L::LS + j] = pv[q] * alpha;
    }
  } else {
    for (int e = threadIdx.x; e < L::ELEMS; e += L::THREADS) Vs[e] = Ps[e] * alpha;
  }
  if constexpr (PV_FIRST && !KEEP) load_pa();

  v4f acc[L::TW];
  if constexpr (PV_FIRST) {
    __syncthreads();  // P fully read (registers) and V0 written before slot P becomes T
    float* Ts = Ps;
    const int t0v = (wave % WPR) * L::TW, li = lane & 15, lk = lane >> 4;
    // VA (one live row, two or four waves per strip): U = V T takes its A operand (the
    // strip's V rows; row r1 on the row waves) from registers loaded while T is
    // computed, so no wave reads V from LDS after T is complete and the update
    // needs no barrier ahead of it.
    constexpr bool VA = fwd_va<NP, WPR, KL>();
    float va[L::NT][4];
    auto load_va = [&]() {
      const int i = rowv ? r1 : 16 * (wave / WPR) + li;
#pragma unroll
      for (int kb = 0; kb < L::NT; ++kb) {
        const float4 v = *reinterpret_cast<const float4*>(&Vs[i * L::LS + 16 * kb + 4 * lk]);
        va[kb][0] = v.x; va[kb][1] = v.y; va[kb][2] = v.z; va[kb][3] = v.w;
      }
    };
    for (int it = 0; it < iters; ++it) {
      if (rowv) {
#pragma unroll
        for (int t = 0; t < L::TW; ++t) {  // T[r1][j] = sum_k P[r1][k] V[k][j]
          const int j = 16 * (t0v + t) + li;
          float sum = 0.f;
#pragma unroll
          for (int kb = 0; kb < L::NT; ++kb)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (kb + 1 < L::NT || q < KL) sum += pa[kb][q] * Vs[(16 * kb + 4 * lk + q) * L::LS + j];
          sum = sum_rows4(sum);
          if (lk == 0) Ts[j * L::LS + r1] = sum;
        }
        if constexpr (VA) load_va();
      } else {
        mfma_rowstrip_areg<NP, WPR, KL>(pa, Vs, wave, lane, acc);       // T = P V
        if constexpr (VA) load_va();  // behind T's operand reads, ahead of its barrier
        store_strip_t<NP, WPR>(Ts, wave, lane, acc);                     // slot T holds T^T
      }
      __syncthreads();
      float u[L::TW];
      if (rowv) {
#pragma unroll
        for (int t = 0; t < L::TW; ++t) {  // U[r1][j] = sum_k V[r1][k] T[k][j], T[k][j] = Ts[j][k]
          const int j = 16 * (t0v + t) + li;
          float sum = 0.f;
#pragma unroll
          for (int kb = 0; kb < L::NT; ++kb) {
            float vr[4];
            if constexpr (VA) {
#pragma unroll
              for (int q = 0; q < 4; ++q) vr[q] = va[kb][q];
            } else {
              const float4 vv = *reinterpret_cast<const float4*>(&Vs[r1 * L::LS + 16 * kb + 4 * lk]);
              vr[0] = vv.x; vr[1] = vv.y; vr[2] = vv.z; vr[3] = vv.w;
            }
            const float4 tt = *reinterpret_cast<const float4*>(&Ts[j * L::LS + 16 * kb + 4 * lk]);
            const float ta[4] = {tt.x, tt.y, tt.z, tt.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (kb + 1 < L::NT || q < KL) sum += vr[q] * ta[q];
          }
          u[t] = sum_rows4(sum);
        }
      } else if constexpr (VA) {
        mfma_rowstrip_areg<NP, WPR, KL, true>(va, Ts, wave, lane, acc);    // U = V T
      } else {
        mfma_rowstrip<NP, WPR, false, true, KL>(Vs, Ts, wave, lane, acc);  // U = V T (own V rows only)
      }
      // With WPR > 1 the waves of a strip read all of its V rows and each then
      // updates part of them: every read first (done before T was complete with VA).
      if constexpr (WPR > 1 && !VA) __syncthreads();
      if (rowv) {
        if (lk == 0)
#pragma unroll
          for (int t = 0; t < L::TW; ++t) {
            float* p = &Vs[r1 * L::LS + 16 * (t0v + t) + li];
            *p = 2.0f * (*p) - u[t];
          }
      } else {
        update_strip<NP, WPR>(Vs, wave, lane, acc);                    // V = 2V - U
      }
      __syncthreads();
    }
  } else {
    __syncthreads();
    for (int it = 0; it < iters; ++it) {
      mfma_rowstrip<NP, WPR, false, false>(Vs, Ps, wave, lane, acc);  // W = V P
      __syncthreads();                                                 // P reads done
      store_strip<NP, WPR>(Ps, wave, lane, acc);
      __syncthreads();
      mfma_rowstrip<NP, WPR, false, false>(Ps, Vs, wave, lane, acc);  // U = W V
      __syncthreads();                                                 // V reads done
      update_strip<NP, WPR>(Vs, wave, lane, acc);
      if (it + 1 < iters) load_P<T, NP, WPR>(Ps, Mg, n);               // padding of slot P is still zero
      __syncthreads();
    }
  }
  // Row i by wave i mod NW, columns by lane: no division by the runtime n.
  for (int i = hw; i < n; i += L::NW)
    for (int j = lane; j < n; j += 64) Og[i * n + j] = from_acc<T>(Vs[i * L::LS + j]);
}

// One 16 x 16 tile of X Y (X's 16 rows in registers as in mfma_rowstrip_areg,
// Y in LDS: rows k, or TRANS_Y: Y[k][j] read from Ys[j][k]) for column tile t,
// with n = 16 m + 1 (KL = 1: one live k in the last block).
template <bool TRANS_Y>
__device__ __forceinline__ v4f mfma_tile_areg64(const float (&pa)[4][4], const float* __restrict__ Ys, int t, int lane) {
  constexpr int LS = NsLayout<64>::LS;
  const int li = lane & 15, lk = lane >> 4, j = 16 * t + li;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  float b[4][4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int k = 16 * kb + 4 * lk;
    if constexpr (TRANS_Y) {
      if (kb < 3) {
        const float4 v = *reinterpret_cast<const float4*>(&Ys[j * LS + k]);
        b[kb][0] = v.x; b[kb][1] = v.y; b[kb][2] = v.z; b[kb][3] = v.w;
      } else {
        b[kb][0] = Ys[j * LS + k];
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (kb < 3 || q == 0) b[kb][q] = Ys[(k + q) * LS + j];
    }
  }
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (kb < 3 || q == 0) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[kb][q], b[kb][q], acc, 0, 0, 0);
  return acc;
}

// NewtonInverse for fp32 n = 49 (the 64 bucket with one live row in the last
// strip) when P is symmetric, which the workgroup checks on the staged P (else
// it runs newton_fwd_body). Every iterate V is then a polynomial in P, so V, T = PV
// and U = VT are symmetric: the iteration (the reference's V <- 2V - V(PV) order)
// computes the six 16 x 16 tiles (r, t), r <= t < 3, on the matrix cores, row 48 on
// the VALU, and writes each tile and its mirror (the diagonal tiles and row 48
// from their upper halves, so every iterate is exactly symmetric): half the
// matrix-core tiles of the general path (twelve), which computes the column-48
// tiles as well. NW waves: 6 tile waves (two per SIMD on SIMDs 0 and 1, one on 2
// and 3), NW = 8: 2 row-48 waves of 32 columns, NW = 16: 4 of 16 (6 idle).
template <int NW>
__device__ __forceinline__ void newton_fwd_sym_body(const float* __restrict__ mat, float* __restrict__ out, int n,
                                                    int iters) {
  constexpr int NP = 64, WPR = NW / 4, R = NW == 8 ? 2 : 4, TWR = 4 / R;
  using L = NsLayout<NP, WPR>;
  static_assert(L::THREADS == 64 * NW && (NW == 8 || NW == 16), "8 or 16 waves");
  extern __shared__ __align__(16) float nsm[];
  __shared__ float red[16];
  float* Ps = nsm;             // P; then T (stored transposed: Ts[j][k] = T[k][j])
  float* Vs = nsm + L::ELEMS;  // V
  const int hw = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63, li = lane & 15, lk = lane >> 4;
  const float* Mg = mat + (size_t)blockIdx.x * n * n;
  float* Og = out + (size_t)blockIdx.x * n * n;
  constexpr int PER = NP * NP / L::THREADS;
  float pv[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + q * L::THREADS, i = e / NP, j = e - i * NP;
    float v = 0.f;
    if (i < n && j < n) v = Mg[i * n + j] + (i == j ? 0.01f : 0.f);
    Ps[i * L::LS + j] = v;
    pv[q] = v;
  }
  __syncthreads();
  int asym = 0;
  for (int e = threadIdx.x; e < n * n; e += L::THREADS) {
    const int i = e / n, j = e - i * n;
    if (j > i && Ps[i * L::LS + j] != Ps[j * L::LS + i]) asym = 1;
  }
  if (__syncthreads_or(asym)) {  // not symmetric: the general iteration
    newton_fwd_body<float, NP, true, WPR, 1>(mat, out, n, iters);
    return;
  }
  constexpr int r1 = NP - 16;  // the last strip's live row (48)
  // Tile waves hw < 6: (r, t) = (0,0) (0,1) (0,2) (1,1) (1,2) (2,2); row waves 6 .. 6 + R - 1.
  const bool tilew = hw < 6, roww = hw >= 6 && hw < 6 + R;
  const int tr = hw < 3 ? 0 : hw < 5 ? 1 : 2;
  const int tc = hw < 3 ? hw : hw < 5 ? hw - 2 : 2;
  const int c0 = (hw - 6) * TWR;  // row waves: first column tile
  float pa[4][4];
  {
    const int i = roww ? r1 : 16 * tr + li;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 v = *reinterpret_cast<const float4*>(&Ps[i * L::LS + 16 * kb + 4 * lk]);
      pa[kb][0] = v.x; pa[kb][1] = v.y; pa[kb][2] = v.z; pa[kb][3] = v.w;
    }
  }
  const float alpha = compute_alpha<NP, WPR>(Ps, n, red);
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + q * L::THREADS, i = e / NP, j = e - i * NP;
    Vs[i * L::LS + j] = pv[q] * alpha;
  }
  __syncthreads();  // P read, V0 written: slot P takes T
  float* Ts = Ps;
  float va[4][4];
  auto load_va = [&]() {
    const int i = roww ? r1 : 16 * tr + li;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 v = *reinterpret_cast<const float4*>(&Vs[i * L::LS + 16 * kb + 4 * lk]);
      va[kb][0] = v.x; va[kb][1] = v.y; va[kb][2] = v.z; va[kb][3] = v.w;
    }
  };
  // Tile (r, c) and its mirror, from the lanes' 16 x 16 values val[row 4 lk + q][col li]:
  // off the diagonal, D[16r + a][16c + b] and D[16c + b][16r + a] (the transposed one as a
  // 16-byte store); on it, both from the upper half (a <= b) only.
  auto store_sym = [&](float* D, int r, int c, const float (&val)[4]) {
    if (r != c) {
#pragma unroll
      for (int q = 0; q < 4; ++q) D[(16 * r + 4 * lk + q) * L::LS + 16 * c + li] = val[q];
      *reinterpret_cast<float4*>(&D[(16 * c + li) * L::LS + 16 * r + 4 * lk]) = float4{val[0], val[1], val[2], val[3]};
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int a = 4 * lk + q, b = li;
        if (a <= b) {
          D[(16 * r + a) * L::LS + 16 * c + b] = val[q];
          D[(16 * c + b) * L::LS + 16 * r + a] = val[q];
        }
      }
    }
  };
  // Row 48 of X Y on the VALU (X's row in xr, Y row-major in LDS or TRANS_Y), for the
  // row wave's columns 16 (c0 + u) + li, summed over k by the lane groups.
  auto row48 = [&](const float (&xr)[4][4], const float* Ys, bool transY, float (&res)[TWR]) {
#pragma unroll
    for (int u = 0; u < TWR; ++u) {
      const int j = 16 * (c0 + u) + li;
      float sum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (kb < 3 || q == 0) {
            const int k = 16 * kb + 4 * lk + q;
            sum += xr[kb][q] * (transY ? Ys[j * L::LS + k] : Ys[k * L::LS + j]);
          }
      res[u] = sum_rows4(sum);
    }
  };
  for (int it = 0; it < iters; ++it) {
    if (tilew) {
      const v4f acc = mfma_tile_areg64<false>(pa, Vs, tc, lane);  // T(r, c) = P(r, :) V(:, c)
      load_va();
      // Ts holds T transposed: T(r, c) goes to Ts block (c, r) transposed, i.e. the
      // mirror of a symmetric T: Ts[16c + b][16r + a] = T[16r + a][16c + b].
      const float val[4] = {acc[0], acc[1], acc[2], acc[3]};
      store_sym(Ts, tr, tc, val);
    } else if (roww) {
      float res[TWR];
      row48(pa, Vs, false, res);  // T[48][j]
      load_va();
      if (lk == 0)
#pragma unroll
        for (int u = 0; u < TWR; ++u) {
          const int j = 16 * (c0 + u) + li;
          if (j <= r1) {
            Ts[j * L::LS + r1] = res[u];
            Ts[r1 * L::LS + j] = res[u];
          }
        }
    }
    __syncthreads();
    if (tilew) {
      const v4f acc = mfma_tile_areg64<true>(va, Ts, tc, lane);  // U(r, c) = V(r, :) T(:, c)
      float val[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) val[q] = 2.0f * Vs[(16 * tr + 4 * lk + q) * L::LS + 16 * tc + li] - acc[q];
      store_sym(Vs, tr, tc, val);
    } else if (roww) {
      float res[TWR];
      row48(va, Ts, true, res);  // U[48][j]
      if (lk == 0)
#pragma unroll
        for (int u = 0; u < TWR; ++u) {
          const int j = 16 * (c0 + u) + li;
          if (j <= r1) {
            const float v = 2.0f * Vs[r1 * L::LS + j] - res[u];
            Vs[r1 * L::LS + j] = v;
            Vs[j * L::LS + r1] = v;
          }
        }
    }
    __syncthreads();
  }
  for (int i = hw; i < n; i += L::NW)
    for (int j = lane; j < n; j += 64) Og[i * n + j] = Vs[i * L::LS + j];
}

template <int NW>
__global__ void __launch_bounds__(64 * NW)
newton_fwd_sym_kernel(const float* __restrict__ mat, float* __restrict__ out, int n, int iters) {
  newton_fwd_sym_body<NW>(mat, out, n, iters);
}

template <typename T, int NP, bool PV_FIRST, int WPR = 1, int KL = 4>
__global__ void __launch_bounds__(NP * 4 * WPR)
newton_fwd_kernel(const T* __restrict__ mat, T* __restrict__ out, int n, int iters) {
  newton_fwd_body<T, NP, PV_FIRST, WPR, KL>(mat, out, n, iters);
}

// ---------------------------------------------------------------------------
// The attention layer's landmark products around NewtonInverse (no reference
// counterpart: the reference ships the operators only). With Kmm the layer's
// m x m landmark kernel, 48 < m <= 64 (the 64 bucket), d <= 64, fp32:
//   forward:  X = NewtonInverse(Kmm) beside the tall product's per-workgroup
//             partials of K_km^T V in one launch (newton_fwd_tall_kernel);
//             then kv = sum of the partials (in workgroup order), W = X kv
//             (landmark_kv_w_kernel)                     (X, kv, W written)
//   backward: dw = sum of the partials of K_qm^T G; then
//             dX = dw kv^T,  dkv = X^T dw,  dKmm = -(X^T dX) X^T
//             (newton_bwd_mul_kernel, one workgroup per slice; dkv, dKmm written)
// so that the m x m products and the inverse's gradient input never make a
// round trip through HBM or a launch of their own.
// Partials: [slice][per][64][64] fp32, entry [p][q] (landmark p, channel q);
// entries outside m x d are not read as data (set to zero here).

// Sum of the slice's `per` partials (in order) into an LDS tile [64][LS]:
// rows < m and columns < d, zero elsewhere.
template <int NP, int WPR>
__device__ __forceinline__ void sum_partials(float* __restrict__ Ds, const float* __restrict__ part, int per, int m,
                                             int d) {
  using L = NsLayout<NP, WPR>;
  static_assert(NP == 64, "64-column tiles");
  const float* src = part + (size_t)blockIdx.x * per * 64 * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += L::THREADS) {
    const int i = e >> 6, j = e & 63;
    float sum = 0.0f;
    if (i < m && j < d)
      for (int x = 0; x < per; ++x) sum += src[(size_t)x * 64 * 64 + e];
    Ds[i * L::LS + j] = sum;
  }
}

// Rows < m, columns < d of this wave's tiles, row-major with d columns.
template <int NP, int WPR>
__device__ __forceinline__ void store_tiles(float* __restrict__ dst, int wave, int lane, const v4f (&acc)[NP / 16 / WPR],
                                            int m, int d) {
  using L = NsLayout<NP, WPR>;
  const int strip = wave / WPR, t0 = (wave % WPR) * L::TW;
#pragma unroll
  for (int t = 0; t < L::TW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * strip + 4 * (lane >> 4) + r, j = 16 * (t0 + t) + (lane & 15);
      if (i < m && j < d) dst[(size_t)i * d + j] = acc[t][r];
    }
}

// The landmark forward in two launches. First, workgroups [0, bh) run
// NewtonInverse on the bh landmark matrices (newton_fwd_body, writing the
// inverse) and workgroups [bh, bh (1 + per)) the tall product's partials of
// K_km^T V (tall_t_bf16_body, per workgroups per slice): the two sets share
// nothing, so the memory-bound tall product runs on the CUs that the
// latency-bound iterations leave free. Then landmark_kv_w_kernel sums the
// partials into kv (in workgroup order) and forms W = inv kv. One block size
// serves both roles: 512 threads, two waves per 16-row strip of NewtonInverse
// (the tall body needs more registers than 1024-thread blocks allow).
template <int NP, int KL, typename TB>
__global__ void __launch_bounds__(NP * 8)
newton_fwd_tall_kernel(const float* __restrict__ kmm, float* __restrict__ inv, int n, int iters, int bh,
                       const float* __restrict__ A, const TB* __restrict__ B, float* __restrict__ part, int N, int P,
                       int Q, int per) {
  if ((int)blockIdx.x < bh) {
    if constexpr (KL == 1 && NP == 64)
      newton_fwd_sym_body<8>(kmm, inv, n, iters);
    else
      newton_fwd_body<float, NP, true, 2, KL>(kmm, inv, n, iters);
  } else {
    extern __shared__ __align__(16) float nsm[];
    const int t = (int)blockIdx.x - bh;
    tall_t_bf16_body<TB>(A, B, part, N, P, Q, nsm, t / per, t % per, per);
  }
}

template <int NP, int WPR, int KL>
__global__ void __launch_bounds__(NP * 4 * WPR)
landmark_kv_w_kernel(const float* __restrict__ inv, const float* __restrict__ part, int per, int n, int d,
                     float* __restrict__ kvOut, float* __restrict__ wOut) {
  using L = NsLayout<NP, WPR>;
  extern __shared__ __align__(16) float nsm[];
  float* KVs = nsm;
  float* Vs = nsm + L::ELEMS;
  static_assert(NP == 64 && L::THREADS == 1024, "four elements of each 64 x 64 slot per thread");
  // Every load in flight before the first LDS write: the inverse (zero padded to 64 x 64) and the
  // partials, summed in workgroup order as sum_partials does.
  const float* Vg = inv + (size_t)blockIdx.x * n * n;
  const float* src = part + (size_t)blockIdx.x * per * 64 * 64;
  float vi[4], ks[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = threadIdx.x + 1024 * q, i = e >> 6, j = e & 63;
    vi[q] = (i < n && j < n) ? Vg[i * n + j] : 0.f;
  }
  int x = 0;
  for (; x + 2 <= per; x += 2) {
    float a[4], b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = threadIdx.x + 1024 * q;
      a[q] = src[(size_t)x * 4096 + e];
      b[q] = src[(size_t)(x + 1) * 4096 + e];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) ks[q] = (ks[q] + a[q]) + b[q];
  }
  for (; x < per; ++x)
#pragma unroll
    for (int q = 0; q < 4; ++q) ks[q] += src[(size_t)x * 4096 + threadIdx.x + 1024 * q];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = threadIdx.x + 1024 * q, i = e >> 6, j = e & 63;
    Vs[i * L::LS + j] = vi[q];
    KVs[i * L::LS + j] = (i < n && j < d) ? ks[q] : 0.f;
  }
  __syncthreads();
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  float* kvs = kvOut + (size_t)blockIdx.x * n * d;
  for (int e = threadIdx.x; e < n * 64; e += L::THREADS) {
    const int i = e >> 6, j = e & 63;
    if (j < d) kvs[i * d + j] = KVs[i * L::LS + j];
  }
  v4f acc[L::TW];
  mfma_rowstrip<NP, WPR, false, false, KL>(Vs, KVs, wave, lane, acc);  // W = X kv (k < n)
  store_tiles<NP, WPR>(wOut + (size_t)blockIdx.x * n * d, wave, lane, acc, n, d);
}

template <int NP, int WPR, int KL>
__device__ __forceinline__ void newton_bwd_mul_body(const float* __restrict__ part, int per, const float* __restrict__ kv,
                                                    const float* __restrict__ inv, float* __restrict__ dkv,
                                                    float* __restrict__ gmat, int n, int d) {
  using L = NsLayout<NP, WPR>;
  extern __shared__ __align__(16) float nsm[];
  float* Vs = nsm;                   // X
  float* Gs = nsm + L::ELEMS;        // dX^T, then S = X^T dX
  float* DWs = nsm + 2 * L::ELEMS;   // dw
  float* KVs = nsm + 3 * L::ELEMS;   // kv
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const size_t off = (size_t)blockIdx.x * n * n, offd = (size_t)blockIdx.x * n * d;
  for (int e = threadIdx.x; e < NP * NP; e += L::THREADS) {
    const int i = e / NP, j = e - i * NP;
    Vs[i * L::LS + j] = i < n && j < n ? inv[off + (size_t)i * n + j] : 0.0f;
    KVs[i * L::LS + j] = i < n && j < d ? kv[offd + (size_t)i * d + j] : 0.0f;
  }
  sum_partials<NP, WPR>(DWs, part, per, n, d);
  __syncthreads();
  v4f acc[L::TW];
  mfma_rowstrip<NP, WPR, false, true, 4>(DWs, KVs, wave, lane, acc);   // dX = dw kv^T (k < d)
  store_strip_t<NP, WPR>(Gs, wave, lane, acc);                          // slot G holds dX^T
  mfma_rowstrip<NP, WPR, true, false, KL>(Vs, DWs, wave, lane, acc);   // dkv = X^T dw (k < n)
  store_tiles<NP, WPR>(dkv + offd, wave, lane, acc, n, d);
  __syncthreads();
  mfma_rowstrip<NP, WPR, true, true, KL>(Vs, Gs, wave, lane, acc);     // S = X^T dX (B read from dX^T)
  __syncthreads();
  store_strip<NP, WPR>(Gs, wave, lane, acc);
  __syncthreads();
  mfma_rowstrip<NP, WPR, false, true, KL>(Gs, Vs, wave, lane, acc);    // R = S X^T
  const int strip = wave / WPR, t0 = (wave % WPR) * L::TW;
#pragma unroll
  for (int t = 0; t < L::TW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * strip + 4 * (lane >> 4) + r, j = 16 * (t0 + t) + (lane & 15);
      if (i < n && j < n) gmat[off + (size_t)i * n + j] = -acc[t][r];
    }
}

template <int NP, int WPR, int KL>
__global__ void __launch_bounds__(NP * 4 * WPR)
newton_bwd_mul_kernel(const float* __restrict__ part, int per, const float* __restrict__ kv,
                      const float* __restrict__ inv, float* __restrict__ dkv, float* __restrict__ gmat, int n, int d) {
  newton_bwd_mul_body<NP, WPR, KL>(part, per, kv, inv, dkv, gmat, n, d);
}

// The landmark backward's first launch after the tall product: workgroups [0, bh)
// run newton_bwd_mul_body (dkv and dKmm), the others the row product
// dK_qm = g W^T (mix_rows_bf16_body, 16 waves, `per` workgroups per slice), which
// needs neither: it runs on the CUs the one-workgroup-per-slice products leave
// free. The other two row products, which read dkv, follow in one launch.
template <int KL, typename TA, bool DIRECT>
__global__ void __launch_bounds__(1024)
newton_bwd_mix_kernel(const float* __restrict__ part, int per, const float* __restrict__ kv,
                      const float* __restrict__ inv, float* __restrict__ dkv, float* __restrict__ dkmm, int n, int d,
                      int bh, const TA* __restrict__ g, const float* __restrict__ w, float* __restrict__ dkqm, int N,
                      int permix) {
  if ((int)blockIdx.x < bh) {
    newton_bwd_mul_body<64, 4, KL>(part, per, kv, inv, dkv, dkmm, n, d);
  } else {
    const int t = (int)blockIdx.x - bh;
    mix_rows_bf16_body<TA, float, DIRECT, 16>(g, w, dkqm, N, d, n, d, 1, (int64_t)n * d, t / permix, t % permix,
                                              permix);
  }
}

template <typename T, int NP, int WPR = 1, int KL = 4>
__global__ void __launch_bounds__(NP * 4 * WPR)
newton_bwd_kernel(const T* __restrict__ gout, const T* __restrict__ inv, T* __restrict__ gmat, int n) {
  using L = NsLayout<NP, WPR>;
  extern __shared__ __align__(16) float nsm[];
  float* Vs = nsm;
  float* Gs = nsm + L::ELEMS;  // G^T, then S = V^T G
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const size_t off = (size_t)blockIdx.x * n * n;
  if (n < NP) {
    // Live block and zero padding of both NP x NP slots in one pass.
    for (int e = threadIdx.x; e < NP * NP; e += L::THREADS) {
      const int i = e / NP, j = e - i * NP;
      float v = 0.f, g = 0.f;
      if (i < n && j < n) {
        v = to_acc(inv[off + (size_t)i * n + j]);
        g = to_acc(gout[off + (size_t)i * n + j]);
      }
      Vs[i * L::LS + j] = v;
      Gs[j * L::LS + i] = g;
    }
  } else {
    // Whole 4-element groups of a row (NP is a multiple of 16).
    for (int e = threadIdx.x; e < NP * NP / 4; e += L::THREADS) {
      const int i = e / (NP / 4), j = 4 * (e - i * (NP / 4));
      float v[4], g[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[c] = to_acc(inv[off + (size_t)i * NP + j + c]);
        g[c] = to_acc(gout[off + (size_t)i * NP + j + c]);
      }
      *reinterpret_cast<float4*>(&Vs[i * L::LS + j]) = float4{v[0], v[1], v[2], v[3]};
#pragma unroll
      for (int c = 0; c < 4; ++c) Gs[(j + c) * L::LS + i] = g[c];
    }
  }
  __syncthreads();
  v4f acc[L::TW];
  mfma_rowstrip<NP, WPR, true, true, KL>(Vs, Gs, wave, lane, acc);  // S = V^T G (B read from G^T)
  __syncthreads();
  store_strip<NP, WPR>(Gs, wave, lane, acc);
  __syncthreads();
  mfma_rowstrip<NP, WPR, false, true, KL>(Gs, Vs, wave, lane, acc);  // R = S V^T
  if (n == NP) {
    // Through LDS (slot V, free once every wave's products are done): whole
    // rows leave as 4-element groups.
    __syncthreads();
    store_strip<NP, WPR>(Vs, wave, lane, acc);
    __syncthreads();
    for (int e = threadIdx.x; e < NP * NP / 4; e += L::THREADS) {
      const int i = e / (NP / 4), j = 4 * (e - i * (NP / 4));
      const float4 v = *reinterpret_cast<const float4*>(&Vs[i * L::LS + j]);
      const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) gmat[off + (size_t)i * NP + j + c] = from_acc<T>(-vv[c]);
    }
    return;
  }
  const int strip = wave / WPR, t0 = (wave % WPR) * L::TW;
#pragma unroll
  for (int t = 0; t < L::TW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * strip + 4 * (lane >> 4) + r, j = 16 * (t0 + t) + (lane & 15);
      if (i < n && j < n) gmat[off + (size_t)i * n + j] = from_acc<T>(-acc[t][r]);
    }
}

// The chained product pair of one wave (strip w) on full NP x NP matrices in LDS
// (V row-major, G^T row-major, row stride NP + 4): acc2 = R[16w.., :] = (V^T G V^T)
// rows, lane (i, g) holding R[16w + 4g + r][16 t + i] in acc2[t][r]. Each k block's
// operands are read while the previous block's MFMAs run (two register sets; the
// scheduling fences keep the reads ahead), and consecutive MFMAs go to different
// accumulators.
template <int NP>
__device__ __forceinline__ void chain_products(const float* __restrict__ Vs, const float* __restrict__ Gts, int w,
                                               int lane, v4f (&acc2)[NP / 16]) {
  using L = NsLayout<NP, 1>;
  constexpr int NT = L::NT;
  const int li = lane & 15, lg = lane >> 4;
  v4f acc1[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc1[t] = v4f{0.f, 0.f, 0.f, 0.f};
  // S^T[:, 16w..16w+16) = G^T V[:, 16w..16w+16): k over the rows of G and V.
  float4 a[2][NT];
  float b[2][4];
#pragma unroll
  for (int kk = 0; kk <= NT; ++kk) {
    if (kk < NT) {
      const int kb = 16 * kk + 4 * lg, nb = kk & 1;
#pragma unroll
      for (int s = 0; s < 4; ++s) b[nb][s] = Vs[(kb + s) * L::LS + 16 * w + li];
#pragma unroll
      for (int t = 0; t < NT; ++t) a[nb][t] = *reinterpret_cast<const float4*>(&Gts[(16 * t + li) * L::LS + kb]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (kk > 0) {
      const int cb = (kk - 1) & 1;
#pragma unroll
      for (int t = 0; t < NT; ++t) acc1[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[cb][t].x, b[cb][0], acc1[t], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc1[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[cb][t].y, b[cb][1], acc1[t], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc1[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[cb][t].z, b[cb][2], acc1[t], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc1[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[cb][t].w, b[cb][3], acc1[t], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // R = S V^T: block t's A operand is acc1[t] (k = 16t + 4g + r), B = V rows as 16-byte reads.
#pragma unroll
  for (int t = 0; t < NT; ++t) acc2[t] = v4f{0.f, 0.f, 0.f, 0.f};
  float4 vb[2][NT];
#pragma unroll
  for (int kk = 0; kk <= NT; ++kk) {
    if (kk < NT) {
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2)
        vb[kk & 1][t2] = *reinterpret_cast<const float4*>(&Vs[(16 * t2 + li) * L::LS + 16 * kk + 4 * lg]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (kk > 0) {
      const int t = kk - 1, cb = t & 1;
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) acc2[t2] = __builtin_amdgcn_mfma_f32_16x16x4f32(acc1[t][0], vb[cb][t2].x, acc2[t2], 0, 0, 0);
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) acc2[t2] = __builtin_amdgcn_mfma_f32_16x16x4f32(acc1[t][1], vb[cb][t2].y, acc2[t2], 0, 0, 0);
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) acc2[t2] = __builtin_amdgcn_mfma_f32_16x16x4f32(acc1[t][2], vb[cb][t2].z, acc2[t2], 0, 0, 0);
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) acc2[t2] = __builtin_amdgcn_mfma_f32_16x16x4f32(acc1[t][3], vb[cb][t2].w, acc2[t2], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Four consecutive elements at p (16-byte aligned for float, 8-byte for the 16-bit types) as fp32.
template <typename T>
__device__ __forceinline__ float4 load4_acc(const T* __restrict__ p) {
  if constexpr (std::is_same<T, float>::value) {
    return *reinterpret_cast<const float4*>(p);
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    T e[4];
    __builtin_memcpy(e, &u, sizeof(e));
    return float4{to_acc(e[0]), to_acc(e[1]), to_acc(e[2]), to_acc(e[3])};
  }
}

// Bounded wait on a workgroup counter in LDS: returns once *c >= target. Every
// counter this kernel waits on is raised by waves of the same workgroup whose own
// waits point only at earlier matrices, so every wait ends.
__device__ __forceinline__ void lds_wait_ge(int* c, int target) {
  while (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(1);
}

__device__ __forceinline__ void lds_raise(int* c, int lane) {
  if (lane == 0) __hip_atomic_fetch_add(c, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Four matrices' slots of two NP x (NP + 4) fp32 buffers and 9 counters.
template <int NP> constexpr size_t pipe_lds() { return 4 * 2 * (size_t)NsLayout<NP>::ELEMS * 4 + 12 * sizeof(int); }

// NewtonInverse backward for full 64 x 64 matrices, dA = -(V^T G) V^T, several per
// CU: one persistent workgroup per CU of four teams (4 waves each), team q taking
// the workgroup's matrices r = q, q + 4, ... through LDS slot q.
// * The two products chain in registers (chain_products): wave w of a team computes
//   the column strip w of S^T = G^T V, which is the A operand of its rows of
//   R = S V^T, so S never goes through LDS and the team meets only once per matrix,
//   after staging V row-major and G transposed.
// * Matrix r's loads are issued only after every wave has issued matrix r - 1's, so
//   a CU's requests reach the memory system in matrix order (all of them in flight
//   at once); each team's products start as soon as its own matrix is in LDS.
// Counters (each raised once per wave and matrix): issued (loads issued, in matrix
// order), ready[q] (waves of team q that wrote their share of the slot) and done[q]
// (waves of team q that finished reading it).
template <typename T, int NP>
__global__ void __launch_bounds__(1024)
newton_bwd_pipe_kernel(const T* __restrict__ gout, const T* __restrict__ inv, T* __restrict__ gmat, int64_t bh,
                       int per) {
  using L = NsLayout<NP, 1>;
  constexpr int NT = L::NT, TEAM_THREADS = NP * 4;
  static_assert(NP == 64, "four teams of four waves");
  extern __shared__ __align__(16) float nsm[];
  int* ready = reinterpret_cast<int*>(nsm + 4 * 2 * L::ELEMS);
  int* done = ready + 4;
  int* issued = ready + 8;
  const int team = uniform(threadIdx.x >> 8), w = uniform((threadIdx.x >> 6) & 3), lane = threadIdx.x & 63;
  const int tt = threadIdx.x & (TEAM_THREADS - 1);
  const int li = lane & 15, lg = lane >> 4;
  if (threadIdx.x < 9) ready[threadIdx.x] = 0;
  __syncthreads();
  const int64_t m0 = (int64_t)blockIdx.x * per;
  const int cnt = (int)(bh - m0 < per ? bh - m0 : per);
  float* Vs = nsm + team * 2 * L::ELEMS;
  float* Gts = Vs + L::ELEMS;
  constexpr int GROUPS = NP * NP / 4, PER = GROUPS / TEAM_THREADS;
  for (int r = team, k = 0; r < cnt; r += 4, ++k) {
    // Issue order only (no data is read through this counter), so relaxed.
    while (__hip_atomic_load(issued, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 4 * r) __builtin_amdgcn_s_sleep(1);
    const size_t off = (size_t)(m0 + r) * NP * NP;
    float4 vv[PER], gg[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int c = q * TEAM_THREADS + tt;
      vv[q] = load4_acc(inv + off + (size_t)(c / (NP / 4)) * NP + 4 * (c % (NP / 4)));
      gg[q] = load4_acc(gout + off + (size_t)(8 * (c >> 7) + ((c & 63) >> 3)) * NP + 32 * ((c >> 6) & 1) + 4 * (c & 7));
    }
    __builtin_amdgcn_sched_barrier(0);  // raised after the load instructions, not after their data
    if (lane == 0) __hip_atomic_fetch_add(issued, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (k > 0) lds_wait_ge(&done[team], 4 * k);  // the team's previous matrix has left the slot
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int c = q * TEAM_THREADS + tt;
      *reinterpret_cast<float4*>(&Vs[(c / (NP / 4)) * L::LS + 4 * (c % (NP / 4))]) = vv[q];
      const int gi = 8 * (c >> 7) + ((c & 63) >> 3), gj = 32 * ((c >> 6) & 1) + 4 * (c & 7);
      Gts[(gj + 0) * L::LS + gi] = gg[q].x;
      Gts[(gj + 1) * L::LS + gi] = gg[q].y;
      Gts[(gj + 2) * L::LS + gi] = gg[q].z;
      Gts[(gj + 3) * L::LS + gi] = gg[q].w;
    }
    lds_raise(&ready[team], lane);
    lds_wait_ge(&ready[team], 4 * (k + 1));
    v4f acc2[NT];
    chain_products<NP>(Vs, Gts, w, lane, acc2);
    lds_raise(&done[team], lane);
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2)
#pragma unroll
      for (int r2 = 0; r2 < 4; ++r2)
        gmat[off + (size_t)(16 * w + 4 * lg + r2) * NP + 16 * t2 + li] = from_acc<T>(-acc2[t2][r2]);
  }
}

// ---------------------------------------------------------------------------
// fp64: VALU products, 2-buffer (VP)V order, one workgroup of 256 threads per
// matrix. Slot A holds P, then W = VP; P is reloaded each iteration.
// ---------------------------------------------------------------------------
constexpr int kF64Threads = 256;

__device__ __forceinline__ void f64_matmul(const double* X, const double* Y, int np, int ls,
                                           bool transX, bool transY, double* outv, int perThread) {
  for (int q = 0; q < perThread; ++q) {
    const int e = threadIdx.x + q * kF64Threads;
    double s = 0.0;
    if (e < np * np) {
      const int i = e / np, j = e - i * np;
      for (int k = 0; k < np; ++k) {
        const double x = transX ? X[k * ls + i] : X[i * ls + k];
        const double y = transY ? Y[j * ls + k] : Y[k * ls + j];
        s = fma(x, y, s);
      }
    }
    outv[q] = s;
  }
}

constexpr int kF64MaxPer = 37;  // ceil(96*96 / 256)

__global__ void __launch_bounds__(kF64Threads)
newton_fwd_f64_kernel(const double* __restrict__ mat, double* __restrict__ out, int n, int np, int iters) {
  extern __shared__ __align__(16) double dsm[];
  __shared__ double redd[kF64Threads / 64];
  const int ls = np + 1, elems = np * ls;
  double* As = dsm;
  double* Vs = dsm + elems;
  const double* Mg = mat + (size_t)blockIdx.x * n * n;
  double* Og = out + (size_t)blockIdx.x * n * n;
  const int per = (np * np + kF64Threads - 1) / kF64Threads;
  auto loadP = [&]() {
    for (int e = threadIdx.x; e < n * n; e += kF64Threads) {
      const int i = e / n, j = e - i * n;
      As[i * ls + j] = Mg[e] + (i == j ? 0.01 : 0.0);
    }
  };
  for (int e = threadIdx.x; e < 2 * elems; e += kF64Threads) dsm[e] = 0.0;
  __syncthreads();
  loadP();
  __syncthreads();
  double row = -1e300;
  if ((int)threadIdx.x < n) {
    double s = 0.0;
    for (int j = 0; j < n; ++j) s += As[threadIdx.x * ls + j];
    row = s;
  }
  for (int o = 32; o > 0; o >>= 1) row = fmax(row, __shfl_xor(row, o));
  if ((threadIdx.x & 63) == 0) redd[threadIdx.x >> 6] = row;
  __syncthreads();
  double m = redd[0];
  for (int w = 1; w < kF64Threads / 64; ++w) m = fmax(m, redd[w]);
  const double alpha = 1.8 / (m * m);
  for (int e = threadIdx.x; e < elems; e += kF64Threads) Vs[e] = As[e] * alpha;
  __syncthreads();
  double tmp[kF64MaxPer];
  for (int it = 0; it < iters; ++it) {
    f64_matmul(Vs, As, np, ls, false, false, tmp, per);  // W = V P
    __syncthreads();
    for (int q = 0; q < per; ++q) {
      const int e = threadIdx.x + q * kF64Threads;
      if (e < np * np) As[(e / np) * ls + e % np] = tmp[q];
    }
    __syncthreads();
    f64_matmul(As, Vs, np, ls, false, false, tmp, per);  // U = W V
    __syncthreads();
    for (int q = 0; q < per; ++q) {
      const int e = threadIdx.x + q * kF64Threads;
      if (e < np * np) {
        double* p = &Vs[(e / np) * ls + e % np];
        *p = 2.0 * (*p) - tmp[q];
      }
    }
    // Restore P in slot A (padding rows/cols of W are zero already).
    if (it + 1 < iters) loadP();
    __syncthreads();
  }
  for (int e = threadIdx.x; e < n * n; e += kF64Threads) Og[e] = Vs[(e / n) * ls + e % n];
}

__global__ void __launch_bounds__(kF64Threads)
newton_bwd_f64_kernel(const double* __restrict__ gout, const double* __restrict__ inv,
                      double* __restrict__ gmat, int n, int np) {
  extern __shared__ __align__(16) double dsm[];
  const int ls = np + 1, elems = np * ls;
  double* Vs = dsm;
  double* Gs = dsm + elems;
  const size_t off = (size_t)blockIdx.x * n * n;
  const int per = (np * np + kF64Threads - 1) / kF64Threads;
  for (int e = threadIdx.x; e < 2 * elems; e += kF64Threads) dsm[e] = 0.0;
  __syncthreads();
  for (int e = threadIdx.x; e < n * n; e += kF64Threads) {
    Vs[(e / n) * ls + e % n] = inv[off + e];
    Gs[(e / n) * ls + e % n] = gout[off + e];
  }
  __syncthreads();
  double tmp[kF64MaxPer];
  f64_matmul(Vs, Gs, np, ls, true, false, tmp, per);  // S = V^T G
  __syncthreads();
  for (int q = 0; q < per; ++q) {
    const int e = threadIdx.x + q * kF64Threads;
    if (e < np * np) Gs[(e / np) * ls + e % np] = tmp[q];
  }
  __syncthreads();
  f64_matmul(Gs, Vs, np, ls, false, true, tmp, per);  // R = S V^T
  for (int q = 0; q < per; ++q) {
    const int e = threadIdx.x + q * kF64Threads;
    if (e < np * np) {
      const int i = e / np, j = e - i * np;
      if (i < n && j < n) gmat[off + (size_t)i * n + j] = -tmp[q];
    }
  }
}

// ---------------------------------------------------------------------------
// Large matrices, 128 < n <= 256 (no reference counterpart: the reference
// rejects n > 128). An n x n fp32 matrix no longer fits one workgroup's LDS
// with its iterate, so each Newton-Schulz step is two batched GEMMs on the
// matrix cores over fp32 copies in a caller workspace, zero-padded to
// NP = 64*ceil(n/64):  T = P V,  V' = 2V - V T  (the V(PV) order, ping-pong V).
// ---------------------------------------------------------------------------
constexpr int kBgTile = 64;  // padding granule of NP (and the smallest workgroup tile side)
constexpr int kBgK = 16;     // k per LDS stage

constexpr int kBgMaxNP = 256;  // largest padded size of the GEMM path
constexpr int kInitRows = 16;  // rows per workgroup of the init kernel

// P = f32(mat) + 0.01 I, zero-padded to NP x NP, and the signed row sums of P
// in ascending j (one thread per row, as the LDS-resident kernel forms them)
// into rowsum[m][i]; padding rows get -FLT_MAX so that they never give the max.
// alpha = 1.8 / max_i(rowsum)^2 is formed by the kernels that apply it (V0 = alpha P
// never goes to memory). Grid (NP/16 row blocks, matrices), 256 threads: the 16
// rows pass through LDS, so both the matrix reads and the P writes are coalesced.
template <typename T>
__global__ void __launch_bounds__(256)
newton_big_init_kernel(const T* __restrict__ mat, float* __restrict__ P, float* __restrict__ rowsum, int n, int NP) {
  __shared__ float rows[kInitRows][kBgMaxNP + 1];
  const int r0 = blockIdx.x * kInitRows;
  const size_t m = blockIdx.y;
  const T* M = mat + m * n * n;
  float* Pm = P + m * NP * NP;
  for (int e = threadIdx.x; e < kInitRows * NP; e += blockDim.x) {
    const int r = e / NP, j = e - r * NP, i = r0 + r;
    float p = 0.0f;
    if (i < n && j < n) p = to_acc(M[(size_t)i * n + j]) + (i == j ? 0.01f : 0.0f);
    Pm[(size_t)i * NP + j] = p;
    rows[r][j] = p;
  }
  __syncthreads();
  if (threadIdx.x < kInitRows) {
    const int i = r0 + threadIdx.x;
    float sum = -3.4e38f;
    if (i < n) {
      sum = 0.0f;
      for (int j = 0; j < n; ++j) sum += rows[threadIdx.x][j];
    }
    rowsum[m * NP + i] = sum;
  }
}

// alpha = 1.8 / (max of the NP row sums)^2, computed by every thread of a
// 256-thread workgroup (contains one barrier).
__device__ float big_alpha(const float* __restrict__ rs, int NP) {
  __shared__ float red[4];
  float v = -3.4e38f;
  for (int i = threadIdx.x; i < NP; i += 256) v = fmaxf(v, rs[i]);
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  return 1.8f / (mx * mx);
}

// f32 copy of an n x n matrix, zero-padded to NP x NP.
template <typename T>
__global__ void __launch_bounds__(256)
newton_big_pack_kernel(const T* __restrict__ src, float* __restrict__ dst, int n, int NP) {
  const size_t m = blockIdx.y;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= NP * NP) return;
  const int i = e / NP, j = e - i * NP;
  dst[m * NP * NP + e] = (i < n && j < n) ? to_acc(src[m * n * n + (size_t)i * n + j]) : 0.0f;
}

// dst[i][j] = src[i][j] (i, j < n), rounded once to T; SIGN = -1 negates;
// SCALED multiplies by alpha from the row sums (dst = V0 = alpha P).
template <typename T, int SIGN, bool SCALED>
__global__ void __launch_bounds__(256)
newton_big_unpack_kernel(const float* __restrict__ src, T* __restrict__ dst, const float* __restrict__ rowsum,
                         int n, int NP) {
  const size_t m = blockIdx.y;
  float scale = (float)SIGN;
  if constexpr (SCALED) scale = big_alpha(rowsum + m * NP, NP);
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n * n) return;
  const int i = e / n, j = e - i * n;
  dst[m * n * n + e] = from_acc<T>(scale * src[m * NP * NP + (size_t)i * NP + j]);
}

// Batched D = f(op(X) op(Y)) over NP x NP fp32 matrices (row-major, matrix
// stride NP*NP), op = transpose when TX / TY. MODE 0: D = XY; 1: D = 2E - XY;
// 2: D = -XY. SCALED multiplies the result by the matrix's alpha (from the
// init kernel's row sums). One TM x TN output tile per 4-wave workgroup (2 x 2
// waves of TM/2 x TN/2). Grid: (NP/TM)(NP/TN) tiles x matrices, flattened so that
// all tiles of a matrix share blockIdx.x mod 8 (workgroups are dealt to the 8
// XCDs round robin, so a matrix's tiles share one L2). Both operands are staged
// k-major in LDS ([k][TM], [k][TN]) with the columns of row k XOR-swizzled by
// 16 * ((k + k/4) mod 4): the 4 k rows of an MFMA operand read then fall on 4
// different 16-bank groups, and so do the 4 rows of a transposing store
// (conflict-free both ways, no padding). Two LDS stages, one
// barrier per stage; global loads run two stages ahead of the MFMAs through
// two register sets, so each load has two stages of MFMA work to land in.
template <int TM, int TN, bool TX, bool TY, int MODE, bool SCALED>
__global__ void __launch_bounds__(256)
newton_big_gemm_kernel(const float* __restrict__ X, const float* __restrict__ Y, const float* __restrict__ E,
                       const float* __restrict__ rowsum, float* __restrict__ D, int NP, int K, int nMat) {
  static_assert(TM % 64 == 0 && TN % 64 == 0, "tile sides are multiples of 64");
  constexpr int RT = TM / 32, CT = TN / 32;     // 16x16 accumulators per wave (2 x 2 waves)
  constexpr int LA = TM / 64, LB = TN / 64;     // float4 staging loads per thread per operand
  __shared__ __align__(16) float As[2][kBgK][TM];
  __shared__ __align__(16) float Bs[2][kBgK][TN];
  auto sw = [](int k) { return 16 * ((k + (k >> 2)) & 3); };
  const int ntm = NP / TM, ntn = NP / TN;
  const int tiles = ntm * ntn;
  // Inverse of the flattening: id = (m % 8) + 8 * (t + tiles * (m / 8)).
  const int id = blockIdx.x;
  const int lo = id & 7, hi = id >> 3;
  const int t = hi % tiles, mg = hi / tiles;
  const int m = mg * 8 + lo;
  if (m >= nMat) return;  // whole workgroup
  const int ti = t / ntn, tj = t - ti * ntn;
  const size_t mo = (size_t)m * NP * NP;
  const float* Xm = X + mo;
  const float* Ym = Y + mo;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wr = (wave >> 1) * (TM / 2), wc = (wave & 1) * (TN / 2);
  float alpha = 1.0f;
  if constexpr (SCALED) alpha = big_alpha(rowsum + (size_t)m * NP, NP);

  // Global -> register staging of one k stage: TM x 16 of op(X) and 16 x TN of op(Y).
  auto load = [&](float4 (&ra)[LA], float4 (&rb)[LB], int k0) {
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      if (TX) {  // A[i][k] = X[k][i]: 16 rows of X, TM contiguous columns
        const int e = tid + 256 * u, k = e / (TM / 4), iq = (e % (TM / 4)) * 4;
        ra[u] = *reinterpret_cast<const float4*>(Xm + (size_t)(k0 + k) * NP + ti * TM + iq);
      } else {   // A[i][k] = X[i][k]: TM rows of X, 16 contiguous columns
        const int i = (tid >> 2) + 64 * u, kq = (tid & 3) * 4;
        ra[u] = *reinterpret_cast<const float4*>(Xm + (size_t)(ti * TM + i) * NP + k0 + kq);
      }
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      if (TY) {  // B[k][j] = Y[j][k]
        const int j = (tid >> 2) + 64 * u, kq = (tid & 3) * 4;
        rb[u] = *reinterpret_cast<const float4*>(Ym + (size_t)(tj * TN + j) * NP + k0 + kq);
      } else {   // B[k][j] = Y[k][j]
        const int e = tid + 256 * u, k = e / (TN / 4), jq = (e % (TN / 4)) * 4;
        rb[u] = *reinterpret_cast<const float4*>(Ym + (size_t)(k0 + k) * NP + tj * TN + jq);
      }
    }
  };
  auto store = [&](const float4 (&ra)[LA], const float4 (&rb)[LB], int b) {
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      if (TX) {
        const int e = tid + 256 * u, k = e / (TM / 4), iq = (e % (TM / 4)) * 4;
        *reinterpret_cast<float4*>(&As[b][k][iq ^ sw(k)]) = ra[u];
      } else {
        const int i = (tid >> 2) + 64 * u, kq = (tid & 3) * 4;
        As[b][kq + 0][i ^ sw(kq + 0)] = ra[u].x; As[b][kq + 1][i ^ sw(kq + 1)] = ra[u].y;
        As[b][kq + 2][i ^ sw(kq + 2)] = ra[u].z; As[b][kq + 3][i ^ sw(kq + 3)] = ra[u].w;
      }
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      if (TY) {
        const int j = (tid >> 2) + 64 * u, kq = (tid & 3) * 4;
        Bs[b][kq + 0][j ^ sw(kq + 0)] = rb[u].x; Bs[b][kq + 1][j ^ sw(kq + 1)] = rb[u].y;
        Bs[b][kq + 2][j ^ sw(kq + 2)] = rb[u].z; Bs[b][kq + 3][j ^ sw(kq + 3)] = rb[u].w;
      } else {
        const int e = tid + 256 * u, k = e / (TN / 4), jq = (e % (TN / 4)) * 4;
        *reinterpret_cast<float4*>(&Bs[b][k][jq ^ sw(k)]) = rb[u];
      }
    }
  };

  v4f acc[RT][CT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[r][c] = v4f{0.f, 0.f, 0.f, 0.f};
  const int li = lane & 15, lk = lane >> 4;
  auto compute = [&](int b) {
#pragma unroll
    for (int ks = 0; ks < kBgK; ks += 4) {
      float a[RT], bb[CT];
#pragma unroll
      for (int r = 0; r < RT; ++r) a[r] = As[b][ks + lk][(wr + 16 * r + li) ^ sw(ks + lk)];
#pragma unroll
      for (int c = 0; c < CT; ++c) bb[c] = Bs[b][ks + lk][(wc + 16 * c + li) ^ sw(ks + lk)];
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], bb[c], acc[r][c], 0, 0, 0);
    }
  };

  // The products run over k < K = 32 * ceil(n / 32) <= NP (columns and rows from n
  // on are zero padding and contribute nothing). nk = K / 16 is even: stages go in
  // pairs, even stages through LDS buffer 0 and register set 0, odd ones through
  // buffer 1 and set 1.
  const int nk = K / kBgK;
  float4 ra0[LA], rb0[LB], ra1[LA], rb1[LB];
  load(ra0, rb0, 0);
  load(ra1, rb1, kBgK);
  store(ra0, rb0, 0);
  __syncthreads();
  for (int kc = 0; kc < nk; kc += 2) {
    if (kc + 2 < nk) load(ra0, rb0, (kc + 2) * kBgK);
    compute(0);
    store(ra1, rb1, 1);
    __syncthreads();
    if (kc + 3 < nk) load(ra1, rb1, (kc + 3) * kBgK);
    compute(1);
    if (kc + 2 < nk) store(ra0, rb0, 0);
    __syncthreads();
  }

  float* Dm = D + mo;
  const float* Em = MODE == 1 ? E + mo : nullptr;
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = ti * TM + wr + 16 * r + 4 * lk + q;
        const int j = tj * TN + wc + 16 * c + li;
        const size_t o = (size_t)i * NP + j;
        float v = acc[r][c][q];
        if (MODE == 1) v = 2.0f * Em[o] - v;
        if (MODE == 2) v = -v;
        if (SCALED) v = alpha * v;
        Dm[o] = v;
      }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {

constexpr int kMaxLdsN = 128;  // LDS-resident kernels (the reference's envelope)
constexpr int kMaxN = 256;     // fp32 / fp16 / bf16 through the batched GEMM path
constexpr int kF64MaxN = 96;   // two fp64 96x97 buffers fill most of gfx950's 160 KB LDS

int big_np(int64_t n) { return (int)((n + kBgTile - 1) / kBgTile) * kBgTile; }

// fp32 NP x NP buffers per matrix the GEMM path uses: P, V, V', T (forward),
// V, G, S (backward); then NP row sums per matrix (forward).
constexpr int kBigBuffers = 4;
size_t big_workspace_bytes(int64_t bh, int64_t n) {
  const size_t np = (size_t)big_np(n);
  return (size_t)bh * (kBigBuffers * np * np + np) * 4;
}

unsigned big_gemm_blocks(int np, int tm, int tn, int64_t bh) {
  const int tiles = (np / tm) * (np / tn);
  return (unsigned)(8 * tiles * ((bh + 7) / 8));  // matrices rounded up to a multiple of 8
}

// fp32 matrices with n == NP (and 16-byte aligned) already have the padded
// layout: the GEMMs then read the caller's tensors and write the result in place
// of the workspace copies (no pack / unpack pass).
template <typename T>
bool big_direct(int n, int np, std::initializer_list<const void*> ptrs) {
  if (!std::is_same<T, float>::value || n != np) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15) return false;
  return true;
}

// Tiles: 128 x 64 for the forward's products (neither operand transposed) when
// 128 divides NP, measured 10 % faster than 64 x 64 at 128 x 256^2; 64 x 64
// otherwise (the backward's transposed products measured 15 % slower at 128 x 64).
template <int MODE, bool SCALED, bool TX = false, bool TY = false>
void big_gemm(const float* X, const float* Y, const float* E, const float* rowsum, float* D, int np, int n,
              int64_t bh, hipStream_t st) {
  const int K = std::min(np, (n + 31) / 32 * 32);
  if (!TX && !TY && np % 128 == 0)
    hipLaunchKernelGGL((newton_big_gemm_kernel<128, 64, TX, TY, MODE, SCALED>),
                       dim3(big_gemm_blocks(np, 128, 64, bh)), dim3(256), 0, st, X, Y, E, rowsum, D, np, K, (int)bh);
  else
    hipLaunchKernelGGL((newton_big_gemm_kernel<64, 64, TX, TY, MODE, SCALED>),
                       dim3(big_gemm_blocks(np, 64, 64, bh)), dim3(256), 0, st, X, Y, E, rowsum, D, np, K, (int)bh);
}

template <typename T>
int big_fwd(const T* mat, T* out, int64_t bh, int n, int iters, float* ws, hipStream_t st) {
  const int np = big_np(n);
  const size_t mat_elems = (size_t)np * np;
  float* P = ws;
  float* Va = ws + (size_t)bh * mat_elems;
  float* Vb = ws + 2 * (size_t)bh * mat_elems;
  float* Tm = ws + 3 * (size_t)bh * mat_elems;
  float* rs = ws + 4 * (size_t)bh * mat_elems;
  const bool direct = big_direct<T>(n, np, {out});
  hipLaunchKernelGGL(newton_big_init_kernel<T>, dim3((unsigned)(np / kInitRows), (unsigned)bh), dim3(256), 0, st,
                     mat, P, rs, n, np);
  int s = check_launch("newton forward init");
  if (s) return s;
  dim3 ug(ceil_div(n * n, 256), (unsigned)bh);
  if (iters == 0) {  // V0 = alpha P
    hipLaunchKernelGGL((newton_big_unpack_kernel<T, 1, true>), ug, dim3(256), 0, st, P, out, rs, n, np);
    return check_launch("newton forward output");
  }
  for (int it = 0; it < iters; ++it) {
    float* dst = (direct && it == iters - 1) ? reinterpret_cast<float*>(out) : Vb;
    if (it == 0) {  // V0 = alpha P:  T = alpha (P P),  V1 = alpha (2P - P T)
      big_gemm<0, true>(P, P, nullptr, rs, Tm, np, n, bh, st);
      big_gemm<1, true>(P, Tm, P, rs, dst, np, n, bh, st);
    } else {        // T = P V,  V' = 2V - V T
      big_gemm<0, false>(P, Va, nullptr, nullptr, Tm, np, n, bh, st);
      big_gemm<1, false>(Va, Tm, Va, nullptr, dst, np, n, bh, st);
    }
    if ((s = check_launch("newton forward step"))) return s;
    std::swap(Va, Vb);
  }
  if (direct) return LFAMD_OK;
  hipLaunchKernelGGL((newton_big_unpack_kernel<T, 1, false>), ug, dim3(256), 0, st, Va, out,
                     static_cast<const float*>(nullptr), n, np);
  return check_launch("newton forward output");
}

template <typename T>
int big_bwd(const T* g, const T* inv, T* out, int64_t bh, int n, float* ws, hipStream_t st) {
  const int np = big_np(n);
  const size_t mat_elems = (size_t)np * np;
  float* S = ws + 2 * (size_t)bh * mat_elems;
  // The second product reads V while it writes out: direct only when they do not overlap.
  const size_t bytes = (size_t)bh * n * n * sizeof(T);
  const uintptr_t o = reinterpret_cast<uintptr_t>(out), v = reinterpret_cast<uintptr_t>(inv);
  const bool apart = o + bytes <= v || v + bytes <= o;
  if (apart && big_direct<T>(n, np, {g, inv, out})) {  // S = V^T G,  out = -S V^T
    const float* Vf = reinterpret_cast<const float*>(inv);
    big_gemm<0, false, true, false>(Vf, reinterpret_cast<const float*>(g), nullptr, nullptr, S, np, n, bh, st);
    big_gemm<2, false, false, true>(S, Vf, nullptr, nullptr, reinterpret_cast<float*>(out), np, n, bh, st);
    return check_launch("newton backward products");
  }
  float* Vf = ws;
  float* Gf = ws + (size_t)bh * mat_elems;
  dim3 pg(ceil_div(np * np, 256), (unsigned)bh);
  hipLaunchKernelGGL(newton_big_pack_kernel<T>, pg, dim3(256), 0, st, inv, Vf, n, np);
  hipLaunchKernelGGL(newton_big_pack_kernel<T>, pg, dim3(256), 0, st, g, Gf, n, np);
  big_gemm<0, false, true, false>(Vf, Gf, nullptr, nullptr, S, np, n, bh, st);  // S = V^T G
  big_gemm<2, false, false, true>(S, Vf, nullptr, nullptr, Gf, np, n, bh, st);  // -S V^T (into G's slot)
  int s = check_launch("newton backward products");
  if (s) return s;
  dim3 ug(ceil_div(n * n, 256), (unsigned)bh);
  hipLaunchKernelGGL((newton_big_unpack_kernel<T, 1, false>), ug, dim3(256), 0, st, Gf, out,
                     static_cast<const float*>(nullptr), n, np);
  return check_launch("newton backward output");
}

int bucket(int64_t n) { return (int)((n + 15) / 16) * 16; }

// Two NP x (NP+4) fp32 matrices in either order (P, then T or W; and V).
template <int NP> constexpr size_t fwd_lds() { return 2 * (size_t)NsLayout<NP>::ELEMS * 4; }

template <typename Kern>
int set_lds(Kern k, size_t bytes) {
  if (bytes > (size_t)max_lds_bytes())
    return fail(LFAMD_ERR_UNSUPPORTED, "NewtonInverse needs %zu bytes of LDS, device allows %d", bytes, max_lds_bytes());
  return set_dyn_lds(reinterpret_cast<const void*>(k), bytes, "NewtonInverse");
}

// Waves per 16-row strip: the most (up to 4) that split the strip's tiles evenly
// within 16 waves per workgroup.
template <int NP> constexpr int pick_wpr() {
  constexpr int nt = NP / 16;
  return (nt % 4 == 0 && nt * 4 <= 16) ? 4 : (nt % 2 == 0 && nt * 2 <= 16) ? 2 : 1;
}

// fp32 matrices with n = 16 m + 1 (e.g. 49 = 7 x 7 landmarks) take the
// instantiations whose last k block runs one MFMA step of four.
template <typename T, int NP> constexpr bool has_kl1() { return std::is_same<T, float>::value && NP >= 32 && NP < 128; }

template <typename T, int NP, int WPR>
int fwd_np_w(const T* m, T* o, int64_t bh, int n, int iters, hipStream_t st) {
  // fp32 n = 49: the symmetric iteration when P is symmetric (the kernel checks; else the general one).
  if constexpr (std::is_same<T, float>::value && NP == 64) {
    if (n == NP - 15) {
      auto k = newton_fwd_sym_kernel<WPR * 4>;
      int s = set_lds(k, fwd_lds<NP>());
      if (s) return s;
      hipLaunchKernelGGL(k, dim3((unsigned)bh), dim3(NP * 4 * WPR), fwd_lds<NP>(), st, m, o, n, iters);
      return check_launch("newton forward");
    }
  }
  // The reference's association order per bucket: V(PV) below 128, (VP)V at 128.
  if constexpr (has_kl1<T, NP>()) {
    if (n == NP - 15) {
      auto k = newton_fwd_kernel<T, NP, true, WPR, 1>;
      int s = set_lds(k, fwd_lds<NP>());
      if (s) return s;
      hipLaunchKernelGGL(k, dim3((unsigned)bh), dim3(NP * 4 * WPR), fwd_lds<NP>(), st, m, o, n, iters);
      return check_launch("newton forward");
    }
  }
  if (NP < 128) {
    auto k = newton_fwd_kernel<T, NP, true, WPR>;
    int s = set_lds(k, fwd_lds<NP>());
    if (s) return s;
    hipLaunchKernelGGL(k, dim3((unsigned)bh), dim3(NP * 4 * WPR), fwd_lds<NP>(), st, m, o, n, iters);
  } else {
    auto k = newton_fwd_kernel<T, NP, false, WPR>;
    int s = set_lds(k, fwd_lds<NP>());
    if (s) return s;
    hipLaunchKernelGGL(k, dim3((unsigned)bh), dim3(NP * 4 * WPR), fwd_lds<NP>(), st, m, o, n, iters);
  }
  return check_launch("newton forward");
}

// 64 x 64 fp32 matrices, 2 to 8 per CU: the persistent issue-ordered kernel (1024 x 64^2:
// 14.25 against 14.6 us; 600 and 1000 matrices 4.6-6 % faster; at 16 per CU, 44.8 against
// 44.1 us, the one-matrix-per-workgroup kernel stays).
template <typename T, int NP>
bool use_pipe(int64_t bh, int n) {
  return std::is_same<T, float>::value && NP == 64 && n == NP && bh > (int64_t)num_cus() &&
         bh <= 8 * (int64_t)num_cus();
}

template <typename T, int NP>
int bwd_np_pipe(const T* g, const T* v, T* o, int64_t bh, hipStream_t st) {
  auto k = newton_bwd_pipe_kernel<T, NP>;
  int s = set_lds(k, pipe_lds<NP>());
  if (s) return s;
  const int64_t cus = num_cus();
  const int per = (int)((bh + cus - 1) / cus);
  const int64_t grid = (bh + per - 1) / per;
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(1024), pipe_lds<NP>(), st, g, v, o, bh, per);
  return check_launch("newton backward");
}

template <typename T, int NP, int WPR>
int bwd_np_w(const T* g, const T* v, T* o, int64_t bh, int n, hipStream_t st) {
  if constexpr (std::is_same<T, float>::value && NP == 64)
    if (use_pipe<T, NP>(bh, n)) return bwd_np_pipe<T, NP>(g, v, o, bh, st);
  auto k = newton_bwd_kernel<T, NP, WPR>;
  if constexpr (has_kl1<T, NP>())
    if (n == NP - 15) k = newton_bwd_kernel<T, NP, WPR, 1>;
  const size_t lds = 2 * (size_t)NsLayout<NP>::ELEMS * 4;
  int s = set_lds(k, lds);
  if (s) return s;
  hipLaunchKernelGGL(k, dim3((unsigned)bh), dim3(NP * 4 * WPR), lds, st, g, v, o, n);
  return check_launch("newton backward");
}

// Four waves per strip only while there are fewer than two matrices per CU
// (latency-bound); with more, two per strip keep more matrices resident.
template <int NP> bool use_wide(int64_t bh) { return pick_wpr<NP>() == 4 && bh < 2 * (int64_t)num_cus(); }
template <int NP> constexpr int narrow_wpr() { return pick_wpr<NP>() == 4 ? 2 : pick_wpr<NP>(); }

template <typename T, int NP>
int fwd_np(const T* m, T* o, int64_t bh, int n, int iters, hipStream_t st) {
  if (use_wide<NP>(bh)) return fwd_np_w<T, NP, pick_wpr<NP>()>(m, o, bh, n, iters, st);
  return fwd_np_w<T, NP, narrow_wpr<NP>()>(m, o, bh, n, iters, st);
}

// The backward's two products per matrix are latency-bound at any matrix count
// (four waves per strip: 14.5 against 15.2 us at 1024 x 64^2, where the forward's
// twelve iterations prefer two per strip).
template <typename T, int NP>
int bwd_np(const T* g, const T* v, T* o, int64_t bh, int n, hipStream_t st) {
  if (pick_wpr<NP>() == 4) return bwd_np_w<T, NP, pick_wpr<NP>()>(g, v, o, bh, n, st);
  return bwd_np_w<T, NP, narrow_wpr<NP>()>(g, v, o, bh, n, st);
}

template <typename T>
int fwd_t(const void* m, void* o, int64_t bh, int n, int iters, hipStream_t st) {
  auto M = static_cast<const T*>(m);
  auto O = static_cast<T*>(o);
  switch (bucket(n)) {
    case 16: return fwd_np<T, 16>(M, O, bh, n, iters, st);
    case 32: return fwd_np<T, 32>(M, O, bh, n, iters, st);
    case 48: return fwd_np<T, 48>(M, O, bh, n, iters, st);
    case 64: return fwd_np<T, 64>(M, O, bh, n, iters, st);
    case 80: return fwd_np<T, 80>(M, O, bh, n, iters, st);
    case 96: return fwd_np<T, 96>(M, O, bh, n, iters, st);
    case 112: return fwd_np<T, 112>(M, O, bh, n, iters, st);
    default: return fwd_np<T, 128>(M, O, bh, n, iters, st);
  }
}

template <typename T>
int bwd_t(const void* g, const void* v, void* o, int64_t bh, int n, hipStream_t st) {
  auto G = static_cast<const T*>(g);
  auto V = static_cast<const T*>(v);
  auto O = static_cast<T*>(o);
  switch (bucket(n)) {
    case 16: return bwd_np<T, 16>(G, V, O, bh, n, st);
    case 32: return bwd_np<T, 32>(G, V, O, bh, n, st);
    case 48: return bwd_np<T, 48>(G, V, O, bh, n, st);
    case 64: return bwd_np<T, 64>(G, V, O, bh, n, st);
    case 80: return bwd_np<T, 80>(G, V, O, bh, n, st);
    case 96: return bwd_np<T, 96>(G, V, O, bh, n, st);
    case 112: return bwd_np<T, 112>(G, V, O, bh, n, st);
    default: return bwd_np<T, 128>(G, V, O, bh, n, st);
  }
}

int check_common(int dtype, int64_t bh, int64_t n, const char* who) {
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "%s: unsupported dtype %d", who, dtype);
  if (bh < 0 || n < 0) return fail(LFAMD_ERR_ARG, "%s: negative size", who);
  if (n < 1 || n > kMaxN)
    return fail(LFAMD_ERR_UNSUPPORTED, "NewtonInverse: N=%lld is not supported on this device (insufficient smem or out of range)", (long long)n);
  if (bh > INT32_MAX / 64) return fail(LFAMD_ERR_UNSUPPORTED, "%s: too many matrices", who);
  if (dtype == LFAMD_F64 && n > kF64MaxN)
    return fail(LFAMD_ERR_UNSUPPORTED, "NewtonInverse: fp64 N=%lld needs more LDS than this device allows (fp64 limit %d)", (long long)n, kF64MaxN);
  return LFAMD_OK;
}

size_t workspace_for(int dtype, int64_t bh, int64_t n) {
  if (dtype == LFAMD_F64 || n <= kMaxLdsN || n > kMaxN || bh <= 0) return 0;
  return big_workspace_bytes(bh, n);
}

int check_workspace(int dtype, int64_t bh, int64_t n, const void* ws, size_t bytes, const char* who) {
  const size_t need = workspace_for(dtype, bh, n);
  if (need && (!ws || bytes < need))
    return fail(LFAMD_ERR_ARG, "%s: N=%lld needs a workspace of %zu bytes, %zu given", who, (long long)n, need,
                ws ? bytes : (size_t)0);
  if (need && (reinterpret_cast<uintptr_t>(ws) & 15) != 0)
    return fail(LFAMD_ERR_ARG, "%s: workspace must be 16-byte aligned", who);
  return LFAMD_OK;
}

}  // namespace
}  // namespace lfamd

using namespace lfamd;

// The attention layer's fused landmark kernels (48 < m <= 64: the 64 bucket).
constexpr size_t kMulBwdLds = 4 * (size_t)NsLayout<64>::ELEMS * 4;

template <int KL>
int launch_fwd_tall(int v_dtype, const float* kmm, float* inv, int64_t bh, int m, int iters, const float* kkm,
                    const void* v, float* part, int64_t rows, int d, int per, hipStream_t st) {
  const size_t lds = std::max<size_t>(fwd_lds<64>(), (size_t)tall_lds_floats() * 4);
  const dim3 grid((unsigned)(bh * (1 + per))), block(64 * 8);
  auto go = [&](auto k, const auto* B) -> int {
    if (int s = check_fit(reinterpret_cast<const void*>(k), 64 * 8, lds, "attention landmarks forward")) return s;
    if (int s = set_lds(k, lds)) return s;
    hipLaunchKernelGGL(k, grid, block, lds, st, kmm, inv, m, iters, (int)bh, kkm, B, part, (int)rows, m, d, per);
    return check_launch("attention landmarks forward");
  };
  switch (v_dtype) {
    case LFAMD_F32: return go(newton_fwd_tall_kernel<64, KL, float>, static_cast<const float*>(v));
    case LFAMD_F16: return go(newton_fwd_tall_kernel<64, KL, f16s>, static_cast<const f16s*>(v));
    default: return go(newton_fwd_tall_kernel<64, KL, bf16s>, static_cast<const bf16s*>(v));
  }
}

template <int KL>
int launch_kv_w(const float* inv, const float* part, int per, int64_t bh, int m, int d, float* kv, float* w,
                hipStream_t st) {
  auto k = landmark_kv_w_kernel<64, 4, KL>;
  if (int s = check_fit(reinterpret_cast<const void*>(k), 64 * 16, fwd_lds<64>(), "attention landmarks forward")) return s;
  if (int s = set_lds(k, fwd_lds<64>())) return s;
  hipLaunchKernelGGL(k, dim3((unsigned)bh), dim3(64 * 16), fwd_lds<64>(), st, inv, part, per, m, d, kv, w);
  return check_launch("attention landmarks forward (kv, W)");
}

template <int KL>
int launch_bwd_mul(const float* part, int per, const float* kv, const float* inv, float* dkv, float* dkmm, int64_t bh,
                   int m, int d, hipStream_t st) {
  auto k = newton_bwd_mul_kernel<64, 4, KL>;
  if (int s = check_fit(reinterpret_cast<const void*>(k), 64 * 16, kMulBwdLds, "attention landmarks backward")) return s;
  if (int s = set_lds(k, kMulBwdLds)) return s;
  hipLaunchKernelGGL(k, dim3((unsigned)bh), dim3(64 * 16), kMulBwdLds, st, part, per, kv, inv, dkv, dkmm, m, d);
  return check_launch("attention landmarks backward");
}

// Launch 1 of the landmark backward after the tall product (newton_bwd_mix_kernel);
// LFAMD_ERR_UNSUPPORTED (nothing launched) where the row kernel does not take g.
template <int KL>
int launch_bwd_mix(int dtype, const float* part, int per, const float* kv, const float* inv, float* dkv, float* dkmm,
                   int64_t bh, int m, int d, const void* g, const float* w, float* dkqm, int64_t rows,
                   hipStream_t st) {
  const int64_t es = dtype == LFAMD_F32 ? 4 : 2;
  const bool aligned = (reinterpret_cast<uintptr_t>(g) & 15) == 0;
  const bool direct = aligned && d == kMixPMax, rows16 = aligned && (rows * d * es) % 16 == 0;
  if (!(direct || rows16) || rows > INT32_MAX / 2)
    return fail(LFAMD_ERR_UNSUPPORTED, "attention landmarks backward: g not 16-byte aligned by rows");
  const int64_t groups = (rows + kMixGroup - 1) / kMixGroup, cus = num_cus();
  const int permix = (int)std::max<int64_t>(1, std::min<int64_t>((groups + 15) / 16, (cus - bh + bh - 1) / bh));
  const dim3 grid((unsigned)(bh * (1 + permix))), block(1024);
  auto go = [&](auto k, const auto* G) -> int {
    if (int s = check_fit(reinterpret_cast<const void*>(k), 1024, kMulBwdLds, "attention landmarks backward")) return s;
    if (int s = set_lds(k, kMulBwdLds)) return s;
    hipLaunchKernelGGL(k, grid, block, kMulBwdLds, st, part, per, kv, inv, dkv, dkmm, m, d, (int)bh, G, w, dkqm,
                       (int)rows, permix);
    return check_launch("attention landmarks backward");
  };
#define LFAMD_BWDMIX(TA)                                                                          \
  return direct ? go(newton_bwd_mix_kernel<KL, TA, true>, static_cast<const TA*>(g))             \
                : go(newton_bwd_mix_kernel<KL, TA, false>, static_cast<const TA*>(g))
  switch (dtype) {
    case LFAMD_F32: LFAMD_BWDMIX(float);
    case LFAMD_F16: LFAMD_BWDMIX(f16s);
    default: LFAMD_BWDMIX(bf16s);
  }
#undef LFAMD_BWDMIX
}

int check_landmarks(int dt, int64_t slices, int64_t rows, int m, int d, const char* who) {
  if (dt != LFAMD_F32 && dt != LFAMD_F16 && dt != LFAMD_BF16) return fail(LFAMD_ERR_DTYPE, "%s: unsupported dtype %d", who, dt);
  if (slices < 0 || slices > 65535 || rows < 1 || rows > (int64_t)1 << 30 || m < 1 || d < 1)
    return fail(LFAMD_ERR_ARG, "%s: bad sizes (slices=%lld rows=%lld m=%d d=%d)", who, (long long)slices,
                (long long)rows, m, d);
  if (m <= 48 || m > 64 || d > 64)
    return fail(LFAMD_ERR_UNSUPPORTED, "%s: landmark count %d or width %d outside (48, 64] / 64", who, m, d);
  return LFAMD_OK;
}

extern "C" {

int lfamd_attention_landmarks_forward(const float* kmm, const float* kkm, int v_dtype, const void* v, float* inv,
                                      float* kv, float* w, int64_t slices, int64_t rows, int m, int d, int iters,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = check_landmarks(v_dtype, slices, rows, m, d, "attention landmarks forward")) return s;
  if (slices == 0) return ok();
  if (!kmm || !kkm || !v || !inv || !kv || !w || !workspace)
    return fail(LFAMD_ERR_ARG, "attention landmarks forward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int per = 0;
  float* part = static_cast<float*>(workspace);
  if (iters < 0) iters = 0;
  if (int s = tall_t_check(v_dtype, kkm, v, workspace_bytes, slices, rows, m, d, &per)) return s;
  if (int s = (m == 49 ? launch_fwd_tall<1>(v_dtype, kmm, inv, slices, m, iters, kkm, v, part, rows, d, per, st)
                       : launch_fwd_tall<4>(v_dtype, kmm, inv, slices, m, iters, kkm, v, part, rows, d, per, st)))
    return s;
  return m == 49 ? launch_kv_w<1>(inv, part, per, slices, m, d, kv, w, st)
                 : launch_kv_w<4>(inv, part, per, slices, m, d, kv, w, st);
}

int lfamd_attention_landmarks_backward(const float* kqm, int dtype, const void* g, const void* v, const float* kkm,
                                       const float* w, const float* kv, const float* inv, float* dkqm, float* dkkm,
                                       void* dv, float* dkv, float* dkmm, int64_t slices, int64_t rows, int m, int d,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = check_landmarks(dtype, slices, rows, m, d, "attention landmarks backward")) return s;
  if (slices == 0) return ok();
  if (!kqm || !g || !v || !kkm || !w || !kv || !inv || !dkqm || !dkkm || !dv || !dkv || !dkmm || !workspace)
    return fail(LFAMD_ERR_ARG, "attention landmarks backward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int per = 0;
  float* part = static_cast<float*>(workspace);
  if (int s = tall_t_partials(dtype, kqm, g, part, workspace_bytes, slices, rows, m, d, st, &per)) return s;
  const int64_t md = (int64_t)m * d;
  const void* as[3] = {g, v, kkm};
  const float* bs[3] = {w, dkv, dkv};
  void* cs[3] = {dkqm, dkkm, dv};
  const int P[2] = {d, m}, Q[2] = {m, d};
  const int64_t sq[2] = {d, 1}, sp[2] = {1, d}, bstr[2] = {md, md};
  // dK_qm = g w^T beside the inverse's products, then dK_km = v dkv^T and dv = K_km dkv in one launch.
  int s = m == 49 ? launch_bwd_mix<1>(dtype, part, per, kv, inv, dkv, dkmm, slices, m, d, g, w, dkqm, rows, st)
                  : launch_bwd_mix<4>(dtype, part, per, kv, inv, dkv, dkmm, slices, m, d, g, w, dkqm, rows, st);
  if (s == LFAMD_OK) {
    s = mix_rows_trio(dtype, as, bs, cs, slices, rows, P, Q, sq, sp, bstr, st, 1);
    if (s != LFAMD_ERR_UNSUPPORTED) return s;
    if ((s = lfamd_mix_rows(dtype, v, dkv, LFAMD_F32, dkkm, slices, rows, d, m, d, 1, md, st))) return s;
    return lfamd_mix_rows(LFAMD_F32, kkm, dkv, dtype, dv, slices, rows, m, d, 1, d, md, st);
  }
  if (s != LFAMD_ERR_UNSUPPORTED) return s;
  // g the row kernel does not take as a whole: the inverse's products, then the row products
  // one call each.
  if ((s = (m == 49 ? launch_bwd_mul<1>(part, per, kv, inv, dkv, dkmm, slices, m, d, st)
                    : launch_bwd_mul<4>(part, per, kv, inv, dkv, dkmm, slices, m, d, st))))
    return s;
  s = mix_rows_trio(dtype, as, bs, cs, slices, rows, P, Q, sq, sp, bstr, st);
  if (s != LFAMD_ERR_UNSUPPORTED) return s;
  if ((s = lfamd_mix_rows(dtype, g, w, LFAMD_F32, dkqm, slices, rows, d, m, d, 1, md, st))) return s;
  if ((s = lfamd_mix_rows(dtype, v, dkv, LFAMD_F32, dkkm, slices, rows, d, m, d, 1, md, st))) return s;
  return lfamd_mix_rows(LFAMD_F32, kkm, dkv, dtype, dv, slices, rows, m, d, 1, d, md, st);
}

int lfamd_newton_is_supported(int64_t n) { return n >= 1 && n <= kMaxN ? 1 : 0; }

size_t lfamd_newton_workspace_size(int dtype, int64_t batch_heads, int64_t n) {
  if (!valid_dtype(dtype) || n < 1 || n > kMaxN) return 0;
  return workspace_for(dtype, batch_heads, n);
}

int lfamd_newton_forward(int dtype, const void* mat, void* output, int64_t batch_heads,
                         int64_t n, int iters, void* workspace, size_t workspace_bytes, void* stream) {
  int s = check_common(dtype, batch_heads, n, "newton forward");
  if (s) return s;
  if (batch_heads == 0) return ok();
  if (!mat || !output) return fail(LFAMD_ERR_ARG, "newton forward: null pointer");
  if ((s = check_workspace(dtype, batch_heads, n, workspace, workspace_bytes, "newton forward"))) return s;
  if (iters < 0) iters = 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n > kMaxLdsN) {
    float* ws = static_cast<float*>(workspace);
    switch (dtype) {
      case LFAMD_F32: return big_fwd<float>(static_cast<const float*>(mat), static_cast<float*>(output), batch_heads, (int)n, iters, ws, st);
      case LFAMD_F16: return big_fwd<f16s>(static_cast<const f16s*>(mat), static_cast<f16s*>(output), batch_heads, (int)n, iters, ws, st);
      default: return big_fwd<bf16s>(static_cast<const bf16s*>(mat), static_cast<bf16s*>(output), batch_heads, (int)n, iters, ws, st);
    }
  }
  switch (dtype) {
    case LFAMD_F32: return fwd_t<float>(mat, output, batch_heads, (int)n, iters, st);
    case LFAMD_F16: return fwd_t<f16s>(mat, output, batch_heads, (int)n, iters, st);
    case LFAMD_BF16: return fwd_t<bf16s>(mat, output, batch_heads, (int)n, iters, st);
    default: {
      const int np = bucket(n);
      const size_t lds = 2 * (size_t)np * (np + 1) * 8;
      if ((s = set_lds(newton_fwd_f64_kernel, lds))) return s;
      hipLaunchKernelGGL(newton_fwd_f64_kernel, dim3((unsigned)batch_heads), dim3(kF64Threads), lds, st,
                         static_cast<const double*>(mat), static_cast<double*>(output), (int)n, np, iters);
      return check_launch("newton forward fp64");
    }
  }
}

int lfamd_newton_backward(int dtype, const void* grad_output, const void* inverse,
                          void* grad_mat, int64_t batch_heads, int64_t n, void* workspace,
                          size_t workspace_bytes, void* stream) {
  int s = check_common(dtype, batch_heads, n, "newton backward");
  if (s) return s;
  if (batch_heads == 0) return ok();
  if (!grad_output || !inverse || !grad_mat) return fail(LFAMD_ERR_ARG, "newton backward: null pointer");
  if ((s = check_workspace(dtype, batch_heads, n, workspace, workspace_bytes, "newton backward"))) return s;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n > kMaxLdsN) {
    float* ws = static_cast<float*>(workspace);
    switch (dtype) {
      case LFAMD_F32: return big_bwd<float>(static_cast<const float*>(grad_output), static_cast<const float*>(inverse), static_cast<float*>(grad_mat), batch_heads, (int)n, ws, st);
      case LFAMD_F16: return big_bwd<f16s>(static_cast<const f16s*>(grad_output), static_cast<const f16s*>(inverse), static_cast<f16s*>(grad_mat), batch_heads, (int)n, ws, st);
      default: return big_bwd<bf16s>(static_cast<const bf16s*>(grad_output), static_cast<const bf16s*>(inverse), static_cast<bf16s*>(grad_mat), batch_heads, (int)n, ws, st);
    }
  }
  switch (dtype) {
    case LFAMD_F32: return bwd_t<float>(grad_output, inverse, grad_mat, batch_heads, (int)n, st);
    case LFAMD_F16: return bwd_t<f16s>(grad_output, inverse, grad_mat, batch_heads, (int)n, st);
    case LFAMD_BF16: return bwd_t<bf16s>(grad_output, inverse, grad_mat, batch_heads, (int)n, st);
    default: {
      const int np = bucket(n);
      const size_t lds = 2 * (size_t)np * (np + 1) * 8;
      if ((s = set_lds(newton_bwd_f64_kernel, lds))) return s;
      hipLaunchKernelGGL(newton_bwd_f64_kernel, dim3((unsigned)batch_heads), dim3(kF64Threads), lds, st,
                         static_cast<const double*>(grad_output), static_cast<const double*>(inverse),
                         static_cast<double*>(grad_mat), (int)n, np);
      return check_launch("newton backward fp64");
    }
  }
}

}  // extern "C"

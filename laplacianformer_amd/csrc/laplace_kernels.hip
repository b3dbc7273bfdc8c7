// LaplaceSubtraction on gfx950: pairwise L1 distance and its sign-weighted
// backward, on the vector ALU.
//
// Reference semantics (src/LaplaceSubtraction_cuda_kernel.cu):
//   forward  out[i,j] = cast(sum_c |f32(q[i,c]) - f32(k[c,j])|), c ascending      (:84-140)
//   dq       dq[i,c]  = cast(sum_j f32(g[i,j]) * sgn(f32(q[i,c]) - f32(k[c,j])))   (:183-266)
//   dk       dk[c,j]  = cast(-sum_i f32(g[i,j]) * sgn(f32(q[i,c]) - f32(k[c,j])))  (:309-392)
//   sgn(0) = 0 (:34-38); fp32 accumulation, fp64 for double (:17-19).
//
// Forward mapping: one wave = 64 consecutive query rows (one per lane) x JB key
// columns; the key tile sits in LDS and every lane reads the same address
// (broadcast), so each (c, j) step costs one subtract and one |.|-add per lane.
// For fp16 the subtract is v_fma_mix_f32 on the packed halves: no conversions.
//
// Backward mapping: one lane per channel c, one wave per run of query rows,
// key column held in registers, the grad_output row broadcast from LDS. dq is a
// lane-local sum over j; dk is a lane-local sum over the wave's rows, reduced
// across the workgroup's waves in LDS in a fixed order and across workgroups by
// a second small kernel (fixed order again), so results are deterministic. A
// kernel boundary rather than device-scope fences: with one L2 per XCD, an
// agent-scope release/acquire writes back / invalidates a whole L2.
#include <algorithm>

#include "lf_common.h"
#include "lf_internal.h"

namespace lfamd {

// ---------------------------------------------------------------------------
// Staged element type for the forward key tile.
// ---------------------------------------------------------------------------
template <typename T> struct StageOf { using type = float; };
template <> struct StageOf<f16s> { using type = uint16_t; };
template <> struct StageOf<double> { using type = double; };

__device__ __forceinline__ float stage_val(float v) { return v; }
__device__ __forceinline__ float stage_val(bf16s v) { return to_acc(v); }
__device__ __forceinline__ uint16_t stage_val(f16s v) { return v.bits; }
__device__ __forceinline__ double stage_val(double v) { return v; }

constexpr int kFwdKC = 64;  // minimum channels staged per LDS pass

// Query elements per 16-byte vector load in the forward.
template <typename T> struct QChunk { static constexpr int value = 16 / sizeof(T); };

// Forward launch flags.
constexpr int kFwdVecQ = 1;    // query rows start on 16 bytes and C % QChunk == 0
constexpr int kFwdVecOut = 2;  // output tile of whole rows starts on 16 bytes

// One wave = 64 query rows (one per lane) x JB key columns; one workgroup =
// W column blocks (one per wave) x `rowBlocks` consecutive 64-row blocks, so the
// staged key tile is reused for several row blocks. KC = channels staged per
// LDS pass (all of C when it fits, which is the common case).
// Waves per forward workgroup: wide column blocks need more registers.
__host__ __device__ constexpr int fwd_max_waves(int jb) { return jb >= 32 ? 8 : 16; }

template <typename T, int JB>
__global__ void __launch_bounds__(64 * fwd_max_waves(JB))
laplace_fwd_kernel(const T* __restrict__ query, const T* __restrict__ key, T* __restrict__ out,
                   int N, int M, int C, int colsPerGroup, int rowBlocks, int KC, int flags) {
  using S = typename StageOf<T>::type;
  using A = typename AccOf<T>::type;
  constexpr int SV = 16 / (int)sizeof(S);  // staged elements per 16-byte LDS read
  constexpr int JBP = round_up(JB, SV);
  constexpr int CK = QChunk<T>::value;
  constexpr bool kF16 = std::is_same<T, f16s>::value;

  const int W = blockDim.x >> 6;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.z;
  const int jg0 = blockIdx.y * colsPerGroup;
  const int ldsCols = W * JBP;
  const int nChunks = ceil_div(C, KC);
  const bool vecq = flags & kFwdVecQ;

  extern __shared__ __align__(16) unsigned char smem[];
  S* kt = reinterpret_cast<S*>(smem);                                          // [W][KC][JBP]
  T* ot = reinterpret_cast<T*>(smem + (size_t)KC * ldsCols * sizeof(S));      // [64][colsPerGroup]

  const T* kb = key + (size_t)bh * C * M;
  const S* kw = kt + (size_t)wave * KC * JBP;

  // Stages key channels [c0, c0 + KC) for this workgroup's columns. One
  // column per lane, so the index arithmetic is per column, not per element.
  auto stage = [&](int c0) {
    const int kc = min(KC, C - c0);
    for (int u = lane; u < ldsCols; u += 64) {
      const int wb = u / JBP, jj = u - wb * JBP;
      const int col = jg0 + wb * JB + jj;
      const bool ok = jj < JB && col < M;
      for (int cc = wave; cc < KC; cc += W)
        kt[((size_t)wb * KC + cc) * JBP + jj] = (ok && cc < kc) ? stage_val(kb[(size_t)(c0 + cc) * M + col]) : S(0);
    }
  };

  const int nrb = ceil_div(N, 64);
  const int rb0 = blockIdx.x * rowBlocks;
  for (int rbi = 0; rbi < rowBlocks && rb0 + rbi < nrb; ++rbi) {
    const int row0 = (rb0 + rbi) * 64;
    const int row = row0 + lane;
    const T* qrow = query + ((size_t)bh * N + (row < N ? row : N - 1)) * C;  // rows past N are never stored

    A acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[j] = A(0);

    for (int ch = 0; ch < nChunks; ++ch) {
      const int c0 = ch * KC;
      const int kc = min(KC, C - c0);
      if (nChunks > 1 || rbi == 0) {
        __syncthreads();
        stage(c0);
        __syncthreads();
      }
      for (int cc = 0; cc < kc; cc += CK) {
        const int cg = c0 + cc;
        if constexpr (kF16) {
          uint32_t qh[4];
          if (vecq) {
            const uint4 v = *reinterpret_cast<const uint4*>(qrow + cg);
            qh[0] = v.x; qh[1] = v.y; qh[2] = v.z; qh[3] = v.w;
          } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const uint32_t lo = (cg + 2 * p < C) ? qrow[cg + 2 * p].bits : 0u;
              const uint32_t hi = (cg + 2 * p + 1 < C) ? qrow[cg + 2 * p + 1].bits : 0u;
              qh[p] = lo | (hi << 16);
            }
          }
#pragma unroll
          for (int u = 0; u < CK; ++u) {
            uint32_t kwv[JBP / 2];
            const uint4* kr = reinterpret_cast<const uint4*>(kw + (cc + u) * JBP);
#pragma unroll
            for (int t = 0; t < JBP / 8; ++t) {
              const uint4 v = kr[t];
              kwv[4 * t] = v.x; kwv[4 * t + 1] = v.y; kwv[4 * t + 2] = v.z; kwv[4 * t + 3] = v.w;
            }
            const uint32_t qp = qh[u >> 1];
#pragma unroll
            for (int j = 0; j < JB; ++j) {
              const uint32_t kp = kwv[j >> 1];
              float d;
              if (u & 1) d = (j & 1) ? mix_sub_hh<1, 1>(qp, kp) : mix_sub_hh<1, 0>(qp, kp);
              else       d = (j & 1) ? mix_sub_hh<0, 1>(qp, kp) : mix_sub_hh<0, 0>(qp, kp);
              acc[j] += fabsf(d);
            }
          }
        } else {
          A qf[CK];
          if (vecq) {
            if constexpr (std::is_same<T, bf16s>::value) {
              const uint4 v = *reinterpret_cast<const uint4*>(qrow + cg);
              const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
              for (int p = 0; p < 4; ++p) {
                qf[2 * p] = __builtin_bit_cast(float, w[p] << 16);
                qf[2 * p + 1] = __builtin_bit_cast(float, w[p] & 0xffff0000u);
              }
            } else {
              const T* src = qrow + cg;
#pragma unroll
              for (int p = 0; p < CK; ++p) qf[p] = to_acc(src[p]);
            }
          } else {
#pragma unroll
            for (int p = 0; p < CK; ++p) qf[p] = (cg + p < C) ? to_acc(qrow[cg + p]) : A(0);
          }
#pragma unroll
          for (int u = 0; u < CK; ++u) {
            const S* kr = kw + (cc + u) * JBP;
            S kv[JBP];
#pragma unroll
            for (int t = 0; t < JBP; ++t) kv[t] = kr[t];
            const A qv = qf[u];
#pragma unroll
            for (int j = 0; j < JB; ++j) acc[j] += fabs(qv - (A)kv[j]);
          }
        }
      }
    }

    // Stage the 64 x colsPerGroup tile in LDS, then store it row-contiguously.
    if (rbi > 0) __syncthreads();  // previous block's stores have read ot
#pragma unroll
    for (int j = 0; j < JB; ++j) ot[lane * colsPerGroup + wave * JB + j] = from_acc<T>(acc[j]);
    __syncthreads();
    const int colsValid = min(colsPerGroup, M - jg0);
    const int rowsValid = min(64, N - row0);
    T* ob = out + ((size_t)bh * N + row0) * M + jg0;
    if (colsPerGroup == M) {
      // Whole rows: the tile is one contiguous range of rowsValid * M elements.
      const int total = rowsValid * M;
      int done = 0;
      if (flags & kFwdVecOut) {
        constexpr int VE = 16 / (int)sizeof(T);
        const int nv = total / VE;
        for (int e = threadIdx.x; e < nv; e += blockDim.x)
          reinterpret_cast<uint4*>(ob)[e] = reinterpret_cast<const uint4*>(ot)[e];
        done = nv * VE;
      }
      for (int e = done + threadIdx.x; e < total; e += blockDim.x) ob[e] = ot[e];
    } else {
      for (int r = wave; r < rowsValid; r += W)
        for (int cidx = lane; cidx < colsValid; cidx += 64) ob[(size_t)r * M + cidx] = ot[r * colsPerGroup + cidx];
    }
  }
}

// ---------------------------------------------------------------------------
// Forward with the key broadcast from LDS. Lane = query row, R rows per lane;
// a workgroup is the W = ceil(M / JB) waves that share one block of 64*R rows,
// wave w owning key columns [w*JB, w*JB + JB). The key is widened to fp32 once
// per workgroup into LDS; per channel a wave reads its JB key values as
// wave-wide broadcasts (ds_read_b128: one read feeds 8*R VALU instructions) and
// does |q - k| + acc as v_sub_f32 and v_add_f32 with an |.| modifier, both with
// VGPR operands only (full issue rate; an SGPR operand halves it on gfx950).
// The query is widened once per channel per row. Channels are summed in
// ascending order in fp32 (fp64 is not handled here), the reference's serial
// order, so results are bit-identical to it. The output tile of the 64*R rows
// is staged in LDS and written as one contiguous span. Requires C % 8 == 0 and a
// 16-byte aligned query (checked on the host).
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float elem_f32(const uint4& v, int e);
template <> __device__ __forceinline__ float elem_f32<f16s>(const uint4& v, int e) {
  const uint32_t w = (&v.x)[e >> 1];
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> (16 * (e & 1))));
}
template <> __device__ __forceinline__ float elem_f32<bf16s>(const uint4& v, int e) {
  const uint32_t w = (&v.x)[e >> 1];
  return __builtin_bit_cast(float, (e & 1) ? (w & 0xffff0000u) : (w << 16));
}
template <> __device__ __forceinline__ float elem_f32<float>(const uint4& v, int e) {
  return __builtin_bit_cast(float, (&v.x)[e]);
}

constexpr int kFbKC = 8;  // channels per query chunk of the broadcast forward

__host__ __device__ constexpr int fb_pitch(int jb) { return (jb + 3) & ~3; }

// Epilogue of the broadcast forward: the distance rounded to the element type,
// or the Laplacian kernel exp(-scale * distance) in fp32 (LaplacianFormer's
// K_xy; fp32 because the distance rounded to fp16 would move it by ~0.4 %).
enum FwdEpi { kEpiDist = 0, kEpiExp = 1 };
template <typename T, int EPI> struct FwdOut { using type = T; };
template <typename T> struct FwdOut<T, kEpiExp> { using type = float; };

// Channel sums of the broadcast forward for the first RR of a lane's R row sets
// (RR = 1 for a block of at most 64 rows: the second set would be idle lanes that
// still cost every instruction). acc[r][j] accumulates |q - k| over c ascending.
template <typename T, int JB, int R, int RR>
__device__ __forceinline__ void fb_sums(float (&acc)[R][JB], const uint4* qsm, const float* ksm, int rows,
                                        int wave, int lane, int KP, int QP, int C) {
  constexpr int JBS = fb_pitch(JB);
  constexpr int NG = JBS / 4;
  constexpr int EV = 16 / (int)sizeof(T);
  constexpr int NVC = kFbKC / EV;
  // Rows past the block's end read row 0 of the tile (their results are not stored).
  const uint4* qrow[RR];
#pragma unroll
  for (int r = 0; r < RR; ++r) qrow[r] = qsm + (r * 64 + lane < rows ? r * 64 + lane : 0) * QP;
  const float4* kw = reinterpret_cast<const float4*>(ksm + wave * JBS);
  const int KP4 = KP / 4;
  const int nChunks = C / kFbKC;
  // Key values one channel ahead and query vectors one chunk ahead of the
  // arithmetic; a compiler memory barrier per channel keeps it from hoisting a
  // whole chunk's reads (registers).
  uint4 qv[RR][NVC];
#pragma unroll
  for (int r = 0; r < RR; ++r)
#pragma unroll
    for (int v = 0; v < NVC; ++v) qv[r][v] = qrow[r][v];
  float4 kcur[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) kcur[g] = kw[g];
  for (int kc = 0; kc < nChunks; ++kc) {
    uint4 qn[RR][NVC];
    const int kn = min(kc + 1, nChunks - 1);
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int v = 0; v < NVC; ++v) qn[r][v] = qrow[r][kn * NVC + v];
#pragma unroll
    for (int cc = 0; cc < kFbKC; ++cc) {
      const int cnext = min(kc * kFbKC + cc + 1, C - 1);
      float4 knext[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        knext[g] = kw[cnext * KP4 + g];
        // Use the padding lane too, so the read stays one ds_read_b128 (a
        // narrower split, e.g. b96 + b32, costs more LDS cycles than b128).
        asm volatile("" ::"v"(knext[g].w));
      }
      float qf[RR];
#pragma unroll
      for (int r = 0; r < RR; ++r) qf[r] = elem_f32<T>(qv[r][cc / EV], cc % EV);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float k4[4] = {kcur[g].x, kcur[g].y, kcur[g].z, kcur[g].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (g * 4 + t < JB) {
#pragma unroll
            for (int r = 0; r < RR; ++r) acc[r][g * 4 + t] += fabsf(qf[r] - k4[t]);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < NG; ++g) kcur[g] = knext[g];
      asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int v = 0; v < NVC; ++v) qv[r][v] = qn[r][v];
  }

}

template <typename T, int JB, int R, int EPI = kEpiDist>
__global__ void __launch_bounds__(1024)
laplace_fwd_bcast_kernel(const T* __restrict__ query, const T* __restrict__ key,
                         typename FwdOut<T, EPI>::type* __restrict__ out, int N, int Mg, int Mtot, int C,
                         float scale) {
  using O = typename FwdOut<T, EPI>::type;
  constexpr int JBS = fb_pitch(JB);
  constexpr int NG = JBS / 4;
  constexpr int EV = 16 / (int)sizeof(T);  // elements per 16-byte vector
  constexpr int NVC = kFbKC / EV;          // vectors per row per chunk
  const int W = blockDim.x >> 6;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // Workgroup -> (slice, row block): every slice's full blocks first, the
  // partial last blocks (N not a multiple of 64R) after all of them, so the
  // workgroups dispatched last, onto CUs that already hold their share, are
  // the short ones.
  // Column groups are the fastest grid index, so that the groups of one row
  // block run next to each other and share its query rows in L2.
  const int CG = (Mtot + Mg - 1) / Mg;
  const int cg = blockIdx.x % CG;
  const int nFull = N / (64 * R);
  const int BH = gridDim.y;
  const int id = blockIdx.y * (gridDim.x / CG) + blockIdx.x / CG;
  int bh, blk;
  if (id < BH * nFull) {
    bh = id / nFull;
    blk = id - bh * nFull;
  } else {
    bh = id - BH * nFull;
    blk = nFull;
  }
  const int i0 = blk * 64 * R;
  const int rows = min(64 * R, N - i0);
  // Column group cg: columns [cb0, cb0 + M) of the Mtot (the row stride
  // of key and output); one group covers all columns unless the tiles of all of
  // them would keep the workgroup to one per CU.
  const int cb0 = cg * Mg;
  const int M = min(Mg, Mtot - cb0);
  const int KP = W * JBS;              // key tile pitch (floats per channel)
  const int QV = C / EV;               // 16-byte vectors per query row
  const int QP = QV + 1;               // query tile pitch in vectors (padding: fewer bank conflicts)

  extern __shared__ __align__(16) unsigned char smem[];
  float* ksm = reinterpret_cast<float*>(smem);                  // [C][W*JBS] key, fp32
  uint4* qsm = reinterpret_cast<uint4*>(ksm + (size_t)C * KP);  // [64R][QP] query rows, raw
  O* otile = reinterpret_cast<O*>(qsm);                         // [64R][M] output (after the sums)

  // The block's query rows are one contiguous span: coalesced 16-byte copies.
  const uint4* qsrc = reinterpret_cast<const uint4*>(query + ((size_t)bh * N + i0) * C);
  for (int u = threadIdx.x; u < rows * QV; u += blockDim.x) {
    const int row = u / QV, v = u - row * QV;
    qsm[row * QP + v] = qsrc[u];
  }
  // Key tile, fp32, zero outside [0, M); channel c staged by wave c % W.
  const T* kb = key + (size_t)bh * C * Mtot + cb0;
  for (int c = wave; c < C; c += W) {
    for (int t = lane; t < KP; t += 64) {
      const int w = t / JBS, jj = t - w * JBS;
      const int col = w * JB + jj;
      ksm[c * KP + t] = (jj < JB && col < M) ? to_acc(kb[(size_t)c * Mtot + col]) : 0.0f;
    }
  }
  __syncthreads();

  float acc[R][JB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[r][j] = 0.0f;
  if (R > 1 && rows <= 64)
    fb_sums<T, JB, R, 1>(acc, qsm, ksm, rows, wave, lane, KP, QP, C);
  else
    fb_sums<T, JB, R, R>(acc, qsm, ksm, rows, wave, lane, KP, QP, C);

  __syncthreads();  // every wave is done with the query tile, which becomes the output tile
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const int col = wave * JB + j;
      if (col < M) {
        if constexpr (EPI == kEpiExp)
          otile[(r * 64 + lane) * M + col] = expf(-scale * acc[r][j]);
        else
          otile[(r * 64 + lane) * M + col] = from_acc<T>(acc[r][j]);
      }
    }
  __syncthreads();
  constexpr int OV = 16 / (int)sizeof(O);  // output elements per 16-byte vector
  O* dst = out + ((size_t)bh * N + i0) * Mtot + cb0;
  if (M != Mtot) {  // a column group: rows of M elements, Mtot apart
    if ((M % OV) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0 && (Mtot % OV) == 0) {
      const int vr = M / OV;
      const uint4* src4 = reinterpret_cast<const uint4*>(otile);
      for (int t = threadIdx.x; t < rows * vr; t += blockDim.x) {
        const int r = t / vr;
        reinterpret_cast<uint4*>(dst + (size_t)r * Mtot)[t - r * vr] = src4[t];
      }
    } else {
      for (int t = threadIdx.x; t < rows * M; t += blockDim.x) {
        const int r = t / M;
        dst[(size_t)r * Mtot + (t - r * M)] = otile[t];
      }
    }
    return;
  }
  // Rows [i0, i0 + rows) are one contiguous span of rows*M elements.
  const int n = rows * M;
  int done = 0;
  if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    const int nv = n / OV;
    const uint4* src4 = reinterpret_cast<const uint4*>(otile);
    uint4* dst4 = reinterpret_cast<uint4*>(dst);
    for (int t = threadIdx.x; t < nv; t += blockDim.x) dst4[t] = src4[t];
    done = nv * OV;
  }
  for (int t = done + threadIdx.x; t < n; t += blockDim.x) dst[t] = otile[t];
}

// ---------------------------------------------------------------------------
// Backward.
// ---------------------------------------------------------------------------
// sgn(q - k) with sgn(0) = 0. For fp16 inputs both operands are pre-scaled by
// 2^24, which makes every non-zero difference at least 1 in magnitude, so a
// clamp to [-1, 1] is the exact sign. For fp32/bf16 the difference is first
// scaled by 2^200 (ldexp; overflow to +-inf is fine) for the same effect.
template <typename T> struct SignOps {
  static __device__ __forceinline__ float scale(float v) { return v; }
  static __device__ __forceinline__ float sgn(float d) {
    return __builtin_amdgcn_fmed3f(ldexpf(d, 200), -1.0f, 1.0f);
  }
};
template <> struct SignOps<f16s> {
  static __device__ __forceinline__ float scale(float v) { return v * 16777216.0f; }
  static __device__ __forceinline__ float sgn(float d) {
    return __builtin_amdgcn_fmed3f(d, -1.0f, 1.0f);
  }
};
template <> struct SignOps<double> {
  static __device__ __forceinline__ double scale(double v) { return v; }
  static __device__ __forceinline__ double sgn(double d) {
    return (double)((d > 0.0) - (d < 0.0));
  }
};

constexpr int kBwdRB = 8;  // grad_output rows staged per LDS batch

// grad_output as staged in LDS: raw fp16 bits (consumed by v_fma_mix_f32),
// otherwise the accumulation type.
template <typename T> struct GStageOf { using type = typename AccOf<T>::type; };
template <> struct GStageOf<f16s> { using type = uint16_t; };
__device__ __forceinline__ float gstage(float v) { return v; }
__device__ __forceinline__ double gstage(double v) { return v; }
__device__ __forceinline__ float gstage(bf16s v) { return to_acc(v); }
__device__ __forceinline__ uint16_t gstage(f16s v) { return v.bits; }

template <typename T> constexpr int gstage_vec() { return 16 / (int)sizeof(typename GStageOf<T>::type); }

template <typename T, int JB, bool DQ, bool DK>
__global__ void __launch_bounds__(512)
laplace_bwd_kernel(const T* __restrict__ gout, const T* __restrict__ query,
                   const T* __restrict__ key, T* __restrict__ dq, T* __restrict__ dk,
                   typename AccOf<T>::type* __restrict__ partial, int N, int M, int C, int rowsPerWave) {
  using A = typename AccOf<T>::type;
  using SO = SignOps<T>;
  using GS = typename GStageOf<T>::type;
  constexpr bool kHalfG = std::is_same<T, f16s>::value;
  constexpr int GV = gstage_vec<T>();
  constexpr int JBP = round_up(JB, GV);

  const int W = blockDim.x >> 6;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.z;
  const int cb = blockIdx.y;
  const int x = blockIdx.x;
  const int nx = gridDim.x;
  const int slice = bh * gridDim.y + cb;
  const int c = cb * 64 + lane;
  const bool cval = c < C;
  const int rowBeg = (x * W + wave) * rowsPerWave;
  const int rowEnd = min(N, rowBeg + rowsPerWave);
  const bool multiJ = M > JB;

  extern __shared__ __align__(16) unsigned char smem[];
  GS* gsm = reinterpret_cast<GS*>(smem);               // [W][kBwdRB][JBP]  grad_output rows
  A* qsm = reinterpret_cast<A*>(gsm + (size_t)W * kBwdRB * JBP);  // [W][kBwdRB][64] scaled query values
  A* ksm = qsm + (size_t)W * kBwdRB * 64;              // [JB][64]          scaled key tile
  A* red = ksm + JB * 64;                              // [JB][64]          (DK)
  A* dqp = red + (DK ? JB * 64 : 0);                   // [W][rowsPerWave][64] (DQ && multiJ)

  const T* qb = query + (size_t)bh * N * C;
  const T* gb = gout + (size_t)bh * N * M;
  const T* kb = key + (size_t)bh * C * M;
  GS* gw = gsm + (size_t)wave * kBwdRB * JBP;
  A* qw = qsm + (size_t)wave * kBwdRB * 64;

  for (int jb0 = 0; jb0 < M; jb0 += JB) {
    const bool lastJ = jb0 + JB >= M;
    // Key tile [64 channels][JB columns] staged through LDS with coalesced loads,
    // then each lane keeps its channel's JB scaled values in registers.
    __syncthreads();  // previous j-block's readers of ksm are done
    for (int t = threadIdx.x; t < 64 * JB; t += blockDim.x) {
      const int cl = t / JB, j = t - cl * JB;
      const int cc = cb * 64 + cl, col = jb0 + j;
      ksm[j * 64 + cl] = (cc < C && col < M) ? SO::scale(to_acc(kb[(size_t)cc * M + col])) : A(0);
    }
    __syncthreads();
    A kreg[JB];
    A dka[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      kreg[j] = ksm[j * 64 + lane];
      dka[j] = A(0);
    }

    // Software pipeline: the next batch's grad_output elements and query values
    // are loaded into registers while the current batch is computed from LDS.
    constexpr int NSTG = ceil_div(kBwdRB * JBP, 64);
    T gpre[NSTG];
    T qpre[kBwdRB];
    auto fetch = [&](int rb) {
      const int nr = min(kBwdRB, rowEnd - rb);
#pragma unroll
      for (int s = 0; s < NSTG; ++s) {
        const int e = lane + 64 * s;
        const int r = e / JBP, jj = e - r * JBP;
        const int col = jb0 + jj;
        gpre[s] = (r < nr && jj < JB && col < M) ? gb[(size_t)(rb + r) * M + col] : T{};
      }
#pragma unroll
      for (int r = 0; r < kBwdRB; ++r) qpre[r] = (r < nr && cval) ? qb[(size_t)(rb + r) * C + c] : T{};
    };
    if (rowBeg < rowEnd) fetch(rowBeg);

    for (int rb = rowBeg; rb < rowEnd; rb += kBwdRB) {
      const int nr = min(kBwdRB, rowEnd - rb);
#pragma unroll
      for (int s = 0; s < NSTG; ++s) {
        const int e = lane + 64 * s;
        if (e < kBwdRB * JBP) gw[e] = gstage(gpre[s]);
      }
#pragma unroll
      for (int r = 0; r < kBwdRB; ++r) qw[r * 64 + lane] = SO::scale(to_acc(qpre[r]));
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (rb + kBwdRB < rowEnd) fetch(rb + kBwdRB);

      for (int r = 0; r < nr; ++r) {
        const int i = rb + r;
        const A qv = qw[r * 64 + lane];
        A dqa = A(0);
        if (DQ && multiJ && jb0 > 0) dqa = dqp[((size_t)wave * rowsPerWave + (i - rowBeg)) * 64 + lane];
        const GS* gr = gw + r * JBP;
        if constexpr (kHalfG) {
          // 8 halves per 16-byte broadcast read; v_fma_mix_f32 widens them in place.
#pragma unroll
          for (int j0 = 0; j0 < JBP; j0 += 8) {
            const uint4 v = *reinterpret_cast<const uint4*>(gr + j0);
            const uint32_t gw4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const int j = j0 + t;
              if (j < JB) {
                const float s = SO::sgn(qv - kreg[j]);
                const uint32_t gp = gw4[t >> 1];
                if (t & 1) {
                  if (DQ) dqa = mix_fma_fh<1>(s, gp, dqa);
                  if (DK) dka[j] = mix_fms_fh<1>(s, gp, dka[j]);
                } else {
                  if (DQ) dqa = mix_fma_fh<0>(s, gp, dqa);
                  if (DK) dka[j] = mix_fms_fh<0>(s, gp, dka[j]);
                }
              }
            }
          }
        } else {
#pragma unroll
          for (int j0 = 0; j0 < JBP; j0 += GV) {
            A gv[GV];
#pragma unroll
            for (int t = 0; t < GV; ++t) gv[t] = gr[j0 + t];
#pragma unroll
            for (int t = 0; t < GV; ++t) {
              const int j = j0 + t;
              if (j < JB) {
                const A s = SO::sgn(qv - kreg[j]);
                if (DQ) dqa = fma(s, gv[t], dqa);
                if (DK) dka[j] = fma(s, -gv[t], dka[j]);
              }
            }
          }
        }
        if (DQ) {
          if (lastJ) {
            if (cval) dq[((size_t)bh * N + i) * C + c] = from_acc<T>(dqa);
          } else {
            dqp[((size_t)wave * rowsPerWave + (i - rowBeg)) * 64 + lane] = dqa;
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    if (DK) {
      // Fold the waves' partial sums in wave order (deterministic).
      for (int w = 0; w < W; ++w) {
        if (wave == w) {
#pragma unroll
          for (int j = 0; j < JB; ++j)
            red[j * 64 + lane] = (w == 0 ? A(0) : red[j * 64 + lane]) + dka[j];
        }
        __syncthreads();
      }
      // partial[slice][x][c_local][M]
      A* pb = partial + ((size_t)slice * nx + x) * 64 * M;
      for (int t = threadIdx.x; t < 64 * JB; t += blockDim.x) {
        const int cl = t / JB, j = t - cl * JB;
        const int col = jb0 + j;
        if (col < M) pb[(size_t)cl * M + col] = red[j * 64 + cl];
      }
      __syncthreads();
    }
  }

}

// ---------------------------------------------------------------------------
// Backward with every key column in registers (M in {16, 32, 49} for fp16,
// {16, 49} for fp32 / bf16), every per-triple instruction at the full VALU rate.
//
// With q' = 2^24 q and k' = 2^24 k (exact for fp16 values, whose nonzero
// differences are at least 2^-24), d = q' - k' is 0 or at least 1 in magnitude,
// so y = clamp(d/2 + 1/2) is exactly (sgn(q - k) + 1) / 2 and sgn = 2y - 1:
//   grad_query[i,c] = sum_j (2 g_ij) y_ijc - sum_j g_ij
//   grad_key[c,j]   = sum_i g_ij - sum_i (2 g_ij) y_ijc
// Per triple: v_sub, v_fma+clamp, two v_fma, all with VGPR operands (an SGPR
// operand, v_med3 or v_fma_mix would issue at half rate on gfx950). fp32 and
// bf16 scale the difference twice by 2^100 instead (every nonzero fp32
// difference is at least 2^-149, so |d| 2^200 >= 2^51; overflow to +-inf clamps
// correctly): one v_mul more per triple.
//
// Lane = channel, key' and the grad_key sums of the MC columns in registers.
// Each wave owns a row range and stages its grad rows, scaled by 2, in a private
// LDS batch of RB rows; every lane reads them as wave-wide broadcasts (one
// ds_read_b128 feeds 16 VALU instructions). The row sums sum_j g_ij and column
// sums sum_i g_ij come from the same batch. No cross-wave synchronisation until
// the final, wave-ordered grad_key reduction. Requires N*MC even and a 4-byte
// aligned grad_output (checked on the host).
// ---------------------------------------------------------------------------
constexpr int kBcRB = 8;  // grad rows per LDS batch
constexpr int kBcBufs = 4;  // LDS accumulators of the workgroup grad_key reduction

// Workgroup sum of the per-wave grad_key partials v[MC] (lane = channel), in a
// fixed order: wave w adds into LDS accumulator w % kBcBufs in rounds of
// increasing w / kBcBufs, then the accumulators are summed 0, 1, ... and the
// result is written to `out` column-major, [MC][64] (channel fastest: LDS reads
// without bank conflicts, coalesced stores). Every read of a round is issued
// before its writes. Needs kBcBufs * MC * 64 floats of LDS at `red`.
template <int MC>
__device__ __forceinline__ void bcast_reduce_dk(const float (&v)[MC], float* red, int W, int wave, int lane,
                                                float* __restrict__ out) {
  const int nb = min(W, kBcBufs);
  float* buf = red + (wave % nb) * MC * 64;
  __syncthreads();  // every wave is done with the LDS it used before
  for (int round = 0; round * nb < W; ++round) {
    if (wave / nb == round) {
      if (round == 0) {
#pragma unroll
        for (int j = 0; j < MC; ++j) buf[j * 64 + lane] = v[j];
      } else {
        float pv[MC];
#pragma unroll
        for (int j = 0; j < MC; ++j) pv[j] = buf[j * 64 + lane];
#pragma unroll
        for (int j = 0; j < MC; ++j) buf[j * 64 + lane] = pv[j] + v[j];
      }
    }
    __syncthreads();
  }
  for (int t = threadIdx.x; t < 64 * MC; t += blockDim.x) {
    float s = red[t];
    for (int b = 1; b < nb; ++b) s += red[b * MC * 64 + t];
    out[t] = s;
  }
}

__host__ __device__ constexpr int bcast_max_waves(int mc) { return mc <= 16 ? 16 : 12; }
// Row pitch (floats) of a staged grad row: whole 16-byte groups, an even number
// of them (the row loop keeps two groups in flight in a two-slot ring).
__host__ __device__ constexpr int bcast_pitch(int mc) { return (mc + 7) & ~7; }

// Where the backward's grad_output comes from: fp16 elements, or (LaplacianFormer's
// kernel K = exp(-s * dist)) the gradient of K in fp32 together with K, from which
// the distance's gradient g = -s * gK * K is formed while a batch is staged.
enum BwdGrad { kGradF16 = 0, kGradKernel = 1 };

template <typename T, int MC, bool DQ, bool DK, int GSRC = kGradF16>
__global__ void __launch_bounds__(64 * bcast_max_waves(MC))
laplace_bwd_bcast_kernel(const T* __restrict__ gout, const float* __restrict__ gkern,
                         const float* __restrict__ kern, float gscale, const T* __restrict__ query,
                         const T* __restrict__ key, T* __restrict__ dq, T* __restrict__ dk,
                         float* __restrict__ partial, int N, int C, int rowsPerWave) {
  constexpr int RB = kBcRB;
  constexpr int MP = bcast_pitch(MC);            // LDS row pitch (floats)
  constexpr bool kF16 = std::is_same<T, f16s>::value;
  constexpr int EPW = sizeof(T) == 2 ? 2 : 1;    // grad elements per 32-bit word
  static_assert(GSRC == kGradF16 || kF16, "the kernel-gradient source is instantiated for fp16 only");
  constexpr int GD = GSRC == kGradF16 ? RB * MC / EPW : RB * MC;  // grad words of a full batch
  constexpr int NL = (GD + 63) / 64;             // words per lane per batch
  const int W = blockDim.x >> 6;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.z, cb = blockIdx.y, x = blockIdx.x, nx = gridDim.x;
  const int slice = bh * gridDim.y + cb;
  const int c = cb * 64 + lane;
  const bool cval = c < C;
  const int rowBeg = uniform((x * W + wave) * rowsPerWave);
  const int rowEnd = uniform(min(N, rowBeg + rowsPerWave));

  extern __shared__ __align__(16) unsigned char smem[];
  float* ksm = reinterpret_cast<float*>(smem);             // [MC][64] key tile, then grad_key sums
  // This wave's batch: [RB][MP] 2g, [RB] -sum_j g, [MP] column sums, [RB][64] scaled query.
  float* gsm = ksm + MC * 64 + wave * (RB * MP + RB + MP + RB * 64);
  float* gneg = gsm + RB * MP;
  float* hsm = gneg + RB;
  float* qsm = hsm + MP;

  const T* qb = query + (size_t)bh * N * C;
  const uint32_t* gw = reinterpret_cast<const uint32_t*>(gout + (size_t)bh * N * MC);
  const T* kb = key + (size_t)bh * C * MC;

  uint32_t gpre[NL];
  float kpre[GSRC == kGradKernel ? NL : 1];
  const float gscale2 = -2.0f * gscale;  // 2 * (-s * gK) * K == (-2s * gK) * K exactly
  int kwords = 0;                        // valid words of the fetched kernel-gradient batch
  T qpre[RB];
  auto fetch = [&](int rb) {
    if constexpr (GSRC == kGradF16) {
      const int words = min(RB, rowEnd - rb) * MC / EPW;
      const uint32_t* src = gw + (size_t)rb * MC / EPW;
#pragma unroll
      for (int t = 0; t < NL; ++t) {
        const int e = lane + 64 * t;
        gpre[t] = e < words ? src[e] : 0u;
      }
    } else {
      // Branch-free: lanes past the batch re-read its last element (rb < rowEnd,
      // so words >= MC >= 1) and are zeroed when the batch is staged.
      const int words = min(RB, rowEnd - rb) * MC;
      const float* gs = gkern + ((size_t)bh * N + rb) * MC;
      const float* ks = kern + ((size_t)bh * N + rb) * MC;
#pragma unroll
      for (int t = 0; t < NL; ++t) {
        const int e = min(lane + 64 * t, words - 1);
        gpre[t] = __builtin_bit_cast(uint32_t, gs[e]);
        kpre[t] = ks[e];
      }
      kwords = words;
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) qpre[r] = (cval && rb + r < rowEnd) ? qb[(size_t)(rb + r) * C + c] : T{};
  };
  // The first batch's loads are in flight while the key tile is staged.
  if (rowBeg < rowEnd) fetch(rowBeg);

  for (int t = threadIdx.x; t < 64 * MC; t += blockDim.x) {
    const int cl = t & 63, j = t >> 6;
    const int cc = cb * 64 + cl;
    ksm[j * 64 + cl] = cc < C ? to_acc(kb[(size_t)cc * MC + j]) * (kF16 ? 16777216.0f : 1.0f) : 0.0f;
  }
  __syncthreads();
  float kreg[MC], dka[MC];
#pragma unroll
  for (int j = 0; j < MC; ++j) {
    kreg[j] = ksm[j * 64 + lane];
    if (DK) dka[j] = 0.0f;
  }
  float hsum = 0.0f;  // lane j < MC: sum over this wave's rows of g[i][j]
  // fp32 / bf16: the difference is scaled twice by 2^100 (a VGPR operand: an
  // SGPR one would halve the issue rate) before the clamped half step.
  float scl = 0x1p100f;
  asm volatile("" : "+v"(scl));

  for (int rb = rowBeg; rb < rowEnd; rb += RB) {
    const int nr = min(RB, rowEnd - rb);  // uniform
    // Stage this batch: 2g as fp32, row-major [RB][MP] (exact for fp16 g; for the
    // kernel gradient g = -s * gK * K, rounded once, then doubled exactly).
    if constexpr (GSRC == kGradF16 && EPW == 2) {
#pragma unroll
      for (int t = 0; t < NL; ++t) {
        const int e = 2 * (lane + 64 * t);
        if (e < RB * MC) {
          const int r0 = e / MC, j0 = e - r0 * MC;
          const int r1 = (e + 1) / MC, j1 = e + 1 - r1 * MC;
          float lo, hi;
          if constexpr (kF16) {
            lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(gpre[t] & 0xffffu));
            hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(gpre[t] >> 16));
          } else {  // bf16
            lo = __builtin_bit_cast(float, gpre[t] << 16);
            hi = __builtin_bit_cast(float, gpre[t] & 0xffff0000u);
          }
          gsm[r0 * MP + j0] = 2.0f * lo;
          gsm[r1 * MP + j1] = 2.0f * hi;
        }
      }
    } else if constexpr (GSRC == kGradF16) {  // fp32: one element per word
#pragma unroll
      for (int t = 0; t < NL; ++t) {
        const int e = lane + 64 * t;
        if (e < RB * MC) {
          const int r = e / MC, j = e - r * MC;
          gsm[r * MP + j] = 2.0f * __builtin_bit_cast(float, gpre[t]);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < NL; ++t) {
        const int e = lane + 64 * t;
        if (e < RB * MC) {
          const int r = e / MC, j = e - r * MC;
          const float v = (gscale2 * __builtin_bit_cast(float, gpre[t])) * kpre[t];
          gsm[r * MP + j] = e < kwords ? v : 0.0f;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) qsm[r * 64 + lane] = to_acc(qpre[r]) * (kF16 ? 16777216.0f : 1.0f);
    wave_sync();
    // Row sums (lane r) for grad_query and column sums (lane j) for grad_key.
    // Rows past nr are zero in the batch. All reads of a sum are issued before
    // the additions, so no chain of dependent LDS round trips.
    if (DQ) {
      const float4* rowp = reinterpret_cast<const float4*>(gsm + min(lane, RB - 1) * MP);
      float4 v[MP / 4];
#pragma unroll
      for (int jq = 0; jq < MP / 4; ++jq) v[jq] = rowp[jq];
      float sum = 0.0f;
#pragma unroll
      for (int jq = 0; jq < MP / 4; ++jq) {
        const float e[4] = {v[jq].x, v[jq].y, v[jq].z, v[jq].w};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (jq * 4 + t < MC) sum += e[t];
      }
      if (lane < RB) gneg[lane] = -0.5f * sum;
    }
    if (DK) {
      float hv[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) hv[r] = gsm[r * MP + min(lane, MC - 1)];
#pragma unroll
      for (int r = 0; r < RB; ++r) hsum += hv[r];
    }
    wave_sync();
    if (rb + RB < rowEnd) fetch(rb + RB);

    // Row loop, software-pipelined two broadcast reads ahead (LDS latency under
    // load exceeds one column group's VALU time); the next row's query value,
    // initial sum and first two grad groups are read during the current row's
    // last groups. The scheduling barriers keep the compiler from computing
    // every column's step up front (MC more registers).
    constexpr int NQ = MP / 4;
    static_assert(NQ >= 2 && NQ % 2 == 0, "two groups in flight, slots aligned at every row start");
    float qn = qsm[lane];
    float accn = DQ ? gneg[0] : 0.0f;
    float4 gq[2] = {reinterpret_cast<const float4*>(gsm)[0], reinterpret_cast<const float4*>(gsm)[1]};
#pragma unroll 1
    for (int r = 0; r < nr; ++r) {
      const float4* g4 = reinterpret_cast<const float4*>(gsm + r * MP);
      const float4* g4n = reinterpret_cast<const float4*>(gsm + min(r + 1, RB - 1) * MP);
      const float qv = qn;
      // grad_query of the row as four independent partial sums (columns j = t
      // mod 4), combined once at the end: a single chain of MC dependent FMAs
      // would stall a wave on every column.
      float acc[4] = {accn, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int jq = 0; jq < NQ; ++jq) {
        const float4 gv = gq[jq & 1];
        if (jq + 2 < NQ) gq[jq & 1] = g4[jq + 2];
        else gq[jq & 1] = g4n[jq + 2 - NQ];
        if (jq == NQ - 1) {
          qn = qsm[min(r + 1, RB - 1) * 64 + lane];
          if (DQ) accn = gneg[min(r + 1, RB - 1)];
        }
        const float gg[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int j = jq * 4 + t;
          if (j < MC) {
            float y;
            if constexpr (kF16) {
              y = half_step(qv - kreg[j]);
            } else {
              const float e = (qv - kreg[j]) * scl;
              y = __builtin_amdgcn_fmed3f(__builtin_fmaf(e, scl, 0.5f), 0.0f, 1.0f);
            }
            if (DQ) acc[t] = fmaf(gg[t], y, acc[t]);
            if (DK) {
              dka[j] = fmaf(gg[t], y, dka[j]);
              asm volatile("" : "+v"(dka[j]));  // update in place, not after the row
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (DQ) {
        float total = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        // Materialise the sum here: sunk into the store's branch, the
        // accumulation would keep every column's step value live.
        asm volatile("" : "+v"(total));
        if (cval) dq[((size_t)bh * N + rb + r) * C + c] = from_acc<T>(total);
      }
    }
    wave_sync();
  }

  if (DK) {
    // This wave's grad_key partial: column sums of g minus the accumulated 2g*step.
    if (lane < MC) hsm[lane] = 0.5f * hsum;
    wave_sync();
#pragma unroll
    for (int j = 0; j < MC; ++j) dka[j] = hsm[j] - dka[j];
    bcast_reduce_dk<MC>(dka, reinterpret_cast<float*>(smem), W, wave, lane,
                        partial + ((size_t)slice * nx + x) * 64 * MC);
  }
}

// ---------------------------------------------------------------------------
// Backward for 17 <= M <= 256 columns in CB = ceil(M / 32) blocks of 32, fp16 /
// bf16 / fp32 (the last block zero-padded when M is not a multiple of 32).
//
// A workgroup is RG row groups of CB waves; wave (g, b) of a group takes the
// 32 columns [32b, 32b + 32) of every row batch (RB rows) of its group, with
// its columns' key values and grad_key sums in registers, as the fp16 kernel
// above does for all columns. A row's grad_query is the sum of the CB waves'
// column-block partials: each wave leaves its partials in LDS (double-buffered
// by batch parity), and after one workgroup barrier per batch each wave of the
// group sums RB/CB of the batch's rows in column-block order (deterministic).
// grad_key: the RG groups' sums in group order, then the workgroup partials
// summed over the slice by the reduction kernel.
//
// Step y = (sgn(q - k) + 1)/2 at the full VALU rate: fp16 operands pre-scaled
// by 2^24 (d = 0 or |d| >= 1, y = clamp(d/2 + 1/2)); bf16/fp32 by scaling the
// difference twice by 2^100 (every nonzero fp32 difference is >= 2^-149, so
// |d| * 2^200 >= 2^51; overflow to +-inf clamps correctly), five instructions
// per triple instead of four.
// ---------------------------------------------------------------------------
constexpr int kMbMC = 32;  // columns per wave
constexpr int kMbRB = 8;   // rows per batch

template <typename T, int CB, bool DQ, bool DK, int GSRC = kGradF16>
__global__ void __launch_bounds__(1024)
laplace_bwd_mb_kernel(const T* __restrict__ gout, const T* __restrict__ query, const T* __restrict__ key,
                      T* __restrict__ dq, float* __restrict__ partial, int N, int C, int rowsPerWG, int Mt,
                      const float* __restrict__ gkern, const float* __restrict__ kern, float gscale) {
  // M = CB * 32 columns in registers and LDS; the tensors have Mt <= M columns (the
  // last block is partial when Mt is not a multiple of 32: its columns from Mt on
  // have zero grad and key, so they add nothing and are not stored).
  constexpr int MC = kMbMC, RB = kMbRB, M = CB * MC;
  constexpr int MP = MC;                       // LDS row pitch of a staged batch (floats)
  // 16-bit inputs take the ordered-pattern step (tmap16): y = clamp(T(q) + (1/2 - T(k))).
  constexpr bool k16 = std::is_same<T, f16s>::value || std::is_same<T, bf16s>::value;
  // Grad elements per fetched 32-bit word: 2 for 16-bit grads, 1 for fp32 grads and
  // for the kernel-gradient source (fp32 gK and K, g = -s * gK * K formed at staging).
  static_assert(GSRC == kGradF16 || std::is_same<T, f16s>::value, "kernel-gradient source: fp16 only");
  constexpr int EPW = GSRC == kGradKernel ? 1 : (4 / (int)sizeof(T) > 0 ? 4 / (int)sizeof(T) : 1);
  constexpr int GW = RB * MC / EPW;            // grad words of a batch (this wave's columns)
  constexpr int NL = (GW + 63) / 64;           // words per lane
  static_assert(GW % 64 == 0, "whole words per lane");
  const int W = blockDim.x >> 6;
  const int RG = W / CB;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cbk = wave % CB, grp = wave / CB;
  const int bh = blockIdx.z, chb = blockIdx.y, x = blockIdx.x, nx = gridDim.x;
  const int slice = bh * gridDim.y + chb;
  const int c = chb * 64 + lane;
  const bool cval = c < C;
  const int cq = min(c, C - 1);
  const int r0wg = x * rowsPerWG;
  const int rowsWG = max(0, min(N, r0wg + rowsPerWG) - r0wg);
  const int nb = (rowsWG + RB - 1) / RB;        // batches of the workgroup
  const int rounds = (nb + RG - 1) / RG;        // batch t goes to group t % RG

  extern __shared__ __align__(16) unsigned char smem[];
  float* big = reinterpret_cast<float*>(smem);  // key tile [M][64] at the start, then the
                                                // grad_query partials [2][W][RB][64]
  const int bigFloats = max(M * 64, 2 * W * RB * 64);
  float* gsm = big + bigFloats + wave * (RB * MP + RB + RB * 64);  // this wave: [RB][MP] 2g,
  float* gneg = gsm + RB * MP;                                      // [RB] -sum_j g,
  float* qsm = gneg + RB;                                           // [RB][64] query values

  const T* qb = query + (size_t)bh * N * C;
  const T* kb = key + (size_t)bh * C * Mt;

  // Next batch of this group: this wave's 32 columns of RB rows (clamped to the
  // last valid row; rows past the batch are zeroed at staging) and RB query values.
  uint32_t gpre[NL];
  float kpre[GSRC == kGradKernel ? NL : 1];
  const float gscale2 = -2.0f * gscale;  // 2 * (-s * gK) * K == (-2s * gK) * K exactly
  T qpre[RB];
  int fnr = 0;
  auto fetch = [&](int t) {
    const int rb = r0wg + t * RB;
    const int nr = min(RB, r0wg + rowsWG - rb);
#pragma unroll
    for (int s = 0; s < NL; ++s) {
      const int w = lane + 64 * s;               // word of the batch block
      const int r = min(w / (MC / EPW), nr - 1), jw = w - (w / (MC / EPW)) * (MC / EPW);
      const int col = cbk * MC + jw * EPW;
      if constexpr (GSRC == kGradKernel) {
        const size_t o = ((size_t)bh * N + rb + r) * Mt + min(col, Mt - 1);
        gpre[s] = col < Mt ? __builtin_bit_cast(uint32_t, gkern[o]) : 0u;
        kpre[s] = col < Mt ? kern[o] : 0.0f;
        continue;
      }
      const T* rowp = gout + ((size_t)bh * N + rb + r) * Mt;
      if constexpr (EPW == 2) {
        if (Mt & 1) {  // odd row length: rows do not start on 4-byte words, two 16-bit loads
          const uint32_t lo = col < Mt ? rowp[min(col, Mt - 1)].bits : 0u;
          const uint32_t hi = col + 1 < Mt ? rowp[min(col + 1, Mt - 1)].bits : 0u;
          gpre[s] = lo | (hi << 16);
          continue;
        }
      }
      // Even row length (or fp32): a word is all in or all out of the row.
      gpre[s] = col < Mt ? *reinterpret_cast<const uint32_t*>(rowp + min(col, Mt - EPW)) : 0u;
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) qpre[r] = qb[(size_t)min(rb + r, rb + nr - 1) * C + cq];
    fnr = nr;
  };
  int t0 = grp;  // this group's first batch
  if (t0 < nb) fetch(t0);

  // Key tile (global [C][M], coalesced over j): 16-bit keys as the step terms
  // 1/2 - T(k) (see tmap16), fp32 keys as values. Columns past Mt have zero grad.
  for (int t = threadIdx.x; t < 64 * M; t += blockDim.x) {
    const int cl = t / M, j = t - cl * M;
    const int cc = chb * 64 + cl;
    const bool in = cc < C && j < Mt;
    const T kv = kb[(size_t)min(cc, C - 1) * Mt + min(j, Mt - 1)];
    if constexpr (k16)
      big[j * 64 + cl] = in ? 0.5f - tmap16(kv.bits) : 0.0f;
    else
      big[j * 64 + cl] = in ? to_acc(kv) : 0.0f;
  }
  __syncthreads();
  float kreg[MC], dka[MC];
#pragma unroll
  for (int j = 0; j < MC; ++j) {
    kreg[j] = big[(cbk * MC + j) * 64 + lane];
    if (DK) dka[j] = 0.0f;
  }
  __syncthreads();  // the key tile's LDS becomes the partial buffers
  float scl = 0x1p100f;
  asm volatile("" : "+v"(scl));  // VGPR operand: an SGPR one would halve the issue rate
  float hsum = 0.0f;  // lane j < MC: sum over this wave's rows of 2 g[i][j]

  for (int round = 0; round < rounds; ++round) {
    const int t = round * RG + grp;
    const bool have = t < nb;                          // uniform per wave
    const int nr = have ? fnr : 0;
    float* dqp = big + ((round & 1) * W + wave) * RB * 64;  // this wave's partials of this batch
    if (have) {
      // Stage: 2g as fp32 [RB][MP], rows past nr zero.
#pragma unroll
      for (int s = 0; s < NL; ++s) {
        const int w = lane + 64 * s;
        const int r = w / (MC / EPW), jw = w - r * (MC / EPW);
        const bool ok = r < nr;
        if constexpr (EPW == 2) {
          const float lo = std::is_same<T, f16s>::value
                               ? (float)__builtin_bit_cast(_Float16, (uint16_t)(gpre[s] & 0xffffu))
                               : __builtin_bit_cast(float, gpre[s] << 16);
          const float hi = std::is_same<T, f16s>::value
                               ? (float)__builtin_bit_cast(_Float16, (uint16_t)(gpre[s] >> 16))
                               : __builtin_bit_cast(float, gpre[s] & 0xffff0000u);
          gsm[r * MP + 2 * jw] = ok ? 2.0f * lo : 0.0f;
          gsm[r * MP + 2 * jw + 1] = ok ? 2.0f * hi : 0.0f;
        } else if constexpr (GSRC == kGradKernel) {
          gsm[r * MP + jw] = ok ? (gscale2 * __builtin_bit_cast(float, gpre[s])) * kpre[s] : 0.0f;
        } else {
          gsm[r * MP + jw] = ok ? 2.0f * __builtin_bit_cast(float, gpre[s]) : 0.0f;
        }
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        if constexpr (k16)
          qsm[r * 64 + lane] = tmap16(qpre[r].bits);
        else
          qsm[r * 64 + lane] = to_acc(qpre[r]);
      }
      wave_sync();
      if (DQ) {
        const float4* rowp = reinterpret_cast<const float4*>(gsm + min(lane, RB - 1) * MP);
        float4 v[MP / 4];
#pragma unroll
        for (int jq = 0; jq < MP / 4; ++jq) v[jq] = rowp[jq];
        float sum = 0.0f;
#pragma unroll
        for (int jq = 0; jq < MP / 4; ++jq) sum += (v[jq].x + v[jq].y) + (v[jq].z + v[jq].w);
        if (lane < RB) gneg[lane] = -0.5f * sum;
      }
      if (DK) {
        float hv[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) hv[r] = gsm[r * MP + min(lane, MC - 1)];
#pragma unroll
        for (int r = 0; r < RB; ++r) hsum += hv[r];
      }
      wave_sync();
      if (t + RG < nb) fetch(t + RG);

      // Row loop as in the fp16 kernel: grad values two 16-byte groups ahead,
      // four partial sums per row, grad_key sums updated in place.
      constexpr int NQ = MP / 4;
      float qn = qsm[lane];
      float accn = DQ ? gneg[0] : 0.0f;
      float4 gq[2] = {reinterpret_cast<const float4*>(gsm)[0], reinterpret_cast<const float4*>(gsm)[1]};
#pragma unroll 1
      for (int r = 0; r < nr; ++r) {
        const float4* g4 = reinterpret_cast<const float4*>(gsm + r * MP);
        const float4* g4n = reinterpret_cast<const float4*>(gsm + min(r + 1, RB - 1) * MP);
        const float qv = qn;
        float acc[4] = {accn, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int jq = 0; jq < NQ; ++jq) {
          const float4 gv = gq[jq & 1];
          if (jq + 2 < NQ) gq[jq & 1] = g4[jq + 2];
          else gq[jq & 1] = g4n[jq + 2 - NQ];
          if (jq == NQ - 1) {
            qn = qsm[min(r + 1, RB - 1) * 64 + lane];
            if (DQ) accn = gneg[min(r + 1, RB - 1)];
          }
          const float gg[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int j = jq * 4 + u;
            float y;
            if constexpr (k16) {
              y = __builtin_amdgcn_fmed3f(qv + kreg[j], 0.0f, 1.0f);  // one clamped add
            } else {
              const float e = (qv - kreg[j]) * scl;
              y = __builtin_amdgcn_fmed3f(__builtin_fmaf(e, scl, 0.5f), 0.0f, 1.0f);
            }
            if (DQ) acc[u] = fmaf(gg[u], y, acc[u]);
            if (DK) {
              dka[j] = fmaf(gg[u], y, dka[j]);
              asm volatile("" : "+v"(dka[j]));  // update in place, not after the row
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (DQ) {
          float total = (acc[0] + acc[1]) + (acc[2] + acc[3]);
          asm volatile("" : "+v"(total));
          dqp[r * 64 + lane] = total;
        }
      }
    }
    if (DQ) {
      // Every wave of the workgroup has written this batch's partials (and is
      // done reading the partials of two batches ago, in the other buffer).
      __syncthreads();
      if (have) {
        const int rb = r0wg + t * RB;
        const float* gp = big + ((round & 1) * W + grp * CB) * RB * 64;  // the group's CB waves
        for (int r = cbk; r < nr; r += CB) {
          float sv = 0.0f;
#pragma unroll
          for (int b = 0; b < CB; ++b) sv += gp[(b * RB + r) * 64 + lane];
          if (cval) dq[((size_t)bh * N + rb + r) * C + c] = from_acc<T>(sv);
        }
      }
    }
    if (have) wave_sync();
  }

  if (DK) {
    // This wave's grad_key partial for its 32 columns, then the RG groups' sums in
    // group order into red[M][64], written out as the workgroup's partial.
    if (lane < MC) gsm[lane] = 0.5f * hsum;
    wave_sync();
#pragma unroll
    for (int j = 0; j < MC; ++j) dka[j] = gsm[j] - dka[j];
    __syncthreads();  // every wave is done with the partial buffers
    float* red = big;
    for (int g = 0; g < RG; ++g) {
      if (grp == g) {
#pragma unroll
        for (int j = 0; j < MC; ++j) {
          float* p = &red[(cbk * MC + j) * 64 + lane];
          *p = g == 0 ? dka[j] : *p + dka[j];
        }
      }
      __syncthreads();
    }
    float* out = partial + ((size_t)slice * nx + x) * 64 * Mt;
    for (int tt = threadIdx.x; tt < 64 * Mt; tt += blockDim.x) out[tt] = red[tt];
  }
}

// grad_key = sum over the workgroups of a slice of their partial sums, in
// workgroup order (deterministic). One thread per (channel, column).
template <typename T>
__global__ void __launch_bounds__(256)
laplace_dk_reduce_kernel(const typename AccOf<T>::type* __restrict__ partial, T* __restrict__ dk,
                         int nx, int M, int C) {
  using A = typename AccOf<T>::type;
  const int bh = blockIdx.z, cb = blockIdx.y;
  const int slice = bh * gridDim.y + cb;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 64 * M) return;
  const int cl = t / M, j = t - cl * M;
  const int cc = cb * 64 + cl;
  if (cc >= C) return;
  const A* pb = partial + (size_t)slice * nx * 64 * M + t;
  A s = A(0);
#pragma unroll 8
  for (int x = 0; x < nx; ++x) s += pb[(size_t)x * 64 * M];
  dk[((size_t)bh * C + cc) * M + j] = from_acc<T>(s);
}

// Same sum over column-major partials ([M][64] per workgroup, channel fastest).
template <typename T = f16s>
__global__ void __launch_bounds__(256)
laplace_dk_reduce_cm_kernel(const float* __restrict__ partial, T* __restrict__ dk, int nx, int M, int C) {
  const int bh = blockIdx.z, cb = blockIdx.y;
  const int slice = bh * gridDim.y + cb;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 64 * M) return;
  const int j = t >> 6, cl = t & 63;
  const int cc = cb * 64 + cl;
  if (cc >= C) return;
  const float* pb = partial + (size_t)slice * nx * 64 * M + t;
  float s = 0.0f;
#pragma unroll 8
  for (int x = 0; x < nx; ++x) s += pb[(size_t)x * 64 * M];
  dk[((size_t)bh * C + cc) * M + j] = from_acc<T>(s);
}

// ---------------------------------------------------------------------------
// Legacy reduce forward: one workgroup of bd = min(C, 256) threads per output,
// arithmetic in the element type, halving-tree fold (reference :399-447).
// ---------------------------------------------------------------------------
template <typename T> struct NativeOf { using type = float; };
template <> struct NativeOf<f16s> { using type = _Float16; };
template <> struct NativeOf<double> { using type = double; };

template <typename T> __device__ __forceinline__ typename NativeOf<T>::type to_native(T v);
template <> __device__ __forceinline__ float to_native<float>(float v) { return v; }
template <> __device__ __forceinline__ double to_native<double>(double v) { return v; }
template <> __device__ __forceinline__ _Float16 to_native<f16s>(f16s v) {
  return __builtin_bit_cast(_Float16, v.bits);
}
template <> __device__ __forceinline__ float to_native<bf16s>(bf16s v) { return to_acc(v); }

// One rounding to the element type after each native operation (bf16 is
// emulated in fp32 and rounded back; fp32 has enough precision for that to
// equal a direct bf16 operation).
template <typename T> __device__ __forceinline__ typename NativeOf<T>::type round_native(typename NativeOf<T>::type v) { return v; }
template <> __device__ __forceinline__ float round_native<bf16s>(float v) { return to_acc(from_acc<bf16s>(v)); }

template <typename T>
__global__ void __launch_bounds__(256)
laplace_reduce_fwd_kernel(const T* __restrict__ query, const T* __restrict__ key, T* __restrict__ out,
                          int64_t total, int N, int M, int C) {
  using Nt = typename NativeOf<T>::type;
  __shared__ Nt sdata[256];
  const int bd = blockDim.x;
  for (int64_t idx = blockIdx.x; idx < total; idx += gridDim.x) {
    const int64_t bh = idx / ((int64_t)N * M);
    const int64_t rem = idx - bh * N * M;
    const int p = (int)(rem / M), qj = (int)(rem - (int64_t)p * M);
    const T* qr = query + (bh * N + p) * C;
    const T* kc = key + bh * C * M + qj;
    Nt s = Nt(0);
    for (int c = threadIdx.x; c < C; c += bd) {
      Nt diff = round_native<T>(to_native(qr[c]) - to_native(kc[(int64_t)c * M]));
      s = round_native<T>(s + (diff >= Nt(0) ? diff : -diff));
    }
    sdata[threadIdx.x] = s;
    __syncthreads();
    for (int stride = bd / 2; stride > 0; stride >>= 1) {
      if ((int)threadIdx.x < stride) sdata[threadIdx.x] = round_native<T>(sdata[threadIdx.x] + sdata[threadIdx.x + stride]);
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      if constexpr (std::is_same<T, f16s>::value) out[idx] = f16s{__builtin_bit_cast(uint16_t, sdata[0])};
      else if constexpr (std::is_same<T, bf16s>::value) out[idx] = from_acc<bf16s>(sdata[0]);
      else out[idx] = sdata[0];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {

struct Dims {
  int64_t B, H, N, M, C;
  int64_t BH() const { return B * H; }
};

int check_dims(const Dims& d, const char* who) {
  if (d.B < 0 || d.H < 0 || d.N < 0 || d.M < 0 || d.C < 0)
    return fail(LFAMD_ERR_ARG, "%s: negative size", who);
  if (d.N > INT32_MAX / 2 || d.M > INT32_MAX / 2 || d.C > INT32_MAX / 2 || d.BH() > 65535)
    return fail(LFAMD_ERR_UNSUPPORTED, "%s: sizes too large (B*H must be <= 65535)", who);
  return LFAMD_OK;
}

bool empty(const Dims& d) { return d.BH() == 0 || d.N == 0 || d.M == 0; }

// ---- forward ----
template <typename T> constexpr int stage_bytes() { return (int)sizeof(typename StageOf<T>::type); }

template <typename T, int JB>
int launch_fwd_jb(const T* q, const T* k, T* o, const Dims& d, hipStream_t st) {
  constexpr int SV = 16 / stage_bytes<T>();
  constexpr int JBP = round_up(JB, SV);
  constexpr int CK = QChunk<T>::value;
  const int M = (int)d.M, N = (int)d.N, C = (int)d.C;
  const size_t ldsBudget = 64 * 1024;
  int W = std::min(fwd_max_waves(JB), ceil_div(M, JB));
  // Channels staged per pass: all of C (rounded to the query chunk) when it fits.
  auto lds = [&](int w, int kc) {
    return (size_t)kc * w * JBP * stage_bytes<T>() + (size_t)64 * w * JB * sizeof(T);
  };
  while (W > 1 && lds(W, kFwdKC) > ldsBudget) --W;
  int KC = round_up(C, CK);
  while (KC > kFwdKC && lds(W, KC) > ldsBudget) KC = std::max(kFwdKC, round_up(KC / 2, CK));
  const int cols = W * JB;
  const int colGroups = ceil_div(M, cols);
  const int nrb = ceil_div(N, 64);
  // Row blocks per workgroup: reuse the staged key tile while keeping ~6 waves per SIMD.
  const int64_t target = 6LL * 4 * num_cus();
  const int64_t waves1 = (int64_t)nrb * colGroups * d.BH() * W;
  const int rowBlocks = (int)std::max<int64_t>(1, std::min<int64_t>(nrb, waves1 / target));
  dim3 grid(ceil_div(nrb, rowBlocks), colGroups, (unsigned)d.BH());
  dim3 block(64 * W);
  int flags = 0;
  if (C % CK == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0) flags |= kFwdVecQ;
  // Whole-row tiles start at ((bh*N + row0) * M) elements: 16-byte aligned for every
  // tile when the base is and 64*M*sizeof(T) and N*M*sizeof(T) are multiples of 16.
  if (cols == M && (reinterpret_cast<uintptr_t>(o) & 15) == 0 && (64 * (size_t)M * sizeof(T)) % 16 == 0 &&
      ((size_t)N * M * sizeof(T)) % 16 == 0)
    flags |= kFwdVecOut;
  hipLaunchKernelGGL((laplace_fwd_kernel<T, JB>), grid, block, lds(W, KC), st, q, k, o, N, M, C, cols, rowBlocks,
                     KC, flags);
  return check_launch("laplace forward");
}

// Column block: the candidate with the least padding, ties to the larger block.
int pick_fwd_jb(int64_t M) {
  const int cands[4] = {7, 8, 16, 32};
  int best = 32;
  int64_t bestPad = INT64_MAX;
  for (int jb : cands) {
    const int64_t pad = ceil_div((int)M, jb) * (int64_t)jb - M;
    if (pad < bestPad || (pad == bestPad && jb > best)) { bestPad = pad; best = jb; }
  }
  return best;
}

// Column block: the least padding W*JB - M with W = ceil(M/JB) <= 16 waves,
// ties to the block count nearest 8 waves.
int pick_fb_jb(int64_t M) {
  int best = 16, bestWaste = 1 << 30, bestDist = 1 << 30;
  for (int jb : {4, 7, 8, 16}) {
    const int w = ceil_div((int)M, jb);
    if (w > 16) continue;
    const int waste = w * jb - (int)M, dist = std::abs(w - 8);
    if (waste < bestWaste || (waste == bestWaste && dist < bestDist)) {
      best = jb;
      bestWaste = waste;
      bestDist = dist;
    }
  }
  return best;
}

constexpr int kFbR = 2;  // query rows per lane of the broadcast forward

template <typename T> constexpr int dtype_of();
template <> constexpr int dtype_of<float>() { return LFAMD_F32; }
template <> constexpr int dtype_of<f16s>() { return LFAMD_F16; }
template <> constexpr int dtype_of<bf16s>() { return LFAMD_BF16; }
template <> constexpr int dtype_of<double>() { return LFAMD_F64; }

// LDS of the broadcast forward: fp32 key tile [C][W*JBS], then the query tile
// [64R][C/EV + 1] 16-byte vectors, which the output tile [64R][M] (elements of
// out_bytes) reuses.
size_t fb_lds_bytes_g(int dtype, const Dims& d, size_t out_bytes, int mg) {
  const int jb = pick_fb_jb(d.M);
  const int W = ceil_div(mg, jb);
  const size_t es = dtype_size(dtype);
  const size_t qtile = (size_t)64 * kFbR * (d.C * es / 16 + 1) * 16;
  const size_t otile = (size_t)64 * kFbR * mg * out_bytes;
  return (size_t)W * d.C * fb_pitch(jb) * 4 + std::max(qtile, otile);
}

// Columns per workgroup: all M, or half of them (a multiple of the per-wave
// block) when the tiles of all M would leave room for only one workgroup per CU
// and there are row blocks for several rounds of the chip, or when all M do not
// fit one workgroup's LDS at all (fp32 output at M = 256). Config 4 (bf16,
// M = 256, 4096 row blocks): 662 -> 560 us; with a single round of row blocks
// the split measured slower (31 -> 34 us at 256 blocks), so it is not taken there.
int fb_group_cols(int dtype, const Dims& d, size_t out_bytes) {
  const int jb = pick_fb_jb(d.M);
  const int half = ceil_div(ceil_div((int)d.M, 2), jb) * jb;
  const int64_t blocks = (int64_t)ceil_div((int)d.N, 64 * kFbR) * d.BH();
  const size_t full = fb_lds_bytes_g(dtype, d, out_bytes, (int)d.M), lim = (size_t)max_lds_bytes();
  if (half < d.M && (full > lim || (2 * full > lim && blocks >= 4 * (int64_t)num_cus()))) return half;
  return (int)d.M;
}

size_t fb_lds_bytes(int dtype, const Dims& d, size_t out_bytes) {
  return fb_lds_bytes_g(dtype, d, out_bytes, fb_group_cols(dtype, d, out_bytes));
}

// Broadcast forward: a non-fp64 type, C % 8 == 0, 16-byte aligned query,
// M <= 256 and the key and output tiles within the LDS of one workgroup.
bool fwd_bcast_ok(int dtype, const Dims& d, const void* q, size_t out_bytes) {
  if (dtype == LFAMD_F64 || d.C % kFbKC != 0 || d.M > 256) return false;
  if ((reinterpret_cast<uintptr_t>(q) & 15) != 0) return false;
  return fb_lds_bytes(dtype, d, out_bytes) <= (size_t)max_lds_bytes();
}

template <typename T, int JB, int EPI>
int launch_fwd_bcast_jb(const void* q, const void* k, void* o, const Dims& d, float scale, hipStream_t st) {
  using O = typename FwdOut<T, EPI>::type;
  const int mg = fb_group_cols(dtype_of<T>(), d, sizeof(O));
  const int W = ceil_div(mg, JB);
  const size_t lds = fb_lds_bytes_g(dtype_of<T>(), d, sizeof(O), mg);
  auto kern = laplace_fwd_bcast_kernel<T, JB, kFbR, EPI>;
  if (lds > 65536)
    if (int s = set_dyn_lds(reinterpret_cast<const void*>(kern), lds, "laplace forward")) return s;
  dim3 grid(ceil_div((int)d.N, 64 * kFbR) * ceil_div((int)d.M, mg), (unsigned)d.BH());
  hipLaunchKernelGGL(kern, grid, dim3(64 * W), lds, st, static_cast<const T*>(q), static_cast<const T*>(k),
                     static_cast<O*>(o), (int)d.N, mg, (int)d.M, (int)d.C, scale);
  return check_launch("laplace forward");
}

template <typename T, int EPI = kEpiDist>
int launch_fwd_bcast(const void* q, const void* k, void* o, const Dims& d, hipStream_t st, float scale = 0.0f) {
  switch (pick_fb_jb(d.M)) {
    case 4: return launch_fwd_bcast_jb<T, 4, EPI>(q, k, o, d, scale, st);
    case 7: return launch_fwd_bcast_jb<T, 7, EPI>(q, k, o, d, scale, st);
    case 8: return launch_fwd_bcast_jb<T, 8, EPI>(q, k, o, d, scale, st);
    default: return launch_fwd_bcast_jb<T, 16, EPI>(q, k, o, d, scale, st);
  }
}

template <typename T>
int launch_fwd(const void* q, const void* k, void* o, const Dims& d, hipStream_t st) {
  const T* qq = static_cast<const T*>(q);
  const T* kk = static_cast<const T*>(k);
  T* oo = static_cast<T*>(o);
  switch (pick_fwd_jb(d.M)) {
    case 7: return launch_fwd_jb<T, 7>(qq, kk, oo, d, st);
    case 8: return launch_fwd_jb<T, 8>(qq, kk, oo, d, st);
    case 16: return launch_fwd_jb<T, 16>(qq, kk, oo, d, st);
    default: return launch_fwd_jb<T, 32>(qq, kk, oo, d, st);
  }
}

// ---- backward ----
struct BwdPlan {
  int JB;           // key columns per register block
  int W;            // waves per workgroup
  int nx;           // workgroups per (bh, channel block) slice
  int rowsPerWave;
  int ncb;          // channel blocks of 64
  size_t lds;
  size_t partialElems;
};

int pick_bwd_jb(int64_t M) {
  if (M <= 16) return 16;
  if (M <= 32) return 32;
  if (M == 49) return 49;
  return 64;
}

BwdPlan plan_bwd(const Dims& d, bool dq, bool dkey, size_t accBytes, size_t gBytes) {
  BwdPlan p{};
  p.JB = pick_bwd_jb(d.M);
  p.ncb = ceil_div((int)d.C, 64);
  const int GV = 16 / (int)gBytes;
  const int JBP = round_up(p.JB, GV);
  const bool multiJ = d.M > p.JB;
  const int64_t slices = d.BH() * p.ncb;
  const int N = (int)std::max<int64_t>(d.N, 1);
  // One round of resident waves: 2 per SIMD (the kernel may use up to 256
  // registers), at least 8 rows per wave.
  const int target = 8 * num_cus();
  int64_t wps = std::max<int64_t>(1, ceil_div(target, (int)std::min<int64_t>(slices, target)));
  wps = std::min<int64_t>(wps, ceil_div(N, 8));
  int rows = ceil_div(N, (int)wps);
  if (dq && multiJ) rows = std::min(rows, 64);
  wps = ceil_div(N, rows);
  const size_t budget = 96 * 1024;
  auto lds = [&](int w) {
    size_t b = (size_t)w * kBwdRB * (JBP * gBytes + 64 * accBytes) + (size_t)p.JB * 64 * accBytes;
    if (dkey) b += (size_t)p.JB * 64 * accBytes;
    if (dq && multiJ) b += (size_t)w * rows * 64 * accBytes;
    return b;
  };
  int W = (int)std::min<int64_t>(8, wps);
  while (W > 1 && lds(W) > budget) --W;
  p.W = W;
  p.nx = ceil_div((int)wps, W);
  p.rowsPerWave = ceil_div(N, p.nx * W);
  if (dq && multiJ) p.rowsPerWave = std::min(p.rowsPerWave, rows);
  p.lds = lds(W);
  p.partialElems = dkey ? (size_t)slices * p.nx * 64 * (size_t)d.M : 0;
  return p;
}

// Plan of the register-resident-column backward: 3 waves per SIMD resident (4 for M <= 16).
struct BcPlan {
  int W, nx, rowsPerWave, ncb;
  size_t lds, partialElems;
};

// (M = 64 runs faster on the column-block kernel below: 57 vs 62 us at B=32 N=3136.)
// fp32 / bf16 with M = 32 (a column block) run the column-block kernel.
bool bcast_bwd_ok(int dtype, const Dims& d, const void* g) {
  if (dtype == LFAMD_F16) {
    if (!(d.M == 16 || d.M == 32 || d.M == 49)) return false;
  } else if (dtype == LFAMD_F32 || dtype == LFAMD_BF16) {
    if (!(d.M == 16 || d.M == 49)) return false;
  } else {
    return false;
  }
  if (dtype != LFAMD_F32 && (d.N * d.M) % 2 != 0) return false;
  return (reinterpret_cast<uintptr_t>(g) & 3) == 0;
}

BcPlan plan_bcast(const Dims& d, bool dkey) {
  BcPlan p{};
  p.ncb = ceil_div((int)d.C, 64);
  const int64_t slices = d.BH() * p.ncb;
  const int N = (int)std::max<int64_t>(d.N, 1);
  const int wmax = bcast_max_waves((int)d.M);
  const int target = wmax * num_cus();
  int64_t wps = std::max<int64_t>(1, ceil_div(target, (int)std::min<int64_t>(slices, target)));
  wps = std::min<int64_t>(wps, ceil_div(N, 8));
  const int W = (int)std::min<int64_t>(wmax, wps);
  p.W = W;
  p.nx = ceil_div((int)wps, W);
  p.rowsPerWave = round_up(ceil_div(N, p.nx * W), 2);
  const int mp = bcast_pitch((int)d.M);
  p.lds = ((size_t)d.M * 64 + (size_t)W * (kBcRB * mp + kBcRB + mp + kBcRB * 64)) * 4;
  if (dkey) p.lds = std::max(p.lds, (size_t)std::min(W, kBcBufs) * d.M * 64 * 4);
  p.partialElems = dkey ? (size_t)slices * p.nx * 64 * (size_t)d.M : 0;
  return p;
}

// Kernel-gradient source of the backward (LaplacianFormer's K = exp(-s * dist)).
struct KernGrad {
  const float* gk = nullptr;
  const float* kv = nullptr;
  float scale = 0.0f;
};

template <typename T, int MC, bool DQ, bool DK, int GSRC = kGradF16>
int launch_bcast_bwd_mc(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, const Dims& d,
                        const BcPlan& p, hipStream_t st, KernGrad kg = {}) {
  dim3 grid(p.nx, p.ncb, (unsigned)d.BH());
  hipLaunchKernelGGL((laplace_bwd_bcast_kernel<T, MC, DQ, DK, GSRC>), grid, dim3(64 * p.W), p.lds, st,
                     static_cast<const T*>(g), kg.gk, kg.kv, kg.scale, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<T*>(dq), static_cast<T*>(dk),
                     static_cast<float*>(ws), (int)d.N, (int)d.C, p.rowsPerWave);
  int s = check_launch("laplace backward");
  if (s || !DK) return s;
  dim3 rgrid(ceil_div(64 * MC, 256), p.ncb, (unsigned)d.BH());
  hipLaunchKernelGGL(laplace_dk_reduce_cm_kernel<T>, rgrid, dim3(256), 0, st, static_cast<const float*>(ws),
                     static_cast<T*>(dk), p.nx, MC, (int)d.C);
  return check_launch("laplace backward_key reduction");
}

template <typename T, bool DQ, bool DK, int GSRC = kGradF16>
int launch_bcast_bwd_t(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, const Dims& d,
                       const BcPlan& p, hipStream_t st, KernGrad kg) {
  if constexpr (std::is_same<T, f16s>::value) {
    switch (d.M) {
      case 16: return launch_bcast_bwd_mc<T, 16, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
      case 32: return launch_bcast_bwd_mc<T, 32, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
      default: return launch_bcast_bwd_mc<T, 49, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    }
  } else {
    if (d.M == 16) return launch_bcast_bwd_mc<T, 16, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    return launch_bcast_bwd_mc<T, 49, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
  }
}

// The kernel-gradient source (fp32 gK and K) is fp16-only.
template <bool DQ, bool DK, int GSRC = kGradF16>
int launch_bcast_bwd(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk, void* ws,
                     const Dims& d, const BcPlan& p, hipStream_t st, KernGrad kg = {}) {
  if constexpr (GSRC == kGradF16) {
    if (dtype == LFAMD_F32) return launch_bcast_bwd_t<float, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    if (dtype == LFAMD_BF16) return launch_bcast_bwd_t<bf16s, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
  }
  return launch_bcast_bwd_t<f16s, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
}

// ---- backward for 17 <= M <= 256 in column blocks of 32 (fp16 / bf16 / fp32) ----
struct MbPlan {
  int CB, RG, W, nx, ncb, rowsPerWG;
  size_t lds, partialElems;
};

// Any 17 <= M <= 256; a last column block of fewer than 32 columns is
// zero-padded. (16-bit grad rows of odd length are fetched element by element.)
bool mb_bwd_ok(int dtype, const Dims& d, const void* g) {
  if (!(dtype == LFAMD_F16 || dtype == LFAMD_BF16 || dtype == LFAMD_F32)) return false;
  if (d.M < 17 || d.M > 8 * kMbMC) return false;
  // Word loads need 4-byte rows; odd 16-bit rows are read element by element.
  const bool elementwise = dtype != LFAMD_F32 && d.M % 2 != 0;
  return (reinterpret_cast<uintptr_t>(g) & (elementwise ? 1 : 3)) == 0;
}

MbPlan plan_mb(const Dims& d, bool dkey) {
  MbPlan p{};
  p.ncb = ceil_div((int)d.C, 64);
  p.CB = ceil_div((int)d.M, kMbMC);
  p.RG = std::max(1, 16 / p.CB);
  p.W = p.CB * p.RG;
  const int64_t slices = d.BH() * p.ncb;
  const int N = (int)std::max<int64_t>(d.N, 1);
  // One workgroup per CU when the slices allow it, each with at least one batch per row group.
  int nx = (int)std::max<int64_t>(1, ceil_div(num_cus(), (int)std::min<int64_t>(slices, num_cus())));
  nx = std::min(nx, std::max(1, N / (kMbRB * p.RG)));
  p.rowsPerWG = round_up(ceil_div(N, nx), kMbRB);
  p.nx = ceil_div(N, p.rowsPerWG);
  const size_t bigFloats = std::max<size_t>((size_t)p.CB * kMbMC * 64, (size_t)2 * p.W * kMbRB * 64);
  p.lds = (bigFloats + (size_t)p.W * (kMbRB * kMbMC + kMbRB + kMbRB * 64)) * 4;
  p.partialElems = dkey ? (size_t)slices * p.nx * 64 * (size_t)d.M : 0;
  return p;
}

template <typename T, int CB, bool DQ, bool DK, int GSRC = kGradF16>
int launch_mb_cb(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, const Dims& d,
                 const MbPlan& p, hipStream_t st, KernGrad kg = {}) {
  auto kern = laplace_bwd_mb_kernel<T, CB, DQ, DK, GSRC>;
  if (p.lds > 65536)
    if (int s = set_dyn_lds(reinterpret_cast<const void*>(kern), p.lds, "laplace backward")) return s;
  dim3 grid(p.nx, p.ncb, (unsigned)d.BH());
  hipLaunchKernelGGL(kern, grid, dim3(64 * p.W), p.lds, st, static_cast<const T*>(g), static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<T*>(dq), static_cast<float*>(ws), (int)d.N, (int)d.C,
                     p.rowsPerWG, (int)d.M, kg.gk, kg.kv, kg.scale);
  int s = check_launch("laplace backward");
  if (s || !DK) return s;
  dim3 rgrid(ceil_div(64 * (int)d.M, 256), p.ncb, (unsigned)d.BH());
  hipLaunchKernelGGL(laplace_dk_reduce_cm_kernel<T>, rgrid, dim3(256), 0, st, static_cast<const float*>(ws),
                     static_cast<T*>(dk), p.nx, (int)d.M, (int)d.C);
  return check_launch("laplace backward_key reduction");
}

template <typename T, bool DQ, bool DK, int GSRC = kGradF16>
int launch_mb_t(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, const Dims& d,
                const MbPlan& p, hipStream_t st, KernGrad kg = {}) {
  switch (p.CB) {
    case 1: return launch_mb_cb<T, 1, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    case 2: return launch_mb_cb<T, 2, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    case 3: return launch_mb_cb<T, 3, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    case 4: return launch_mb_cb<T, 4, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    case 5: return launch_mb_cb<T, 5, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    case 6: return launch_mb_cb<T, 6, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    case 7: return launch_mb_cb<T, 7, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
    default: return launch_mb_cb<T, 8, DQ, DK, GSRC>(g, q, k, dq, dk, ws, d, p, st, kg);
  }
}

template <bool DQ, bool DK>
int launch_mb(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk, void* ws,
              const Dims& d, const MbPlan& p, hipStream_t st) {
  switch (dtype) {
    case LFAMD_F16: return launch_mb_t<f16s, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    case LFAMD_BF16: return launch_mb_t<bf16s, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    default: return launch_mb_t<float, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
  }
}

// The fused kernel-gradient backward (fp16): M in {16, 32, 49} on the
// register-resident-column kernel, any other 17 <= M <= 256 on the column-block
// kernel (the former spills at M = 64: 94 us there against 87 us composed).
bool kernel_bwd_bcast(const Dims& d) { return d.M == 16 || d.M == 32 || d.M == 49; }
bool kernel_bwd_ok(int dtype, const Dims& d) {
  return dtype == LFAMD_F16 && (kernel_bwd_bcast(d) || (d.M >= 17 && d.M <= 8 * kMbMC));
}

template <typename T, int JB, bool DQ, bool DK>
int launch_bwd_jb(const T* g, const T* q, const T* k, T* dq, T* dk, void* ws, const Dims& d,
                  const BwdPlan& p, hipStream_t st) {
  using A = typename AccOf<T>::type;
  dim3 grid(p.nx, p.ncb, (unsigned)d.BH());
  dim3 block(64 * p.W);
  hipLaunchKernelGGL((laplace_bwd_kernel<T, JB, DQ, DK>), grid, block, p.lds, st, g, q, k, dq, dk,
                     static_cast<A*>(ws), (int)d.N, (int)d.M, (int)d.C, p.rowsPerWave);
  int s = check_launch("laplace backward");
  if (s || !DK) return s;
  dim3 rgrid(ceil_div(64 * (int)d.M, 256), p.ncb, (unsigned)d.BH());
  hipLaunchKernelGGL(laplace_dk_reduce_kernel<T>, rgrid, dim3(256), 0, st, static_cast<const A*>(ws), dk,
                     p.nx, (int)d.M, (int)d.C);
  return check_launch("laplace backward_key reduction");
}

template <typename T, bool DQ, bool DK>
int launch_bwd_t(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws,
                 const Dims& d, const BwdPlan& p, hipStream_t st) {
  auto G = static_cast<const T*>(g);
  auto Q = static_cast<const T*>(q);
  auto K = static_cast<const T*>(k);
  auto DQp = static_cast<T*>(dq);
  auto DKp = static_cast<T*>(dk);
  switch (p.JB) {
    case 16: return launch_bwd_jb<T, 16, DQ, DK>(G, Q, K, DQp, DKp, ws, d, p, st);
    case 32: return launch_bwd_jb<T, 32, DQ, DK>(G, Q, K, DQp, DKp, ws, d, p, st);
    case 49: return launch_bwd_jb<T, 49, DQ, DK>(G, Q, K, DQp, DKp, ws, d, p, st);
    default: return launch_bwd_jb<T, 64, DQ, DK>(G, Q, K, DQp, DKp, ws, d, p, st);
  }
}

template <bool DQ, bool DK>
int launch_bwd(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk, void* ws,
               const Dims& d, const BwdPlan& p, hipStream_t st) {
  switch (dtype) {
    case LFAMD_F32: return launch_bwd_t<float, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    case LFAMD_F16: return launch_bwd_t<f16s, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    case LFAMD_BF16: return launch_bwd_t<bf16s, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    default: return launch_bwd_t<double, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
  }
}

// Fills `n` elements of `p` with zero (used when the reduction length is 0).
template <typename T>
__global__ void fill_zero_kernel(T* __restrict__ p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = T{};
}

int zero_fill(void* p, int64_t bytes, hipStream_t st) {
  if (bytes <= 0) return LFAMD_OK;
  const int64_t words = bytes / 2;  // every element type is a multiple of 2 bytes
  const int blocks = (int)std::min<int64_t>(1024, (words + 255) / 256);
  hipLaunchKernelGGL(fill_zero_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, static_cast<uint16_t*>(p), words);
  return check_launch("zero fill");
}

int bwd_common(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk,
               const Dims& d, void* ws, size_t wsBytes, void* stream, bool doDq, bool doDk,
               const char* who) {
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "%s: unsupported dtype %d", who, dtype);
  int s = check_dims(d, who);
  if (s) return s;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t es = dtype_size(dtype);
  if (d.BH() == 0 || d.C == 0) return ok();
  if (d.M == 0 || d.N == 0) {
    // Empty reduction: the gradients are zero (the output is empty when N or M is 0).
    if (doDq && (s = zero_fill(dq, d.BH() * d.N * d.C * (int64_t)es, st))) return s;
    if (doDk && (s = zero_fill(dk, d.BH() * d.C * d.M * (int64_t)es, st))) return s;
    return ok();
  }
  if (!g || !q || !k || (doDq && !dq) || (doDk && !dk)) return fail(LFAMD_ERR_ARG, "%s: null pointer", who);
  const size_t acc = dtype == LFAMD_F64 ? 8 : 4;
  if (doDk && ws && (reinterpret_cast<uintptr_t>(ws) & (acc - 1)))
    return fail(LFAMD_ERR_ARG, "%s: workspace not %zu-byte aligned", who, acc);
  if (b2_ok(dtype, d.BH(), d.N, d.M, d.C) && (reinterpret_cast<uintptr_t>(q) & 3) == 0)
    return b2_launch(dtype, g, q, k, doDq ? dq : nullptr, doDk ? dk : nullptr, ws, wsBytes, d.BH(), d.N, d.M, d.C,
                     st, who);
  if (bcast_bwd_ok(dtype, d, g)) {
    const BcPlan sp = plan_bcast(d, doDk);
    if (doDk && (!ws || wsBytes < sp.partialElems * 4))
      return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, sp.partialElems * 4, wsBytes);
    if (doDq && doDk) return launch_bcast_bwd<true, true>(dtype, g, q, k, dq, dk, ws, d, sp, st);
    if (doDq) return launch_bcast_bwd<true, false>(dtype, g, q, k, dq, dk, ws, d, sp, st);
    return launch_bcast_bwd<false, true>(dtype, g, q, k, dq, dk, ws, d, sp, st);
  }
  if (mb_bwd_ok(dtype, d, g)) {
    const MbPlan mp = plan_mb(d, doDk);
    if (doDk && (!ws || wsBytes < mp.partialElems * 4))
      return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, mp.partialElems * 4, wsBytes);
    if (doDq && doDk) return launch_mb<true, true>(dtype, g, q, k, dq, dk, ws, d, mp, st);
    if (doDq) return launch_mb<true, false>(dtype, g, q, k, dq, dk, ws, d, mp, st);
    return launch_mb<false, true>(dtype, g, q, k, dq, dk, ws, d, mp, st);
  }
  const BwdPlan p = plan_bwd(d, doDq, doDk, acc, dtype == LFAMD_F16 ? 2 : acc);
  if (doDk) {
    const size_t need = p.partialElems * acc;
    if (!ws || wsBytes < need)
      return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, need, wsBytes);
  }
  if (doDq && doDk) return launch_bwd<true, true>(dtype, g, q, k, dq, dk, ws, d, p, st);
  if (doDq) return launch_bwd<true, false>(dtype, g, q, k, dq, dk, ws, d, p, st);
  return launch_bwd<false, true>(dtype, g, q, k, dq, dk, ws, d, p, st);
}

}  // namespace
}  // namespace lfamd

using namespace lfamd;

extern "C" {

int lfamd_laplace_forward(int dtype, const void* query, const void* key, void* output,
                          int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                          int64_t channels, void* stream) {
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "laplace forward: unsupported dtype %d", dtype);
  const Dims d{batch, heads, q_len, k_len, channels};
  int s = check_dims(d, "laplace forward");
  if (s) return s;
  if (empty(d)) return ok();
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d.C == 0) return zero_fill(output, d.BH() * d.N * d.M * (int64_t)dtype_size(dtype), st);
  if (!query || !key || !output) return fail(LFAMD_ERR_ARG, "laplace forward: null pointer");
  if (f2_ok(dtype, d.BH(), d.N, d.M, d.C, query))
    return f2_launch(dtype, false, query, key, output, d.BH(), d.N, d.C, 0.0f, st);
  if (f3_ok(dtype, d.BH(), d.N, d.M, d.C, query, output))
    return f3_launch(dtype, query, key, output, d.BH(), d.N, d.M, d.C, st);
  if (fwd_bcast_ok(dtype, d, query, dtype_size(dtype))) {
    switch (dtype) {
      case LFAMD_F32: return launch_fwd_bcast<float>(query, key, output, d, st);
      case LFAMD_F16: return launch_fwd_bcast<f16s>(query, key, output, d, st);
      default: return launch_fwd_bcast<bf16s>(query, key, output, d, st);
    }
  }
  switch (dtype) {
    case LFAMD_F32: return launch_fwd<float>(query, key, output, d, st);
    case LFAMD_F16: return launch_fwd<f16s>(query, key, output, d, st);
    case LFAMD_BF16: return launch_fwd<bf16s>(query, key, output, d, st);
    default: return launch_fwd<double>(query, key, output, d, st);
  }
}

int lfamd_laplace_backward_query(int dtype, const void* grad_output, const void* query,
                                 const void* key, void* grad_query, int64_t batch,
                                 int64_t heads, int64_t q_len, int64_t k_len,
                                 int64_t channels, void* stream) {
  return bwd_common(dtype, grad_output, query, key, grad_query, nullptr,
                    Dims{batch, heads, q_len, k_len, channels}, nullptr, 0, stream, true, false,
                    "laplace backward_query");
}

size_t lfamd_laplace_backward_workspace_size(int dtype, int64_t batch, int64_t heads,
                                             int64_t q_len, int64_t k_len, int64_t channels) {
  const Dims d{batch, heads, q_len, k_len, channels};
  if (!valid_dtype(dtype) || check_dims(d, "workspace") || d.BH() == 0 || d.N == 0 || d.M == 0 || d.C == 0)
    return 0;
  const size_t acc = dtype == LFAMD_F64 ? 8 : 4;
  // Any of the backward paths may run (which one also depends on pointer alignment).
  size_t bytes = plan_bwd(d, true, true, acc, dtype == LFAMD_F16 ? 2 : acc).partialElems * acc;
  if (dtype != LFAMD_F64) bytes = std::max(bytes, plan_bcast(d, true).partialElems * 4);
  if (dtype != LFAMD_F64 && d.M >= 17 && d.M <= 8 * kMbMC)
    bytes = std::max(bytes, plan_mb(d, true).partialElems * 4);
  if (b2_ok(dtype, d.BH(), d.N, d.M, d.C)) bytes = std::max(bytes, b2_workspace_elems(d.BH(), d.N, d.M, d.C) * 4);
  return bytes;
}

int lfamd_laplace_backward_key(int dtype, const void* grad_output, const void* query,
                               const void* key, void* grad_key, int64_t batch,
                               int64_t heads, int64_t q_len, int64_t k_len,
                               int64_t channels, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return bwd_common(dtype, grad_output, query, key, nullptr, grad_key,
                    Dims{batch, heads, q_len, k_len, channels}, workspace, workspace_bytes, stream,
                    false, true, "laplace backward_key");
}

int lfamd_laplace_backward(int dtype, const void* grad_output, const void* query,
                           const void* key, void* grad_query, void* grad_key,
                           int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                           int64_t channels, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return bwd_common(dtype, grad_output, query, key, grad_query, grad_key,
                    Dims{batch, heads, q_len, k_len, channels}, workspace, workspace_bytes, stream,
                    true, true, "laplace backward");
}

int lfamd_laplace_kernel_forward(int dtype, const void* query, const void* key, float* output,
                                 int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                                 int64_t channels, float scale, void* stream) {
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "laplace kernel forward: unsupported dtype %d", dtype);
  const Dims d{batch, heads, q_len, k_len, channels};
  int s = check_dims(d, "laplace kernel forward");
  if (s) return s;
  if (empty(d)) return ok();
  if (d.C == 0 || !fwd_bcast_ok(dtype, d, query, sizeof(float)))
    return fail(LFAMD_ERR_UNSUPPORTED, "laplace kernel forward: no fused path for dtype %d, M=%lld, C=%lld",
                dtype, (long long)d.M, (long long)d.C);
  if (!query || !key || !output) return fail(LFAMD_ERR_ARG, "laplace kernel forward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (f2_ok(dtype, d.BH(), d.N, d.M, d.C, query))
    return f2_launch(dtype, true, query, key, output, d.BH(), d.N, d.C, scale, st);
  switch (dtype) {
    case LFAMD_F32: return launch_fwd_bcast<float, kEpiExp>(query, key, output, d, st, scale);
    case LFAMD_F16: return launch_fwd_bcast<f16s, kEpiExp>(query, key, output, d, st, scale);
    default: return launch_fwd_bcast<bf16s, kEpiExp>(query, key, output, d, st, scale);
  }
}

int lfamd_laplace_kernel_forward_multi(int dtype, int num_sources, const void* const* queries,
                                       const int64_t* q_lens, const void* key, float* const* outputs,
                                       int64_t batch, int64_t heads, int64_t k_len, int64_t channels,
                                       float scale, void* stream) {
  const char* who = "laplace kernel forward (several sources)";
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "%s: unsupported dtype %d", who, dtype);
  if (num_sources < 1 || num_sources > 3 || !queries || !q_lens || !outputs)
    return fail(LFAMD_ERR_ARG, "%s: 1 to 3 sources with their arrays expected", who);
  for (int i = 0; i < num_sources; ++i)
    if (q_lens[i] < 1 || !queries[i] || !outputs[i]) return fail(LFAMD_ERR_ARG, "%s: source %d empty or null", who, i);
  const Dims d{batch, heads, 1, k_len, channels};
  int s = check_dims(d, who);
  if (s) return s;
  if (d.BH() == 0) return ok();
  if (!key) return fail(LFAMD_ERR_ARG, "%s: null pointer", who);
  for (int i = 0; i < num_sources; ++i)
    if (!f2_ok(dtype, d.BH(), q_lens[i], d.M, d.C, queries[i]))
      return fail(LFAMD_ERR_UNSUPPORTED, "%s: no single-launch path (dtype %d, M=%lld, C=%lld, source %d)", who,
                  dtype, (long long)d.M, (long long)d.C, i);
  return f2_launch_multi(dtype, num_sources, queries, q_lens, key, outputs, d.BH(), d.C, scale,
                         static_cast<hipStream_t>(stream));
}

namespace {
// The segmented fused-kernel backward applies: fp16, M = 49, C % 64 == 0,
// 1 to 3 sources of at least one row, 4-byte aligned queries.
int multi_bwd_check(int dtype, int nsrc, const int64_t* q_lens, const void* const* queries, const Dims& d,
                    const char* who) {
  if (nsrc < 1 || nsrc > 3 || !q_lens) return fail(LFAMD_ERR_ARG, "%s: 1 to 3 sources expected", who);
  for (int i = 0; i < nsrc; ++i)
    if (q_lens[i] < 1) return fail(LFAMD_ERR_ARG, "%s: source %d has no rows", who, i);
  if (dtype != LFAMD_F16 || d.M != 49 || d.C <= 0 || d.C % 64 != 0 || d.BH() < 1 || d.C / 64 > 65535)
    return fail(LFAMD_ERR_UNSUPPORTED, "%s: no single-launch path (dtype %d, M=%lld, C=%lld)", who, dtype,
                (long long)d.M, (long long)d.C);
  // The kernel holds row counts and its linear workgroup id in 32-bit ints.
  for (int i = 0; i < nsrc; ++i)
    if (q_lens[i] > INT32_MAX / 2)
      return fail(LFAMD_ERR_UNSUPPORTED, "%s: source %d has %lld rows (at most %d)", who, i, (long long)q_lens[i],
                  INT32_MAX / 2);
  if (b2_multi_workgroups(nsrc, q_lens, d.BH(), d.C) > INT32_MAX)
    return fail(LFAMD_ERR_UNSUPPORTED, "%s: too many workgroups for one launch", who);
  if (queries)
    for (int i = 0; i < nsrc; ++i)
      if (reinterpret_cast<uintptr_t>(queries[i]) & 3)
        return fail(LFAMD_ERR_UNSUPPORTED, "%s: query %d not 4-byte aligned", who, i);
  return LFAMD_OK;
}
}  // namespace

size_t lfamd_laplace_kernel_backward_multi_workspace_size(int dtype, int num_sources, const int64_t* q_lens,
                                                          int64_t batch, int64_t heads, int64_t k_len,
                                                          int64_t channels) {
  const Dims d{batch, heads, 1, k_len, channels};
  if (check_dims(d, "laplace kernel backward (several sources)") ||
      multi_bwd_check(dtype, num_sources, q_lens, nullptr, d, "laplace kernel backward (several sources)"))
    return 0;
  return b2_workspace_elems_multi(num_sources, q_lens, d.BH(), d.C) * 4;
}

int lfamd_laplace_kernel_backward_multi(int dtype, int num_sources, const float* const* grad_kernels,
                                        const float* const* kernels, const void* const* queries,
                                        const int64_t* q_lens, const void* key, void* const* grad_queries,
                                        void* grad_key, int64_t batch, int64_t heads, int64_t k_len,
                                        int64_t channels, float scale, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  const char* who = "laplace kernel backward (several sources)";
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "%s: unsupported dtype %d", who, dtype);
  const Dims d{batch, heads, 1, k_len, channels};
  int s = check_dims(d, who);
  if (s) return s;
  if (!grad_kernels || !kernels || !queries || !grad_queries || !key || !grad_key)
    return fail(LFAMD_ERR_ARG, "%s: null pointer", who);
  if ((s = multi_bwd_check(dtype, num_sources, q_lens, queries, d, who))) return s;
  for (int i = 0; i < num_sources; ++i)
    if (!grad_kernels[i] || !kernels[i] || !grad_queries[i]) return fail(LFAMD_ERR_ARG, "%s: null pointer", who);
  return b2_launch_multi(num_sources, grad_kernels, kernels, queries, grad_queries, q_lens, key, grad_key, workspace,
                         workspace_bytes, d.BH(), d.C, scale, static_cast<hipStream_t>(stream), who);
}

int lfamd_laplace_kernel_backward(int dtype, const float* grad_kernel, const float* kernel,
                                  const void* query, const void* key, void* grad_query, void* grad_key,
                                  int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                                  int64_t channels, float scale, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  const char* who = "laplace kernel backward";
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "%s: unsupported dtype %d", who, dtype);
  const Dims d{batch, heads, q_len, k_len, channels};
  int s = check_dims(d, who);
  if (s) return s;
  const bool doDq = grad_query != nullptr, doDk = grad_key != nullptr;
  if (d.BH() == 0 || d.C == 0 || !(doDq || doDk)) return ok();
  if (d.N == 0 || !kernel_bwd_ok(dtype, d))
    return fail(LFAMD_ERR_UNSUPPORTED, "%s: no fused path for dtype %d, N=%lld, M=%lld", who, dtype,
                (long long)d.N, (long long)d.M);
  if (!grad_kernel || !kernel || !query || !key) return fail(LFAMD_ERR_ARG, "%s: null pointer", who);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (b2_ok(dtype, d.BH(), d.N, d.M, d.C) && (reinterpret_cast<uintptr_t>(query) & 3) == 0)
    return b2_launch(dtype, nullptr, query, key, grad_query, grad_key, workspace, workspace_bytes, d.BH(), d.N, d.M,
                     d.C, st, who, B2Grad{grad_kernel, kernel, scale});
  const KernGrad kg{grad_kernel, kernel, scale};
  if (!kernel_bwd_bcast(d)) {
    const MbPlan mp = plan_mb(d, doDk);
    if (doDk && (!workspace || workspace_bytes < mp.partialElems * 4))
      return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, mp.partialElems * 4,
                  workspace_bytes);
    if (doDq && doDk)
      return launch_mb_t<f16s, true, true, kGradKernel>(nullptr, query, key, grad_query, grad_key, workspace, d, mp, st, kg);
    if (doDq)
      return launch_mb_t<f16s, true, false, kGradKernel>(nullptr, query, key, grad_query, nullptr, workspace, d, mp, st, kg);
    return launch_mb_t<f16s, false, true, kGradKernel>(nullptr, query, key, nullptr, grad_key, workspace, d, mp, st, kg);
  }
  const BcPlan sp = plan_bcast(d, doDk);
  if (doDk && (!workspace || workspace_bytes < sp.partialElems * 4))
    return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, sp.partialElems * 4,
                workspace_bytes);
  if (doDq && doDk)
    return launch_bcast_bwd<true, true, kGradKernel>(LFAMD_F16, nullptr, query, key, grad_query, grad_key, workspace, d, sp, st, kg);
  if (doDq)
    return launch_bcast_bwd<true, false, kGradKernel>(LFAMD_F16, nullptr, query, key, grad_query, nullptr, workspace, d, sp, st, kg);
  return launch_bcast_bwd<false, true, kGradKernel>(LFAMD_F16, nullptr, query, key, nullptr, grad_key, workspace, d, sp, st, kg);
}

int lfamd_laplace_reduce_forward(int dtype, const void* query, const void* key,
                                 void* output, int64_t batch, int64_t heads,
                                 int64_t q_len, int64_t k_len, int64_t channels,
                                 void* stream) {
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "laplace reduce_forward: unsupported dtype %d", dtype);
  const Dims d{batch, heads, q_len, k_len, channels};
  int s = check_dims(d, "laplace reduce_forward");
  if (s) return s;
  if (empty(d)) return ok();
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d.C == 0) return zero_fill(output, d.BH() * d.N * d.M * (int64_t)dtype_size(dtype), st);
  if (!query || !key || !output) return fail(LFAMD_ERR_ARG, "laplace reduce_forward: null pointer");
  const int64_t total = d.BH() * d.N * d.M;
  const int bd = (int)std::min<int64_t>(d.C, 256);
  const unsigned blocks = (unsigned)std::min<int64_t>(total, 1 << 20);
#define LFAMD_REDUCE(T)                                                                        \
  hipLaunchKernelGGL(laplace_reduce_fwd_kernel<T>, dim3(blocks), dim3(bd), 0, st,              \
                     static_cast<const T*>(query), static_cast<const T*>(key), static_cast<T*>(output), \
                     total, (int)d.N, (int)d.M, (int)d.C)
  switch (dtype) {
    case LFAMD_F32: LFAMD_REDUCE(float); break;
    case LFAMD_F16: LFAMD_REDUCE(f16s); break;
    case LFAMD_BF16: LFAMD_REDUCE(bf16s); break;
    default: LFAMD_REDUCE(double); break;
  }
#undef LFAMD_REDUCE
  return check_launch("laplace reduce_forward");
}

}  // extern "C"

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
// Forward, fp32-key path. A pre-pass writes the key once per call as fp32 rows
// padded to `Mp` columns; the forward then reads each channel's JB key values
// with one scalar load (wave-uniform, into SGPRs) and spends two full-rate VALU
// operations per (c, j): v_sub_f32 with the SGPR operand and v_add_f32 with |.|.
// The query row of the lane stays in VGPRs (widened once per channel).
// ---------------------------------------------------------------------------
// Key pre-pass of the SGPR forward: kf[bh][b][c][t] = f32(key[bh][c][b*JB + t]) for
// column block b, channel c < KCp and t < JBS (JB rounded up to 8), zero outside
// the key. Each channel of a block is one run of JBS floats, and two channels of
// an 8-wide block are one 16-dword run: few, wide scalar loads.
template <typename T>
__global__ void __launch_bounds__(256)
laplace_key_f32_kernel(const T* __restrict__ key, float* __restrict__ kf, int64_t BH, int C, int KCp, int M,
                       int JB, int JBS, int nJB) {
  const int64_t total = BH * nJB * KCp * JBS;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = e / JBS;
    const int t = (int)(e - r * JBS);
    const int c = (int)(r % KCp);
    r /= KCp;
    const int b = (int)(r % nJB);
    const int64_t bh = r / nJB;
    const int col = b * JB + t;
    kf[e] = (t < JB && col < M && c < C) ? (float)to_acc(key[(bh * C + c) * M + col]) : 0.0f;
  }
}

constexpr int kFwdSgQV = 16;  // max 16-byte query vectors per row (256 bytes)

// NV = 16-byte query vectors per row (C <= NV*CK; the key copy is zero-padded
// to NV*CK channels and the query vectors past C are zero).
template <typename T, int JB, int NV>
__global__ void __launch_bounds__(1024)
laplace_fwd_sgpr_kernel(const T* __restrict__ query, const float* __restrict__ kf, T* __restrict__ out,
                        int N, int M, int C, int nJB, int colsPerGroup, int flags) {
  constexpr int CK = QChunk<T>::value;
  constexpr int KCp = NV * CK;
  constexpr int JBS = round_up(JB, 8);
  const int W = blockDim.x >> 6;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.z;
  const int jg0 = blockIdx.y * colsPerGroup;
  const int jblk = uniform(blockIdx.y * W + wave);
  const int row0 = blockIdx.x * 64;
  const int row = row0 + lane;
  const int nv = C / CK;

  extern __shared__ __align__(16) unsigned char smem[];
  T* ot = reinterpret_cast<T*>(smem);  // [64][colsPerGroup]

  // The lane's query row (rows past N read row N-1 and are never stored).
  uint4 qv[NV];
  const uint4* src = reinterpret_cast<const uint4*>(query + ((size_t)bh * N + min(row, N - 1)) * C);
#pragma unroll
  for (int t = 0; t < NV; ++t) qv[t] = t < nv ? src[t] : uint4{0u, 0u, 0u, 0u};

  // This wave's column block: channel c's JB key values at kb + c*JBS.
  const float* kb = kf + ((size_t)bh * nJB + min(jblk, nJB - 1)) * KCp * JBS;
  float acc[JB];
#pragma unroll
  for (int j = 0; j < JB; ++j) acc[j] = 0.0f;
  // Channels are processed in groups of KG: the group's key values are loaded
  // (scalar loads, whole 16-byte groups) before any of them is used, so each
  // group costs one scalar-load latency. Scalar loads may return out of order,
  // so every wait is a wait for all of them; one wait per channel would expose
  // the latency channel by channel.
  constexpr int KG = (JBS >= 16 ? 4 : 8) < CK ? (JBS >= 16 ? 4 : 8) : CK;
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    const uint32_t w[4] = {qv[t].x, qv[t].y, qv[t].z, qv[t].w};
#pragma unroll
    for (int u0 = 0; u0 < CK; u0 += KG) {
      float kv[KG][JBS];
#pragma unroll
      for (int g = 0; g < KG; ++g) {
        const float4* kr4 = reinterpret_cast<const float4*>(kb + (t * CK + u0 + g) * JBS);
#pragma unroll
        for (int r = 0; r < JBS / 4; ++r) {
          const float4 v = kr4[r];
          kv[g][4 * r] = v.x; kv[g][4 * r + 1] = v.y; kv[g][4 * r + 2] = v.z; kv[g][4 * r + 3] = v.w;
        }
      }
#pragma unroll
      for (int g = 0; g < KG; ++g) {
        const int u = u0 + g;
        float q;
        if constexpr (std::is_same<T, f16s>::value)
          q = (float)__builtin_bit_cast(_Float16, (uint16_t)((u & 1) ? (w[u >> 1] >> 16) : (w[u >> 1] & 0xffffu)));
        else if constexpr (std::is_same<T, bf16s>::value)
          q = __builtin_bit_cast(float, (u & 1) ? (w[u >> 1] & 0xffff0000u) : (w[u >> 1] << 16));
        else
          q = __builtin_bit_cast(float, w[u]);
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[j] += fabsf(q - kv[g][j]);
      }
    }
  }

#pragma unroll
  for (int j = 0; j < JB; ++j) ot[lane * colsPerGroup + wave * JB + j] = from_acc<T>(acc[j]);
  __syncthreads();
  const int colsValid = min(colsPerGroup, M - jg0);
  const int rowsValid = min(64, N - row0);
  T* ob = out + ((size_t)bh * N + row0) * M + jg0;
  if (colsPerGroup == M) {
    const int total = rowsValid * M;
    int done = 0;
    if (flags & kFwdVecOut) {
      constexpr int VE = 16 / (int)sizeof(T);
      const int nvv = total / VE;
      for (int e = threadIdx.x; e < nvv; e += blockDim.x)
        reinterpret_cast<uint4*>(ob)[e] = reinterpret_cast<const uint4*>(ot)[e];
      done = nvv * VE;
    }
    for (int e = done + threadIdx.x; e < total; e += blockDim.x) ob[e] = ot[e];
  } else {
    for (int r = wave; r < rowsValid; r += W)
      for (int cidx = lane; cidx < colsValid; cidx += 64) ob[(size_t)r * M + cidx] = ot[r * colsPerGroup + cidx];
  }
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
// fp16 backward with the grad_output rows in SGPRs (M == MC known at compile
// time). A group of R2 rows (2 when MC is odd, so that the group starts on a
// dword) is MC*R2/2 dwords: one scalar load, wave-uniform, consumed directly by
// v_fma_mix_f32 with the half selected statically. No LDS traffic for
// grad_output, no VGPRs for it, so 3 waves fit per SIMD. Requires N*MC even
// and a 4-byte aligned grad_output (checked on the host).
// ---------------------------------------------------------------------------
constexpr int kSgRB = 8;  // rows per query-prefetch batch (multiple of 2)

// Waves per workgroup of the SGPR path: the MC <= 49 variants fit 128 VGPRs
// (4 waves per SIMD, one 16-wave workgroup per CU); MC = 64 needs ~154 (3 waves).
__host__ __device__ constexpr int sgpr_max_waves(int mc) { return mc <= 49 ? 16 : 12; }

template <int MC, bool DQ, bool DK>
__global__ void __launch_bounds__(64 * sgpr_max_waves(MC))
laplace_bwd_sgpr_kernel(const f16s* __restrict__ gout, const f16s* __restrict__ query,
                        const f16s* __restrict__ key, f16s* __restrict__ dq, f16s* __restrict__ dk,
                        float* __restrict__ partial, int N, int C, int rowsPerWave) {
  constexpr int R2 = (MC & 1) ? 2 : 1;
  constexpr int GW = MC * R2 / 2;  // dwords per row group
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
  float* ksm = reinterpret_cast<float*>(smem);  // [MC][64] scaled key tile
  float* red = ksm + MC * 64;                   // [MC][64] (DK)

  const f16s* qb = query + (size_t)bh * N * C;
  const uint32_t* gw = reinterpret_cast<const uint32_t*>(gout + (size_t)bh * N * MC);
  const f16s* kb = key + (size_t)bh * C * MC;

  for (int t = threadIdx.x; t < 64 * MC; t += blockDim.x) {
    const int cl = t & 63, j = t >> 6;  // lane-fastest: conflict-free LDS writes
    const int cc = cb * 64 + cl;
    ksm[j * 64 + cl] = cc < C ? to_acc(kb[(size_t)cc * MC + j]) * 16777216.0f : 0.0f;
  }
  __syncthreads();
  float kreg[MC], dka[MC];
#pragma unroll
  for (int j = 0; j < MC; ++j) {
    kreg[j] = ksm[j * 64 + lane];
    dka[j] = 0.0f;
  }

  uint16_t qpre[kSgRB];
  auto fetch_q = [&](int rb) {
#pragma unroll
    for (int r = 0; r < kSgRB; ++r) qpre[r] = (cval && rb + r < rowEnd) ? qb[(size_t)(rb + r) * C + c].bits : 0;
  };
  // The scalar loads of grad rows would each miss to HBM (every row is read by
  // one wave only); one vector load per 128-byte line a batch ahead pulls the
  // next batch's rows into L2 first. The loaded words feed a sink that is
  // stored only under a condition the host never sets (rowsPerWave < 0).
  uint32_t sink = 0;
  auto warm_g = [&](int rb) {
    const int words = min(kSgRB, rowEnd - rb) * MC / 2;
    const uint32_t* nb = gw + (size_t)rb * MC / 2;
    if (lane * 32 < words) sink ^= nb[lane * 32];
  };
  if (rowBeg < rowEnd) {
    fetch_q(rowBeg);
    warm_g(rowBeg);
  }
  for (int rb = rowBeg; rb < rowEnd; rb += kSgRB) {
    float qcur[kSgRB];
#pragma unroll
    for (int r = 0; r < kSgRB; ++r) {
      qcur[r] = (float)__builtin_bit_cast(_Float16, qpre[r]) * 16777216.0f;
      // Keep the widened value in a register: folding the widening into each
      // subtract (v_fma_mix_f32) would put a wait state after every one of them.
      asm volatile("" : "+v"(qcur[r]));
    }
    if (rb + kSgRB < rowEnd) {
      fetch_q(rb + kSgRB);
      warm_g(rb + kSgRB);
    }
#pragma unroll
    for (int r0 = 0; r0 < kSgRB; r0 += R2) {
      if (rb + r0 >= rowEnd) break;  // uniform; rows come in whole groups of R2
      const uint32_t* gp = gw + (size_t)(rb + r0) * MC / 2;
      uint32_t g[GW];
#pragma unroll
      for (int t = 0; t < GW; ++t) g[t] = gp[t];
#pragma unroll
      for (int rr = 0; rr < R2; ++rr) {
        const float qv = qcur[r0 + rr];
        float dqa = 0.0f;
#pragma unroll
        for (int j = 0; j < MC; ++j) {
          const int h = rr * MC + j;  // half index inside the row group (compile-time)
          const float s = __builtin_amdgcn_fmed3f(qv - kreg[j], -1.0f, 1.0f);
          if (h & 1) {
            if (DQ) dqa = mix_fma_fs<1>(s, g[h >> 1], dqa);
            if (DK) dka[j] = mix_fms_fs<1>(s, g[h >> 1], dka[j]);
          } else {
            if (DQ) dqa = mix_fma_fs<0>(s, g[h >> 1], dqa);
            if (DK) dka[j] = mix_fms_fs<0>(s, g[h >> 1], dka[j]);
          }
        }
        if (DQ && cval) dq[((size_t)bh * N + rb + r0 + rr) * C + c] = from_acc<f16s>(dqa);
      }
    }
  }

  if (rowsPerWave < 0) partial[lane] = (float)sink;  // never taken; keeps the warming loads

  if (DK) {
    for (int w = 0; w < W; ++w) {
      if (wave == w) {
#pragma unroll
        for (int j = 0; j < MC; ++j) red[j * 64 + lane] = (w == 0 ? 0.0f : red[j * 64 + lane]) + dka[j];
      }
      __syncthreads();
    }
    float* pb = partial + ((size_t)slice * nx + x) * 64 * MC;
    for (int t = threadIdx.x; t < 64 * MC; t += blockDim.x) {
      const int cl = t / MC, j = t - cl * MC;
      pb[t] = red[j * 64 + cl];
    }
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

bool fwd_sgpr_ok(int dtype, const Dims& d, const void* q) {
  if (dtype == LFAMD_F64) return false;
  const int64_t ck = 16 / (int64_t)dtype_size(dtype);
  return d.C % ck == 0 && d.C / ck <= kFwdSgQV && (reinterpret_cast<uintptr_t>(q) & 15) == 0;
}

// 16-byte query vectors per row rounded up to the instantiated 2, 4, 8, 16.
int fwd_nv(int dtype, int64_t C) {
  const int64_t ck = 16 / (int64_t)dtype_size(dtype);
  const int64_t v = (C + ck - 1) / ck;
  return v <= 2 ? 2 : v <= 4 ? 4 : v <= 8 ? 8 : 16;
}

int pick_fwd_sgpr_jb(int64_t M);

size_t fwd_workspace_bytes(int dtype, const Dims& d) {
  if (dtype == LFAMD_F64) return 0;
  const int64_t kcp = (int64_t)fwd_nv(dtype, d.C) * (16 / (int64_t)dtype_size(dtype));
  const int jb = pick_fwd_sgpr_jb(d.M);
  const int64_t njb = (d.M + jb - 1) / jb;
  return (size_t)d.BH() * njb * kcp * round_up(jb, 8) * sizeof(float);
}

template <typename T, int JB, int NV>
int launch_fwd_sgpr_jb(const T* q, const T* k, T* o, float* kf, const Dims& d, hipStream_t st) {
  const int M = (int)d.M, N = (int)d.N, C = (int)d.C;
  const int KCp = NV * QChunk<T>::value;
  constexpr int JBS = round_up(JB, 8);
  const int nJB = ceil_div(M, JB);
  const int pblocks = (int)std::min<int64_t>(4096, (d.BH() * nJB * KCp * JBS + 255) / 256);
  hipLaunchKernelGGL(laplace_key_f32_kernel<T>, dim3(pblocks), dim3(256), 0, st, k, kf, d.BH(), C, KCp, M, JB, JBS,
                     nJB);
  int s = check_launch("laplace forward key conversion");
  if (s) return s;
  const int W = std::min(16, ceil_div(M, JB));
  const int cols = W * JB;
  dim3 grid(ceil_div(N, 64), ceil_div(M, cols), (unsigned)d.BH());
  int flags = 0;
  if (cols == M && (reinterpret_cast<uintptr_t>(o) & 15) == 0 && ((size_t)N * M * sizeof(T)) % 16 == 0)
    flags |= kFwdVecOut;
  hipLaunchKernelGGL((laplace_fwd_sgpr_kernel<T, JB, NV>), grid, dim3(64 * W), (size_t)64 * cols * sizeof(T), st, q,
                     kf, o, N, M, C, nJB, cols, flags);
  return check_launch("laplace forward");
}

// Column block of the SGPR forward: at most 16 (32 fp32 key values per channel
// would not fit the scalar register file once several channels are in flight).
int pick_fwd_sgpr_jb(int64_t M) {
  const int jb = pick_fwd_jb(M);
  return jb > 16 ? 16 : jb;
}

template <typename T, int NV>
int launch_fwd_sgpr_nv(const T* q, const T* k, T* o, float* kf, const Dims& d, hipStream_t st) {
  switch (pick_fwd_sgpr_jb(d.M)) {
    case 7: return launch_fwd_sgpr_jb<T, 7, NV>(q, k, o, kf, d, st);
    case 8: return launch_fwd_sgpr_jb<T, 8, NV>(q, k, o, kf, d, st);
    default: return launch_fwd_sgpr_jb<T, 16, NV>(q, k, o, kf, d, st);
  }
}

template <typename T>
int launch_fwd_sgpr(const void* q, const void* k, void* o, void* ws, int nv, const Dims& d, hipStream_t st) {
  const T* qq = static_cast<const T*>(q);
  const T* kk = static_cast<const T*>(k);
  T* oo = static_cast<T*>(o);
  float* kf = static_cast<float*>(ws);
  switch (nv) {
    case 2: return launch_fwd_sgpr_nv<T, 2>(qq, kk, oo, kf, d, st);
    case 4: return launch_fwd_sgpr_nv<T, 4>(qq, kk, oo, kf, d, st);
    case 8: return launch_fwd_sgpr_nv<T, 8>(qq, kk, oo, kf, d, st);
    default: return launch_fwd_sgpr_nv<T, 16>(qq, kk, oo, kf, d, st);
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

// Plan of the SGPR fast path: 3 waves per SIMD resident, up to 12 waves per workgroup.
struct SgPlan {
  int W, nx, rowsPerWave, ncb;
  size_t lds, partialElems;
};

bool sgpr_path_ok(int dtype, const Dims& d, const void* g) {
  if (dtype != LFAMD_F16) return false;
  if (!(d.M == 16 || d.M == 32 || d.M == 49 || d.M == 64)) return false;
  if ((d.N * d.M) % 2 != 0) return false;
  return (reinterpret_cast<uintptr_t>(g) & 3) == 0;
}

SgPlan plan_sgpr(const Dims& d, bool dkey) {
  SgPlan p{};
  p.ncb = ceil_div((int)d.C, 64);
  const int64_t slices = d.BH() * p.ncb;
  const int N = (int)std::max<int64_t>(d.N, 1);
  const int wmax = sgpr_max_waves((int)d.M);
  const int target = wmax * num_cus();
  int64_t wps = std::max<int64_t>(1, ceil_div(target, (int)std::min<int64_t>(slices, target)));
  wps = std::min<int64_t>(wps, ceil_div(N, 8));
  const int W = (int)std::min<int64_t>(wmax, wps);
  p.W = W;
  p.nx = ceil_div((int)wps, W);
  p.rowsPerWave = round_up(ceil_div(N, p.nx * W), 2);
  p.lds = (size_t)d.M * 64 * 4 * (dkey ? 2 : 1);
  p.partialElems = dkey ? (size_t)slices * p.nx * 64 * (size_t)d.M : 0;
  return p;
}

template <int MC, bool DQ, bool DK>
int launch_sgpr_mc(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, const Dims& d,
                   const SgPlan& p, hipStream_t st) {
  dim3 grid(p.nx, p.ncb, (unsigned)d.BH());
  hipLaunchKernelGGL((laplace_bwd_sgpr_kernel<MC, DQ, DK>), grid, dim3(64 * p.W), p.lds, st,
                     static_cast<const f16s*>(g), static_cast<const f16s*>(q), static_cast<const f16s*>(k),
                     static_cast<f16s*>(dq), static_cast<f16s*>(dk), static_cast<float*>(ws), (int)d.N, (int)d.C,
                     p.rowsPerWave);
  int s = check_launch("laplace backward");
  if (s || !DK) return s;
  dim3 rgrid(ceil_div(64 * MC, 256), p.ncb, (unsigned)d.BH());
  hipLaunchKernelGGL(laplace_dk_reduce_kernel<f16s>, rgrid, dim3(256), 0, st, static_cast<const float*>(ws),
                     static_cast<f16s*>(dk), p.nx, MC, (int)d.C);
  return check_launch("laplace backward_key reduction");
}

template <bool DQ, bool DK>
int launch_sgpr(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, const Dims& d,
                const SgPlan& p, hipStream_t st) {
  switch (d.M) {
    case 16: return launch_sgpr_mc<16, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    case 32: return launch_sgpr_mc<32, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    case 49: return launch_sgpr_mc<49, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
    default: return launch_sgpr_mc<64, DQ, DK>(g, q, k, dq, dk, ws, d, p, st);
  }
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
  if (sgpr_path_ok(dtype, d, g)) {
    const SgPlan sp = plan_sgpr(d, doDk);
    if (doDk && (!ws || wsBytes < sp.partialElems * 4))
      return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, sp.partialElems * 4, wsBytes);
    if (doDq && doDk) return launch_sgpr<true, true>(g, q, k, dq, dk, ws, d, sp, st);
    if (doDq) return launch_sgpr<true, false>(g, q, k, dq, dk, ws, d, sp, st);
    return launch_sgpr<false, true>(g, q, k, dq, dk, ws, d, sp, st);
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

size_t lfamd_laplace_forward_workspace_size(int dtype, int64_t batch, int64_t heads, int64_t q_len,
                                            int64_t k_len, int64_t channels) {
  const Dims d{batch, heads, q_len, k_len, channels};
  if (!valid_dtype(dtype) || check_dims(d, "workspace") || empty(d) || d.C == 0) return 0;
  return fwd_workspace_bytes(dtype, d);
}

int lfamd_laplace_forward(int dtype, const void* query, const void* key, void* output,
                          int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                          int64_t channels, void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(dtype)) return fail(LFAMD_ERR_DTYPE, "laplace forward: unsupported dtype %d", dtype);
  const Dims d{batch, heads, q_len, k_len, channels};
  int s = check_dims(d, "laplace forward");
  if (s) return s;
  if (empty(d)) return ok();
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d.C == 0) return zero_fill(output, d.BH() * d.N * d.M * (int64_t)dtype_size(dtype), st);
  if (!query || !key || !output) return fail(LFAMD_ERR_ARG, "laplace forward: null pointer");
  if (workspace && workspace_bytes >= fwd_workspace_bytes(dtype, d) && fwd_sgpr_ok(dtype, d, query)) {
    const int nv = fwd_nv(dtype, d.C);
    switch (dtype) {
      case LFAMD_F32: return launch_fwd_sgpr<float>(query, key, output, workspace, nv, d, st);
      case LFAMD_F16: return launch_fwd_sgpr<f16s>(query, key, output, workspace, nv, d, st);
      default: return launch_fwd_sgpr<bf16s>(query, key, output, workspace, nv, d, st);
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
  // Either backward path may run (the fp16 SGPR path also depends on pointer alignment).
  size_t bytes = plan_bwd(d, true, true, acc, dtype == LFAMD_F16 ? 2 : acc).partialElems * acc;
  if (dtype == LFAMD_F16) bytes = std::max(bytes, plan_sgpr(d, true).partialElems * 4);
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

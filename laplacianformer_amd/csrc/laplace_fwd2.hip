// Row-staged forward of LaplaceSubtraction for M = 49 key columns on gfx950.
//
// Reference semantics (src/LaplaceSubtraction_cuda_kernel.cu:84-140):
//   out[i,j] = cast(sum_c |f32(q[i,c]) - f32(k[c,j])|), c ascending, fp32 sums.
// The sums here run over c ascending in fp32 with the same operations, so the
// results are bit-identical to the reference's.
//
// Mapping. A workgroup, one per CU, takes a contiguous range of at most 448
// rows of one (b, h) slice. It stages those query rows in LDS as fp32
// ([row][C + 4]: the padding makes the per-lane 16-byte reads of 16 consecutive
// rows hit distinct banks) and the slice's key as fp32 [C][56] (7 blocks of 7
// columns, padded to 8). A wave computes one key column block for R row sets
// (rows 64 s + lane, lane = row): per 4 channels it reads one 16-byte vector of
// each of its rows and, per channel, the block's 7 key values as two broadcast
// 16-byte reads, which feed 14 R VALU instructions (v_sub_f32 and v_add_f32
// with an |.| modifier, VGPR operands only). The channel loop is the generated
// asm block of l1_asm_gen.h (reads one step ahead with exact wait counts).
// A last partial set of at most 9 rows is a "tail": one lane per (row, column
// block). The host assigns (block, set range, tail) to the waves:
//  * 16 waves (4 per SIMD, 128 VGPRs) when every block's sets split into runs
//    of at most 3: runs placed so that the most loaded SIMD carries the fewest
//    sets (the 392-row share of one CU at B=32, N=3136 or B=64, H=2, N=784 is
//    6 sets + 8 rows per block: 43 set-units, at most 11 per SIMD);
//  * else 8 waves (2 per SIMD): wave b < 7 takes block b for all sets, wave 7
//    the tail.
// The output tile is staged in LDS and written as one contiguous span.
#include <algorithm>
#include <functional>
#include <vector>

#include "lf_common.h"
#include "lf_internal.h"
#include "l1_asm_gen.h"

namespace lfamd {

namespace {

constexpr int kF2M = 49;          // key columns
constexpr int kF2JB = 7;          // key columns per column wave
constexpr int kF2NB = 7;          // column waves
constexpr int kF2KP = 56;         // key tile pitch (floats per channel: 7 blocks of 8)
constexpr int kF2MaxRows = 448;   // most rows of one workgroup
constexpr int kF2MaxC = 64;       // most channels (query tile pitch C + 4)
constexpr int kF2Tail = 9;        // most rows of a last partial set taken by wave 7

enum F2Epi { kF2Dist = 0, kF2Exp = 1 };
template <typename T, int EPI> struct F2Out { using type = T; };
template <typename T> struct F2Out<T, kF2Exp> { using type = float; };

__host__ __device__ constexpr size_t f2_lds_bytes(int C, int rows, size_t outBytes) {
  return (size_t)C * kF2KP * 4 + ((size_t)rows * (C + 4) * 4 > (size_t)rows * kF2M * outBytes
                                      ? (size_t)rows * (C + 4) * 4
                                      : (size_t)rows * kF2M * outBytes);
}

template <typename T> __device__ __forceinline__ void widen16(const uint4& v, float (&f)[16 / sizeof(T)]);
template <> __device__ __forceinline__ void widen16<f16s>(const uint4& v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
}
template <> __device__ __forceinline__ void widen16<bf16s>(const uint4& v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = __builtin_bit_cast(float, (e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
}
template <> __device__ __forceinline__ void widen16<float>(const uint4& v, float (&f)[4]) {
  f[0] = __builtin_bit_cast(float, v.x);
  f[1] = __builtin_bit_cast(float, v.y);
  f[2] = __builtin_bit_cast(float, v.z);
  f[3] = __builtin_bit_cast(float, v.w);
}

// Dispatch to the generated channel loops (l1_asm_gen.h): OCC = 1 for up to
// 256 VGPRs per wave (2 waves per SIMD), 2 for up to 128 (4 waves per SIMD).
template <int R, int OCC> struct F2Sums;
#define LFAMD_F2SUMS(RR, OCC, FN)                                                                     \
  template <> struct F2Sums<RR, OCC> {                                                                \
    __device__ static void run(float (&acc)[RR][kF2JB], const unsigned (&qa)[RR], unsigned ka, int it) { \
      FN(acc, qa, ka, it);                                                                            \
    }                                                                                                 \
  };
LFAMD_F2SUMS(1, 1, fwd2_sums_r1)
LFAMD_F2SUMS(2, 1, fwd2_sums_r2)
LFAMD_F2SUMS(3, 1, fwd2_sums_r3)
LFAMD_F2SUMS(4, 1, fwd2_sums_r4)
LFAMD_F2SUMS(5, 1, fwd2_sums_r5)
LFAMD_F2SUMS(6, 1, fwd2_sums_r6)
LFAMD_F2SUMS(7, 1, fwd2_sums_r7)
LFAMD_F2SUMS(1, 2, fwd2_sums_r1_v128)
LFAMD_F2SUMS(2, 2, fwd2_sums_r2_v128)
LFAMD_F2SUMS(3, 2, fwd2_sums_r3_v128)
#undef LFAMD_F2SUMS


// Per-wave work of a workgroup: wave w computes key column block b for the
// row sets [s0, s0 + R) (rows 64 s + lane), and, with `tail`, the rows
// [64 full, rows) with one lane per (row, column block). Packed as
// b | s0 << 3 | R << 6 | tail << 9.
struct F2Sched {
  uint32_t w[16];
  int full;  // full row sets of the workgroup (the tail starts at row 64 * full)
};

// Up to three row sources sharing one key in one launch (count > 0): source i
// has N[i] rows per slice (query q[i], output o[i]) split over nx[i]
// workgroups per slice with its own schedule sched[i]; the linear workgroup id
// runs source-major (all of source 0's workgroups first). Read only by the
// SEG instantiations (the plain ones take the plain arguments).
struct F2Seg {
  int count;
  int nx[3], N[3];
  const void* q[3];
  void* o[3];
  F2Sched sched[3];
};

// Grid: (nx workgroups per slice, B*H). Workgroup x takes rows
// [x*N/nx, (x+1)*N/nx) of its slice (at most kF2MaxRows); WAVES waves (2 or 4
// per SIMD) run the schedule. Rows past the workgroup's end are computed on
// clamped rows and not stored.
template <typename T, int EPI, int WAVES, bool SEG>
__device__ __forceinline__ void fwd2_body(const T* __restrict__ queryIn, const T* __restrict__ key,
                                          typename F2Out<T, EPI>::type* __restrict__ outIn, int NIn, int C,
                                          float scale, const F2Sched& sched, const F2Seg& sg) {
  using O = typename F2Out<T, EPI>::type;
  constexpr int THREADS = 64 * WAVES;
  constexpr int OCC = WAVES / 8;            // asm register budget: 256 (8 waves) or 128 (16) VGPRs
  constexpr int RMAX = WAVES == 16 ? 3 : 7;
  constexpr int EV = 16 / (int)sizeof(T);  // elements per 16-byte query vector
  const int tid = threadIdx.x;
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  int x = blockIdx.x, nx = gridDim.x, bh = blockIdx.y, N = NIn, si = -1;
  const T* query = queryIn;
  O* out = outIn;
  if constexpr (SEG) {
    const int L = x + nx * bh, S = (int)gridDim.y;
    const int e1 = S * sg.nx[0], e2 = e1 + S * sg.nx[1];
    si = L < e1 ? 0 : (L < e2 ? 1 : 2);
    nx = si == 0 ? sg.nx[0] : si == 1 ? sg.nx[1] : sg.nx[2];
    const int Ls = L - (si == 0 ? 0 : si == 1 ? e1 : e2);
    bh = Ls / nx;
    x = Ls - bh * nx;
    N = si == 0 ? sg.N[0] : si == 1 ? sg.N[1] : sg.N[2];
    query = static_cast<const T*>(si == 0 ? sg.q[0] : si == 1 ? sg.q[1] : sg.q[2]);
    out = static_cast<O*>(si == 0 ? sg.o[0] : si == 1 ? sg.o[1] : sg.o[2]);
  }
  const int sfull = !SEG ? sched.full : si == 0 ? sg.sched[0].full : si == 1 ? sg.sched[1].full : sg.sched[2].full;
  const int P0 = (int)((int64_t)x * N / nx), P1 = (int)((int64_t)(x + 1) * N / nx);
  const int n = P1 - P0;
  const int QP = C + 4;

  extern __shared__ __align__(16) unsigned char smem[];
  float* ktile = reinterpret_cast<float*>(smem);                          // [C][56]
  float* qtile = reinterpret_cast<float*>(smem + (size_t)C * kF2KP * 4);   // [n][C + 4]
  O* otile = reinterpret_cast<O*>(qtile);                                  // [n][49] after the sums

  // All loads first: the query rows (one contiguous span of n*C elements, in
  // 16-byte vectors; C % EV == 0 and a 16-byte aligned query) and the key.
  constexpr int kQL = (kF2MaxRows * kF2MaxC / EV + THREADS - 1) / THREADS;
  const int qvecs = n * C / EV, vpr = C / EV;
  const uint4* qsrc = reinterpret_cast<const uint4*>(query + ((size_t)bh * N + P0) * C);
  uint4 qv[kQL];
#pragma unroll
  for (int i = 0; i < kQL; ++i) qv[i] = qsrc[min(tid + i * THREADS, qvecs - 1)];
  constexpr int kKL = (kF2MaxC * kF2M + THREADS - 1) / THREADS;
  const int kn = C * kF2M;
  const T* ksrc = key + (size_t)bh * C * kF2M;
  T kvv[kKL];
#pragma unroll
  for (int i = 0; i < kKL; ++i) kvv[i] = ksrc[min(tid + i * THREADS, kn - 1)];

  // Key tile: column j of channel c at c*56 + (j / 7)*8 + j % 7; the padding
  // column of each block is zero.
#pragma unroll
  for (int i = 0; i < kKL; ++i) {
    const int t = tid + i * THREADS;
    if (t < kn) {
      const int c = t / kF2M, j = t - c * kF2M;
      ktile[c * kF2KP + (j / kF2JB) * 8 + j % kF2JB] = to_acc(kvv[i]);
    }
  }
  for (int t = tid; t < C * kF2NB; t += THREADS) ktile[(t / kF2NB) * kF2KP + (t % kF2NB) * 8 + 7] = 0.0f;
  // Query tile (fp32).
#pragma unroll
  for (int i = 0; i < kQL; ++i) {
    const int u = tid + i * THREADS;
    if (u < qvecs) {
      const int row = u / vpr, c0 = (u - row * vpr) * EV;
      float f[EV];
      widen16<T>(qv[i], f);
      float4* dst = reinterpret_cast<float4*>(qtile + row * QP + c0);
#pragma unroll
      for (int e = 0; e < EV / 4; ++e) dst[e] = make_float4(f[4 * e], f[4 * e + 1], f[4 * e + 2], f[4 * e + 3]);
    }
  }
  __syncthreads();

  const unsigned kBase = (unsigned)(uintptr_t)ktile, qBase = (unsigned)(uintptr_t)qtile;
  const uint32_t me = wave >= 16 ? 0u
                      : !SEG    ? sched.w[wave]
                      : si == 0 ? sg.sched[0].w[wave]
                      : si == 1 ? sg.sched[1].w[wave]
                                : sg.sched[2].w[wave];
  const int b = uniform((int)(me & 7)), s0 = uniform((int)((me >> 3) & 7)), R = uniform((int)((me >> 6) & 7));
  const bool hasTail = (me >> 9) & 1;
  const int trows = n - 64 * sfull;  // tail rows of this workgroup (may be <= 0)
  float acc[RMAX][kF2JB];
  float acct[1][kF2JB];
  unsigned qa[RMAX];
#pragma unroll
  for (int s = 0; s < RMAX; ++s) qa[s] = qBase + (unsigned)(min(64 * (s0 + s) + lane, n - 1) * QP) * 4;
  const unsigned ka = kBase + (unsigned)b * 32;
  switch (R) {  // wave-uniform
    case 1: F2Sums<1, OCC>::run(reinterpret_cast<float(&)[1][kF2JB]>(acc), reinterpret_cast<const unsigned(&)[1]>(qa), ka, C / 8); break;
    case 2: F2Sums<2, OCC>::run(reinterpret_cast<float(&)[2][kF2JB]>(acc), reinterpret_cast<const unsigned(&)[2]>(qa), ka, C / 8); break;
    case 3: F2Sums<3, OCC>::run(reinterpret_cast<float(&)[3][kF2JB]>(acc), reinterpret_cast<const unsigned(&)[3]>(qa), ka, C / 8); break;
    default:
      if constexpr (RMAX > 3) {
        switch (R) {
          case 4: F2Sums<4, OCC>::run(reinterpret_cast<float(&)[4][kF2JB]>(acc), reinterpret_cast<const unsigned(&)[4]>(qa), ka, C / 8); break;
          case 5: F2Sums<5, OCC>::run(reinterpret_cast<float(&)[5][kF2JB]>(acc), reinterpret_cast<const unsigned(&)[5]>(qa), ka, C / 8); break;
          case 6: F2Sums<6, OCC>::run(reinterpret_cast<float(&)[6][kF2JB]>(acc), reinterpret_cast<const unsigned(&)[6]>(qa), ka, C / 8); break;
          case 7: F2Sums<7, OCC>::run(reinterpret_cast<float(&)[7][kF2JB]>(acc), reinterpret_cast<const unsigned(&)[7]>(qa), ka, C / 8); break;
          default: break;
        }
      }
      break;
  }
  // The tail: one lane per (row, column block), lanes [0, 7 * trows).
  const int bt = lane % kF2NB;
  const int rowt = 64 * sfull + min(lane / kF2NB, max(trows, 1) - 1);
  if (hasTail && trows > 0) {
    const unsigned qt[1] = {qBase + (unsigned)(min(rowt, n - 1) * QP) * 4};
    F2Sums<1, OCC>::run(acct, qt, kBase + (unsigned)bt * 32, C / 8);
  }
  __syncthreads();  // every wave is done with the query tile, which becomes the output tile

  auto emit = [&](float a) -> O {
    if constexpr (EPI == kF2Exp)
      return expf(-scale * a);
    else
      return from_acc<T>(a);
  };
#pragma unroll
  for (int s = 0; s < RMAX; ++s) {
    const int row = 64 * (s0 + s) + lane;
    if (s < R && row < n)
#pragma unroll
      for (int j = 0; j < kF2JB; ++j) otile[row * kF2M + b * kF2JB + j] = emit(acc[s][j]);
  }
  if (hasTail && lane < kF2NB * trows) {
#pragma unroll
    for (int j = 0; j < kF2JB; ++j) otile[rowt * kF2M + bt * kF2JB + j] = emit(acct[0][j]);
  }
  __syncthreads();

  // Rows [P0, P1) of the slice are one contiguous span of n*49 outputs.
  O* const dst = out + ((size_t)bh * N + P0) * kF2M;
  const int total = n * kF2M;
  constexpr int OV = 16 / (int)sizeof(O);
  int done = 0;
  if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    const int nv = total / OV;
    const uint4* s4 = reinterpret_cast<const uint4*>(otile);
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    for (int t = tid; t < nv; t += THREADS) d4[t] = s4[t];
    done = nv * OV;
  } else if (sizeof(O) == 2 && (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
    const int nv = total / 2;
    const uint32_t* s4 = reinterpret_cast<const uint32_t*>(otile);
    uint32_t* d4 = reinterpret_cast<uint32_t*>(dst);
    for (int t = tid; t < nv; t += THREADS) d4[t] = s4[t];
    done = nv * 2;
  }
  for (int t = done + tid; t < total; t += THREADS) dst[t] = otile[t];
}

// The plain kernel (one row source) and the segmented one (up to three sources
// sharing the key, F2Seg); both run fwd2_body.
template <typename T, int EPI, int WAVES>
__global__ void __launch_bounds__(64 * WAVES, 1)
laplace_fwd2_kernel(const T* __restrict__ query, const T* __restrict__ key, typename F2Out<T, EPI>::type* __restrict__ out,
                    int N, int C, float scale, F2Sched sched) {
  fwd2_body<T, EPI, WAVES, false>(query, key, out, N, C, scale, sched, F2Seg{});
}

template <typename T, int EPI, int WAVES>
__global__ void __launch_bounds__(64 * WAVES, 1)
laplace_fwd2_seg_kernel(const T* __restrict__ key, int C, float scale, F2Seg sg) {
  fwd2_body<T, EPI, WAVES, true>(nullptr, key, nullptr, 0, C, scale, sg.sched[0], sg);
}

struct F2Plan {
  int nx, waves;
  size_t lds;
  F2Sched sched;
};

// Schedule of a 16-wave workgroup (wave w on SIMD w % 4): each column block's
// F row sets split into runs of at most maxR (the 128-VGPR channel loops), the
// tail (if any) a wave of its own or added to a run of at most 2, runs placed
// longest first on the least loaded SIMD with a free wave. The split that
// minimizes the most loaded SIMD wins. Returns false when no split fits 16 waves.
bool f2_schedule16(int F, bool tail, int maxR, F2Sched& out) {
  std::vector<std::vector<int>> opts;  // partitions of F into at most 4 parts <= maxR, descending
  for (int a = 0; a <= maxR; ++a)
    for (int b2 = 0; b2 <= maxR; ++b2)
      for (int c = 0; c <= maxR; ++c)
        for (int d = 0; d <= maxR; ++d) {
          if (a + b2 + c + d != F) continue;
          if (!(a >= b2 && b2 >= c && c >= d)) continue;
          std::vector<int> v;
          for (int e : {a, b2, c, d})
            if (e > 0) v.push_back(e);
          opts.push_back(v);
        }
  if (F == 0) opts.push_back({});
  int best = 1 << 30;
  std::vector<int> choice(kF2NB, 0), bestChoice;
  int bestTailMode = 0;
  // Blocks are interchangeable: enumerate nondecreasing option indices.
  std::function<void(int, int)> rec = [&](int blk, int from) {
    if (blk == kF2NB) {
      std::vector<int> parts;
      for (int i = 0; i < kF2NB; ++i)
        for (int e : opts[choice[i]]) parts.push_back(e);
      for (int tailMode = 0; tailMode < (tail ? 2 : 1); ++tailMode) {  // 0: own wave, 1: attached
        std::vector<int> ps = parts;
        if (tail && tailMode == 0) ps.push_back(1);
        if ((int)ps.size() > 16) continue;
        std::sort(ps.begin(), ps.end(), std::greater<int>());
        int load[4] = {0, 0, 0, 0}, cnt[4] = {0, 0, 0, 0};
        bool attached = !(tail && tailMode == 1);
        for (int e : ps) {
          int sm = -1;
          for (int q = 0; q < 4; ++q)
            if (cnt[q] < 4 && (sm < 0 || load[q] < load[sm])) sm = q;
          load[sm] += e;
          ++cnt[sm];
        }
        if (!attached) {  // add the tail to the least loaded SIMD that has a run of <= 2 (approximation: any)
          int sm = 0;
          for (int q = 1; q < 4; ++q)
            if (load[q] < load[sm]) sm = q;
          load[sm] += 1;
        }
        const int mx = std::max(std::max(load[0], load[1]), std::max(load[2], load[3]));
        if (mx < best) {
          best = mx;
          bestChoice = choice;
          bestTailMode = tailMode;
        }
      }
      return;
    }
    for (int o = from; o < (int)opts.size(); ++o) {
      choice[blk] = o;
      rec(blk + 1, o);
    }
  };
  rec(0, 0);
  if (best == (1 << 30)) return false;
  // Materialize: runs (block, s0, R), longest first onto the least loaded SIMD.
  struct Run { int b, s0, R; bool tail; };
  std::vector<Run> runs;
  for (int i = 0; i < kF2NB; ++i) {
    int s0 = 0;
    for (int e : opts[bestChoice[i]]) {
      runs.push_back({i, s0, e, false});
      s0 += e;
    }
  }
  if (tail && bestTailMode == 0) runs.push_back({0, 0, 0, true});
  std::stable_sort(runs.begin(), runs.end(), [](const Run& a, const Run& b) { return std::max(a.R, 1) > std::max(b.R, 1); });
  int load[4] = {0, 0, 0, 0}, cnt[4] = {0, 0, 0, 0};
  for (int i = 0; i < 16; ++i) out.w[i] = 0;
  int slotOf[16];
  int nslots = 0;
  for (const Run& r : runs) {
    int sm = -1;
    for (int q = 0; q < 4; ++q)
      if (cnt[q] < 4 && (sm < 0 || load[q] < load[sm])) sm = q;
    const int w = sm + 4 * cnt[sm];
    ++cnt[sm];
    load[sm] += std::max(r.R, 1);
    out.w[w] = (uint32_t)r.b | (uint32_t)r.s0 << 3 | (uint32_t)r.R << 6 | (r.tail ? 1u << 9 : 0u);
    slotOf[nslots++] = w;
  }
  if (tail && bestTailMode == 1) {
    // Attach to the oldest wave (lowest index) of the least loaded SIMD: a SIMD
    // issues its oldest ready waves first, so its youngest wave runs last and
    // partly alone, and should hold the least work.
    int bw = -1, bl = 1 << 30;
    for (int i = 0; i < nslots; ++i) {
      const int w = slotOf[i];
      if (load[w % 4] < bl || (load[w % 4] == bl && w < bw)) {
        bl = load[w % 4];
        bw = w;
      }
    }
    if (bw < 0) return false;
    out.w[bw] |= 1u << 9;
  }
  return true;
}

// Workgroups per slice: one per CU where the rows allow, at most kF2MaxRows
// rows each. Full row sets F = rows / 64; a last partial set of at most
// kF2Tail rows is a tail (one lane per row and column block), a longer one a
// set of its own. 16 waves (4 per SIMD: ~1.4x the VALU rate of 2 per SIMD)
// when the schedule fits runs of at most 3 sets, else 8 waves (7 column waves
// with every set, wave 7 the tail).
F2Plan plan_f2(int64_t BH, int64_t N, int64_t C, size_t outBytes) {
  F2Plan p{};
  const int64_t per = std::max<int64_t>(1, num_cus() / std::max<int64_t>(BH, 1));
  p.nx = (int)std::max<int64_t>((N + kF2MaxRows - 1) / kF2MaxRows, std::min<int64_t>(per, (N + 63) / 64));
  const int rows = (int)((N + p.nx - 1) / p.nx), minRows = (int)(N / p.nx);
  int full = rows / 64;
  const int part = rows % 64;
  const bool tail = full >= 1 && part > 0 && part <= kF2Tail && minRows / 64 == full;
  if (!tail && part > 0) ++full;
  p.lds = f2_lds_bytes((int)C, rows, outBytes);
  p.sched.full = full;
  // The schedule depends on (full, tail) only: searched once per pair and host thread.
  struct Memo {
    bool done, ok;
    F2Sched s;
  };
  constexpr int kMemo = kF2MaxRows / 64 + 2;
  static thread_local Memo memo[kMemo][2] = {};
  Memo local{};
  Memo& m = full < kMemo ? memo[full][tail ? 1 : 0] : local;
  if (!m.done) {
    m.s = p.sched;
    m.ok = f2_schedule16(full, tail, 3, m.s);
    m.done = true;
  }
  if (m.ok) {
    for (int w = 0; w < 16; ++w) p.sched.w[w] = m.s.w[w];
    p.waves = 16;
    return p;
  }
  p.waves = 8;
  for (int w = 0; w < 16; ++w) p.sched.w[w] = 0;
  for (int w = 0; w < kF2NB; ++w) p.sched.w[w] = (uint32_t)w | (uint32_t)full << 6;
  if (tail) p.sched.w[7] = 1u << 9;
  return p;
}

template <typename T, int EPI, int WAVES, bool SEG>
int launch_f2_w(const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t C, float scale,
                const F2Plan& p, hipStream_t st, const F2Seg& sg) {
  using O = typename F2Out<T, EPI>::type;
  if constexpr (SEG) {
    auto kern = laplace_fwd2_seg_kernel<T, EPI, WAVES>;
    if (int s = check_fit(reinterpret_cast<const void*>(kern), 64 * WAVES, p.lds, "laplace forward")) return s;
    if (p.lds > 65536)
      if (int s = set_dyn_lds(reinterpret_cast<const void*>(kern), p.lds, "laplace forward")) return s;
    hipLaunchKernelGGL(kern, dim3(p.nx, (unsigned)BH), dim3(64 * WAVES), p.lds, st, static_cast<const T*>(k),
                       (int)C, scale, sg);
  } else {
    auto kern = laplace_fwd2_kernel<T, EPI, WAVES>;
    if (int s = check_fit(reinterpret_cast<const void*>(kern), 64 * WAVES, p.lds, "laplace forward")) return s;
    if (p.lds > 65536)
      if (int s = set_dyn_lds(reinterpret_cast<const void*>(kern), p.lds, "laplace forward")) return s;
    hipLaunchKernelGGL(kern, dim3(p.nx, (unsigned)BH), dim3(64 * WAVES), p.lds, st, static_cast<const T*>(q),
                       static_cast<const T*>(k), static_cast<O*>(o), (int)N, (int)C, scale, p.sched);
  }
  return check_launch("laplace forward (row-staged)");
}

template <typename T, int EPI, bool SEG = false>
int launch_f2_t(const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t C, float scale,
                const F2Plan& p, hipStream_t st, const F2Seg& sg = F2Seg{}) {
  if (p.waves == 16) return launch_f2_w<T, EPI, 16, SEG>(q, k, o, BH, N, C, scale, p, st, sg);
  return launch_f2_w<T, EPI, 8, SEG>(q, k, o, BH, N, C, scale, p, st, sg);
}

// ---------------------------------------------------------------------------
// Wide landmark sets, M in {128, 256} (M = 256). A workgroup
// of WAVES waves (128 VGPRs each; 16: one workgroup per CU, 8: two per CU for
// C <= 16) takes 192 rows (3 row sets) of one slice:
// the rows staged as fp32 [row][C + 4] as above, the slice's key as fp32 with a
// fixed pitch of 256 columns per channel. Wave w computes the 8-column blocks
// w, w + WAVES, ... for the 3 sets with the generated channel loop
// (fwd3_sums_r3_v128: per channel the block's 8 keys as two broadcast 16-byte reads
// feed 48 VALU instructions), c ascending in fp32 (bit-identical to the
// reference's order). A lane's 8 results of a row are one 16-byte store for
// 16-bit outputs (two for fp32), written from registers: the output tile
// would not fit in the LDS beside the key.
constexpr int kF3Sets = 3;
constexpr int kF3Rows = 64 * kF3Sets;
constexpr int kF3KP = 256;

__host__ __device__ constexpr size_t f3_lds_bytes(int C) {
  return (size_t)C * kF3KP * 4 + (size_t)kF3Rows * (C + 4) * 4;
}

template <typename T>
__device__ __forceinline__ void store8(T* dst, const float (&a)[8]);
template <>
__device__ __forceinline__ void store8<float>(float* dst, const float (&a)[8]) {
  reinterpret_cast<float4*>(dst)[0] = make_float4(a[0], a[1], a[2], a[3]);
  reinterpret_cast<float4*>(dst)[1] = make_float4(a[4], a[5], a[6], a[7]);
}
template <typename T>
__device__ __forceinline__ void store8(T* dst, const float (&a)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w[e] = (uint32_t)from_acc<T>(a[2 * e]).bits | ((uint32_t)from_acc<T>(a[2 * e + 1]).bits << 16);
  *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Grid: (workgroups per slice = ceil(N / 192), B*H). WAVES = 16 (one workgroup
// per CU) or 8 (two per CU, for small C: the two workgroups' load, compute and
// store phases overlap).
template <typename T, int WAVES>
__global__ void __launch_bounds__(64 * WAVES, 16 / WAVES)
laplace_fwd3_kernel(const T* __restrict__ query, const T* __restrict__ key, T* __restrict__ out, int N, int M,
                    int C) {
  constexpr int THREADS = 64 * WAVES;
  constexpr int EV = 16 / (int)sizeof(T);
  const int tid = threadIdx.x;
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int x = blockIdx.x, bh = blockIdx.y;
  const int P0 = x * kF3Rows, n = min(kF3Rows, N - P0);
  const int QP = C + 4;

  extern __shared__ __align__(16) unsigned char smem[];
  float* ktile = reinterpret_cast<float*>(smem);                          // [C][256]
  float* qtile = reinterpret_cast<float*>(smem + (size_t)C * kF3KP * 4);   // [n][C + 4]

  constexpr int kQL = (kF3Rows * kF2MaxC / EV + THREADS - 1) / THREADS;
  const int qvecs = n * C / EV, vpr = C / EV;
  const uint4* qsrc = reinterpret_cast<const uint4*>(query + ((size_t)bh * N + P0) * C);
  uint4 qv[kQL];
#pragma unroll
  for (int i = 0; i < kQL; ++i) qv[i] = qsrc[min(tid + i * THREADS, qvecs - 1)];
  constexpr int kKL = (kF2MaxC * kF3KP + THREADS - 1) / THREADS;
  const int kn = C * M;
  const T* ksrc = key + (size_t)bh * C * M;
  T kvv[kKL];
#pragma unroll
  for (int i = 0; i < kKL; ++i) kvv[i] = ksrc[min(tid + i * THREADS, kn - 1)];
#pragma unroll
  for (int i = 0; i < kKL; ++i) {
    const int t = tid + i * THREADS;
    if (t < kn) {
      const int c = t / M, j = t - c * M;
      ktile[c * kF3KP + j] = to_acc(kvv[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < kQL; ++i) {
    const int u = tid + i * THREADS;
    if (u < qvecs) {
      const int row = u / vpr, c0 = (u - row * vpr) * EV;
      float f[EV];
      widen16<T>(qv[i], f);
      float4* dst = reinterpret_cast<float4*>(qtile + row * QP + c0);
#pragma unroll
      for (int e = 0; e < EV / 4; ++e) dst[e] = make_float4(f[4 * e], f[4 * e + 1], f[4 * e + 2], f[4 * e + 3]);
    }
  }
  __syncthreads();

  const unsigned kBase = (unsigned)(uintptr_t)ktile, qBase = (unsigned)(uintptr_t)qtile;
  unsigned qa[kF3Sets];
#pragma unroll
  for (int s = 0; s < kF3Sets; ++s) qa[s] = qBase + (unsigned)(min(64 * s + lane, n - 1) * QP) * 4;
  const int nblk = M / 8;
  // Blocks wave, wave + WAVES, ...: the waves writing one row's 16-byte pieces
  // run concurrently (measured 1.6x faster stores than adjacent blocks per wave).
  for (int b = wave; b < nblk; b += WAVES) {  // wave-uniform
    float acc[kF3Sets][8];
    fwd3_sums_r3_v128(acc, qa, kBase + (unsigned)b * 32, C / 8);
#pragma unroll
    for (int s = 0; s < kF3Sets; ++s) {
      const int row = 64 * s + lane;
      if (row < n) store8<T>(out + ((size_t)bh * N + P0 + row) * M + 8 * b, acc[s]);
    }
  }
}

// Small channel counts (C in {8, 16}) with M = 64 MG landmarks, where the
// output (2 bytes per (i, j) against 2 C VALU instructions) bounds the time:
// every store instruction writes whole 128-byte lines. Lane (rsub, chunk) =
// (lane / 16, lane % 16) computes 4 consecutive columns [4 chunk, 4 chunk + 4)
// of a 64-column group for row rsub of each 4-row step, so the 16 lanes of a
// row write 64 consecutive outputs (one line of 16-bit outputs, two of fp32).
// Wave w of the 4-wave workgroup takes column group w % MG and, for MG = 2, one
// half of the workgroup's rows; each lane keeps its columns' keys for all C
// channels in registers (from the workgroup's fp32 key tile) and reads the query
// row of each step as a broadcast from the fp32 query tile. Sums over c
// ascending in fp32: the reference's order, bit-identical to the serial oracle.
constexpr int kF4Rows = 256;   // rows per workgroup

// Two fp32 values rounded to nearest even into one word of 16-bit outputs, as
// one v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 (the same rounding as from_acc; a
// NaN comes out as a quiet NaN of its own sign where from_acc writes 0x7fc0 for
// bf16).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<f16s>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack2<bf16s>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

template <typename T, int C, int MG>
__global__ void __launch_bounds__(256)
laplace_fwd4_kernel(const T* __restrict__ query, const T* __restrict__ key, T* __restrict__ out, int N) {
  constexpr int M = 64 * MG, QP = C + 4, WPG = 4 / MG, RPW = kF4Rows / WPG;
  __shared__ __align__(16) float qs[kF4Rows * QP];
  __shared__ __align__(16) float ks[C * M];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int cg = wave % MG, rw = wave / MG, chunk = lane & 15, rsub = lane >> 4;
  const int bh = blockIdx.y, r0 = blockIdx.x * kF4Rows;
  const T* qsl = query + (size_t)bh * N * C;
#pragma unroll
  for (int i = 0; i < kF4Rows * C / 256; ++i) {
    const int e = tid + 256 * i, r = e / C, c = e - r * C;
    qs[r * QP + c] = to_acc(qsl[(size_t)min(r0 + r, N - 1) * C + c]);
  }
#pragma unroll
  for (int i = 0; i < C * M / 256; ++i) ks[tid + 256 * i] = to_acc(key[(size_t)bh * C * M + tid + 256 * i]);
  __syncthreads();
  float kr[C][4];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float4 v = *reinterpret_cast<const float4*>(ks + c * M + cg * 64 + 4 * chunk);
    kr[c][0] = v.x;
    kr[c][1] = v.y;
    kr[c][2] = v.z;
    kr[c][3] = v.w;
  }
  T* const o = out + ((size_t)bh * N + r0) * M + cg * 64 + 4 * chunk;
#pragma unroll 4
  for (int t = 0; t < RPW / 4; ++t) {
    const int r = rw * RPW + 4 * t + rsub;
    float qv[C];
#pragma unroll
    for (int c4 = 0; c4 < C / 4; ++c4) {
      const float4 v = *reinterpret_cast<const float4*>(qs + r * QP + 4 * c4);
      qv[4 * c4] = v.x;
      qv[4 * c4 + 1] = v.y;
      qv[4 * c4 + 2] = v.z;
      qv[4 * c4 + 3] = v.w;
    }
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += __builtin_fabsf(qv[c] - kr[c][j]);
    if (r0 + r < N) {
      if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(o + (size_t)r * M) = make_float4(acc[0], acc[1], acc[2], acc[3]);
      } else {
        *reinterpret_cast<uint2*>(o + (size_t)r * M) = make_uint2(pack2<T>(acc[0], acc[1]), pack2<T>(acc[2], acc[3]));
      }
    }
  }
}

template <typename T, int C, int MG>
int launch_f4(const void* q, const void* k, void* o, int64_t BH, int64_t N, hipStream_t st) {
  auto kern = laplace_fwd4_kernel<T, C, MG>;
  if (int s = check_fit(reinterpret_cast<const void*>(kern), 256, 0, "laplace forward (small d)")) return s;
  hipLaunchKernelGGL(kern, dim3((unsigned)((N + kF4Rows - 1) / kF4Rows), (unsigned)BH), dim3(256), 0, st,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<T*>(o), (int)N);
  return check_launch("laplace forward (small d)");
}

template <typename T>
int launch_f4_t(const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t M, int64_t C, hipStream_t st) {
  if (C == 8) return M == 256 ? launch_f4<T, 8, 4>(q, k, o, BH, N, st) : launch_f4<T, 8, 2>(q, k, o, BH, N, st);
  return M == 256 ? launch_f4<T, 16, 4>(q, k, o, BH, N, st) : launch_f4<T, 16, 2>(q, k, o, BH, N, st);
}

template <typename T, int WAVES>
int launch_f3_w(const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t M, int64_t C, hipStream_t st) {
  auto kern = laplace_fwd3_kernel<T, WAVES>;
  const size_t lds = f3_lds_bytes((int)C);
  if (int s = check_fit(reinterpret_cast<const void*>(kern), 64 * WAVES, lds, "laplace forward")) return s;
  if (lds > 65536)
    if (int s = set_dyn_lds(reinterpret_cast<const void*>(kern), lds, "laplace forward")) return s;
  const int64_t nx = (N + kF3Rows - 1) / kF3Rows;
  hipLaunchKernelGGL(kern, dim3((unsigned)nx, (unsigned)BH), dim3(64 * WAVES), lds, st, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<T*>(o), (int)N, (int)M, (int)C);
  return check_launch("laplace forward (wide landmarks)");
}

template <typename T>
int launch_f3(const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t M, int64_t C, hipStream_t st) {
  if (2 * f3_lds_bytes((int)C) <= (size_t)max_lds_bytes() && C <= 16)
    return launch_f3_w<T, 8>(q, k, o, BH, N, M, C, st);
  return launch_f3_w<T, 16>(q, k, o, BH, N, M, C, st);
}

}  // namespace

// The row-staged forward: fp32 / fp16 / bf16, M = 49, 8 <= C <= 64 with
// C % 8 == 0, a 16-byte aligned query and N >= 1.
bool f2_ok(int dtype, int64_t BH, int64_t N, int64_t M, int64_t C, const void* q) {
  if (!(dtype == LFAMD_F32 || dtype == LFAMD_F16 || dtype == LFAMD_BF16)) return false;
  if (M != kF2M || C < 8 || C > kF2MaxC || C % 8 != 0 || N <= 0 || BH <= 0 || BH > 65535) return false;
  if ((reinterpret_cast<uintptr_t>(q) & 15) != 0) return false;
  return N <= INT32_MAX / kF2M;
}

// The wide-landmark forward: fp32 / fp16 / bf16, M in {128, 256}, 8 <= C <= 64
// with C % 8 == 0, 16-byte aligned query and output, N >= 1.
bool f3_ok(int dtype, int64_t BH, int64_t N, int64_t M, int64_t C, const void* q, const void* out) {
  if (!(dtype == LFAMD_F32 || dtype == LFAMD_F16 || dtype == LFAMD_BF16)) return false;
  if (!(M == 128 || M == 256) || C < 8 || C > kF2MaxC || C % 8 != 0 || N <= 0 || BH <= 0 || BH > 65535) return false;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) & 15) != 0) return false;
  return N <= INT32_MAX / M && f3_lds_bytes((int)C) <= (size_t)max_lds_bytes();
}

int f3_launch(int dtype, const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t M, int64_t C,
              hipStream_t st) {
  if (C == 8 || C == 16) {  // output-bound: the line-coalesced small-d kernel
    if (dtype == LFAMD_F32) return launch_f4_t<float>(q, k, o, BH, N, M, C, st);
    if (dtype == LFAMD_F16) return launch_f4_t<f16s>(q, k, o, BH, N, M, C, st);
    return launch_f4_t<bf16s>(q, k, o, BH, N, M, C, st);
  }
  if (dtype == LFAMD_F32) return launch_f3<float>(q, k, o, BH, N, M, C, st);
  if (dtype == LFAMD_F16) return launch_f3<f16s>(q, k, o, BH, N, M, C, st);
  return launch_f3<bf16s>(q, k, o, BH, N, M, C, st);
}

namespace {
const F2Plan& f2_plan_cached(int dtype, bool kernelEpi, int64_t BH, int64_t N, int64_t C) {
  // The plan's schedule search (~80 us of host time for six row sets) is
  // cached per shape, per host thread, for the last kPlanCache shapes (a layer
  // step alternates three; the CU count is per device, so the device is part
  // of the key).
  struct Key {
    int64_t BH, N, C;
    size_t ob;
    int dev, cus;
    bool operator==(const Key& o) const {
      return BH == o.BH && N == o.N && C == o.C && ob == o.ob && dev == o.dev && cus == o.cus;
    }
  };
  constexpr int kPlanCache = 8;
  static thread_local Key keys[kPlanCache] = {};
  static thread_local F2Plan plans[kPlanCache];
  static thread_local int used = 0, next = 0;
  int dev = 0;
  (void)hipGetDevice(&dev);
  const Key key{BH, N, C, kernelEpi ? 4 : dtype_size(dtype), dev, num_cus()};
  int slot = -1;
  for (int i = 0; i < used; ++i)
    if (keys[i] == key) slot = i;
  if (slot < 0) {
    slot = used < kPlanCache ? used++ : next;
    next = (slot + 1) % kPlanCache;
    plans[slot] = plan_f2(BH, N, C, key.ob);
    keys[slot] = key;
  }
  return plans[slot];
}
}  // namespace

int f2_launch(int dtype, bool kernelEpi, const void* q, const void* k, void* o, int64_t BH, int64_t N, int64_t C,
              float scale, hipStream_t st) {
  const F2Plan& p = f2_plan_cached(dtype, kernelEpi, BH, N, C);
  if (p.lds > (size_t)max_lds_bytes()) return fail(LFAMD_ERR_UNSUPPORTED, "laplace forward: LDS plan too large");
  if (kernelEpi) {
    if (dtype == LFAMD_F32) return launch_f2_t<float, kF2Exp>(q, k, o, BH, N, C, scale, p, st);
    if (dtype == LFAMD_F16) return launch_f2_t<f16s, kF2Exp>(q, k, o, BH, N, C, scale, p, st);
    return launch_f2_t<bf16s, kF2Exp>(q, k, o, BH, N, C, scale, p, st);
  }
  if (dtype == LFAMD_F32) return launch_f2_t<float, kF2Dist>(q, k, o, BH, N, C, scale, p, st);
  if (dtype == LFAMD_F16) return launch_f2_t<f16s, kF2Dist>(q, k, o, BH, N, C, scale, p, st);
  return launch_f2_t<bf16s, kF2Dist>(q, k, o, BH, N, C, scale, p, st);
}

// The fused-kernel forward over up to three row sources sharing one key, one
// launch: each source keeps its own plan (workgroups per slice, wave schedule);
// LFAMD_ERR_UNSUPPORTED when their wave counts differ or the LDS plan is too
// large. Needs f2_ok for every source.
int f2_launch_multi(int dtype, int nsrc, const void* const* q, const int64_t* n, const void* k, float* const* o,
                    int64_t BH, int64_t C, float scale, hipStream_t st) {
  F2Seg sg{};
  F2Plan p{};
  sg.count = nsrc;
  for (int i = 0; i < nsrc; ++i) {
    const F2Plan& pi = f2_plan_cached(dtype, true, BH, n[i], C);
    if (i > 0 && pi.waves != p.waves)
      return fail(LFAMD_ERR_UNSUPPORTED, "laplace kernel forward (several sources): plans of different widths");
    p.waves = pi.waves;
    p.lds = std::max(p.lds, pi.lds);
    p.nx += pi.nx;
    sg.nx[i] = pi.nx;
    sg.N[i] = (int)n[i];
    sg.q[i] = q[i];
    sg.o[i] = o[i];
    sg.sched[i] = pi.sched;
  }
  if (p.lds > (size_t)max_lds_bytes()) return fail(LFAMD_ERR_UNSUPPORTED, "laplace forward: LDS plan too large");
  if (dtype == LFAMD_F32) return launch_f2_t<float, kF2Exp, true>(nullptr, k, nullptr, BH, 0, C, scale, p, st, sg);
  if (dtype == LFAMD_F16) return launch_f2_t<f16s, kF2Exp, true>(nullptr, k, nullptr, BH, 0, C, scale, p, st, sg);
  return launch_f2_t<bf16s, kF2Exp, true>(nullptr, k, nullptr, BH, 0, C, scale, p, st, sg);
}

}  // namespace lfamd

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
// Mapping. A workgroup is WAVES waves, one workgroup per CU: 12 (3 per SIMD,
// 168 VGPRs each) for M = 49, whose row loop keeps its grad_key sums and the
// inputs it consumes in its own registers, else 8 (2 per SIMD, 256 VGPRs). A
// SIMD issues two VALU instructions per 4 cycles only from two different
// waves: the row loop reaches ~2.8 cycles per instruction with two waves and
// about 10 % less with three. The workgroup takes a contiguous range of at most
// 512 rows of one (b, h) slice and one channel block of 64 channels. Lane
// (h, p), h = lane / 32, p = lane % 32, owns channels 2p + h and 2p + 1 - h (in
// that order) and the key columns of parity h (column 2j + h, j < JC =
// ceil(M / 2)); its key terms and grad_key sums stay in registers, and its
// grad_query is that of channel 2p + h (the other column half's partial comes
// from lane (1 - h, p)).
//
// The workgroup stages the key terms in LDS (the only barrier before the row
// loops); each wave stages its own grad rows: one 2-byte load per lane per row
// (lane = column), all in flight at once, written as 2g in fp32 to row r, half
// h = col % 2, slot col / 2 (consecutive lanes write consecutive LDS words),
// each half 16-byte aligned with that half's sum of g in slot JC. The wave
// then adds the half-row sums and column sums of its rows and runs its row
// loop: the generated asm block of l1_asm_gen.h, in which every 16-byte
// wave-wide grad read (two addresses, one per half) feeds 24 VALU instructions
// (two channels x four columns x three), query rows are prefetched four rows
// ahead, and the T(q) of the next row and the grad_query of the previous row
// are interleaved with the current row's arithmetic.
//
// grad_key: per wave, half its column sums of 2g minus its accumulated 2g y,
// summed over the waves in LDS in wave order; the workgroup partials of a slice
// are summed in workgroup order by laplace_dk_reduce_t_kernel. Results are
// deterministic.
#include <algorithm>

#include "lf_common.h"
#include "lf_internal.h"
#include "l1_asm_gen.h"
#include "b2_plan.h"

namespace lfamd {

namespace {

constexpr int kB2Unroll = 4;    // rows per iteration of the asm row loop (its query prefetch depth)
constexpr int kB2SoloRows = 64;  // slices up to this many rows take one workgroup each

// Waves per workgroup for key count M (12 needs the 168-VGPR row loops).
__host__ __device__ constexpr int b2_waves(int M) { return M == 49 ? 12 : 8; }

// Rows of a workgroup's range before wave w (w = WAVES: all n), split by the
// kB2P0 : kB2P1 : kB2P2 weights of b2_plan.h for 12 waves, evenly otherwise.
template <int WAVES>
__device__ __forceinline__ int b2_wave_start(int w, int n) {
  if constexpr (WAVES == 12) {
    const int pl = w >> 2, k = w & 3;  // w = 12: pl = 3, k = 0
    int units = k * (pl == 0 ? kB2P0 : pl == 1 ? kB2P1 : kB2P2);
    if (pl > 0) units += 4 * kB2P0;
    if (pl > 1) units += 4 * kB2P1;
    if (pl > 2) units += 4 * kB2P2;
    return (int)((int64_t)units * n / kB2PSum);
  } else {
    return (int)((int64_t)w * n / WAVES);
  }
}

// Layout constants shared by the kernel and the host plan.
struct B2Shape {
  int M, W, JC, HP, PITCH, NKK;
  __host__ __device__ constexpr B2Shape(int m, int w)
      : M(m), W(w), JC((m + 1) / 2), HP((((m + 1) / 2) + 1 + 3) / 4 * 4),
        PITCH(2 * ((((m + 1) / 2) + 1 + 3) / 4 * 4) + 4), NKK((2 * ((m + 1) / 2) + 3) / 4) {}
  // LDS: the waves' column sums of 2g [W][M] | key-term table [NKK][65][4]
  // (lane-major 16-byte groups, one spare group per table row so that the
  // scatter into it spreads over the banks) | staged rows [kB2MaxRows + 1][PITCH].
  // After the row loops the waves' grad_key sums ([W][M][65], channel fastest,
  // padded) overwrite the table and rows.
  __host__ __device__ constexpr int colsum_bytes() const { return (W * M * 4 + 15) / 16 * 16; }
  __host__ __device__ constexpr int kk_off() const { return colsum_bytes(); }
  __host__ __device__ constexpr int rows_off() const { return kk_off() + NKK * 65 * 16; }
  __host__ __device__ constexpr int red_bytes() const { return W * M * 65 * 4; }
  __host__ __device__ constexpr int lds_bytes() const {
    return rows_off() + (kB2MaxRows + 1) * PITCH * 4 > colsum_bytes() + red_bytes()
               ? rows_off() + (kB2MaxRows + 1) * PITCH * 4
               : colsum_bytes() + red_bytes();
  }
};


template <typename T> __device__ __forceinline__ float g2f(uint16_t b);
template <> __device__ __forceinline__ float g2f<f16s>(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
template <> __device__ __forceinline__ float g2f<bf16s>(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// Dispatch to the generated row loops (grad_query and grad_key together or
// alone; the _v168 forms for 12-wave workgroups).
template <typename T, int M, bool DQ, bool DK, int WAVES> struct B2Rows;
#define LFAMD_B2ROWS(TY, MM, DQ_, DK_, WW, FN)                                                           \
  template <> struct B2Rows<TY, MM, DQ_, DK_, WW> {                                                       \
    __device__ static void run(float (&dk)[2 * ((MM + 1) / 2)], const void* q3, const void* ql, void* dq,  \
                               unsigned qs, int rows, unsigned wpar, unsigned rda, unsigned vq4,           \
                               unsigned vqs, unsigned kka, unsigned paddr, const unsigned (&shf)[4],       \
                               const unsigned (&q0)[kB2Unroll]) {                                          \
      FN(dk, q3, ql, dq, qs, rows, wpar, rda, vq4, vqs, kka, paddr, shf, q0);                             \
    }                                                                                                     \
  };
#define LFAMD_B2ALL(TY, TN, MM)                                        \
  LFAMD_B2ROWS(TY, MM, true, true, 8, bwd2_rows_##TN##_m##MM##_qk)      \
  LFAMD_B2ROWS(TY, MM, true, false, 8, bwd2_rows_##TN##_m##MM##_q)      \
  LFAMD_B2ROWS(TY, MM, false, true, 8, bwd2_rows_##TN##_m##MM##_k)
#define LFAMD_B2ALL12(TY, TN, MM)                                       \
  LFAMD_B2ROWS(TY, MM, true, true, 12, bwd2_rows_##TN##_m##MM##_qk_v168) \
  LFAMD_B2ROWS(TY, MM, true, false, 12, bwd2_rows_##TN##_m##MM##_q_v168) \
  LFAMD_B2ROWS(TY, MM, false, true, 12, bwd2_rows_##TN##_m##MM##_k_v168)
LFAMD_B2ALL12(f16s, f16, 49)
LFAMD_B2ALL12(bf16s, bf16, 49)
LFAMD_B2ALL(f16s, f16, 32)
LFAMD_B2ALL(bf16s, bf16, 32)
LFAMD_B2ALL(f16s, f16, 16)
LFAMD_B2ALL(bf16s, bf16, 16)
#undef LFAMD_B2ALL12
#undef LFAMD_B2ALL
#undef LFAMD_B2ROWS

// Loads `count` >= 1 16-bit elements from `src` as 4-byte words: word b of the
// workgroup in thread b % THREADS, slot b / THREADS. The first word may
// start one element before `src` and the last end one after the span (never
// outside the 4-byte-aligned words holding the span's own bytes); slots past
// the last word load it again. Returns the number of elements before `src` in
// word 0 (0 or 1).
template <int THREADS, int MAXW>
__device__ __forceinline__ int load_words(const uint16_t* src, int count, int tid, uint32_t (&wd)[MAXW]) {
  const int skew = (int)(reinterpret_cast<uintptr_t>(src) & 3) >> 1;
  const uint32_t* base = reinterpret_cast<const uint32_t*>(src - skew);
  const int last = ((count + skew + 1) >> 1) - 1;
#pragma unroll
  for (int i = 0; i < MAXW; ++i) wd[i] = base[min(tid + i * THREADS, last)];
  return skew;
}

// a where c, else b, as one v_cndmask on a lane mask (a plain select lets the
// compiler branch around the computation of a).
__device__ __forceinline__ int select_lanes(bool c, int a, int b) {
  const unsigned long long m = __builtin_amdgcn_ballot_w64(c);
  int r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(b), "v"(a), "s"(m));
  return r;
}

// Calls f(row, col, valid, bits) for both 16-bit halves of every word loaded by
// load_words: (row, col) = (e / M, e % M) for the element index e of the half,
// valid = e in [0, count) (f is to route an invalid element to a dummy
// location). (row, col) advance incrementally from word to word; there are no
// branches. In each call of a wave the lanes hold elements two apart.
template <int M, int THREADS, int MAXW, typename F>
__device__ __forceinline__ void scatter_words(const uint32_t (&wd)[MAXW], int skew, int count, int tid, F f) {
  constexpr int kStep = 2 * THREADS, kDR = kStep / M, kDC = kStep % M;
  int e = 2 * tid - skew;            // >= -1
  int row = (e + M) / M - 1;         // -1 for e = -1
  int col = e - row * M;
#pragma unroll
  for (int i = 0; i < MAXW; ++i) {
    f(row, col, (unsigned)e < (unsigned)count, (uint16_t)(wd[i] & 0xffff));
    const int wrap = col == M - 1 ? 1 : 0;
    f(row + wrap, wrap ? 0 : col + 1, (unsigned)(e + 1) < (unsigned)count, (uint16_t)(wd[i] >> 16));
    e += kStep;
    col += kDC;
    row += kDR;
    const int carry = col >= M ? 1 : 0;
    col -= carry * M;
    row += carry;
  }
}

// Grid: (nx workgroups per slice, channel blocks, B*H). Workgroup x takes rows
// [x*N/nx, (x+1)*N/nx) of its slice, at most kB2MaxRows of them (the host
// plan sizes nx for that), split evenly over the WAVES = b2_waves(M) waves.
//
// GK: the gradient is that of the fused Laplacian kernel K = exp(-s * distance)
// (fp32 gk = dL/dK and kv = K instead of gout): the staged 2g is
// (-2s * gk) * kv, i.e. 2 * fl(fl(-s * gk) * kv) exactly.
// Up to three row sources sharing one key in one launch (fused-kernel gradient
// only): the slice's workgroups are segments of nx[i] workgroups over source
// i's N[i] rows (gk[i], kv[i], query q[i], grad_query dq[i]); every workgroup
// writes a partial, so grad_key sums all sources' rows. Read only by the SEG
// instantiations.
// With cat set, the slice's rows are instead taken as one list (source 0's,
// then source 1's, then source 2's) cut into nx equal workgroup ranges, so that
// every workgroup carries the same work whatever the sources' lengths; each
// wave keeps to one source, and wv[x * 12 + w] gives wave w of workgroup x its
// rows: source (bits 0-1), row count (2-8), first LDS row (9-18) and first row
// within the source (19-31).
struct B2Seg {
  int count;
  int nx[3], N[3];
  const float* gk[3];
  const float* kv[3];
  const void* q[3];
  void* dq[3];
  int cat;
  uint32_t wv[kB2CatSlots * 12];
};

template <typename T, int M, bool DQ, bool DK, bool GK, bool SEG>
__device__ __forceinline__ void bwd2_body(const T* __restrict__ gout, const float* __restrict__ gkIn,
                                          const float* __restrict__ kvIn, float gscale, const T* __restrict__ queryIn,
                                          const T* __restrict__ key, T* __restrict__ dqIn, float* __restrict__ partial,
                                          T* __restrict__ dkOut, int NIn, int C, const B2Seg& sg) {
  constexpr int WAVES = b2_waves(M), THREADS = 64 * WAVES;
  constexpr B2Shape S{M, WAVES};
  constexpr int JC = S.JC, HP = S.HP, PITCH = S.PITCH, NKK = S.NKK;
  static_assert(M >= 2, "M >= 2");
  const int tid = threadIdx.x;
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int nxg = gridDim.x, ncb = gridDim.y;
  int xg = blockIdx.x, cb = blockIdx.y, bh = blockIdx.z;
  // This workgroup's source and its place among that source's workgroups.
  int x = xg, nx = nxg, N = NIn;
  const float* gk = gkIn;
  const float* kv = kvIn;
  const T* query = queryIn;
  T* dq = dqIn;
  // With a concatenated plan: this wave's rows (first LDS row, first source row).
  int catW0 = 0, catRows = 0, catStart = 0;
  if constexpr (SEG) {
    if (sg.cat) {
      const uint32_t e = sg.wv[xg * 12 + wave];
      const int si = (int)(e & 3u);
      catRows = (int)((e >> 2) & 127u);
      catW0 = (int)((e >> 9) & 1023u);
      catStart = (int)(e >> 19);
      N = si == 0 ? sg.N[0] : si == 1 ? sg.N[1] : sg.N[2];
      gk = si == 0 ? sg.gk[0] : si == 1 ? sg.gk[1] : sg.gk[2];
      kv = si == 0 ? sg.kv[0] : si == 1 ? sg.kv[1] : sg.kv[2];
      query = static_cast<const T*>(si == 0 ? sg.q[0] : si == 1 ? sg.q[1] : sg.q[2]);
      dq = static_cast<T*>(si == 0 ? sg.dq[0] : si == 1 ? sg.dq[1] : sg.dq[2]);
    }
  }
  if constexpr (SEG) if (!sg.cat) {
    // Source-major order of the linear workgroup id (dispatch order): all of
    // source 0's workgroups, then source 1's, then source 2's. (Slice-major
    // order left a third round of big workgroups on half the CUs; callers put
    // a small source first, whose workgroups end early and let the big ones in.)
    const int S = ncb * (int)gridDim.z;
    const int L = xg + nxg * (cb + ncb * bh);
    const int e1 = S * sg.nx[0], e2 = e1 + S * sg.nx[1];
    const int si = L < e1 ? 0 : (L < e2 ? 1 : 2);
    nx = si == 0 ? sg.nx[0] : si == 1 ? sg.nx[1] : sg.nx[2];
    const int Ls = L - (si == 0 ? 0 : si == 1 ? e1 : e2);
    const int slice = Ls / nx;
    x = Ls - slice * nx;
    cb = slice % ncb;
    bh = slice / ncb;
    xg = x + (si == 0 ? 0 : si == 1 ? sg.nx[0] : sg.nx[0] + sg.nx[1]);  // the slice's partial slot
    N = si == 0 ? sg.N[0] : si == 1 ? sg.N[1] : sg.N[2];
    gk = si == 0 ? sg.gk[0] : si == 1 ? sg.gk[1] : sg.gk[2];
    kv = si == 0 ? sg.kv[0] : si == 1 ? sg.kv[1] : sg.kv[2];
    query = static_cast<const T*>(si == 0 ? sg.q[0] : si == 1 ? sg.q[1] : sg.q[2]);
    dq = static_cast<T*>(si == 0 ? sg.dq[0] : si == 1 ? sg.dq[1] : sg.dq[2]);
  }

  extern __shared__ __align__(16) unsigned char smem[];
  const unsigned ldsBase = (unsigned)(uintptr_t)smem;
  float* colsum = reinterpret_cast<float*>(smem);                     // [WAVES][M]: column sums of 2g
  float* kkt = reinterpret_cast<float*>(smem + S.kk_off());           // [NKK][65][4]
  float* rowsA = reinterpret_cast<float*>(smem + S.rows_off());       // [rows + 1][PITCH]
  const unsigned rowsBase = ldsBase + S.rows_off();

  const bool cat = SEG && sg.cat;
  // P0 + (LDS row) is the source row: the workgroup's first row, or for a
  // concatenated plan the wave's first source row less its first LDS row.
  const int P0 = cat ? catStart - catW0 : (int)((int64_t)x * N / nx);
  const int n = cat ? 0 : (int)((int64_t)(x + 1) * N / nx) - P0;
  const uint16_t* qsl = reinterpret_cast<const uint16_t*>(query) + (size_t)bh * N * C + cb * 64;

  // All loads first: the key block [64][M] of the channel block (the whole
  // workgroup), this wave's own grad rows (lane = column: RPI rows of M
  // columns per load) and the first query pairs of its row loop.
  constexpr int kKeyW = (64 * M + 2 + 2 * THREADS - 1) / (2 * THREADS);
  uint32_t kwd[kKeyW];
  const int kskew = load_words<THREADS>(reinterpret_cast<const uint16_t*>(key) + ((size_t)bh * C + cb * 64) * M, 64 * M, tid, kwd);
  const int w0 = uniform(cat ? catW0 : b2_wave_start<WAVES>(wave, n));
  const int w1 = uniform(cat ? catW0 + catRows : b2_wave_start<WAVES>(wave + 1, n));
  const int rows = w1 - w0;  // at most b2_max_wave_rows(WAVES)
  const int h = lane >> 5, p = lane & 31;
  constexpr int RPI = 64 / M;                                         // rows per load instruction
  constexpr int kOwnLoads = (b2_max_wave_rows(WAVES) + RPI - 1) / RPI;
  constexpr int kGkSplit = (2 * kOwnLoads + 2) / 3;
  const int lrow = lane / M, lcol = lane - lrow * M;
  uint16_t gv[GK ? 1 : kOwnLoads];
  float ga[GK ? kOwnLoads : 1], ka[GK ? kOwnLoads : 1];
  {
    // Unconditional loads, the row clamped to the wave's last (its first when
    // it has none, w0 < n): a clamped lane holds the value of the row it is
    // later stored to, so the stores need no lane mask.
    const size_t e0 = ((size_t)bh * N + P0 + w0) * M + lcol;
    const int rlast = max(rows, 1) - 1;
    if constexpr (GK) {
      // Two fp32 loads per element: the first two thirds of the rows are
      // combined into 2g before the rest is loaded (so that the register file
      // never holds more than about two thirds of the rows' pairs).
#pragma unroll
      for (int i = 0; i < kGkSplit; ++i) {
        const size_t e = e0 + (size_t)min(i * RPI + lrow, rlast) * M;
        ga[i] = gk[e];
        ka[i] = kv[e];
      }
#pragma unroll
      for (int i = 0; i < kGkSplit; ++i) ga[i] = (-2.0f * gscale * ga[i]) * ka[i];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = kGkSplit; i < kOwnLoads; ++i) {
        const size_t e = e0 + (size_t)min(i * RPI + lrow, rlast) * M;
        ga[i] = gk[e];
        ka[i] = kv[e];
      }
    } else {
      const uint16_t* gw = reinterpret_cast<const uint16_t*>(gout) + e0;
#pragma unroll
      for (int i = 0; i < kOwnLoads; ++i) gv[i] = gw[(size_t)min(i * RPI + lrow, rlast) * M];
    }
  }
  unsigned q0[kB2Unroll];
  {
    const uint32_t* qpair = reinterpret_cast<const uint32_t*>(qsl + (size_t)(P0 + w0) * C) + p;
#pragma unroll
    for (int k = 0; k < kB2Unroll; ++k) q0[k] = rows > 0 ? qpair[(size_t)min(k, rows - 1) * (C / 2)] : 0u;
  }

  // Key terms 0.5 - T(k[c][col]) for lane (h, p): entry [c][j] of the lane
  // (channel 2p + (c ^ h): the lane's own channel first, column 2j + h) at
  // kkt[((e / 4) * 65 + lane) * 4 + e % 4], e = c*JC + j; entries without a
  // key column are zero. (Invalid elements go to the spare entry [0][64][0].)
  scatter_words<M, THREADS>(kwd, kskew, 64 * M, tid, [&](int ch, int col, bool valid, uint16_t bits) {
    const int hc = col & 1;
    const int l = (ch >> 1) + 32 * hc, e = ((ch & 1) ^ hc) * JC + (col >> 1);
    const int a = ((e >> 2) * 65 + l) * 4 + (e & 3);
    kkt[select_lanes(valid, a, 64 * 4)] = 0.5f - tmap16(bits);
  });
  if (tid < 64) {
#pragma unroll
    for (int e = 2 * JC; e < 4 * NKK; ++e) kkt[((e >> 2) * 65 + tid) * 4 + (e & 3)] = 0.0f;
    if (M % 2 && tid >= 32) {
      kkt[(((JC - 1) >> 2) * 65 + tid) * 4 + ((JC - 1) & 3)] = 0.0f;
      kkt[(((2 * JC - 1) >> 2) * 65 + tid) * 4 + ((2 * JC - 1) & 3)] = 0.0f;
    }
  }
  __syncthreads();  // the key-term table is complete

  // Each wave stages and completes its own rows (its LDS operations are
  // performed in order, so its row loop below sees them without a barrier).
  // Grad rows as 2g: column col of row r at rowsA[r*PITCH + (col % 2)*HP + col / 2]
  // (the row pitch is 16 bytes more than the two halves, so that lanes reading
  // consecutive rows spread over the banks). The column sums of 2g over the
  // wave's rows are taken from the same registers, in row order.
  float csum = 0.0f;
  {
    float* dst = rowsA + w0 * PITCH + (lcol & 1) * HP + (lcol >> 1);
#pragma unroll
    for (int i = 0; i < kOwnLoads; ++i) {
      if (i * RPI < rows) {  // wave-uniform; lanes past the last row rewrite it with its own value
        float v2;
        if constexpr (GK) {
          v2 = i < kGkSplit ? ga[i] : (-2.0f * gscale * ga[i]) * ka[i];
        } else {
          const float v = g2f<T>(gv[i]);
          v2 = v + v;
        }
        const int r = i * RPI + lrow;
        dst[min(r, rows - 1) * PITCH] = v2;
        if (DK) csum += r < rows ? v2 : 0.0f;
      }
    }
  }
  if (DK) {
    // Lanes lcol + M t (t < 64 / M) hold the same column when M divides 64.
    if constexpr (64 % M == 0) {
#pragma unroll
      for (int m = M; m < 64; m <<= 1) csum += __shfl_xor(csum, m);
    }
    if (lane < M) colsum[wave * M + lane] = csum;
  }
  if (lane < rows) {
    // Each half's sum of g (half of the sum of its staged 2g) into its slot JC,
    // read as 16-byte groups; an odd M's missing column of half 1 (slot JC - 1)
    // is zeroed.
    float* rp = rowsA + (w0 + lane) * PITCH;
    if (DQ) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int cols = hh == 0 ? JC : M - JC;
        float s2 = 0.0f;
#pragma unroll
        for (int g = 0; g * 4 < cols; ++g) {
          const float4 a = *reinterpret_cast<const float4*>(rp + hh * HP + 4 * g);
          const float b = (4 * g + 1 < cols ? a.x + a.y : a.x) + (4 * g + 3 < cols ? a.z + a.w : 4 * g + 2 < cols ? a.z : 0.0f);
          s2 += b;
        }
        rp[hh * HP + JC] = 0.5f * s2;
      }
    }
    if (M % 2) rp[HP + JC - 1] = 0.0f;
  }
  float dk[2 * JC];
#pragma unroll
  for (int j = 0; j < 2 * JC; ++j) dk[j] = 0.0f;
  if (rows > 0) {
    const unsigned rda = rowsBase + (unsigned)(w0 * PITCH + h * HP) * 4;
    const uint16_t* q3 = uniform_ptr(qsl + (size_t)(P0 + w0 + kB2Unroll - 1) * C);
    const uint16_t* ql = uniform_ptr(qsl + (size_t)(P0 + w1 - 1) * C);
    uint16_t* dqrow = uniform_ptr(reinterpret_cast<uint16_t*>(dq) + ((size_t)bh * N + P0 + w0) * C + cb * 64);
    // Bit offsets of the lane's channels in a query pair (own channel 2p + h first).
    const unsigned shf[4] = {16u * h, 16u * h + 15u, 16u - 16u * h, 31u - 16u * h};
    // wpar: the wave's place among the waves of its SIMD (wave w runs on SIMD w % 4).
    B2Rows<T, M, DQ, DK, WAVES>::run(dk, q3, ql, dqrow, (unsigned)C * 2, rows, (unsigned)uniform(wave >> 2), rda,
                                     (unsigned)p * 4, (unsigned)(2 * p + h) * 2,
                                     ldsBase + S.kk_off() + (unsigned)lane * 16, (unsigned)(lane ^ 32) * 4, shf,
                                     q0);
  }
  if constexpr (!DK) return;

  // Workgroup grad_key partial: per wave, half its column sums of 2g minus its
  // accumulated 2g y; summed over the waves in wave order and written
  // channel-major. (A wave's column sums were written by its own lanes.)
  // Channel c sits at slot (c >> 1) + 32 (c & 1) of its column's 65: the
  // lanes of each half-wave write 32 consecutive slots (the own and the
  // partner channel of lane (h, p) are both at slot p of a half), and the
  // final sum reads consecutive columns at stride 65, without bank conflicts.
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem + S.colsum_bytes());   // [WAVES][M][65]
  {
    // All column sums first: the stores below may alias them as far as the
    // compiler knows, and would otherwise wait for one read each.
    float cs[JC];
#pragma unroll
    for (int j = 0; j < JC; ++j) cs[j] = colsum[wave * M + min(2 * j + h, M - 1)];
    float* buf = red + wave * M * 65;
#pragma unroll
    for (int j = 0; j < JC; ++j) {
      const int col = 2 * j + h;
      if (col < M) {
        buf[col * 65 + p + 32 * h] = 0.5f * cs[j] - dk[j];            // own channel 2p + h
        buf[col * 65 + p + 32 - 32 * h] = 0.5f * cs[j] - dk[JC + j];  // partner's channel 2p + 1 - h
      }
    }
  }
  __syncthreads();
  // [64][M] channel-major: the workgroup's partial, or with one workgroup per
  // slice (dkOut) grad_key itself, rounded once.
  for (int t = tid; t < 64 * M; t += THREADS) {
    const int c = t / M, col = t - c * M;
    const int slot = col * 65 + (c >> 1) + 32 * (c & 1);
    float s2 = red[slot];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) s2 += red[w * M * 65 + slot];
    if (dkOut)
      dkOut[((size_t)bh * C + cb * 64) * M + t] = from_acc<T>(s2);
    else
      partial[(((size_t)bh * ncb + cb) * nxg + xg) * 64 * M + t] = s2;
  }
}

// The plain kernel (one row source) and the segmented one (up to three sources
// sharing the key, B2Seg; fused-kernel gradient, dq and dk); both run bwd2_body.
template <typename T, int M, bool DQ, bool DK, bool GK = false>
__global__ void __launch_bounds__(64 * b2_waves(M), 1)
laplace_bwd2_kernel(const T* __restrict__ gout, const float* __restrict__ gk, const float* __restrict__ kv,
                    float gscale, const T* __restrict__ query, const T* __restrict__ key, T* __restrict__ dq,
                    float* __restrict__ partial, T* __restrict__ dkOut, int N, int C) {
  bwd2_body<T, M, DQ, DK, GK, false>(gout, gk, kv, gscale, query, key, dq, partial, dkOut, N, C, B2Seg{});
}

template <typename T, int M>
__global__ void __launch_bounds__(64 * b2_waves(M), 1)
laplace_bwd2_seg_kernel(const T* __restrict__ key, float* __restrict__ partial, int C, float gscale, B2Seg sg) {
  bwd2_body<T, M, true, true, true, true>(nullptr, nullptr, nullptr, gscale, nullptr, key, nullptr, partial, nullptr,
                                          0, C, sg);
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
  int i = 0;
  for (; i + 8 <= nx; i += 8) {  // eight loads in flight, summed in order
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = p[(size_t)(i + k) * n];
#pragma unroll
    for (int k = 0; k < 8; ++k) s += v[k];
  }
  for (; i < nx; ++i) s += p[(size_t)i * n];
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
  // One workgroup per CU where the rows allow (at least 8 rows each), and never
  // more than kB2MaxRows rows per workgroup (its LDS holds that many). Up to
  // kB2SoloRows rows a slice takes one workgroup, which writes grad_key itself
  // (no partials, no reduction launch).
  p.nx = N <= kB2SoloRows
             ? 1
             : (int)std::max<int64_t>((N + kB2MaxRows - 1) / kB2MaxRows,
                                      std::max<int64_t>(1, std::min<int64_t>(num_cus() / std::max<int64_t>(slices, 1),
                                                                             (N + 7) / 8)));
  p.lds = (size_t)B2Shape((int)M, b2_waves((int)M)).lds_bytes();
  p.partialElems = p.nx == 1 ? 0 : (size_t)slices * p.nx * 64 * (size_t)M;
  return p;
}

template <typename T, int M, bool DQ, bool DK>
int launch_b2_m(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, int64_t BH, int64_t N,
                int64_t C, const B2Plan& p, hipStream_t st, const B2Grad& kg, const B2Seg& sg = B2Seg{}) {
  dim3 grid(p.nx, p.ncb, (unsigned)BH);
  T* dkOut = DK && p.nx == 1 && sg.count == 0 ? static_cast<T*>(dk) : nullptr;
  const void* fn = kg.gk && sg.count > 0 ? reinterpret_cast<const void*>(laplace_bwd2_seg_kernel<T, M>)
                   : kg.gk              ? reinterpret_cast<const void*>(laplace_bwd2_kernel<T, M, DQ, DK, true>)
                                        : reinterpret_cast<const void*>(laplace_bwd2_kernel<T, M, DQ, DK, false>);
  if (int s = check_fit(fn, 64 * b2_waves(M), p.lds, "laplace backward (column-split)")) return s;
  if (kg.gk && sg.count > 0) {
    if constexpr (M == 49 && DQ && DK)
      hipLaunchKernelGGL((laplace_bwd2_seg_kernel<T, M>), grid, dim3(64 * b2_waves(M)), p.lds, st,
                         static_cast<const T*>(k), static_cast<float*>(ws), (int)C, kg.scale, sg);
    else
      return fail(LFAMD_ERR_UNSUPPORTED, "laplace backward: several sources need M = 49 with dq and dk");
  } else if (kg.gk)
    hipLaunchKernelGGL((laplace_bwd2_kernel<T, M, DQ, DK, true>), grid, dim3(64 * b2_waves(M)), p.lds, st,
                       static_cast<const T*>(g), kg.gk, kg.kv, kg.scale, static_cast<const T*>(q),
                       static_cast<const T*>(k), static_cast<T*>(dq), static_cast<float*>(ws), dkOut, (int)N, (int)C);
  else
    hipLaunchKernelGGL((laplace_bwd2_kernel<T, M, DQ, DK, false>), grid, dim3(64 * b2_waves(M)), p.lds, st,
                       static_cast<const T*>(g), kg.gk, kg.kv, kg.scale, static_cast<const T*>(q),
                       static_cast<const T*>(k), static_cast<T*>(dq), static_cast<float*>(ws), dkOut, (int)N, (int)C);
  int s = check_launch("laplace backward (column-split)");
  if (s || !DK || dkOut) return s;
  dim3 rgrid((64 * M + 255) / 256, p.ncb, (unsigned)BH);
  hipLaunchKernelGGL(laplace_dk_reduce_t_kernel<T>, rgrid, dim3(256), 0, st, static_cast<const float*>(ws),
                     static_cast<T*>(dk), p.nx, M, (int)C);
  return check_launch("laplace backward_key reduction");
}

template <typename T, bool DQ, bool DK>
int launch_b2_t(const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, int64_t BH, int64_t N,
                int64_t M, int64_t C, const B2Plan& p, hipStream_t st, const B2Grad& kg) {
  switch (M) {
    case 16: return launch_b2_m<T, 16, DQ, DK>(g, q, k, dq, dk, ws, BH, N, C, p, st, kg);
    case 32: return launch_b2_m<T, 32, DQ, DK>(g, q, k, dq, dk, ws, BH, N, C, p, st, kg);
    default: return launch_b2_m<T, 49, DQ, DK>(g, q, k, dq, dk, ws, BH, N, C, p, st, kg);
  }
}

template <bool DQ, bool DK>
int launch_b2(int dtype, const void* g, const void* q, const void* k, void* dq, void* dk, void* ws, int64_t BH,
              int64_t N, int64_t M, int64_t C, const B2Plan& p, hipStream_t st, const B2Grad& kg) {
  if (dtype == LFAMD_BF16) return launch_b2_t<bf16s, DQ, DK>(g, q, k, dq, dk, ws, BH, N, M, C, p, st, kg);
  return launch_b2_t<f16s, DQ, DK>(g, q, k, dq, dk, ws, BH, N, M, C, p, st, kg);
}

}  // namespace

// grad_query and / or grad_key on the column-split kernel (null dq or dk: that
// half is skipped): fp16 / bf16, M in {16, 32, 49}, C a multiple of 64 (one
// channel block per 64 channels), N >= 1. The caller also needs the query
// 4-byte aligned (it is read as channel pairs).
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
              int64_t BH, int64_t N, int64_t M, int64_t C, hipStream_t st, const char* who, const B2Grad& kg) {
  const B2Plan p = plan_b2(BH, N, M, C);
  if (dk && p.partialElems && (!ws || wsBytes < p.partialElems * 4))
    return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, p.partialElems * 4, wsBytes);
  if (kg.gk && dtype != LFAMD_F16) return fail(LFAMD_ERR_UNSUPPORTED, "%s: fused kernel gradient needs fp16", who);
  if (dq && dk) return launch_b2<true, true>(dtype, g, q, k, dq, dk, ws, BH, N, M, C, p, st, kg);
  if (dq) return launch_b2<true, false>(dtype, g, q, k, dq, dk, ws, BH, N, M, C, p, st, kg);
  return launch_b2<false, true>(dtype, g, q, k, dq, dk, ws, BH, N, M, C, p, st, kg);
}

namespace {
// Workgroups per source of a segmented launch and the partials they write.
// The concatenated plan (B2Seg::cat) for sources of n[i] rows: nx workgroups
// per slice (b2_cat_nx), zero when the sources do not fit it (then each source
// takes its own workgroups). The wave tables (b2_cat_tables) are searched once
// per shape and host thread (~0.8 ms) and kept for the last few shapes.
int plan_b2_cat(int nsrc, const int64_t* n, int64_t BH, int64_t C, uint32_t* wv) {
  if (nsrc < 2) return 0;
  const int nx = b2_cat_nx(nsrc, n, BH * (C / 64), num_cus());
  if (nx == 0) return 0;
  struct Key {
    int nsrc, nx;
    int64_t n[3];
  };
  constexpr int kCache = 4;
  static thread_local Key keys[kCache] = {};
  static thread_local uint32_t tabs[kCache][kB2CatSlots * 12];
  static thread_local int okay[kCache] = {};
  static thread_local int used = 0, next = 0;
  const Key key{nsrc, nx, {n[0], nsrc > 1 ? n[1] : 0, nsrc > 2 ? n[2] : 0}};
  for (int i = 0; i < used; ++i)
    if (keys[i].nsrc == key.nsrc && keys[i].nx == key.nx && keys[i].n[0] == key.n[0] && keys[i].n[1] == key.n[1] &&
        keys[i].n[2] == key.n[2]) {
      std::copy(tabs[i], tabs[i] + kB2CatSlots * 12, wv);
      return okay[i] ? nx : 0;
    }
  const int slot = used < kCache ? used++ : next;
  next = (slot + 1) % kCache;
  keys[slot] = key;
  const bool ok = b2_cat_tables(nsrc, n, nx, tabs[slot]);
  okay[slot] = ok;
  std::copy(tabs[slot], tabs[slot] + kB2CatSlots * 12, wv);
  return ok ? nx : 0;
}

B2Plan plan_b2_multi(int nsrc, const int64_t* n, int64_t BH, int64_t C, B2Seg& sg) {
  B2Plan p{};
  sg.count = nsrc;
  if (const int nx = plan_b2_cat(nsrc, n, BH, C, sg.wv)) {
    sg.cat = 1;
    for (int i = 0; i < nsrc; ++i) sg.N[i] = (int)n[i];
    const B2Plan p0 = plan_b2(BH, n[0], 49, C);
    p.nx = nx;
    p.ncb = p0.ncb;
    p.lds = p0.lds;
    p.partialElems = (size_t)BH * p.ncb * p.nx * 64 * 49;
    return p;
  }
  sg.cat = 0;
  for (int i = 0; i < nsrc; ++i) {
    const B2Plan pi = plan_b2(BH, n[i], 49, C);
    sg.nx[i] = pi.nx;
    sg.N[i] = (int)n[i];
    p.nx += pi.nx;
    p.ncb = pi.ncb;
    p.lds = pi.lds;
  }
  p.partialElems = (size_t)BH * p.ncb * p.nx * 64 * 49;
  return p;
}
}  // namespace

size_t b2_workspace_elems_multi(int nsrc, const int64_t* n, int64_t BH, int64_t C) {
  B2Seg sg{};
  return plan_b2_multi(nsrc, n, BH, C, sg).partialElems;
}

int64_t b2_multi_workgroups(int nsrc, const int64_t* n, int64_t BH, int64_t C) {
  int64_t total = 0;
  for (int i = 0; i < nsrc; ++i) total += (int64_t)plan_b2(BH, n[i], 49, C).nx;
  return total * (C / 64) * BH;
}

int b2_launch_multi(int nsrc, const float* const* gk, const float* const* kv, const void* const* q, void* const* dq,
                    const int64_t* n, const void* k, void* dk, void* ws, size_t wsBytes, int64_t BH, int64_t C, float scale,
                    hipStream_t st, const char* who) {
  B2Seg sg{};
  const B2Plan p = plan_b2_multi(nsrc, n, BH, C, sg);
  for (int i = 0; i < nsrc; ++i) {
    sg.gk[i] = gk[i];
    sg.kv[i] = kv[i];
    sg.q[i] = q[i];
    sg.dq[i] = dq[i];
  }
  if (!ws || wsBytes < p.partialElems * 4)
    return fail(LFAMD_ERR_ARG, "%s: workspace of %zu bytes needed, %zu given", who, p.partialElems * 4, wsBytes);
  return launch_b2_m<f16s, 49, true, true>(nullptr, nullptr, k, nullptr, dk, ws, BH, 0, C, p, st,
                                           B2Grad{gk[0], kv[0], scale}, sg);
}

}  // namespace lfamd

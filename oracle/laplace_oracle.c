/*
 * CPU restatement of LaplaceSubtraction (forward, backward-query,
 * backward-key) in the reference's exact accumulation order.
 *
 * TEST INFRASTRUCTURE ONLY: this file is the parity checker (and the timed
 * CPU "port" baseline of bench.py). Nothing in the laplacianformer_amd product
 * path links, loads or calls it.
 *
 * Inputs are fp32 (fp16/bf16 tensors are widened exactly by the caller) or
 * fp64; outputs are the unrounded accumulators, which the caller rounds once to
 * the element type (reference from_acc at the store).
 *
 *   forward   out[i,j] = sum_c |q[i,c] - k[c,j]|, c ascending
 *             (src/LaplaceSubtraction_cuda_kernel.cu:84-125, store :137)
 *   dq        dq[i,c]  = sum_j g[i,j] * sgn(q[i,c] - k[c,j]), j ascending
 *             (:206-249 without split-K; sgn per :34-38, sgn(0) = 0)
 *   dk        dk[c,j]  = -sum_i g[i,j] * sgn(q[i,c] - k[c,j]), i ascending
 *             (:332-375 without split-P)
 * Layouts: q [BH,N,C], k [BH,C,M] (channel-major key), g/out [BH,N,M],
 * dq [BH,N,C], dk [BH,C,M] (src/LaplaceSubtraction_cuda.cu:12-28,59-63).
 * Parallel over (bh, row) with OpenMP; each output is still summed serially in
 * the order above, so the result does not depend on the thread count.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>

#define SGN(v) (((v) > 0) - ((v) < 0))

/* The reference is built with nvcc --use_fast_math (setup.py:29), which implies
 * -ftz=true: single-precision instructions read denormal operands as zero and
 * flush denormal results to zero (sign kept). The f32ftz entry points restate
 * that build: every fp32 input and every operation's result passes FTZ. The
 * plain f32 / f64 entry points are IEEE (fast math does not flush fp64). */
static inline float ftz_f(float x) { return fabsf(x) < FLT_MIN ? copysignf(0.0f, x) : x; }
#define ID(x) (x)

#define DEFINE_ORACLE(T, SUF, FZ)                                                      \
  void lf_oracle_forward_##SUF(const T* q, const T* k, T* out, int64_t BH, int64_t N,  \
                               int64_t M, int64_t C) {                                 \
    _Pragma("omp parallel for collapse(2) schedule(static)")                           \
    for (int64_t b = 0; b < BH; ++b)                                                   \
      for (int64_t i = 0; i < N; ++i) {                                                \
        const T* qi = q + (b * N + i) * C;                                             \
        const T* kb = k + b * C * M;                                                   \
        T* oi = out + (b * N + i) * M;                                                 \
        for (int64_t j = 0; j < M; ++j) {                                              \
          T acc = 0;                                                                   \
          for (int64_t c = 0; c < C; ++c) {                                            \
            T d = FZ(FZ(qi[c]) - FZ(kb[c * M + j]));                                   \
            acc = FZ(acc + (d < 0 ? -d : d));                                          \
          }                                                                            \
          oi[j] = acc;                                                                 \
        }                                                                              \
      }                                                                                \
  }                                                                                    \
                                                                                       \
  void lf_oracle_backward_query_##SUF(const T* g, const T* q, const T* k, T* dq,       \
                                      int64_t BH, int64_t N, int64_t M, int64_t C) {   \
    _Pragma("omp parallel for collapse(2) schedule(static)")                           \
    for (int64_t b = 0; b < BH; ++b)                                                   \
      for (int64_t i = 0; i < N; ++i) {                                                \
        const T* qi = q + (b * N + i) * C;                                             \
        const T* gi = g + (b * N + i) * M;                                             \
        const T* kb = k + b * C * M;                                                   \
        for (int64_t c = 0; c < C; ++c) {                                              \
          T acc = 0;                                                                   \
          for (int64_t j = 0; j < M; ++j)                                              \
            acc = FZ(acc + FZ(gi[j]) * (T)SGN(FZ(FZ(qi[c]) - FZ(kb[c * M + j]))));     \
          dq[(b * N + i) * C + c] = acc;                                               \
        }                                                                              \
      }                                                                                \
  }                                                                                    \
                                                                                       \
  /* i is the outer loop so that rows stream; each dk[c,j] is still summed in  */ \
  /* ascending i.                                                              */ \
  void lf_oracle_backward_key_##SUF(const T* g, const T* q, const T* k, T* dk,         \
                                    int64_t BH, int64_t N, int64_t M, int64_t C) {     \
    _Pragma("omp parallel for collapse(2) schedule(static)")                           \
    for (int64_t b = 0; b < BH; ++b)                                                   \
      for (int64_t c = 0; c < C; ++c) {                                                \
        const T* kc = k + (b * C + c) * M;                                             \
        T* acc = dk + (b * C + c) * M;                                                 \
        for (int64_t j = 0; j < M; ++j) acc[j] = 0;                                    \
        for (int64_t i = 0; i < N; ++i) {                                              \
          const T qv = q[(b * N + i) * C + c];                                         \
          const T* gi = g + (b * N + i) * M;                                           \
          for (int64_t j = 0; j < M; ++j)                                              \
            acc[j] = FZ(acc[j] - FZ(gi[j]) * (T)SGN(FZ(FZ(qv) - FZ(kc[j]))));          \
        }                                                                              \
      }                                                                                \
  }

DEFINE_ORACLE(float, f32, ID)
DEFINE_ORACLE(float, f32ftz, ftz_f)
DEFINE_ORACLE(double, f64, ID)

int lf_oracle_max_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}

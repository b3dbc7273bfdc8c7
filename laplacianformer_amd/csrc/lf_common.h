// Shared device helpers for the gfx950 LaplaceSubtraction / NewtonInverse kernels.
//
// Storage types: f16s / bf16s wrap the 16-bit patterns so that every
// conversion is explicit. Arithmetic is fp32 for f32/f16/bf16 storage and fp64
// for double storage (reference AccT, src/LaplaceSubtraction_cuda_kernel.cu:17-19,
// src/NewtonInverse_cuda_kernel.cu:17-19).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lfamd {

struct f16s { uint16_t bits; };
struct bf16s { uint16_t bits; };

template <typename T> struct AccOf { using type = float; };
template <> struct AccOf<double> { using type = double; };

// ---- element conversions ---------------------------------------------------
__device__ __forceinline__ float to_acc(float x) { return x; }
__device__ __forceinline__ double to_acc(double x) { return x; }
__device__ __forceinline__ float to_acc(f16s x) {
  return (float)__builtin_bit_cast(_Float16, x.bits);
}
__device__ __forceinline__ float to_acc(bf16s x) {
  return __builtin_bit_cast(float, (uint32_t)x.bits << 16);
}

// Round-to-nearest-even narrowing (the rounding of a C++ cast on both vendors).
template <typename T> __device__ __forceinline__ T from_acc(typename AccOf<T>::type v);
template <> __device__ __forceinline__ float from_acc<float>(float v) { return v; }
template <> __device__ __forceinline__ double from_acc<double>(double v) { return v; }
template <> __device__ __forceinline__ f16s from_acc<f16s>(float v) {
  return f16s{__builtin_bit_cast(uint16_t, (_Float16)v)};
}
template <> __device__ __forceinline__ bf16s from_acc<bf16s>(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16s{(uint16_t)0x7fc0};  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16s{(uint16_t)(u >> 16)};
}

// ---- v_fma_mix_f32: fp32 result from fp16 halves, no separate conversion ----
// d = f32(a.half[AS]) - f32(b.half[BS]), computed exactly then rounded once to
// fp32, i.e. the same value as (float)a - (float)b. AS/BS select the low (0) or
// high (1) 16 bits of each packed register.
template <int AS, int BS>
__device__ __forceinline__ float mix_sub_hh(uint32_t a, uint32_t b) {
  float d;
  if constexpr (AS == 0 && BS == 0)
    asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,0] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  else if constexpr (AS == 0 && BS == 1)
    asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  else if constexpr (AS == 1 && BS == 0)
    asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[1,0,0] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  return d;
}

// acc + s * f32(g.half[GS]) and acc - s * f32(g.half[GS]), one rounding each.
template <int GS>
__device__ __forceinline__ float mix_fma_fh(float s, uint32_t g, float acc) {
  float r;
  if constexpr (GS == 0)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(s), "v"(g), "v"(acc));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(s), "v"(g), "v"(acc));
  return r;
}
template <int GS>
__device__ __forceinline__ float mix_fms_fh(float s, uint32_t g, float acc) {
  float r;
  if constexpr (GS == 0)
    asm("v_fma_mix_f32 %0, %1, -%2, %3 op_sel:[0,0,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(s), "v"(g), "v"(acc));
  else
    asm("v_fma_mix_f32 %0, %1, -%2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(s), "v"(g), "v"(acc));
  return r;
}

// Wave-uniform value hint (moves a VGPR that is known to be uniform to an SGPR).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Pointer form of uniform().
template <typename P>
__device__ __forceinline__ P* uniform_ptr(P* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<P*>(((uint64_t)hi << 32) | lo);
}

// Orders the LDS accesses of one wave around this point: what any lane of the
// wave wrote before it is visible to every lane of the wave after it.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Half step of a scaled difference: clamp(0.5 * d + 0.5) to [0, 1]. The
// compiler folds the median into the clamp output modifier of the v_fma_f32
// (kernels run with DX10 clamping), one full-rate VALU instruction with inline
// constants. For a d that is 0 or at least 1 in magnitude the result is exactly
// 0 (d < 0), 0.5 (d == 0) or 1 (d > 0), i.e. (sgn(d) + 1) / 2.
// Ordered map of a 16-bit float pattern (fp16 or bf16): T = 2^22 + 2^14 + t / 2,
// the fp32 bit pattern 0x4a808000 + t, with t the signed magnitude of the pattern
// (+0 and -0 both 0). T is strictly increasing in the value over every non-NaN
// pattern (infinities included) and its values are multiples of 1/2 in [2^22, 2^23),
// so T(q) + (1/2 - T(k)) is exact and clamps to exactly 0, 1/2 or 1 =
// (sgn(q - k) + 1) / 2. A NaN pattern orders beyond the infinities by its sign bit.
__device__ __forceinline__ float tmap16(uint16_t bits) {
  const int t = (bits & 0x8000) ? -(int)(bits & 0x7fff) : (int)bits;
  return __builtin_bit_cast(float, (uint32_t)(0x4a808000 + t));
}

__device__ __forceinline__ float half_step(float d) {
  return __builtin_amdgcn_fmed3f(__builtin_fmaf(d, 0.5f, 0.5f), 0.0f, 1.0f);
}

__host__ __device__ constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int round_up(int a, int b) { return ceil_div(a, b) * b; }

}  // namespace lfamd

// PyTorch-facing LaplaceSubtraction API of the MI355X build.
//
// Same namespace, function names, argument order and error texts as the
// reference header (include/LaplaceSubtraction.h:6-108), so C++ includers and
// the pybind11 module keep compiling and behaving the same. The *_cuda
// functions are implemented on the C ABI of include/laplacianformer_amd.h
// (LaplaceSubtraction_hip.cpp); nothing here runs on the CPU.
#pragma once
#include <torch/types.h>

#include <optional>

namespace laplace {

#if defined(WITH_HIP)
void LaplaceSubtraction_forward_cuda(const at::Tensor query, const at::Tensor key, at::Tensor output);
void LaplaceSubtraction_backward_query_cuda(const at::Tensor gradOutput, const at::Tensor query,
                                            const at::Tensor key, at::Tensor gradQuery);
void LaplaceSubtraction_backward_key_cuda(const at::Tensor gradOutput, const at::Tensor query,
                                          const at::Tensor key, at::Tensor gradKey);
void LaplaceSubtraction_reduce_forward_cuda(const at::Tensor query, const at::Tensor key, at::Tensor output);
// Superset: grad_query and grad_key in one pass (no reference counterpart).
void LaplaceSubtraction_backward_cuda(const at::Tensor gradOutput, const at::Tensor query,
                                      const at::Tensor key, at::Tensor gradQuery, at::Tensor gradKey);
// Superset: the Laplacian kernel exp(-scale * dist) in fp32 with the exp fused
// into the forward, and its backward with -scale * gradKernel * kernel formed in
// the backward's staging. Both return false (and write nothing) where the fused
// path does not cover the sizes or type; the caller then composes the ops above.
bool LaplaceKernel_forward_cuda(const at::Tensor query, const at::Tensor key, at::Tensor output, double scale);
bool LaplaceKernel_backward_cuda(const at::Tensor gradKernel, const at::Tensor kernel, const at::Tensor query,
                                 const at::Tensor key, std::optional<at::Tensor> gradQuery,
                                 std::optional<at::Tensor> gradKey, double scale);
// LaplacianFormer attention layer's row products (no reference counterpart):
// C[..., n, q] = sum_p A[..., n, p] * B[..., q, p] for a small B read through its
// strides, inner and output widths <= 64 (lfamd_mix_rows).
void MixRows_cuda(const at::Tensor a, const at::Tensor b, at::Tensor c);
// C[..., p, q] = sum_n A[..., n, p] * B[..., n, q], A and C float32, widths <= 64 (lfamd_tall_t).
void TallT_cuda(const at::Tensor a, const at::Tensor b, at::Tensor c);
#endif

inline void LaplaceSubtraction_forward(const at::Tensor query, const at::Tensor key, at::Tensor output) {
  if (query.is_cuda() && key.is_cuda()) {
#if defined(WITH_HIP)
    return LaplaceSubtraction_forward_cuda(query, key, output);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline void LaplaceSubtraction_backward_query(const at::Tensor gradOutput, const at::Tensor query,
                                              const at::Tensor key, at::Tensor gradQuery) {
  if (gradOutput.is_cuda() && query.is_cuda() && key.is_cuda()) {
#if defined(WITH_HIP)
    return LaplaceSubtraction_backward_query_cuda(gradOutput, query, key, gradQuery);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline void LaplaceSubtraction_backward_key(const at::Tensor gradOutput, const at::Tensor query,
                                            const at::Tensor key, at::Tensor gradKey) {
  if (gradOutput.is_cuda() && query.is_cuda() && key.is_cuda()) {
#if defined(WITH_HIP)
    return LaplaceSubtraction_backward_key_cuda(gradOutput, query, key, gradKey);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline void LaplaceSubtraction_reduce_forward(const at::Tensor query, const at::Tensor key, at::Tensor output) {
  if (query.is_cuda() && key.is_cuda()) {
#if defined(WITH_HIP)
    return LaplaceSubtraction_reduce_forward_cuda(query, key, output);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline void LaplaceSubtraction_backward(const at::Tensor gradOutput, const at::Tensor query,
                                        const at::Tensor key, at::Tensor gradQuery, at::Tensor gradKey) {
  if (gradOutput.is_cuda() && query.is_cuda() && key.is_cuda()) {
#if defined(WITH_HIP)
    return LaplaceSubtraction_backward_cuda(gradOutput, query, key, gradQuery, gradKey);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline bool LaplaceKernel_forward(const at::Tensor query, const at::Tensor key, at::Tensor output, double scale) {
  if (query.is_cuda() && key.is_cuda()) {
#if defined(WITH_HIP)
    return LaplaceKernel_forward_cuda(query, key, output, scale);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline void MixRows(const at::Tensor a, const at::Tensor b, at::Tensor c) {
  if (a.is_cuda() && b.is_cuda() && c.is_cuda()) {
#if defined(WITH_HIP)
    return MixRows_cuda(a, b, c);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline void TallT(const at::Tensor a, const at::Tensor b, at::Tensor c) {
  if (a.is_cuda() && b.is_cuda() && c.is_cuda()) {
#if defined(WITH_HIP)
    return TallT_cuda(a, b, c);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

inline bool LaplaceKernel_backward(const at::Tensor gradKernel, const at::Tensor kernel, const at::Tensor query,
                                   const at::Tensor key, std::optional<at::Tensor> gradQuery,
                                   std::optional<at::Tensor> gradKey, double scale) {
  if (gradKernel.is_cuda() && query.is_cuda() && key.is_cuda()) {
#if defined(WITH_HIP)
    return LaplaceKernel_backward_cuda(gradKernel, kernel, query, key, gradQuery, gradKey, scale);
#else
    AT_ERROR("Not compiled with GPU support");
#endif
  }
  AT_ERROR("Not implemented on the CPU");
}

}  // namespace laplace

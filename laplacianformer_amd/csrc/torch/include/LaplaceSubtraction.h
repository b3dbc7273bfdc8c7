// PyTorch-facing LaplaceSubtraction API of the MI355X build.
//
// Same namespace, function names, argument order and error texts as the
// reference header (include/LaplaceSubtraction.h:6-108), so C++ includers and
// the pybind11 module keep compiling and behaving the same. The *_cuda
// functions are implemented on the C ABI of include/laplacianformer_amd.h
// (LaplaceSubtraction_hip.cpp); nothing here runs on the CPU.
#pragma once
#include <torch/types.h>

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

}  // namespace laplace

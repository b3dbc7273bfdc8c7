// Shared helpers of the PyTorch adapters: dtype mapping, status -> exception,
// device guard and current stream.
#pragma once
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/types.h>

#include "../../../include/laplacianformer_amd.h"

namespace laplace {
namespace detail {

// Element type code of the C ABI; rejects what the ops do not implement with
// the wording of ATen's dispatch macros.
inline int abi_dtype(const at::Tensor& t, const char* op) {
  switch (t.scalar_type()) {
    case at::kFloat: return LFAMD_F32;
    case at::kHalf: return LFAMD_F16;
    case at::kBFloat16: return LFAMD_BF16;
    case at::kDouble: return LFAMD_F64;
    default: TORCH_CHECK(false, '"', op, "\" not implemented for '", toString(t.scalar_type()), "'");
  }
  return -1;
}

inline void same_type(const at::Tensor& ref, const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == ref.scalar_type(), "expected ", name, " to have scalar type ",
              toString(ref.scalar_type()), " but found ", toString(t.scalar_type()));
  TORCH_CHECK(t.is_cuda() && t.device() == ref.device(), name, " must be on the same GPU as the inputs");
}

inline void check_status(int status) {
  TORCH_CHECK(status == LFAMD_OK, lfamd_last_error()[0] ? lfamd_last_error() : lfamd_status_string(status));
}

inline void* stream_of(const at::Tensor& t) {
  return static_cast<void*>(at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

}  // namespace detail
}  // namespace laplace

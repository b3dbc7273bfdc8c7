// Host adapters of NewtonInverse: the reference's checks
// (src/NewtonInverse_cuda_kernel.cu:764-833), then the C ABI of
// include/laplacianformer_amd.h on the tensor's device and current stream.
#include "NewtonInverse.h"

#include "torch_common.h"

namespace laplace {

bool NewtonInverse_supports(int N) { return lfamd_newton_is_supported(N) != 0; }

void NewtonInverse_forward_cuda(const at::Tensor mat, at::Tensor output, int iter) {
  at::hip::HIPGuardMasqueradingAsCUDA guard(mat.device());
  TORCH_CHECK(mat.is_contiguous(), "mat must be contiguous");
  TORCH_CHECK(output.is_contiguous(), "output must be contiguous");
  TORCH_CHECK(mat.sizes() == output.sizes(), "mat and output must have the same shape");
  const int64_t BH = mat.size(0) * mat.size(1), N = mat.size(2);
  TORCH_CHECK(NewtonInverse_supports((int)N), "NewtonInverse: N=", N,
              " is not supported on this device (insufficient smem or out of range)");
  const int dt = detail::abi_dtype(mat, "newton_inverse_forward");
  detail::same_type(mat, output, "output");
  // n > 128 runs as batched GEMMs over fp32 copies in a workspace (0 bytes otherwise).
  const size_t ws_bytes = lfamd_newton_workspace_size(dt, BH, N);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, mat.options().dtype(at::kByte));
  detail::check_status(lfamd_newton_forward(dt, mat.data_ptr(), output.data_ptr(), BH, N, iter,
                                            ws_bytes ? ws.data_ptr() : nullptr, ws_bytes,
                                            detail::stream_of(mat)));
}

void NewtonInverse_backward_cuda(const at::Tensor grad_output, const at::Tensor inverse, at::Tensor grad_mat) {
  at::hip::HIPGuardMasqueradingAsCUDA guard(inverse.device());
  TORCH_CHECK(grad_output.is_contiguous(), "grad_output must be contiguous");
  TORCH_CHECK(inverse.is_contiguous(), "inverse must be contiguous");
  TORCH_CHECK(grad_mat.is_contiguous(), "grad_mat must be contiguous");
  TORCH_CHECK(grad_output.sizes() == inverse.sizes() && inverse.sizes() == grad_mat.sizes(), "shape mismatch");
  const int64_t BH = inverse.size(0) * inverse.size(1), N = inverse.size(2);
  TORCH_CHECK(NewtonInverse_supports((int)N), "NewtonInverse: N=", N,
              " is not supported on this device (insufficient smem or out of range)");
  const int dt = detail::abi_dtype(inverse, "newton_inverse_backward");
  detail::same_type(inverse, grad_output, "grad_output");
  detail::same_type(inverse, grad_mat, "grad_mat");
  const size_t ws_bytes = lfamd_newton_workspace_size(dt, BH, N);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, inverse.options().dtype(at::kByte));
  detail::check_status(lfamd_newton_backward(dt, grad_output.data_ptr(), inverse.data_ptr(),
                                             grad_mat.data_ptr(), BH, N, ws_bytes ? ws.data_ptr() : nullptr,
                                             ws_bytes, detail::stream_of(inverse)));
}

}  // namespace laplace

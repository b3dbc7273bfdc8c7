// Host adapters of LaplaceSubtraction: reference input contract, then the C ABI
// of include/laplacianformer_amd.h on the tensor's device and current stream.
//
// Mirrors src/LaplaceSubtraction_cuda.cu:12-116 (shape_check and size
// extraction: B=q.size(0), H=q.size(1), N=q.size(2), M=k.size(3), C=q.size(3)).
// Stricter than the reference: output / gradient tensors are also checked for
// shape, dtype and device (the reference writes through them unchecked), and a
// non-contiguous grad_output is made contiguous instead of being read raw.
#include "LaplaceSubtraction.h"

#include "torch_common.h"

namespace laplace {

void shape_check(const at::Tensor& query, const at::Tensor& key) {
  TORCH_CHECK(query.ndimension() == 4,
              "4D weight tensor (batch size, head number, sequence length, channel) expected, but got: ",
              query.ndimension());
  TORCH_CHECK(key.ndimension() == 4,
              "4D weight tensor (batch size, head number, sequence length, channel) expected, but got: ",
              key.ndimension());
  TORCH_CHECK(query.is_contiguous(), "query tensor has to be contiguous");
  TORCH_CHECK(key.is_contiguous(), "key tensor has to be contiguous");
  TORCH_CHECK(query.size(0) == key.size(0) && query.size(1) == key.size(1) && query.size(3) == key.size(2),
              "query and key must match their size");
}

namespace {

struct Sizes {
  int64_t B, H, N, M, C;
};

Sizes sizes_of(const at::Tensor& query, const at::Tensor& key) {
  return Sizes{query.size(0), query.size(1), query.size(2), key.size(3), query.size(3)};
}

void check_out(const at::Tensor& ref, const at::Tensor& t, at::IntArrayRef shape, const char* name) {
  detail::same_type(ref, t, name);
  TORCH_CHECK(t.sizes() == shape, name, " must have shape ", shape, " but has ", t.sizes());
  TORCH_CHECK(t.is_contiguous(), name, " has to be contiguous");
}

}  // namespace

void LaplaceSubtraction_forward_cuda(const at::Tensor query, const at::Tensor key, at::Tensor output) {
  shape_check(query, key);
  const int dt = detail::abi_dtype(query, "laplace_forward_tiled");
  detail::same_type(query, key, "key");
  const Sizes s = sizes_of(query, key);
  check_out(query, output, {s.B, s.H, s.N, s.M}, "output");
  at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  detail::check_status(lfamd_laplace_forward(dt, query.data_ptr(), key.data_ptr(), output.data_ptr(), s.B,
                                             s.H, s.N, s.M, s.C, detail::stream_of(query)));
}

void LaplaceSubtraction_backward_query_cuda(const at::Tensor gradOutput, const at::Tensor query,
                                            const at::Tensor key, at::Tensor gradQuery) {
  shape_check(query, key);
  const int dt = detail::abi_dtype(query, "laplace_backward_query_tiled");
  detail::same_type(query, key, "key");
  const Sizes s = sizes_of(query, key);
  check_out(query, gradQuery, {s.B, s.H, s.N, s.C}, "gradQuery");
  detail::same_type(query, gradOutput, "gradOutput");
  TORCH_CHECK(gradOutput.sizes() == at::IntArrayRef({s.B, s.H, s.N, s.M}), "gradOutput must have shape [B,H,N,M]");
  at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  const at::Tensor g = gradOutput.contiguous();
  detail::check_status(lfamd_laplace_backward_query(dt, g.data_ptr(), query.data_ptr(), key.data_ptr(),
                                                    gradQuery.data_ptr(), s.B, s.H, s.N, s.M, s.C,
                                                    detail::stream_of(query)));
}

namespace {
void backward_impl(const at::Tensor& gradOutput, const at::Tensor& query, const at::Tensor& key,
                   at::Tensor* gradQuery, at::Tensor* gradKey, const char* op) {
  shape_check(query, key);
  const int dt = detail::abi_dtype(query, op);
  detail::same_type(query, key, "key");
  const Sizes s = sizes_of(query, key);
  if (gradQuery) check_out(query, *gradQuery, {s.B, s.H, s.N, s.C}, "gradQuery");
  check_out(query, *gradKey, {s.B, s.H, s.C, s.M}, "gradKey");
  detail::same_type(query, gradOutput, "gradOutput");
  TORCH_CHECK(gradOutput.sizes() == at::IntArrayRef({s.B, s.H, s.N, s.M}), "gradOutput must have shape [B,H,N,M]");
  at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  const at::Tensor g = gradOutput.contiguous();
  const size_t ws_bytes = lfamd_laplace_backward_workspace_size(dt, s.B, s.H, s.N, s.M, s.C);
  at::Tensor ws = at::empty({(int64_t)std::max<size_t>(ws_bytes, 1)}, query.options().dtype(at::kByte));
  void* stream = detail::stream_of(query);
  if (gradQuery)
    detail::check_status(lfamd_laplace_backward(dt, g.data_ptr(), query.data_ptr(), key.data_ptr(),
                                                gradQuery->data_ptr(), gradKey->data_ptr(), s.B, s.H, s.N,
                                                s.M, s.C, ws.data_ptr(), ws_bytes, stream));
  else
    detail::check_status(lfamd_laplace_backward_key(dt, g.data_ptr(), query.data_ptr(), key.data_ptr(),
                                                    gradKey->data_ptr(), s.B, s.H, s.N, s.M, s.C,
                                                    ws.data_ptr(), ws_bytes, stream));
}
}  // namespace

void LaplaceSubtraction_backward_key_cuda(const at::Tensor gradOutput, const at::Tensor query,
                                          const at::Tensor key, at::Tensor gradKey) {
  backward_impl(gradOutput, query, key, nullptr, &gradKey, "laplace_backward_key_tiled");
}

void LaplaceSubtraction_backward_cuda(const at::Tensor gradOutput, const at::Tensor query, const at::Tensor key,
                                      at::Tensor gradQuery, at::Tensor gradKey) {
  backward_impl(gradOutput, query, key, &gradQuery, &gradKey, "laplace_backward_fused");
}

namespace {
void check_kernel_tensor(const at::Tensor& query, const at::Tensor& t, const Sizes& s, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be float32");
  TORCH_CHECK(t.is_cuda() && t.device() == query.device(), name, " must be on the same GPU as the inputs");
  TORCH_CHECK(t.sizes() == at::IntArrayRef({s.B, s.H, s.N, s.M}), name, " must have shape [B,H,N,M]");
  TORCH_CHECK(t.is_contiguous(), name, " has to be contiguous");
}

// LFAMD_ERR_UNSUPPORTED means "compose the unfused ops"; any other error raises.
bool fused_status(int status) {
  if (status == LFAMD_ERR_UNSUPPORTED) return false;
  detail::check_status(status);
  return true;
}
}  // namespace

bool LaplaceKernel_forward_cuda(const at::Tensor query, const at::Tensor key, at::Tensor output, double scale) {
  shape_check(query, key);
  const int dt = detail::abi_dtype(query, "laplace_kernel_forward");
  detail::same_type(query, key, "key");
  const Sizes s = sizes_of(query, key);
  check_kernel_tensor(query, output, s, "output");
  at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  return fused_status(lfamd_laplace_kernel_forward(dt, query.data_ptr(), key.data_ptr(),
                                                   output.data_ptr<float>(), s.B, s.H, s.N, s.M, s.C,
                                                   (float)scale, detail::stream_of(query)));
}

bool LaplaceKernel_backward_cuda(const at::Tensor gradKernel, const at::Tensor kernel, const at::Tensor query,
                                 const at::Tensor key, std::optional<at::Tensor> gradQuery,
                                 std::optional<at::Tensor> gradKey, double scale) {
  shape_check(query, key);
  const int dt = detail::abi_dtype(query, "laplace_kernel_backward");
  detail::same_type(query, key, "key");
  const Sizes s = sizes_of(query, key);
  check_kernel_tensor(query, kernel, s, "kernel");
  TORCH_CHECK(gradKernel.scalar_type() == at::kFloat && gradKernel.sizes() == kernel.sizes(),
              "gradKernel must be float32 of the kernel's shape");
  const bool dq = gradQuery.has_value() && gradQuery->defined();
  const bool dk = gradKey.has_value() && gradKey->defined();
  if (dq) check_out(query, *gradQuery, {s.B, s.H, s.N, s.C}, "gradQuery");
  if (dk) check_out(query, *gradKey, {s.B, s.H, s.C, s.M}, "gradKey");
  at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  const at::Tensor gk = gradKernel.contiguous();
  const size_t ws_bytes = dk ? lfamd_laplace_backward_workspace_size(dt, s.B, s.H, s.N, s.M, s.C) : 0;
  at::Tensor ws = at::empty({(int64_t)std::max<size_t>(ws_bytes, 1)}, query.options().dtype(at::kByte));
  return fused_status(lfamd_laplace_kernel_backward(
      dt, gk.data_ptr<float>(), kernel.data_ptr<float>(), query.data_ptr(), key.data_ptr(),
      dq ? gradQuery->data_ptr() : nullptr, dk ? gradKey->data_ptr() : nullptr, s.B, s.H, s.N, s.M, s.C,
      (float)scale, ws.data_ptr(), ws_bytes, detail::stream_of(query)));
}

void LaplaceSubtraction_reduce_forward_cuda(const at::Tensor query, const at::Tensor key, at::Tensor output) {
  shape_check(query, key);
  const int dt = detail::abi_dtype(query, "subtraction_reduce_laplace_forward_cuda");
  detail::same_type(query, key, "key");
  const Sizes s = sizes_of(query, key);
  check_out(query, output, {s.B, s.H, s.N, s.M}, "output");
  at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  detail::check_status(lfamd_laplace_reduce_forward(dt, query.data_ptr(), key.data_ptr(), output.data_ptr(),
                                                    s.B, s.H, s.N, s.M, s.C, detail::stream_of(query)));
}

void MixRows_cuda(const at::Tensor a, const at::Tensor b, at::Tensor c) {
  TORCH_CHECK(a.dim() >= 2 && b.dim() == a.dim() && c.dim() == a.dim(), "mix_rows: a, b, c need the same rank >= 2");
  TORCH_CHECK(a.is_contiguous() && c.is_contiguous(), "mix_rows: a and c must be contiguous");
  TORCH_CHECK(b.scalar_type() == at::kFloat, "mix_rows: b must be float32");
  TORCH_CHECK(a.device() == b.device() && a.device() == c.device(), "mix_rows: tensors on different devices");
  const int nd = (int)a.dim();
  const int64_t N = a.size(nd - 2), P = a.size(nd - 1), Q = b.size(nd - 2);
  TORCH_CHECK(b.size(nd - 1) == P && c.size(nd - 2) == N && c.size(nd - 1) == Q, "mix_rows: shapes ", a.sizes(), " ",
              b.sizes(), " ", c.sizes(), " do not chain");
  int64_t S = 1, bSlice = 0;
  for (int i = nd - 3; i >= 0; --i) {  // leading dims: equal sizes, and b's must collapse to one stride
    TORCH_CHECK(a.size(i) == b.size(i) && a.size(i) == c.size(i), "mix_rows: batch dims differ");
    if (a.size(i) == 1) continue;
    if (S == 1) bSlice = b.stride(i);
    else TORCH_CHECK(b.stride(i) == bSlice * S, "mix_rows: b's batch dims do not collapse to one stride");
    S *= a.size(i);
  }
  const int dt = detail::abi_dtype(a, "mix_rows"), ct = detail::abi_dtype(c, "mix_rows");
  at::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
  detail::check_status(lfamd_mix_rows(dt, a.data_ptr(), b.data_ptr<float>(), ct, c.data_ptr(), S, N, (int)P,
                                      (int)Q, b.stride(nd - 2), b.stride(nd - 1), bSlice, detail::stream_of(a)));
}

void TallT_cuda(const at::Tensor a, const at::Tensor b, at::Tensor c) {
  TORCH_CHECK(a.dim() >= 2 && b.dim() == a.dim() && c.dim() == a.dim(), "tall_t: a, b, c need the same rank >= 2");
  TORCH_CHECK(a.is_contiguous() && b.is_contiguous() && c.is_contiguous(), "tall_t: a, b and c must be contiguous");
  TORCH_CHECK(a.scalar_type() == at::kFloat && c.scalar_type() == at::kFloat, "tall_t: a and c must be float32");
  TORCH_CHECK(a.device() == b.device() && a.device() == c.device(), "tall_t: tensors on different devices");
  const int nd = (int)a.dim();
  const int64_t N = a.size(nd - 2), P = a.size(nd - 1), Q = b.size(nd - 1);
  TORCH_CHECK(b.size(nd - 2) == N && c.size(nd - 2) == P && c.size(nd - 1) == Q, "tall_t: shapes ", a.sizes(), " ",
              b.sizes(), " ", c.sizes(), " do not chain");
  int64_t S = 1;
  for (int i = nd - 3; i >= 0; --i) {
    TORCH_CHECK(a.size(i) == b.size(i) && a.size(i) == c.size(i), "tall_t: batch dims differ");
    S *= a.size(i);
  }
  const int bt = detail::abi_dtype(b, "tall_t");
  at::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
  const size_t ws_bytes = lfamd_tall_t_workspace_size(S, N);
  at::Tensor ws = at::empty({(int64_t)std::max<size_t>(ws_bytes, 1)}, a.options().dtype(at::kByte));
  detail::check_status(lfamd_tall_t(bt, a.data_ptr<float>(), b.data_ptr(), c.data_ptr<float>(), S, N, (int)P, (int)Q,
                                    ws.data_ptr(), ws_bytes, detail::stream_of(a)));
}

}  // namespace laplace

// pybind11 module of the MI355X build. Same module name and the same ten
// exports as the reference module (src/wrapper.cpp:73-99), plus the fused
// backward LaplaceSubtraction_backward and the fused Laplacian-kernel pair
// LaplaceKernel_forward / LaplaceKernel_backward.
#include <torch/extension.h>

#include <sstream>
#include <string>

#include "../../../include/laplacianformer_amd.h"
#include "LaplaceSubtraction.h"
#include "LaplacianAttention.h"
#include "NewtonInverse.h"

namespace laplace {

// HIP runtime version as major*100 + minor (reference src/cuda_version.cu:16-20).
int get_cudart_version() { return lfamd_runtime_version(); }

// "HIP " followed by the version printed the way the reference prints it
// (src/wrapper.cpp:14-37: v/1000 "." v/10%100 ["." v%10]).
std::string get_cuda_version() {
  std::ostringstream oss;
  oss << "HIP ";
  const int v = get_cudart_version();
  oss << (v / 1000) << "." << (v / 10 % 100);
  if (v % 10 != 0) oss << "." << (v % 10);
  return oss.str();
}

// True only for a CUDA build (reference src/wrapper.cpp:39-45): false here.
bool has_cuda() { return false; }

std::string get_compiler_version() {
  std::ostringstream ss;
#if defined(__clang_major__)
  ss << "clang " << __clang_major__ << "." << __clang_minor__ << "." << __clang_patchlevel__;
#elif defined(__GNUC__)
  ss << "GCC " << __GNUC__ << "." << __GNUC_MINOR__;
#endif
  return ss.str();
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("get_compiler_version", &get_compiler_version, "get_compiler_version");
  m.def("get_cuda_version", &get_cuda_version, "get_cuda_version");
  m.def("has_cuda", &has_cuda, "has_cuda");
  m.def("LaplaceSubtraction_forward", &LaplaceSubtraction_forward, "LaplaceSubtraction_forward");
  m.def("LaplaceSubtraction_backward_query", &LaplaceSubtraction_backward_query, "LaplaceSubtraction_backward_query");
  m.def("LaplaceSubtraction_backward_key", &LaplaceSubtraction_backward_key, "LaplaceSubtraction_backward_key");
  m.def("LaplaceSubtraction_reduce_forward", &LaplaceSubtraction_reduce_forward, "LaplaceSubtraction_reduce_forward");
  m.def("NewtonInverse_forward", &NewtonInverse_forward, "NewtonInverse_forward (mat, output, iter)");
  m.def("NewtonInverse_backward", &NewtonInverse_backward, "NewtonInverse_backward (grad_output, inverse, grad_mat)");
  m.def("NewtonInverse_is_supported", &NewtonInverse_is_supported, "NewtonInverse_is_supported (N)");
  m.def("LaplaceSubtraction_backward", &LaplaceSubtraction_backward,
        "LaplaceSubtraction_backward (gradOutput, query, key, gradQuery, gradKey): fused dq+dk");
  m.def("LaplaceKernel_forward", &LaplaceKernel_forward,
        "LaplaceKernel_forward (query, key, output, scale): output = exp(-scale * dist) in float32; "
        "False where the fused path does not apply");
  m.def("LaplaceKernel_backward", &LaplaceKernel_backward,
        "LaplaceKernel_backward (gradKernel, kernel, query, key, gradQuery, gradKey, scale): "
        "gradQuery / gradKey may be None; False where the fused path does not apply");
  m.def("MixRows", &MixRows,
        "MixRows (a, b, c): c[..., n, q] = sum_p a[..., n, p] * b[..., q, p] in float32, widths <= 64 "
        "(the attention layer's products; b is read through its strides)");
  m.def("LaplacianAttention_forward", &LaplacianAttention_forward,
        "LaplacianAttention_forward (q, k, v, gh, gw, pool, iters) -> [out, km, km_cm, k_qm, k_mm, k_km, inv, kv, w] "
        "(the attention layer's forward; the rest is what its backward reads)");
  m.def("LaplacianAttention_backward", &LaplacianAttention_backward,
        "LaplacianAttention_backward (grad_out, saved, gh, gw, pool) -> [d_q, d_k, d_v]");
  m.def("TallT", &TallT,
        "TallT (a, b, c): c[..., p, q] = sum_n a[..., n, p] * b[..., n, q], a and c float32, widths <= 64 "
        "(the attention layer's K^T V products)");
}

}  // namespace laplace

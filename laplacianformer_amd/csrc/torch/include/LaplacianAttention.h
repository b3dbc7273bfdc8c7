// The attention layer's host entry points (no reference counterpart; the layer
// is the caller of LaplaceSubtraction and NewtonInverse, see
// LaplacianAttention_hip.cpp).
#pragma once
#include <torch/types.h>

#include <vector>

namespace laplace {

// {out, km, km_cm, k_qm, k_mm, k_km, inv, kv, w} for q, k, v [B,H,N,d] on a gh x gw token grid.
std::vector<at::Tensor> LaplacianAttention_forward(at::Tensor q, at::Tensor k, at::Tensor v, int64_t gh, int64_t gw,
                                                   int64_t pool, int64_t iters);
// {d_q, d_k, d_v} from grad_output and {q, k, v, km, km_cm, k_qm, k_mm, k_km, inv, kv, w}.
std::vector<at::Tensor> LaplacianAttention_backward(at::Tensor g, std::vector<at::Tensor> saved, int64_t gh,
                                                    int64_t gw, int64_t pool);

}  // namespace laplace

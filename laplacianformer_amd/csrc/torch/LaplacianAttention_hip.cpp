// The LaplacianFormer attention layer's forward and backward as two host
// functions (no reference counterpart: the reference ships the two operators
// only). They issue the operations of the per-op composition in attention.py
// (landmark pooling, three fused Laplacian-kernel distances, NewtonInverse,
// the tall products and the M x M GEMMs), with the pooling and its backward
// (including the sum of the landmarks' gradient parts) as one kernel each, so
// that an eager training step pays one Python call per direction instead of
// about forty: at config 5 the host's per-op dispatch, not the GPU, bounded
// the step.
//
//   Km  = pool x pool mean of K over the gh x gw grid (fp32 sums, input type)
//   K_xy = exp(-s L1(x, y)), s = 1 / sqrt(d), fp32
//   out = K_qm . W,  W = NewtonInverse(K_mm) . (K_km^T V)
#include <ATen/ATen.h>
#include <torch/types.h>

#include <cmath>
#include <tuple>
#include <vector>

#include "LaplaceSubtraction.h"
#include "LaplacianAttention.h"
#include "NewtonInverse.h"
#include "torch_common.h"

namespace laplace {

namespace {

// exp(-scale * L1(query, key_cm)) in fp32: the fused op, or the composition of
// the distance and an exp where the fused path does not take the shape.
at::Tensor kernel_fwd(const at::Tensor& query, const at::Tensor& key_cm, double scale) {
  at::Tensor out = at::empty({query.size(0), query.size(1), query.size(2), key_cm.size(3)},
                             query.options().dtype(at::kFloat));
  if (LaplaceKernel_forward(query, key_cm, out, scale)) return out;
  at::Tensor dist = at::empty_like(out);
  LaplaceSubtraction_forward(query.to(at::kFloat), key_cm.to(at::kFloat), dist);
  return at::exp(dist * -scale);
}

// exp(-scale * L1(x, key_cm)) for the layer's row sets x = km, q, k in one
// launch where the fused path takes them all (K_mm's 49-row slices first: their
// workgroups end early and let the others in); else one call each. Returns
// {K_mm, K_qm, K_km}.
std::vector<at::Tensor> kernel_fwd3(const at::Tensor& km, const at::Tensor& q, const at::Tensor& k,
                                    const at::Tensor& key_cm, double scale) {
  const int64_t B = q.size(0), H = q.size(1), C = q.size(3), M = key_cm.size(3);
  const at::Tensor* xs[3] = {&km, &q, &k};
  std::vector<at::Tensor> outs;
  const void* qp[3];
  float* op[3];
  int64_t n[3];
  for (int i = 0; i < 3; ++i) {
    outs.push_back(at::empty({B, H, xs[i]->size(2), M}, q.options().dtype(at::kFloat)));
    qp[i] = xs[i]->data_ptr();
    op[i] = outs[i].data_ptr<float>();
    n[i] = xs[i]->size(2);
  }
  at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const int st = lfamd_laplace_kernel_forward_multi(detail::abi_dtype(q, "laplacian attention"), 3, qp, n,
                                                    key_cm.data_ptr(), op, B, H, M, C, (float)scale,
                                                    detail::stream_of(q));
  if (st == LFAMD_ERR_UNSUPPORTED)
    return {kernel_fwd(km, key_cm, scale), kernel_fwd(q, key_cm, scale), kernel_fwd(k, key_cm, scale)};
  detail::check_status(st);
  return outs;
}

// (grad_query, grad_key) of exp(-scale * L1(query, key_cm)) for the fp32 dL/dK = grad.
std::pair<at::Tensor, at::Tensor> kernel_bwd(const at::Tensor& grad, const at::Tensor& kern, const at::Tensor& query,
                                             const at::Tensor& key_cm, double scale) {
  at::Tensor dq = at::empty_like(query), dk = at::empty_like(key_cm);
  if (LaplaceKernel_backward(grad, kern, query, key_cm, dq, dk, scale)) return {dq, dk};
  at::Tensor qa = query.to(at::kFloat), ka = key_cm.to(at::kFloat);
  at::Tensor dqa = at::empty_like(qa), dka = at::empty_like(ka);
  LaplaceSubtraction_backward(grad * kern * -scale, qa, ka, dqa, dka);
  return {dqa.to(query.scalar_type()), dka.to(key_cm.scalar_type())};
}

// c[..., n, q] = sum_p a[..., n, p] * b_qp[..., q, p] in fp32, stored as `out`.
at::Tensor mix_rows(const at::Tensor& a, const at::Tensor& b_qp, at::ScalarType out) {
  std::vector<int64_t> shape(a.sizes().begin(), a.sizes().end());
  shape.back() = b_qp.size(-2);
  at::Tensor c = at::empty(shape, a.options().dtype(out));
  MixRows(a.contiguous(), b_qp.to(at::kFloat), c);
  return c;
}

// a^T b over the rows, fp32 [..., P, Q].
at::Tensor tall_t(const at::Tensor& a, const at::Tensor& b) {
  std::vector<int64_t> shape(a.sizes().begin(), a.sizes().end());
  shape[shape.size() - 2] = a.size(-1);
  shape.back() = b.size(-1);
  at::Tensor c = at::empty(shape, a.options().dtype(at::kFloat));
  TallT(a.contiguous(), b.contiguous(), c);
  return c;
}

// inv = NewtonInverse(k_mm), kv = K_km^T V and w = inv kv in two launches (the
// tall product's partials, then the inverse with the partials' sum and the m x m
// product fused in) where the fused path takes the shape; false otherwise.
bool landmarks_forward(const at::Tensor& k_mm, const at::Tensor& k_km, const at::Tensor& v, int64_t iters,
                       at::Tensor& inv, at::Tensor& kv, at::Tensor& w) {
  const int64_t B = v.size(0), H = v.size(1), N = v.size(2), d = v.size(3), M = k_mm.size(2);
  at::hip::HIPGuardMasqueradingAsCUDA guard(v.device());
  const size_t wsb = lfamd_tall_t_workspace_size(B * H, N);
  kv = at::empty({B, H, M, d}, v.options().dtype(at::kFloat));
  w = at::empty_like(kv);
  at::Tensor ws = at::empty({(int64_t)wsb}, v.options().dtype(at::kByte));
  const int st = lfamd_attention_landmarks_forward(
      k_mm.data_ptr<float>(), k_km.data_ptr<float>(), detail::abi_dtype(v, "laplacian attention"), v.data_ptr(),
      inv.data_ptr<float>(), kv.data_ptr<float>(), w.data_ptr<float>(), B * H, N, (int)M, (int)d, (int)iters,
      ws.data_ptr(), wsb, detail::stream_of(v));
  if (st == LFAMD_ERR_UNSUPPORTED) return false;
  detail::check_status(st);
  return true;
}

// Its backward with the row products around it, for the output gradient g:
// d_kmm (the gradient of K_mm, through dw = K_qm^T g, kv and inv), d_kqm = g w^T,
// d_kkm = v dkv^T and d_v = K_km dkv, where the fused path takes the shape;
// false otherwise.
bool landmarks_backward(const at::Tensor& g, const at::Tensor& v, const at::Tensor& k_qm, const at::Tensor& k_km,
                        const at::Tensor& w, const at::Tensor& kv, const at::Tensor& inv, at::Tensor& d_kqm,
                        at::Tensor& d_kkm, at::Tensor& d_v, at::Tensor& d_kmm) {
  const int64_t B = g.size(0), H = g.size(1), N = g.size(2), d = g.size(3), M = inv.size(2);
  for (const at::Tensor* t : {&w, &kv, &inv, &k_qm, &k_km})
    if (!t->is_contiguous() || t->scalar_type() != at::kFloat) return false;
  if (!v.is_contiguous() || !g.is_contiguous() || v.scalar_type() != g.scalar_type()) return false;
  at::hip::HIPGuardMasqueradingAsCUDA guard(g.device());
  const size_t wsb = lfamd_tall_t_workspace_size(B * H, N);
  d_kqm = at::empty_like(k_qm);
  d_kkm = at::empty_like(k_km);
  d_v = at::empty_like(v);
  d_kmm = at::empty_like(inv);
  at::Tensor d_kv = at::empty_like(kv);
  at::Tensor ws = at::empty({(int64_t)wsb}, g.options().dtype(at::kByte));
  const int st = lfamd_attention_landmarks_backward(
      k_qm.data_ptr<float>(), detail::abi_dtype(g, "laplacian attention backward"), g.data_ptr(), v.data_ptr(),
      k_km.data_ptr<float>(), w.data_ptr<float>(), kv.data_ptr<float>(), inv.data_ptr<float>(),
      d_kqm.data_ptr<float>(), d_kkm.data_ptr<float>(), d_v.data_ptr(), d_kv.data_ptr<float>(),
      d_kmm.data_ptr<float>(), B * H, N, (int)M, (int)d, ws.data_ptr(), wsb, detail::stream_of(g));
  if (st == LFAMD_ERR_UNSUPPORTED) return false;
  detail::check_status(st);
  return true;
}

void check_layer(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, int64_t gh, int64_t gw,
                 int64_t pool) {
  // Every launch below takes raw device pointers: inputs on the CPU or on two
  // different GPUs are rejected here, before any of them.
  TORCH_CHECK(q.is_cuda() && k.device() == q.device() && v.device() == q.device(),
              "laplacian attention: q, k, v must be on one GPU");
  TORCH_CHECK(q.dim() == 4 && k.sizes() == q.sizes() && v.sizes() == q.sizes(),
              "laplacian attention: q, k, v must be [B,H,N,d] of one shape");
  TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type(),
              "laplacian attention: q, k, v must have one type");
  TORCH_CHECK(q.scalar_type() == at::kFloat || q.scalar_type() == at::kHalf || q.scalar_type() == at::kBFloat16,
              "laplacian attention: float32, float16 or bfloat16 inputs");
  TORCH_CHECK(pool > 0 && gh > 0 && gw > 0 && gh * gw == q.size(2) && gh % pool == 0 && gw % pool == 0,
              "laplacian attention: token grid ", gh, "x", gw, " does not match N=", q.size(2), " or pool=", pool);
  const int64_t M = (gh / pool) * (gw / pool);
  TORCH_CHECK(q.size(3) <= 64 && M <= 64, "laplacian attention: d and the landmark count must be <= 64");
}

}  // namespace

// Returns {out, km, km_cm, k_qm, k_mm, k_km, inv, kv, w}: the output and what
// the backward reads.
std::vector<at::Tensor> LaplacianAttention_forward(at::Tensor q, at::Tensor k, at::Tensor v, int64_t gh, int64_t gw,
                                                   int64_t pool, int64_t iters) {
  check_layer(q, k, v, gh, gw, pool);
  const at::ScalarType in = q.scalar_type();
  q = q.contiguous();
  k = k.contiguous();
  v = v.contiguous();
  const int64_t B = q.size(0), H = q.size(1), d = q.size(3);
  const double s = 1.0 / std::sqrt((double)d);
  const int64_t M = (gh / pool) * (gw / pool);
  at::Tensor km = at::empty({B, H, M, d}, q.options());          // landmarks [B,H,M,d]
  at::Tensor km_cm = at::empty({B, H, d, M}, q.options());       // and channel-major [B,H,d,M]
  at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  detail::check_status(lfamd_landmark_pool(detail::abi_dtype(k, "laplacian attention"), k.data_ptr(),
                                           km.data_ptr(), km_cm.data_ptr(), B, H, (int)gh, (int)gw, (int)pool,
                                           (int)d, detail::stream_of(k)));
  const std::vector<at::Tensor> kk = kernel_fwd3(km, q, k, km_cm, s);
  const at::Tensor &k_mm = kk[0], &k_qm = kk[1], &k_km = kk[2];
  at::Tensor inv = at::empty_like(k_mm), kv, w;
  if (!landmarks_forward(k_mm, k_km, v, iters, inv, kv, w)) {
    NewtonInverse_forward(k_mm, inv, iters);
    kv = tall_t(k_km, v);                                        // K_km^T V  [B,H,M,d]
    w = at::matmul(inv, kv);                                     // [B,H,M,d]
  }
  at::Tensor out = mix_rows(k_qm, w.transpose(-1, -2), in);      // K_qm W, rounded once
  return {out, km, km_cm, k_qm, k_mm, k_km, inv, kv, w};
}

// saved = {q, k, v, km, km_cm, k_qm, k_mm, k_km, inv, kv, w}; returns {d_q, d_k, d_v}.
std::vector<at::Tensor> LaplacianAttention_backward(at::Tensor g, std::vector<at::Tensor> saved, int64_t gh,
                                                    int64_t gw, int64_t pool) {
  TORCH_CHECK(saved.size() == 11, "laplacian attention backward: 11 saved tensors expected");
  const at::Tensor &q = saved[0], &k = saved[1], &v = saved[2], &km = saved[3], &km_cm = saved[4];
  const at::Tensor &k_qm = saved[5], &k_mm = saved[6], &k_km = saved[7], &inv = saved[8], &kv = saved[9];
  const at::Tensor& w = saved[10];
  check_layer(q, k, v, gh, gw, pool);
  TORCH_CHECK(g.sizes() == q.sizes(), "laplacian attention backward: grad_output must be [B,H,N,d]");
  TORCH_CHECK(g.device() == q.device(), "laplacian attention backward: grad_output must be on the inputs' GPU");
  for (const at::Tensor& t : saved)
    TORCH_CHECK(t.device() == q.device(), "laplacian attention backward: saved tensors must be on the inputs' GPU");
  const int64_t B = k.size(0), H = k.size(1), dd = k.size(3);
  const double s = 1.0 / std::sqrt((double)dd);
  g = g.contiguous();
  at::Tensor d_kqm, d_kkm, d_v, d_kmm;
  if (!landmarks_backward(g, v, k_qm, k_km, w, kv, inv, d_kqm, d_kkm, d_v, d_kmm)) {
    d_kqm = mix_rows(g, w, at::kFloat);                                  // G W^T       [B,H,N,M]
    at::Tensor d_w = tall_t(k_qm, g);                                    // K_qm^T G    [B,H,M,d]
    at::Tensor d_inv = at::matmul(d_w, kv.transpose(-1, -2));            // [B,H,M,M]
    at::Tensor d_kv = at::matmul(inv.transpose(-1, -2), d_w);            // [B,H,M,d]
    d_kmm = at::empty_like(k_mm);
    NewtonInverse_backward(d_inv.contiguous(), inv, d_kmm);
    d_kkm = mix_rows(v, d_kv, at::kFloat);                               // V dkv^T     [B,H,N,M]
    d_v = mix_rows(k_km, d_kv.transpose(-1, -2), v.scalar_type());       // K_km dkv    [B,H,N,d]
  }
  at::hip::HIPGuardMasqueradingAsCUDA guard(k.device());
  const int dt = detail::abi_dtype(k, "laplacian attention backward");
  // The three distances' gradients (K_qm, K_km, K_mm share the key km_cm): one
  // launch whose grad_key is their sum where the fused path takes it (K_mm's
  // 49-row slices first: their workgroups end early and let the others in).
  at::Tensor d_q = at::empty_like(q), d_k = at::empty_like(k), d_km = at::empty_like(km);
  at::Tensor d_cm = at::empty_like(km_cm), d_cm2, d_cm3;
  {
    const float* gks[3] = {d_kmm.data_ptr<float>(), d_kqm.data_ptr<float>(), d_kkm.data_ptr<float>()};
    const float* kvs[3] = {k_mm.data_ptr<float>(), k_qm.data_ptr<float>(), k_km.data_ptr<float>()};
    const void* qs[3] = {km.data_ptr(), q.data_ptr(), k.data_ptr()};
    void* dqs[3] = {d_km.data_ptr(), d_q.data_ptr(), d_k.data_ptr()};
    const int64_t ns[3] = {km.size(2), q.size(2), k.size(2)};
    const size_t wsb = lfamd_laplace_kernel_backward_multi_workspace_size(dt, 3, ns, B, H, km_cm.size(3), dd);
    int st = LFAMD_ERR_UNSUPPORTED;
    if (wsb > 0 && d_kqm.is_contiguous() && d_kkm.is_contiguous() && d_kmm.is_contiguous()) {
      at::Tensor ws = at::empty({(int64_t)wsb}, k.options().dtype(at::kByte));
      st = lfamd_laplace_kernel_backward_multi(dt, 3, gks, kvs, qs, ns, km_cm.data_ptr(), dqs, d_cm.data_ptr(), B, H,
                                               km_cm.size(3), dd, (float)s, ws.data_ptr(), wsb,
                                               detail::stream_of(k));
    }
    if (st == LFAMD_ERR_UNSUPPORTED) {
      std::tie(d_q, d_cm) = kernel_bwd(d_kqm, k_qm, q, km_cm, s);
      std::tie(d_km, d_cm2) = kernel_bwd(d_kmm, k_mm, km, km_cm, s);
      std::tie(d_k, d_cm3) = kernel_bwd(d_kkm, k_km, k, km_cm, s);
    } else {
      detail::check_status(st);
    }
  }
  // The landmarks' gradient, d_km + (d_cm + d_cm2 + d_cm3)^T (the last two absent
  // when the one launch summed them into d_cm), / pool^2 onto each pool x pool
  // patch of k's distance gradient (every step rounded to the type).
  detail::check_status(lfamd_landmark_pool_backward(
      dt, d_k.data_ptr(), d_km.data_ptr(), d_cm.data_ptr(), d_cm2.defined() ? d_cm2.data_ptr() : nullptr,
      d_cm3.defined() ? d_cm3.data_ptr() : nullptr, B, H, (int)gh, (int)gw, (int)pool, (int)dd,
      detail::stream_of(d_k)));
  return {d_q, d_k, d_v};
}

}  // namespace laplace

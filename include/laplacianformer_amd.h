/*
 * laplacianformer_amd.h - C ABI of the MI355X (gfx950) LaplaceSubtraction and
 * NewtonInverse operators.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as void*, a hipStream_t; NULL means the null stream). Nothing here
 * depends on PyTorch. All launches are asynchronous on the given stream; no
 * entry point synchronises the host. Outputs are caller-allocated and are
 * fully overwritten (no pre-zeroing needed), exactly like the reference ops.
 *
 * Tensor layouts (contiguous, row-major), B = batch, H = heads:
 *   query      [B, H, N, C]      key / grad_key  [B, H, C, M]   (channel-major)
 *   output     [B, H, N, M]      grad_output     [B, H, N, M]
 *   grad_query [B, H, N, C]
 *   mat / out / grad [B*H, n, n]
 *
 * Every function returns LFAMD_OK (0) or one of the LFAMD_ERR_* codes;
 * lfamd_last_error() gives a message for the calling thread's last failure.
 */
#ifndef LAPLACIANFORMER_AMD_H
#define LAPLACIANFORMER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. All tensors of one call share one type. */
#define LFAMD_F32 0
#define LFAMD_F16 1
#define LFAMD_BF16 2
#define LFAMD_F64 3

/* Status codes. */
#define LFAMD_OK 0
#define LFAMD_ERR_ARG 1         /* bad size, null pointer or workspace too small */
#define LFAMD_ERR_DTYPE 2       /* element type not supported by this entry point */
#define LFAMD_ERR_UNSUPPORTED 3 /* size outside the supported envelope */
#define LFAMD_ERR_HIP 4         /* HIP runtime or launch failure */

/* ---- LaplaceSubtraction ------------------------------------------------ */

/* out[b,h,i,j] = sum_c |query[b,h,i,c] - key[b,h,c,j]|, fp32 accumulation
 * (fp64 for LFAMD_F64), c ascending, rounded once to the element type.
 * Replaces laplace::LaplaceSubtraction_forward_cuda
 * (reference include/LaplaceSubtraction.h:9-13, src/LaplaceSubtraction_cuda.cu:55-67,
 *  src/LaplaceSubtraction_cuda_kernel.cu:455-485). */
int lfamd_laplace_forward(int dtype, const void* query, const void* key, void* output,
                          int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                          int64_t channels, void* stream);

/* grad_query[b,h,i,c] = sum_j grad_output[b,h,i,j] * sgn(query[b,h,i,c] - key[b,h,c,j]),
 * sgn(0) = 0. Replaces laplace::LaplaceSubtraction_backward_query_cuda
 * (reference include/LaplaceSubtraction.h:15-20, src/LaplaceSubtraction_cuda.cu:69-84,
 *  src/LaplaceSubtraction_cuda_kernel.cu:487-547). */
int lfamd_laplace_backward_query(int dtype, const void* grad_output, const void* query,
                                 const void* key, void* grad_query, int64_t batch,
                                 int64_t heads, int64_t q_len, int64_t k_len,
                                 int64_t channels, void* stream);

/* Bytes of device workspace lfamd_laplace_backward_key / lfamd_laplace_backward
 * need for these sizes (fp32 per-workgroup partial sums of grad_key). No
 * counterpart in the reference, which split-K atomically adds into the output
 * (src/LaplaceSubtraction_cuda_kernel.cu:568-591). */
size_t lfamd_laplace_backward_workspace_size(int dtype, int64_t batch, int64_t heads,
                                             int64_t q_len, int64_t k_len,
                                             int64_t channels);

/* grad_key[b,h,c,j] = -sum_i grad_output[b,h,i,j] * sgn(query[b,h,i,c] - key[b,h,c,j]).
 * Deterministic: per-workgroup fp32 partials in `workspace`, summed in a fixed
 * order by a second small kernel on the same stream, rounded once.
 * Replaces laplace::LaplaceSubtraction_backward_key_cuda
 * (reference include/LaplaceSubtraction.h:22-27, src/LaplaceSubtraction_cuda.cu:86-101,
 *  src/LaplaceSubtraction_cuda_kernel.cu:549-609). */
int lfamd_laplace_backward_key(int dtype, const void* grad_output, const void* query,
                               const void* key, void* grad_key, int64_t batch,
                               int64_t heads, int64_t q_len, int64_t k_len,
                               int64_t channels, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Fused backward: grad_query and grad_key in one pass over (i, j, c), computing
 * sgn(query - key) once per triple. Superset export (no single reference entry
 * point); equals lfamd_laplace_backward_query + lfamd_laplace_backward_key. */
int lfamd_laplace_backward(int dtype, const void* grad_output, const void* query,
                           const void* key, void* grad_query, void* grad_key,
                           int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                           int64_t channels, void* workspace, size_t workspace_bytes,
                           void* stream);

/* lfamd_laplace_backward without a workspace argument and without allocating:
 * the grad_key partials live in a static device array of
 * lfamd_laplace_backward_noalloc_limit() bytes (8 MiB) that each GPU holds until
 * the process ends; sizes needing more workspace return LFAMD_ERR_UNSUPPORTED.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (HIP graph capture, serving loops, harnesses forbidding hipMalloc).
 * Calls that overlap on one GPU share the array and race. */
int lfamd_laplace_backward_noalloc(int dtype, const void* grad_output, const void* query,
                                   const void* key, void* grad_query, void* grad_key,
                                   int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                                   int64_t channels, void* stream);

/* Bytes of the static scratch of lfamd_laplace_backward_noalloc. */
size_t lfamd_laplace_backward_noalloc_limit(void);

/* Legacy "reduce" forward: the same distance, accumulated in the element type
 * by min(C,256) partial sums folded by a halving tree, exactly as the reference
 * kernel does (including its behaviour when min(C,256) is not a power of two).
 * Replaces laplace::LaplaceSubtraction_reduce_forward_cuda
 * (reference include/LaplaceSubtraction.h:29-33, src/LaplaceSubtraction_cuda.cu:103-116,
 *  src/LaplaceSubtraction_cuda_kernel.cu:399-447,611-647). */
int lfamd_laplace_reduce_forward(int dtype, const void* query, const void* key,
                                 void* output, int64_t batch, int64_t heads,
                                 int64_t q_len, int64_t k_len, int64_t channels,
                                 void* stream);

/* ---- Fused Laplacian kernel K = exp(-scale * dist) ----------------------- */

/* output[b,h,i,j] = expf(-scale * dist[b,h,i,j]) in fp32, dist as in
 * lfamd_laplace_forward but kept in fp32 (not rounded to the element type).
 * The exp is applied in the forward's epilogue, so dist never reaches HBM.
 * No single reference counterpart: it replaces the model-side composition
 * torch.exp(-LaplaceSubtraction_forward(...) * scale) around
 * laplace::LaplaceSubtraction_forward_cuda (reference src/wrapper.cpp:81-82).
 * Returns LFAMD_ERR_UNSUPPORTED outside the fused path (fp64, C % 8 != 0 or
 * C == 0, M > 256, a query not 16-byte aligned, tiles beyond one workgroup's
 * LDS); callers then compose the unfused ops. */
int lfamd_laplace_kernel_forward(int dtype, const void* query, const void* key, float* output,
                                 int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                                 int64_t channels, float scale, void* stream);

/* Backward of output = expf(-scale * dist): with g = -scale * grad_kernel * kernel
 * (fp32, formed while staging, never stored), grad_query and grad_key as
 * lfamd_laplace_backward_query / lfamd_laplace_backward_key give for grad_output = g.
 * `kernel` is this op's forward output, `grad_kernel` its gradient, both fp32
 * [B,H,N,M]. Either of grad_query / grad_key may be NULL to skip it; grad_key
 * needs the workspace lfamd_laplace_backward_workspace_size reports. Fused path:
 * LFAMD_F16 with 16 <= M <= 256; LFAMD_ERR_UNSUPPORTED elsewhere. No single
 * reference counterpart (replaces the composition around
 * laplace::LaplaceSubtraction_backward_{query,key}_cuda, reference src/wrapper.cpp:84-88). */
int lfamd_laplace_kernel_backward(int dtype, const float* grad_kernel, const float* kernel,
                                  const void* query, const void* key, void* grad_query, void* grad_key,
                                  int64_t batch, int64_t heads, int64_t q_len, int64_t k_len,
                                  int64_t channels, float scale, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* lfamd_laplace_kernel_forward for up to three queries that share one key, in
 * one launch: source i has q_lens[i] >= 1 rows per (b, h) slice, query
 * queries[i] [B,H,q_lens[i],C] and fp32 output outputs[i] [B,H,q_lens[i],M];
 * each output is what lfamd_laplace_kernel_forward gives for that query alone
 * (the same bits). No reference counterpart: for callers with several kernel
 * matrices against one landmark key (the LaplacianFormer layer's K_qm, K_km and
 * K_mm). LFAMD_ERR_UNSUPPORTED unless M = 49, 8 <= C <= 64 with C % 8 == 0, a
 * float dtype other than fp64 and 16-byte aligned queries; callers then make
 * one call per source. */
int lfamd_laplace_kernel_forward_multi(int dtype, int num_sources, const void* const* queries,
                                       const int64_t* q_lens, const void* key, float* const* outputs,
                                       int64_t batch, int64_t heads, int64_t k_len, int64_t channels,
                                       float scale, void* stream);

/* lfamd_laplace_kernel_backward for up to three row sources that share one key,
 * in one launch: source i has q_lens[i] >= 1 rows per (b, h) slice with fp32
 * grad_kernels[i] and kernels[i] [B,H,q_lens[i],M], fp16 queries[i]
 * [B,H,q_lens[i],C] and grad_queries[i] (its grad_query); grad_key [B,H,C,M]
 * is the sum over all sources (one rounding). Fused path only: LFAMD_F16,
 * M = 49, C % 64 == 0, 4-byte aligned queries; LFAMD_ERR_UNSUPPORTED elsewhere
 * (callers then make one call per source). The workspace is
 * lfamd_laplace_kernel_backward_multi_workspace_size bytes (0 when the path does
 * not apply to that dtype and shape, e.g. any dtype but LFAMD_F16, or a source
 * of more than INT32_MAX / 2 rows). No reference counterpart: for callers with several kernel
 * matrices against one landmark key (the LaplacianFormer layer's K_qm, K_km
 * and K_mm), whose grad_key parts are summed anyway. */
size_t lfamd_laplace_kernel_backward_multi_workspace_size(int dtype, int num_sources, const int64_t* q_lens,
                                                          int64_t batch, int64_t heads, int64_t k_len,
                                                          int64_t channels);
int lfamd_laplace_kernel_backward_multi(int dtype, int num_sources, const float* const* grad_kernels,
                                        const float* const* kernels, const void* const* queries,
                                        const int64_t* q_lens, const void* key, void* const* grad_queries,
                                        void* grad_key, int64_t batch, int64_t heads, int64_t k_len,
                                        int64_t channels, float scale, void* workspace, size_t workspace_bytes,
                                        void* stream);

/* ---- NewtonInverse ------------------------------------------------------ */

/* Bytes of device workspace lfamd_newton_forward / lfamd_newton_backward need:
 * 0 for n <= 128 (matrices stay in LDS) and for fp64; for 128 < n <= 256 four
 * fp32 copies per matrix padded to NP = 64*ceil(n/64) plus NP row sums (the
 * products run as batched GEMMs). No reference counterpart (the reference
 * stops at n = 128). */
size_t lfamd_newton_workspace_size(int dtype, int64_t batch_heads, int64_t n);

/* Newton-Schulz inverse of P = mat + 0.01*I for each of the batch_heads n x n
 * matrices: alpha = 1.8 / (max_i sum_j P_ij)^2, V0 = alpha*P, then `iters`
 * steps V <- 2V - V(PV) (the reference's order for n <= 112 and here for
 * n > 128) or V <- 2V - (VP)V (its order for 112 < n <= 128); fp32 arithmetic
 * (fp64 for LFAMD_F64), one rounding at the store. 1 <= n <= 256 (fp64:
 * n <= 96). `workspace` (16-byte aligned) of lfamd_newton_workspace_size bytes;
 * NULL when that is 0. Replaces laplace::NewtonInverse_forward_cuda
 * (reference include/NewtonInverse.h:9-12, src/NewtonInverse_cuda_kernel.cu:764-794). */
int lfamd_newton_forward(int dtype, const void* mat, void* output, int64_t batch_heads,
                         int64_t n, int iters, void* workspace, size_t workspace_bytes,
                         void* stream);

/* grad_mat = -(V^T G) V^T for V = inverse, G = grad_output; workspace as for
 * lfamd_newton_forward. Replaces laplace::NewtonInverse_backward_cuda
 * (reference include/NewtonInverse.h:14-17, src/NewtonInverse_cuda_kernel.cu:796-833). */
int lfamd_newton_backward(int dtype, const void* grad_output, const void* inverse,
                          void* grad_mat, int64_t batch_heads, int64_t n, void* workspace,
                          size_t workspace_bytes, void* stream);

/* 1 if n is inside the NewtonInverse envelope on this build, else 0.
 * Replaces laplace::NewtonInverse_supports
 * (reference include/NewtonInverse.h:19, src/NewtonInverse_cuda_kernel.cu:753-762). */
int lfamd_newton_is_supported(int64_t n);

/* ---- Attention-layer products ------------------------------------------- */

/* c[s][n][q] = sum_{p < inner} a[s][n][p] * b[s*b_slice_stride + q*b_col_stride + p*b_inner_stride]
 * for s < slices, n < rows, q < cols; fp32 arithmetic, `a` of element type `dtype` and c of
 * element type `c_dtype` (each F32, F16 or BF16; c is the fp32 sum rounded once),
 * a and c contiguous [slices][rows][inner] / [slices][rows][cols], b fp32
 * addressed through the element strides (W and W^T are both read in place). inner, cols <= 64;
 * LFAMD_ERR_UNSUPPORTED beyond. No reference counterpart: these are the LaplacianFormer
 * attention layer's products around the two operators (K_qm.W, grad.W^T, V.grad_kv^T,
 * K_km.grad_kv), which the reference leaves to its caller. */
int lfamd_mix_rows(int dtype, const void* a, const float* b, int c_dtype, void* c, int64_t slices,
                   int64_t rows, int inner, int cols, int64_t b_col_stride, int64_t b_inner_stride,
                   int64_t b_slice_stride, void* stream);

/* Bytes of workspace lfamd_tall_t needs for these sizes (per-workgroup fp32 partials). */
size_t lfamd_tall_t_workspace_size(int64_t slices, int64_t rows);

/* c[s][p][q] = sum_{n < rows} a[s][n][p] * b[s][n][q] for s < slices, p < inner, q < cols:
 * a fp32 [slices][rows][inner], b of element type `b_dtype` (F32, F16 or BF16, used as fp32)
 * [slices][rows][cols], c fp32 [slices][inner][cols], all contiguous; inner, cols <= 64
 * (LFAMD_ERR_UNSUPPORTED beyond). Summed in fp32 over per-workgroup row ranges, then over the
 * workgroups in a fixed order (deterministic). No reference counterpart: the attention layer's
 * K_km^T.V and K_qm^T.grad_out (the reference leaves the layer to its caller). */
int lfamd_tall_t(int b_dtype, const float* a, const void* b, float* c, int64_t slices, int64_t rows,
                 int inner, int cols, void* workspace, size_t workspace_bytes, void* stream);

/* The attention layer's landmark products around NewtonInverse, for m landmarks with 48 < m <= 64
 * and width d <= 64 (else LFAMD_ERR_UNSUPPORTED), fp32 [slices][...] contiguous unless stated.
 * Forward (NewtonInverse and the tall product's partials in one launch, then one for kv and w):
 * inv = NewtonInverse(kmm, iters) (kmm [m][m],
 * as lfamd_newton_forward), kv = kkm^T v (kkm [rows][m], v [rows][d] of element type v_dtype: F32,
 * F16 or BF16; kv [m][d]) and w = inv kv ([m][d]). Backward, for the layer's output gradient g
 * ([rows][d], element type dtype, as v): dw = kqm^T g, dinv = dw kv^T, dkv = inv^T dw ([m][d]),
 * dkmm = -(inv^T dinv) inv^T ([m][m], as lfamd_newton_backward), then, in one launch,
 * dkqm = g w^T, dkkm = v dkv^T ([rows][m]) and dv = kkm dkv ([rows][d], element type dtype). The
 * tall products need 16-byte aligned slices (LFAMD_ERR_UNSUPPORTED otherwise) and
 * lfamd_tall_t_workspace_size(slices, rows) bytes of workspace. No reference counterpart: they
 * replace, for the layer, the tall products' reductions, the three m x m products and the two
 * NewtonInverse launches, run the forward's tall product beside NewtonInverse, and run the three
 * backward row products in one launch. */
int lfamd_attention_landmarks_forward(const float* kmm, const float* kkm, int v_dtype, const void* v, float* inv,
                                      float* kv, float* w, int64_t slices, int64_t rows, int m, int d, int iters,
                                      void* workspace, size_t workspace_bytes, void* stream);
int lfamd_attention_landmarks_backward(const float* kqm, int dtype, const void* g, const void* v, const float* kkm,
                                       const float* w, const float* kv, const float* inv, float* dkqm, float* dkkm,
                                       void* dv, float* dkv, float* dkmm, int64_t slices, int64_t rows, int m, int d,
                                       void* workspace, size_t workspace_bytes, void* stream);

/* km[b][h][m][c] = (sum over the pool x pool patch m of k[b][h][n][c]) / pool^2, summed in fp32 and
 * rounded once to `dtype` (F32, F16 or BF16), for k [B][H][gh*gw][d] on a gh x gw token grid
 * (gh, gw multiples of pool; M = (gh/pool)*(gw/pool), patches row-major); written as km
 * [B][H][M][d] and channel-major as km_cm [B][H][d][M], all contiguous. No reference counterpart:
 * the attention layer's landmark pooling. */
int lfamd_landmark_pool(int dtype, const void* k, void* km, void* km_cm, int64_t B, int64_t H, int gh,
                        int gw, int pool, int d, void* stream);

/* Backward of the pooling with the landmarks' gradient assembled from its parts: with every
 * operation rounded to `dtype`, t = (dcm0 + dcm1) + dcm2 ([B][H][d][M]), u = dkm + t^T
 * ([B][H][M][d]), and dk[b][h][n][c] += u[b][h][m(n)][c] / pool^2 in place ([B][H][gh*gw][d]).
 * dcm1 and dcm2 may be NULL (taken as zero: t = dcm0). No reference counterpart (the attention
 * layer's). */
int lfamd_landmark_pool_backward(int dtype, void* dk, const void* dkm, const void* dcm0, const void* dcm1,
                                 const void* dcm2, int64_t B, int64_t H, int gh, int gw, int pool, int d,
                                 void* stream);

/* ---- Runtime ------------------------------------------------------------ */

/* HIP runtime version as major*100 + minor (e.g. 700 for 7.0), the convention
 * the reference's version probe uses for HIP. Replaces laplace::get_cudart_version
 * (reference src/cuda_version.cu:7-26). */
int lfamd_runtime_version(void);

/* Static text for a status code. No reference counterpart. */
const char* lfamd_status_string(int status);

/* Message for the calling thread's most recent failing call ("" if none).
 * No reference counterpart (the reference printf's launch errors,
 * src/LaplaceSubtraction_cuda_kernel.cu:481-484). */
const char* lfamd_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* LAPLACIANFORMER_AMD_H */

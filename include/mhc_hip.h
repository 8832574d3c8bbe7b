/*
 * mhc_hip.h - C ABI of the MI355X (gfx950) mHC hyper-connection library.
 *
 * This is the drop-in boundary that replaces the reference's native module
 * `mhc_ascend` (src/python/bindings.cpp, pybind11 + ATen + ACL).  Every entry
 * point takes plain device pointers, sizes and a HIP stream (`hipStream_t`
 * passed as `void*`; NULL = the null stream), enqueues its kernels on that
 * stream and returns without synchronising.  Buffers are caller-owned,
 * contiguous, row-major.  Scratch memory is passed in by the caller
 * (`workspace` / `workspace_bytes`, size from the matching *_workspace_size
 * query); the library keeps no hidden device state, so calls are reentrant
 * (the one exception is the allocation-free entry's scratch array, below).
 *
 * Element types: `dtype` arguments take MHC_DTYPE_F32 or MHC_DTYPE_BF16 and
 * describe the storage of the large [B, n, C] / [B, C] tensors; all
 * arithmetic is fp32.  Small parameters (H, M, weights) are fp32.
 *
 * Status: 0 on success; MHC_ERR_* (< 0) for argument errors, with a message
 * from mhc_last_error(); > 0 is the hipError_t of a failed launch.
 *
 * The reference interface each entry replaces is cited as file:line of
 * ParadoxZW/mHC_Ascend.
 */
#ifndef MHC_HIP_H_
#define MHC_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MHC_DTYPE_F32 0
#define MHC_DTYPE_BF16 1

#define MHC_SUCCESS 0
#define MHC_ERR_INVALID (-1)     /* bad pointer, shape or dtype (TORCH_CHECK in the reference) */
#define MHC_ERR_UNSUPPORTED (-2) /* valid request this build has no kernel for (e.g. n > 64) */
#define MHC_ERR_WORKSPACE (-3)   /* workspace smaller than the *_workspace_size query */

/* ABI version: major * 10000 + minor * 100 + patch. */
int mhc_abi_version(void);

/* Message for the last MHC_ERR_* returned on this thread ("" if none). */
const char* mhc_last_error(void);

/* ---- Sinkhorn-Knopp --------------------------------------------------------
 * out = SK_{num_iters, eps}(inp) on [batch, n, n] fp32, dividing rows then
 * columns by (sum + eps) each iteration.
 * Replaces sinkhorn_knopp_fwd (bindings.cpp:155-187). */
int mhc_sinkhorn_knopp_fwd(const float* inp, float* out, int64_t batch, int32_t n, int32_t num_iters, float eps,
                           void* stream);

/* grad_inp = exact VJP of SK at inp.  `out` (the forward result) is accepted
 * for signature parity and may be NULL; the kernel recomputes the forward
 * history in registers.
 * Replaces sinkhorn_knopp_bwd (bindings.cpp:189-231). */
int mhc_sinkhorn_knopp_bwd(const float* grad_out, const float* inp, const float* out, float* grad_inp,
                           int64_t batch, int32_t n, int32_t num_iters, float eps, void* stream);

/* ---- RMSNorm ---------------------------------------------------------------
 * out = inp / rms * weight, rms = sqrt(mean(inp^2) + eps) per row of `hidden`.
 * inp/out [batch, hidden] (dtype), weight [hidden] fp32, rms [batch] fp32.
 * Replaces rmsnorm_fwd (bindings.cpp:237-266); the reference forces bf16
 * storage, here out has the input's dtype. */
int mhc_rmsnorm_fwd(const void* inp, int32_t dtype, const float* weight, void* out, float* rms, int64_t batch,
                    int32_t hidden, float eps, void* stream);

size_t mhc_rmsnorm_bwd_workspace_size(int64_t batch, int32_t hidden, int32_t dtype);

/* grad_inp = w g / rms - inp (sum g w inp) / (hidden rms^3) (dtype);
 * grad_weight = sum_rows g inp / rms (fp32 [hidden], deterministic).
 * grad_out has the input's dtype.  Replaces rmsnorm_bwd (bindings.cpp:268-301). */
int mhc_rmsnorm_bwd(const void* grad_out, const void* inp, int32_t dtype, const float* weight, const float* rms,
                    void* grad_inp, float* grad_weight, void* workspace, size_t workspace_bytes, int64_t batch,
                    int32_t hidden, void* stream);

/* rms[b] = sqrt(mean_k inp[b, k]^2 + eps) for inp [batch, k] (dtype).
 * Replaces compute_rms_fwd (bindings.cpp:543-566). */
int mhc_compute_rms_fwd(const void* inp, int32_t dtype, float* rms, int64_t batch, int64_t k, float eps,
                        void* stream);

/* ---- stream aggregate --------------------------------------------------------
 * h = sigmoid(h_pre_raw[b]), out[b, :] = sum_i h_i inp[b, i, :].
 * inp [batch, n, hidden] and out [batch, hidden] (dtype); h_pre_raw fp32
 * with batch stride 0 (shared) or n; h_pre_act [batch, n] receives h.
 * Replaces stream_aggregate_fwd (bindings.cpp:307-338). */
int mhc_stream_aggregate_fwd(const void* inp, int32_t dtype, const float* h_pre_raw, int64_t h_batch_stride,
                             void* out, float* h_pre_act, int64_t batch, int32_t n, int32_t hidden, void* stream);

/* grad_inp[b, i, :] = grad_out[b, :] h_i (dtype); grad_h_pre_act[b, i] =
 * sum_c grad_out x_i (before the sigmoid derivative, as the reference
 * returns it); grad_h_pre_raw = grad_h_pre_act h (1 - h).  Either fp32
 * output may be NULL.  Replaces stream_aggregate_bwd (bindings.cpp:340-374)
 * and the sigmoid derivative of ops.py:172. */
int mhc_stream_aggregate_bwd(const void* grad_out, const void* inp, int32_t dtype, const float* h_pre_act,
                             int64_t h_batch_stride, void* grad_inp, float* grad_h_pre_act, float* grad_h_pre_raw,
                             int64_t batch, int32_t n, int32_t hidden, void* stream);

/* ---- stream distribute-mix-add ------------------------------------------------
 * h = 2 sigmoid(h_post_raw[b]), out[b, i, :] = h_i y[b, :] + sum_j M[b, i, j] x[b, j, :].
 * y_norm [batch, hidden] and x_inp [batch, n, hidden] (dtype); out fp32;
 * h_post_raw / M fp32 with batch stride 0 or n / n*n; h_post_act [batch, n].
 * Replaces stream_distribute_mix_add_fwd (bindings.cpp:380-416). */
int mhc_stream_distribute_mix_add_fwd(const void* y_norm, const float* h_post_raw, int64_t h_batch_stride,
                                      const float* M, int64_t m_batch_stride, const void* x_inp, int32_t dtype,
                                      float* out, float* h_post_act, int64_t batch, int32_t n, int32_t hidden,
                                      void* stream);

/* For grad_out [batch, n, hidden] fp32: grad_x[b, j] = sum_i M_ij g_i and
 * grad_y = sum_i h_i g_i (dtype); grad_M[b, i, j] = sum_c g_i x_j,
 * grad_h_post_act[b, i] = sum_c g_i y, grad_h_post_raw = grad_h_post_act
 * h (1 - h/2) (fp32; the last two may be NULL).
 * Replaces stream_distribute_mix_add_bwd (bindings.cpp:418-460) and the
 * derivative of ops.py:240-242. */
int mhc_stream_distribute_mix_add_bwd(const float* grad_out, const void* x_inp, const void* y_norm, int32_t dtype,
                                      const float* M, int64_t m_batch_stride, const float* h_post_act,
                                      int64_t h_batch_stride, void* grad_x, void* grad_y, float* grad_M,
                                      float* grad_h_post_act, float* grad_h_post_raw, int64_t batch, int32_t n,
                                      int32_t hidden, void* stream);

/* ---- fused static-H mHC layer ----------------------------------------------
 * x [batch, n, hidden] (x_dtype), weight [hidden] (weight_dtype: the
 * reference keeps it bf16, layer.py:65), h_pre/h_post [n], h_res [n, n] raw
 * (pre-activation) fp32 parameters.
 *   h_pre = sigmoid(H_pre), h_post = 2 sigmoid(H_post), M = SK(exp(H_res))
 *   out[b,i,:] = sum_j M[i,j] x[b,j,:] + h_post[i] * RMSNorm(sum_i h_pre[i] x[b,i,:]) * weight
 * out [batch, n, hidden] fp32; rms [batch] fp32 (may be NULL); `saved`
 * (mhc_layer_static_saved_size bytes) receives h_pre, h_post, M and the fp32
 * weight for the backward.
 * Replaces the static branch of MHCLayer.forward (layer.py:142-170), i.e.
 * stream_aggregate_fwd + rmsnorm_fwd + sinkhorn_knopp_fwd +
 * stream_distribute_mix_add_fwd (bindings.cpp:307, 237, 155, 380). */
size_t mhc_layer_static_saved_size(int32_t n, int32_t hidden);

int mhc_layer_static_fwd(const void* x, int32_t x_dtype, const void* weight, int32_t weight_dtype,
                         const float* h_pre, const float* h_post, const float* h_res, float* out, float* rms,
                         float* saved, int64_t batch, int32_t n, int32_t hidden, int32_t num_iters,
                         float sinkhorn_eps, float rmsnorm_eps, void* stream);

size_t mhc_layer_static_bwd_workspace_size(int64_t batch, int32_t n, int32_t hidden, int32_t x_dtype);

/* Gradients of the static layer for cotangent grad_out [batch, n, hidden]
 * fp32: grad_x (x_dtype), grad_weight [hidden] (weight_dtype), grad_h_pre /
 * grad_h_post [n] and grad_h_res [n, n] fp32 (token-summed).  `saved` is the
 * forward's.  Deterministic (fixed-order reductions, no atomics).
 * Replaces the backward chain of the static layer:
 * stream_distribute_mix_add_bwd, rmsnorm_bwd, stream_aggregate_bwd,
 * sinkhorn_knopp_bwd (bindings.cpp:418, 268, 340, 189) plus the autograd
 * expand/exp/sigmoid backward of layer.py:144-160 and ops.py:172, 240-242. */
int mhc_layer_static_bwd(const float* grad_out, const void* x, int32_t x_dtype, int32_t weight_dtype,
                         const float* h_pre, const float* h_post, const float* h_res, const float* saved,
                         void* grad_x, void* grad_weight, float* grad_h_pre, float* grad_h_post, float* grad_h_res,
                         void* workspace, size_t workspace_bytes, int64_t batch, int32_t n, int32_t hidden,
                         int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps, void* stream);

/* ---- allocation-free static backward ------------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops): the same
 * gradients as mhc_layer_static_bwd, bit for bit, with its workspace in a
 * library-owned device array of mhc_noalloc_scratch_bytes() (16 MiB, one per
 * device, held until the process ends) instead of a caller buffer.  The
 * caller still passes every input and output.  Shapes whose workspace would
 * exceed the array return MHC_ERR_UNSUPPORTED.  Calls that overlap on one
 * device share the array and race: serialise them (one stream, or events). */
size_t mhc_noalloc_scratch_bytes(void);
int mhc_layer_static_bwd_noalloc(const float* grad_out, const void* x, int32_t x_dtype, int32_t weight_dtype,
                                 const float* h_pre, const float* h_post, const float* h_res, const float* saved,
                                 void* grad_x, void* grad_weight, float* grad_h_pre, float* grad_h_post,
                                 float* grad_h_res, int64_t batch, int32_t n, int32_t hidden, int32_t num_iters,
                                 float sinkhorn_eps, float rmsnorm_eps, void* stream);

/* ---- dynamic-H projection ----------------------------------------------------
 * out[b, o] = sum_k inp[b, k] weight[o, k]: inp [batch, k] (dtype), weight
 * [out_dim, k] fp32, out [batch, out_dim] fp32; out_dim <= 8192 (tiles of
 * 32 rows, one pass over inp each), k % 32 == 0.
 * bf16 MFMA on a hi/lo bf16 split of the operands (about fp32 accuracy).
 * Replaces fused_rmsnorm_matmul_fwd (bindings.cpp:480-528), which rounds
 * inputs and result to bf16. */
size_t mhc_fused_rmsnorm_matmul_fwd_workspace_size(int64_t batch, int64_t k, int32_t out_dim);
int mhc_fused_rmsnorm_matmul_fwd(const void* inp, int32_t dtype, const float* weight, float* out, void* workspace,
                                 size_t workspace_bytes, int64_t batch, int64_t k, int32_t out_dim, void* stream);

/* grad_x = grad_out . phi ([batch, k] fp32), grad_phi = grad_out^T . x_flat
 * ([out_dim, k] fp32, deterministic).  Replaces fused_rmsnorm_matmul_bwd
 * (bindings.cpp:530-541). */
size_t mhc_fused_rmsnorm_matmul_bwd_workspace_size(int64_t batch, int64_t k, int32_t out_dim);
int mhc_fused_rmsnorm_matmul_bwd(const float* grad_out, const float* x_flat, const float* phi, float* grad_x,
                                 float* grad_phi, void* workspace, size_t workspace_bytes, int64_t batch, int64_t k,
                                 int32_t out_dim, void* stream);

/* ---- fused dynamic-H mHC layer --------------------------------------------------
 * Per token: x_flat = x[b] (n*hidden), r_h = sqrt(mean(x_flat^2) + rmsnorm_eps),
 * P = x_flat . [phi_pre; phi_post; phi_res]^T, t_k = alpha_k P_k / r_h + b_k,
 * h_pre = sigmoid(t_pre), h_post = 2 sigmoid(t_post), M = SK(exp(t_res)),
 * then the static formulas with per-token h and M.
 * phi_pre / phi_post [n, n*hidden], phi_res [n*n, n*hidden], b_pre / b_post
 * [n], b_res [n, n] fp32; alpha_* are single fp32 values in DEVICE memory
 * (no host synchronisation).  out [batch, n, hidden] fp32; `saved`
 * (mhc_layer_dynamic_saved_size bytes) receives what the backward needs.
 * Replaces mhc_layer_fwd_dynamic (bindings.cpp:880-952) and the inference
 * path of ops.py:337-380. */
size_t mhc_layer_dynamic_saved_size(int64_t batch, int32_t n, int32_t hidden);
size_t mhc_layer_dynamic_fwd_workspace_size(int64_t batch, int32_t n, int32_t hidden);
int mhc_layer_dynamic_fwd(const void* x, int32_t x_dtype, const void* weight, int32_t weight_dtype,
                          const float* phi_pre, const float* phi_post, const float* phi_res, const float* alpha_pre,
                          const float* alpha_post, const float* alpha_res, const float* b_pre, const float* b_post,
                          const float* b_res, float* out, float* saved, void* workspace, size_t workspace_bytes,
                          int64_t batch, int32_t n, int32_t hidden, int32_t num_iters, float sinkhorn_eps,
                          float rmsnorm_eps, void* stream);

/* ---- forward-only dynamic-H layer (inference) ----------------------------------
 * The forward of mhc_layer_dynamic_fwd without the backward's saved state, in
 * two steps.  mhc_layer_dynamic_pack writes what depends on the parameters
 * alone - the fp32 RMSNorm weight and [phi_pre; phi_post; phi_res] as three
 * bf16 planes in the projection kernel's operand order - into `packed`
 * (device memory of mhc_layer_dynamic_packed_size bytes, 256-byte aligned).
 * Pack once per parameter update.  mhc_layer_dynamic_infer then runs the
 * projection, the per-token H and the fused row pass, and writes
 * out [batch, n, hidden] in out_dtype: MHC_DTYPE_F32 as the reference, or
 * MHC_DTYPE_BF16 (rounded to nearest even) to halve the output traffic.
 * `packed` must come from mhc_layer_dynamic_pack with the same n and hidden;
 * alpha_* and b_* are as in mhc_layer_dynamic_fwd.  Results equal
 * mhc_layer_dynamic_fwd's `out` bit for bit at out_dtype F32.
 * Replaces the inference path of ops.py:337-380 (mhc_layer_fwd_dynamic,
 * bindings.cpp:880-952, with its saved outputs dropped). */
size_t mhc_layer_dynamic_packed_size(int32_t n, int32_t hidden);
int mhc_layer_dynamic_pack(const void* weight, int32_t weight_dtype, const float* phi_pre, const float* phi_post,
                           const float* phi_res, void* packed, size_t packed_bytes, int32_t n, int32_t hidden,
                           void* stream);
size_t mhc_layer_dynamic_infer_workspace_size(int64_t batch, int32_t n, int32_t hidden);
int mhc_layer_dynamic_infer(const void* x, int32_t x_dtype, const void* packed, const float* alpha_pre,
                            const float* alpha_post, const float* alpha_res, const float* b_pre, const float* b_post,
                            const float* b_res, void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                            int64_t batch, int32_t n, int32_t hidden, int32_t num_iters, float sinkhorn_eps,
                            float rmsnorm_eps, void* stream);

/* Gradients for grad_out [batch, n, hidden] fp32: grad_x (x_dtype),
 * grad_weight [hidden] (weight_dtype), grad_phi [2n+n^2, n*hidden] (rows
 * pre, post, res), grad_alpha [3] (pre, post, res), grad_b [2n+n^2]
 * (pre, post, res row-major), all fp32 and deterministic.
 * Replaces mhc_layer_bwd_dynamic (bindings.cpp:600-874). */
size_t mhc_layer_dynamic_bwd_workspace_size(int64_t batch, int32_t n, int32_t hidden, int32_t x_dtype);
int mhc_layer_dynamic_bwd(const float* grad_out, const void* x, int32_t x_dtype, int32_t weight_dtype,
                          const float* phi_pre, const float* phi_post, const float* phi_res, const float* alpha_pre,
                          const float* alpha_post, const float* alpha_res, const float* b_pre, const float* b_post,
                          const float* b_res, const float* saved, void* grad_x, void* grad_weight, float* grad_phi,
                          float* grad_alpha, float* grad_b, void* workspace, size_t workspace_bytes, int64_t batch,
                          int32_t n, int32_t hidden, int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps,
                          void* stream);

/* ---- reference-shaped dynamic-H pair ---------------------------------------------
 * The reference's native pair with its own call shape, for a caller that
 * keeps the reference's ops.py (ops.py:425-448, 518-542): the forward
 * returns nine tensors and the backward takes them back with 23 arguments.
 * Both run the fused entries above; the extra tensors cost one more pass
 * over x in the forward and a recomputed projection P in the backward (as
 * the reference's backward recomputes it, bindings.cpp:764-766).
 *
 * mhc_layer_fwd_dynamic - replaces mhc_layer_fwd_dynamic (bindings.cpp:
 * 880-952).  phi_concat [2n+n^2, n*hidden] fp32 = [phi_pre; phi_post;
 * phi_res] (ops.py:416-418); the alphas are host floats.  Outputs (in the
 * reference's order): output [batch, n, hidden] fp32, rms [batch] fp32 (RMS
 * of x_agg), x_agg [batch, hidden] bf16, h_pre_act / h_post_act [batch, n]
 * fp32, M [batch, n, n] fp32, y_norm [batch, hidden] bf16, x_flat
 * [batch, n*hidden] bf16, rms_h [batch] fp32.  All arithmetic is fp32; only
 * the three tensors the reference stores in bf16 are rounded on output. */
size_t mhc_layer_fwd_dynamic_workspace_size(int64_t batch, int32_t n, int32_t hidden);
int mhc_layer_fwd_dynamic(const void* x, int32_t x_dtype, const void* weight, int32_t weight_dtype,
                          const float* phi_concat, float alpha_pre, float alpha_post, float alpha_res,
                          const float* b_pre, const float* b_post, const float* b_res, float* output, float* rms,
                          void* x_agg_bf16, float* h_pre_act, float* h_post_act, float* M, void* y_norm_bf16,
                          void* x_flat_bf16, float* rms_h, void* workspace, size_t workspace_bytes, int64_t batch,
                          int32_t n, int32_t hidden, int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps,
                          void* stream);

/* mhc_layer_bwd_dynamic - replaces mhc_layer_bwd_dynamic (bindings.cpp:
 * 600-874), arguments in its order.  h_pre_act, h_post_act, M and rms_h are
 * used as given; P is recomputed from x; rms, x_agg_bf16, y_norm_bf16 and
 * x_flat_bf16 are not read (the row pass recomputes them in fp32 from x;
 * they may be NULL).  Gradients: grad_x (x_dtype), grad_weight [hidden]
 * fp32 (as the reference's), grad_phi_pre [n, n*hidden], grad_phi_post
 * [n, n*hidden], grad_phi_res [n*n, n*hidden], one fp32 value each for the
 * alphas, grad_b_pre / grad_b_post [n], grad_b_res [n, n]; deterministic. */
size_t mhc_layer_bwd_dynamic_workspace_size(int64_t batch, int32_t n, int32_t hidden, int32_t x_dtype);
int mhc_layer_bwd_dynamic(const float* grad_output, const void* x, int32_t x_dtype, const void* weight,
                          int32_t weight_dtype, const float* rms, const void* x_agg_bf16, const float* h_pre_act,
                          const float* h_post_act, const float* M, const void* y_norm_bf16, const void* x_flat_bf16,
                          const float* rms_h, const float* phi_pre, const float* phi_post, const float* phi_res,
                          float alpha_pre, float alpha_post, float alpha_res, const float* b_pre, const float* b_post,
                          const float* b_res, void* grad_x, float* grad_weight, float* grad_phi_pre,
                          float* grad_phi_post, float* grad_phi_res, float* grad_alpha_pre, float* grad_alpha_post,
                          float* grad_alpha_res, float* grad_b_pre, float* grad_b_post, float* grad_b_res,
                          void* workspace, size_t workspace_bytes, int64_t batch, int32_t n, int32_t hidden,
                          int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps, void* stream);

/* ---- fused MHCResidualWrapper ---------------------------------------------------
 * The wrapper of layer.py:225-329 on residual / branch [tokens, hidden]
 * (dtype): streams X_0 = residual, X_1 = branch and, for i >= 2,
 * X_i = residual * 0.1^(i-1) rounded to dtype (MHC_WRAPPER_DECAY,
 * layer.py:306-308) or 0 (MHC_WRAPPER_ZERO); the mHC layer on X; the mean
 * over the n streams (layer.py:316) -> out [tokens, hidden] fp32.
 * n = 2..32 and hidden % 4 == 0; dynamic H also needs n * hidden % 32 == 0
 * and, past n = 10 (more than 128 projection rows), a backward at Sinkhorn
 * settings under which the H_res gradients vanish (num_iters >= 1 and
 * sinkhorn_eps <= 1e-6, the defaults); others return MHC_ERR_UNSUPPORTED.
 * The row passes rebuild X from residual and branch in registers, so with
 * static H, and with dynamic H at n = 4 and hidden % 32 == 0 (whose
 * projection kernels rebuild it too), X never exists in memory.  For the
 * other dynamic-H shapes the projection forward reads a storage-dtype copy
 * of X from the workspace (except with bf16 storage, n >= 5, tokens >= 1024
 * and hidden % 64 == 0, where it too rebuilds X), and so does the backward
 * (fp32) when the Sinkhorn settings keep the H_res gradients (num_iters == 0
 * or sinkhorn_eps > 1e-6), and for n > 16, or n > 8 with hidden < 2048; the
 * queries below size both.
 * Parameters and `saved` are those of the layer entries above.  Backward:
 * grad_out [tokens, hidden] fp32 -> grad_residual, grad_branch (dtype) and
 * the layer's parameter gradients.
 * Replaces MHCResidualWrapper.forward (layer.py:269-322) over
 * mhc_layer_fwd_dynamic / mhc_layer_bwd_dynamic (bindings.cpp:880-952,
 * 600-874) or the static layer chain. */
#define MHC_WRAPPER_DECAY 0
#define MHC_WRAPPER_ZERO 1

size_t mhc_wrapper_dynamic_saved_size(int64_t tokens, int32_t n, int32_t hidden);
size_t mhc_wrapper_dynamic_fwd_workspace_size(int64_t tokens, int32_t n, int32_t hidden);
/* The forward's workspace for the given storage dtype (the query above
 * covers both): with bf16 storage the run-time-n path mostly rebuilds the
 * streams inside its projection and keeps no stream rows.  No counterpart
 * in the reference; for callers that size the workspace per call. */
size_t mhc_wrapper_dynamic_fwd_workspace_size_for(int64_t tokens, int32_t n, int32_t hidden, int32_t dtype);
int mhc_wrapper_dynamic_fwd(const void* residual, const void* branch, int32_t dtype, int32_t residual_mode,
                            const void* weight, int32_t weight_dtype, const float* phi_pre, const float* phi_post,
                            const float* phi_res, const float* alpha_pre, const float* alpha_post,
                            const float* alpha_res, const float* b_pre, const float* b_post, const float* b_res,
                            float* out, float* saved, void* workspace, size_t workspace_bytes, int64_t tokens,
                            int32_t n, int32_t hidden, int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps,
                            void* stream);
size_t mhc_wrapper_dynamic_bwd_workspace_size(int64_t tokens, int32_t n, int32_t hidden, int32_t dtype,
                                              int32_t residual_mode);
/* The backward's workspace for given Sinkhorn settings: at n != 4 (and
 * n = 4 rows the n = 4 kernels do not take) with num_iters >= 1 and
 * sinkhorn_eps <= 1e-6 no stream rows are kept, and this is smaller than
 * the query above (which covers every setting).  No counterpart in the
 * reference (its op allocates its own buffers); for callers that size the
 * workspace per call. */
size_t mhc_wrapper_dynamic_bwd_workspace_size_for(int64_t tokens, int32_t n, int32_t hidden, int32_t dtype,
                                                  int32_t residual_mode, int32_t num_iters, float sinkhorn_eps);
int mhc_wrapper_dynamic_bwd(const float* grad_out, const void* residual, const void* branch, int32_t dtype,
                            int32_t residual_mode, int32_t weight_dtype, const float* phi_pre, const float* phi_post,
                            const float* phi_res, const float* alpha_pre, const float* alpha_post,
                            const float* alpha_res, const float* b_res, const float* saved, void* grad_residual,
                            void* grad_branch, void* grad_weight, float* grad_phi, float* grad_alpha, float* grad_b,
                            void* workspace, size_t workspace_bytes, int64_t tokens, int32_t n, int32_t hidden,
                            int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps, void* stream);

/* Static H: saved is mhc_layer_static_saved_size(n, hidden) bytes. */
int mhc_wrapper_static_fwd(const void* residual, const void* branch, int32_t dtype, int32_t residual_mode,
                           const void* weight, int32_t weight_dtype, const float* h_pre, const float* h_post,
                           const float* h_res, float* out, float* saved, int64_t tokens, int32_t n, int32_t hidden,
                           int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps, void* stream);
size_t mhc_wrapper_static_bwd_workspace_size(int64_t tokens, int32_t n, int32_t hidden, int32_t dtype,
                                             int32_t residual_mode);
int mhc_wrapper_static_bwd(const float* grad_out, const void* residual, const void* branch, int32_t dtype,
                           int32_t residual_mode, int32_t weight_dtype, const float* h_pre, const float* h_post,
                           const float* h_res, const float* saved, void* grad_residual, void* grad_branch,
                           void* grad_weight, float* grad_h_pre, float* grad_h_post, float* grad_h_res,
                           void* workspace, size_t workspace_bytes, int64_t tokens, int32_t n, int32_t hidden,
                           int32_t num_iters, float sinkhorn_eps, float rmsnorm_eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MHC_HIP_H_ */

// Host-side declarations shared by the kernel translation units and the
// C-ABI layer (abi.hip).  Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#ifdef MHC_KERNEL_TIMING
#include <hip/hip_ext.h>
#endif
#include <stdint.h>
#include <stddef.h>

namespace mhc {

enum DType : int { kF32 = 0, kBF16 = 1 };

inline int dtype_size(int dt) { return dt == kBF16 ? 2 : 4; }

// Per-thread work split of one token row of C channels: `threads` lanes each
// own `vpt` chunks of `wc` channels (chunk q = k * threads + tid).
struct RowTiling {
    int threads;
    int vpt;
};
// Live row state per thread (floats) the row kernels are sized for.
constexpr int kRowStateBudget = 136;
RowTiling choose_row_tiling(int64_t C, int wc, int n_arrays_live, int pref_threads = 256);
// A tiling with at least `need` lanes (kernels whose block reductions hand
// one value per thread; lanes past the row are masked out).
inline RowTiling with_min_threads(RowTiling t, int need) {
    if (t.vpt > 0 && t.threads < need) t.threads = ((need + 63) / 64) * 64;
    return t;
}

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Per-kernel timing, compiled in only for the benchmark's build of the
// library (MHC_KERNEL_TIMING, libmhc_hip_timed.so; include/mhc_hip_timing.h).
// timing_begin(name) opens a scope (returning a token for timing_end) in
// which every launch goes through hipExtLaunchKernel with the scope's
// events: the first launch's dispatch records the start, each launch's end
// the stop, so the scope measures its kernels' own begin-to-end time (event
// markers between launches would also count the queue around them).  All
// launches go through MHC_LAUNCH_GGL / mhc_launch_kernel, which are plain
// hipLaunchKernelGGL / hipLaunchKernel in the product build, where the
// scope functions are empty and the library has no timing state.
#ifdef MHC_KERNEL_TIMING
int timing_begin(const char* name, hipStream_t s);
void timing_end(int token, hipStream_t s);
struct TimingScope {
    hipEvent_t start;
    hipEvent_t stop;
    bool first;
};
TimingScope* timing_scope();  // the calling thread's open scope, or null
hipError_t mhc_launch_kernel(const void* fn, dim3 grid, dim3 block, void** args, size_t shm, hipStream_t s);
#define MHC_LAUNCH_GGL(kernel, grid, block, shm, stream, ...)                                                \
    do {                                                                                                     \
        ::mhc::TimingScope* mhc_ts_ = ::mhc::timing_scope();                                                 \
        if (mhc_ts_) {                                                                                       \
            hipExtLaunchKernelGGL(kernel, grid, block, shm, stream, mhc_ts_->first ? mhc_ts_->start : nullptr, \
                                  mhc_ts_->stop, 0, __VA_ARGS__);                                            \
            mhc_ts_->first = false;                                                                          \
        } else {                                                                                             \
            hipLaunchKernelGGL(kernel, grid, block, shm, stream, __VA_ARGS__);                               \
        }                                                                                                    \
    } while (0)
#else
inline int timing_begin(const char*, hipStream_t) { return -1; }
inline void timing_end(int, hipStream_t) {}
inline hipError_t mhc_launch_kernel(const void* fn, dim3 grid, dim3 block, void** args, size_t shm, hipStream_t s) {
    return hipLaunchKernel(fn, grid, block, args, shm, s);
}
#define MHC_LAUNCH_GGL hipLaunchKernelGGL
#endif

// ---- generic.hip -----------------------------------------------------------
// Expansion rates without a compiled instantiation (n <= kGenMaxN): the
// layer's are n outside {2, 4, 8, 16, 32}, the stream operators' n outside
// {1, 2, 4, 8, 16, 32}.  The layer launchers of layer.hip and dynamic.hip
// and the operator launchers of ops.hip route these n here themselves.
constexpr int kGenMaxN = 64;
bool generic_layer_n(int n);
bool generic_ops_n(int n);
hipError_t launch_gen_static_coef(int n, const float* h_pre, const float* h_post, const float* h_res,
                                  const void* weight, int w_dtype, int64_t C, float* saved, int iters, float sk_eps,
                                  hipStream_t s);
hipError_t launch_gen_layer_fwd(int x_dtype, int out_dtype, int n, const void* x, const float* w, const float* coef,
                                int64_t coef_stride, void* out, float* rms_out, int64_t B, int64_t C, float eps,
                                hipStream_t s);
// Backward rows of the generic kernels: grid = gen_layer_bwd_grid(B)
// persistent workgroups, scratch of gen_layer_bwd_scratch_bytes (each
// workgroup's xa and gy rows); scal_out / dw_part as launch_layer_bwd.
int gen_layer_bwd_grid(int64_t B);
size_t gen_layer_bwd_scratch_bytes(int64_t B, int64_t C);
hipError_t launch_gen_layer_bwd(int x_dtype, int n, int mode, const float* g, const void* x, const float* w,
                                const float* coef, int64_t coef_stride, void* dx, float* dw_part, float* scal_out,
                                int grid, int64_t B, int64_t C, float eps, float* scratch, hipStream_t s);
// hist (hist_bytes, may be null): the Sinkhorn adjoint's per-iteration state,
// used when skw_hist_floats(kWave, n, iters) floats fit.
hipError_t launch_gen_static_finalize(int n, const float* scal_part, int rows, const float* h_pre,
                                      const float* h_post, const float* h_res, float* d_h_pre, float* d_h_post,
                                      float* d_h_res, int iters, float sk_eps, hipStream_t s, float* hist,
                                      size_t hist_bytes);
hipError_t launch_gen_aggregate_fwd(int dt, int n, const void* x, const float* H, int64_t hs, void* out,
                                    float* h_act, int64_t B, int64_t C, hipStream_t s);
hipError_t launch_gen_aggregate_bwd(int dt, int n, const void* g, const void* x, const float* h_act, int64_t hs,
                                    void* gx, float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s);
hipError_t launch_gen_distribute_fwd(int dt, int n, const void* y, const float* H, int64_t hs, const float* M,
                                     int64_t ms, const void* x, float* out, float* h_act, int64_t B, int64_t C,
                                     hipStream_t s);
hipError_t launch_gen_distribute_bwd(int dt, int n, const float* g, const void* x, const void* y, const float* M,
                                     int64_t ms, const float* h_act, int64_t hs, void* gx, void* gy, float* gM,
                                     float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s);

// ---- layer.hip -------------------------------------------------------------
// saved = [coef (2n + n^2) | pad | fp32 weight (C)], weight at saved_w_offset(n) floats
int saved_w_offset(int n);
hipError_t launch_static_coef(int n, const float* h_pre, const float* h_post, const float* h_res,
                              const void* weight, int w_dtype, int64_t C, float* saved, int iters, float sk_eps,
                              hipStream_t s);
// The static forward in one launch (coefficients formed in every
// workgroup, saved state written by workgroup 0): n <= 8 on register rows.
bool layer_static_fwd_fused(int n, int64_t C);
hipError_t launch_layer_static_fwd(int x_dtype, int n, const void* x, const void* weight, int w_dtype,
                                   const float* h_pre, const float* h_post, const float* h_res, float* saved,
                                   int iters, float sk_eps, float* out, float* rms_out, int64_t B, int64_t C,
                                   float eps, hipStream_t s);
// out is [B, n, C] in out_dtype (fp32, or bf16 for the inference entry).
// rms_scratch > 0: rms_out is scratch of that many floats (>= B) whose
// contents the caller does not need; 0: rms_out (when not null) receives r.
hipError_t launch_layer_fwd(int x_dtype, int n, const void* x, const float* w, const float* coef,
                            int64_t coef_stride, void* out, int out_dtype, float* rms_out, int64_t B, int64_t C,
                            float eps, hipStream_t s, int64_t rms_scratch = 0);
// mode 0: static (writes dx, per-workgroup sums of [dM, dh_post_act,
//         dh_pre_act] into scal_out[grid][n*n+2n]);
// mode 1: dx = stream terms only, and per token scal_out[B][n*n+2n+2] =
//         dM, dh_post_act, dh_pre_act, inv_rms, k2.  With bf16 x the stream
//         terms are fp16 against power-of-two scales (part_pack4 in
//         mhc_device.h) with the scale exponents
//         dx_scale[B][layer_bwd_part_groups] (register rows and
//         C % 128 == 0 only: other bf16 x rows are an error here).
// scratch: layer_bwd_scratch_bytes (the channel-chunked wide backward's
// partial row sums; 0 bytes and unused otherwise).
hipError_t launch_layer_bwd(int x_dtype, int n, int mode, const float* g, const void* x, const float* w,
                            const float* coef, int64_t coef_stride, void* dx, float* dw_part, float* scal_out,
                            int grid, int64_t B, int64_t C, float eps, float* scratch, hipStream_t s,
                            int32_t* dx_scale = nullptr);
int layer_bwd_grid(int x_dtype, int n, int64_t B, int64_t C);
// Scale groups per token row of the mode-1 stream part (one per half
// wave of the register-row kernel; 0 when the channel-loop kernels run).
int layer_bwd_part_groups(int x_dtype, int n, int64_t C);
size_t layer_bwd_scratch_bytes(int x_dtype, int n, int64_t B, int64_t C);
// Whether the layer forward / backward of (n, C) runs the channel-loop
// kernels of wide.hip rather than the register rows.
bool layer_fwd_is_wide(int n, int64_t C);
bool layer_bwd_is_wide(int n, int64_t C);
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t s);
// p0[0, n0) and p1[0, n1) = +0 while c[0] + .. + c[nc - 1] is finite, NaN
// otherwise (fill_zero_carry_kernel)
hipError_t launch_fill_zero_carry(float* p0, int64_t n0, float* p1, int64_t n1, const float* c, int nc,
                                  hipStream_t s);
// out[i] = bf16(in[i]) (round to nearest even) for n elements.
hipError_t launch_cast_bf16(const float* in, int64_t n, void* out, hipStream_t s);
// Two-stage deterministic column sum of part[rows][cols]: stage[rsplit][cols].
hipError_t launch_column_partial(const float* part, int rows, int64_t cols, float* stage, int rsplit,
                                 hipStream_t s);
// dw = sum of the rsplit staged rows (stored as w_dtype); with n > 0 also the
// static parameter gradients from scal_part[rows][n*n+2n].
hipError_t launch_layer_finalize(int n, int w_dtype, const float* stage, int rsplit, int64_t cols, void* dw,
                                 const float* scal_part, int rows, const float* h_pre, const float* h_post,
                                 const float* h_res, float* d_h_pre, float* d_h_post, float* d_h_res, int iters,
                                 float sk_eps, hipStream_t s);
// Column sums of part[rows][cols] into dw (w_dtype), plus the static scalar
// gradients when n > 0: one launch when rows is small (the finalize reads the
// partials directly), else a first pass into stage[column_sums_stage_floats].
size_t column_sums_stage_floats(int64_t cols);
// sk_hist (kStaticSkHistBytes, n >= 16 and the generic n; null elsewhere):
// the static Sinkhorn adjoint's history.
hipError_t launch_column_finalize(int n, int w_dtype, const float* part, int rows, int64_t cols, float* stage,
                                  void* dw, const float* scal_part, int scal_rows, const float* h_pre,
                                  const float* h_post, const float* h_res, float* d_h_pre, float* d_h_post,
                                  float* d_h_res, int iters, float sk_eps, hipStream_t s, float* sk_hist = nullptr);

// ---- wide.hip --------------------------------------------------------------
// Channel-loop layer kernels (any C up to kWideMaxC; n in {2, 4, 8, 16, 32}):
// used for n > 8 and where the register rows do not fit C.  The backward's
// dw partial of a workgroup sits in LDS (C floats).
constexpr int kWideMaxC = 12288;
bool wide_supported(int n, int64_t C);
hipError_t launch_wide_fwd(int x_dtype, int out_dtype, int n, const void* x, const float* w, const float* coef,
                           int64_t coef_stride, void* out, float* rms_out, int64_t B, int64_t C, float eps,
                           hipStream_t s, int64_t rms_scratch = 0);
// Partial rows of the backward (mode 0 scalar rows and dw rows): the
// persistent grid, or one per token when a token's channels are split over
// several workgroups (few tokens); then the launch needs scratch of
// wide_bwd_scratch_bytes (0 otherwise).
int wide_bwd_grid(int x_dtype, int n, int64_t B, int64_t C);
size_t wide_bwd_scratch_bytes(int n, int64_t B, int64_t C);
// Same outputs as launch_layer_bwd (mode 0 / 1); for n >= 16 the dM entries
// come from a second kernel on the same stream.
hipError_t launch_wide_bwd(int x_dtype, int n, int mode, const float* g, const void* x, const float* w,
                           const float* coef, int64_t coef_stride, void* dx, float* dw_part, float* scal_out, int grid,
                           int64_t B, int64_t C, float eps, float* scratch, hipStream_t s);
// Standalone operators on rows of any width, n in {1, 2, 4, 8, 16, 32}
// (same outputs as the launch_* of ops.hip; the RMSNorm backward's dw
// partial rows [grid][C] come from wide_rmsnorm_bwd_grid, C <= kWideMaxC).
hipError_t launch_wide_rmsnorm_fwd(int dt, const void* x, const float* w, void* y, float* rms, int64_t B, int64_t C,
                                   float eps, hipStream_t s);
int wide_rmsnorm_bwd_grid(int dt, int64_t B, int64_t C);
hipError_t launch_wide_rmsnorm_bwd(int dt, const void* g, const void* x, const float* w, const float* rms, void* gx,
                                   float* dw_part, int grid, int64_t B, int64_t C, hipStream_t s);
hipError_t launch_wide_compute_rms(int dt, const void* x, float* rms, int64_t B, int64_t K, float eps,
                                   hipStream_t s);
hipError_t launch_wide_aggregate_fwd(int dt, int n, const void* x, const float* H, int64_t hs, void* out,
                                     float* h_act, int64_t B, int64_t C, hipStream_t s);
hipError_t launch_wide_aggregate_bwd(int dt, int n, const void* g, const void* x, const float* h_act, int64_t hs,
                                     void* gx, float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s);
hipError_t launch_wide_distribute_fwd(int dt, int n, const void* y, const float* H, int64_t hs, const float* M,
                                      int64_t ms, const void* x, float* out, float* h_act, int64_t B, int64_t C,
                                      hipStream_t s);
hipError_t launch_wide_distribute_bwd(int dt, int n, const float* g, const void* x, const void* y, const float* M,
                                      int64_t ms, const float* h_act, int64_t hs, void* gx, void* gy, float* gM,
                                      float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s);
// Static H gradients for n >= 16 from scal_part[rows][n^2 + 2n]; the
// Sinkhorn adjoint keeps its history in hist when iters * (n + 1) * n
// floats fit hist_bytes, else recomputes it.
constexpr size_t kStaticSkHistBytes = size_t(4) << 20;
hipError_t launch_wide_static_finalize(int n, const float* scal_part, int rows, const float* h_pre,
                                       const float* h_post, const float* h_res, float* d_h_pre, float* d_h_post,
                                       float* d_h_res, int iters, float sk_eps, float* hist, size_t hist_bytes,
                                       hipStream_t s);

// ---- ops.hip ---------------------------------------------------------------
hipError_t launch_rmsnorm_fwd(int dt, const void* x, const float* w, void* y, float* rms, int64_t B, int64_t C,
                              float eps, hipStream_t s);
int rmsnorm_bwd_grid(int dt, int64_t B, int64_t C);
hipError_t launch_rmsnorm_bwd(int dt, const void* g, const void* x, const float* w, const float* rms, void* gx,
                              float* dw_part, int grid, int64_t B, int64_t C, hipStream_t s);
hipError_t launch_compute_rms(int dt, const void* x, float* rms, int64_t B, int64_t K, float eps, hipStream_t s);
hipError_t launch_aggregate_fwd(int dt, int n, const void* x, const float* H, int64_t hs, void* out, float* h_act,
                                int64_t B, int64_t C, hipStream_t s);
hipError_t launch_aggregate_bwd(int dt, int n, const void* g, const void* x, const float* h_act, int64_t hs,
                                void* gx, float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s);
hipError_t launch_distribute_fwd(int dt, int n, const void* y, const float* H, int64_t hs, const float* M,
                                 int64_t ms, const void* x, float* out, float* h_act, int64_t B, int64_t C,
                                 hipStream_t s);
hipError_t launch_distribute_bwd(int dt, int n, const float* g, const void* x, const void* y, const float* M,
                                 int64_t ms, const float* h_act, int64_t hs, void* gx, void* gy, float* gM,
                                 float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s);

// ---- dynamic.hip -----------------------------------------------------------
typedef uint16_t bf16_raw_t;
// Projection outputs come in tiles of 32 rows (two 16-wide MFMA tiles).
constexpr int kProjTile = 32;
constexpr int proj_tiles(int np) { return (np + kProjTile - 1) / kProjTile; }
// Row stride of the per-token projection cotangent dP [B][dp_stride(np)].
constexpr int dp_stride(int np) { return proj_tiles(np) * kProjTile; }
// Largest number of projection rows (output tiles run one after another).
constexpr int kMaxProjRows = 8192;
// Phi [np rows, K] -> proj_tiles(np) output tiles of three bf16 planes
// (3 * 32 * K bf16 each) in the projection kernel's operand order; with w32
// the same launch converts the RMSNorm weight (C elements of w_dtype) too.
hipError_t launch_phi_split(const float* pre, const float* post, const float* res, int n, int np, int64_t K,
                            bf16_raw_t* phib, hipStream_t s, const void* weight = nullptr, int w_dtype = 0,
                            int64_t C = 0, float* w32 = nullptr);
int proj_ksplit(int64_t B, int64_t K, int np);
// P partials of all proj_tiles(np) output tiles, tile-major:
// p_part[tile][ks][B][32], plus ss_part[ks][B] = partial sums of x^2.
hipError_t launch_proj_mfma(int x_dtype, const void* x, const bf16_raw_t* phib, int np, float* p_part,
                            float* ss_part, int64_t B, int64_t K, int ks, hipStream_t s);
// More than 128 rows (proj_stream_path): the streaming projection reads Phi
// once (fp32 rows from pre / post / res as phi_row, or, when phib is not
// null, the planes of launch_phi_split); fp32 x is first split into
// xplanes (proj_xplanes_bytes) with ss_part.  Same p_part / ss_part layout
// as launch_proj_mfma, ks from proj_ksplit.
bool proj_stream_path(int np);
constexpr size_t proj_xplanes_bytes(int64_t B, int64_t K) { return (size_t)(3 * B * K * 2); }
hipError_t launch_proj_stream(int x_dtype, const void* x, bf16_raw_t* xplanes, const float* phi_pre,
                              const float* phi_post, const float* phi_res, int n_pre, const bf16_raw_t* phib, int np,
                              float* p_part, float* ss_part, int64_t B, int64_t K, int ks, hipStream_t s);
// The streaming projection of the MHCResidualWrapper's stream rows with
// bf16 storage, read from residual / branch ([B][Cw] each, Cw % 64 == 0)
// instead of a stream tensor (decay: streams j >= 2 are bf16(r 0.1^(j-1)),
// else 0); Phi as the planes of launch_phi_split; p_part / ss_part as
// launch_proj_mfma.
hipError_t launch_proj_stream_wrap(bool decay, const void* res, const void* br, int64_t Cw, const bf16_raw_t* phib,
                                   int np, float* p_part, float* ss_part, int64_t B, int64_t K, int ks,
                                   hipStream_t s);
hipError_t launch_proj_reduce(const float* p_part, int ks, int64_t B, int np, float* out, hipStream_t s);
#ifdef MHC_KERNEL_TIMING
// The benchmark build's VALU projection (A/B against launch_proj_mfma): Phi
// [np <= 32, K] fp32 is transposed into phit [K][32], then the same p_part
// [ks][B][32] and ss_part[ks][B] from fp32 FMAs, ks from proj_valu_ksplit.
int proj_valu_ksplit(int64_t B, int64_t K);
hipError_t launch_proj_valu(int x_dtype, const void* x, const float* phi, int np, float* phit, float* p_part,
                            float* ss_part, int64_t B, int64_t K, int ks, hipStream_t s);
#endif
hipError_t launch_dyn_coef_fwd(int n, const float* p_part, const float* ss_part, int ks, int64_t B, int64_t K,
                               const float* a_pre, const float* a_post, const float* a_res, const float* b_pre,
                               const float* b_post, const float* b_res, float* coef, float* p_out, float* rh,
                               int iters, float sk_eps, float rms_eps, hipStream_t s);
int dyn_coef_bwd_blocks(int n, int64_t B);
// n >= 16: the Sinkhorn adjoint's per-iteration history lives in a region
// of kSkHistBytes (hist; null for n < 16), split into token slots of
// iters * (n + 1) * n floats; 0 slots = iters too large for the region.
// Generic n: a region of dyn_coef_gen_hist_bytes(n, B) (at most
// kSkHistBytes; hist may be null), used when one workgroup's token slots fit
// it at the call's iters, else each iteration's state is recomputed.
constexpr size_t kSkHistBytes = size_t(64) << 20;
int dyn_coef_bwd_hist_slots(int n, int64_t B, int iters);
size_t dyn_coef_gen_hist_bytes(int n, int64_t B);
// res_rows = false (any n): dM is taken as zero after
// the Sinkhorn adjoint (the wrapper's column-constant dM,
// wrap_res_grad_vanishes): dP, db and dalpha of the H_res rows are written as
// zeros and no adjoint runs.
hipError_t launch_dyn_coef_bwd(int n, const float* scal, const float* coef, const float* p, const float* rh,
                               int64_t B, int64_t K, const float* a_pre, const float* a_post, const float* a_res,
                               const float* b_res, float* dp_out, float* s_out, float* part, int iters, float sk_eps,
                               float* hist, hipStream_t s, bool res_rows = true);
// Deterministic column sums of several partial matrices in one launch:
// out[c] = sum_r part[r][c] over `rows` <= 512 rows (column_sums_direct),
// columns c < split to `out` (bf16 when out_bf16, else fp32) and the rest to
// out2 (fp32).  phases and blocks are set by the launcher.
constexpr int kMaxColSumJobs = 3;
struct ColSumJob {
    const float* part;
    void* out;
    float* out2;
    int64_t cols;
    int rows;
    int split;
    int out_bf16;
    int phases;
    int blocks;
};
struct ColSumJobs {
    ColSumJob j[kMaxColSumJobs];
    int count;
};
bool column_sums_direct(int rows);
hipError_t launch_multi_column_sum(ColSumJobs jobs, hipStream_t s);
hipError_t launch_small_column_sum(const float* part, int rows, int cols, float* out_db, float* out_da, int np,
                                   hipStream_t s);
// Projection backward (bf16 MFMA, split operands) over the flattened [B, K]
// rows, for the output rows o0 .. o0 + np - 1 (np <= 32; dP points at
// column o0 of its rows):
//   dx[b][k] = (accumulate ? dx[b][k] : 0) + (s ? s[b] x[b][k] : 0) + sum_o dP[b][o] Phi[o0 + o][k]
//   dphi_part[tile][o][k] = sum_{b in tile} dP[b][o] x[b][k]
// Phi row o is phi_row(pre, post, res, n_pre, o): rows < n_pre from `pre`,
// the next n_pre from `post`, the rest from `res`.  K % 32 == 0.
int proj_bwd_tiles(int x_dtype, int64_t B, int64_t K);
// More than one output tile, fp32 x, up to 1024 tokens: dx over all tiles in
// one pass and dPhi written directly (no partials).  scratch holds dP, dP^T
// and x^T as bf16 hi / lo planes (proj_bwd_wide_scratch_bytes).
bool proj_bwd_wide_path(int x_dtype, int np, int64_t B);
size_t proj_bwd_wide_scratch_bytes(int np, int64_t B, int64_t K);
// 32 < np <= 128 at any batch: dx over all output tiles in one pass (one
// workgroup per 128 columns x 32 tokens) and dPhi written directly (one
// workgroup per 64 rows x 128 columns walking all tokens); fp32 x and dx.
// rows (np) launch_proj_bwd_small takes at most
int proj_bwd_small_max_rows();
hipError_t launch_proj_bwd_small(const float* x, const float* dP, int dp_stride, const float* s_tok,
                                 const float* phi_pre, const float* phi_post, const float* phi_res, int n_pre, int np,
                                 float* dx, bool accumulate, float* dphi, int64_t B, int64_t K, hipStream_t s);
hipError_t launch_proj_bwd_wide(const float* x, const float* dP, int dp_stride, const float* s_tok,
                                const float* phi_pre, const float* phi_post, const float* phi_res, int n_pre, int np,
                                float* dx, bool accumulate, float* dphi, void* scratch, int64_t B, int64_t K,
                                hipStream_t s);
// With bf16 x (one output tile, accumulate) the incoming dx is the layer
// backward's fp16 stream part with scale exponents dx_scale[B][groups]
// (groups = layer_bwd_part_groups).
hipError_t launch_proj_bwd(int x_dtype, const void* x, const float* dP, int dp_stride, const float* s_tok,
                           const float* phi_pre, const float* phi_post, const float* phi_res, int n_pre, int o0,
                           int np, void* dx, bool accumulate, float* dphi_part, int tiles, int64_t B, int64_t K,
                           hipStream_t s, const int32_t* dx_scale = nullptr, int groups = 0);
hipError_t launch_weight_f32(const void* w, int w_dtype, int64_t C, float* out, hipStream_t s);

// ---- wrapper.hip -----------------------------------------------------------
// Fused MHCResidualWrapper (n = 4): streams synthesised from (residual,
// branch); decay = 'decay' mode (else 'zero').
// Floats per token of the dynamic backward's stream-part factors
// (cm_0..3, h_pre_0..3, hs, 1/r, k2, one spare slot).
constexpr int kWrapEp = 12;
hipError_t launch_wrap_fwd(int dt, int n, bool decay, const void* res, const void* br, const float* w,
                           const float* coef, int64_t coef_stride, float* out, int64_t B, int64_t C, float eps,
                           hipStream_t s);
int wrap_bwd_grid(int dt, int n, bool decay, int64_t B, int64_t C);
// Static-H backward: per-workgroup sums of [dM, dh_post_act, dh_pre_act] in
// scal_out[grid][n*n+2n], d r / d b and the dw partials dw_part[grid][C].
hipError_t launch_wrap_bwd(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                           const float* w, const float* coef, int64_t coef_stride, void* dres, void* dbr,
                           float* dw_part, float* scal_out, int grid, int64_t B, int64_t C, float eps,
                           hipStream_t s);
// Dynamic-H backward, pass 1 (reads G, r, b only): per-token scalars
// scal_out[B][n*n+2n+2] and stream-part factors ep_out[B][kWrapEp].
hipError_t launch_wrap_bwd_red(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                               const float* w, const float* coef, int64_t coef_stride, float* scal_out,
                               float* ep_out, int64_t B, int64_t C, float eps, hipStream_t s);
int wrap_proj_csplit(int64_t B, int64_t C);
// Phi planes for launch_wrap_proj (n = 4): bf16 storage takes the five-slot
// layout of wrap_phi_pack_kernel, fp32 storage phi_split_kernel's planes;
// phib holds 6 * 32 * n * C bytes either way.
hipError_t launch_wrap_phi_planes(int dt, int n, const float* phi_pre, const float* phi_post, const float* phi_res,
                                  int64_t C, bf16_raw_t* phib, hipStream_t s);
hipError_t launch_wrap_proj(int dt, int n, bool decay, const void* res, const void* br, const bf16_raw_t* phib,
                            float* p_part, float* ss_part, int64_t B, int64_t C, int ks, hipStream_t s);
int wrap_proj_bwd_tiles(int dt, int64_t B, int64_t C);
// Dynamic-H backward, pass 2: d r / d b (written, rounded once), dw_part
// [tiles][C] and dphi_part [tiles][np][n*C] from G, r, b, the factors of
// launch_wrap_bwd_red, dP and s.  res_rows = false: the H_res rows of dP are
// zero and dphi_part holds only the 2n pre / post rows per tile.
hipError_t launch_wrap_proj_bwd(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                                const float* w, const float* ep, const float* dP, const float* s_tok,
                                const float* phi_pre, const float* phi_post, const float* phi_res, void* dres,
                                void* dbr, float* dw_part, float* dphi_part, int tiles, int64_t B, int64_t C,
                                bool res_rows, hipStream_t s);

// ---- wrapper_gen.hip -------------------------------------------------------
// MHCResidualWrapper for n = 2..32 with n at run time (the shapes the n = 4
// kernels above do not take); hidden % 4 == 0.  The dPhi / fold kernels
// (the dynamic-H backward without stream rows) take n <= kWgFoldMaxN.
constexpr int kWgMaxN = 32;
constexpr int kWgFoldMaxN = 16;
// Floats per token of the per-token factors of d r / d b (and h_pre up to
// capacity 8).
constexpr int kWgEp = 16;
bool wgen_supported(int n, int64_t C);
hipError_t launch_wgen_fwd(int dt, int n, bool decay, const void* res, const void* br, const float* w,
                           const float* coef, int64_t coef_stride, float* out, int64_t B, int64_t C, float eps,
                           hipStream_t s);
// Waves of the static-H row sums (rows of its scal_out) are 4 x this grid.
int wgen_red_static_grid(int64_t B);
// Row sums of the backward: stat = false: scal_out[B][n*n+2n+2] per token;
// stat = true: scal_out[4 * wgen_red_static_grid(B)][n*n+2n] per wave.
// Both: ep_out[B][kWgEp].
hipError_t launch_wgen_red(int dt, int n, bool decay, bool stat, const float* g, const void* res, const void* br,
                           const float* w, const float* coef, int64_t coef_stride, float* scal_out, float* ep_out,
                           int64_t B, int64_t C, float eps, hipStream_t s);
int wgen_dx_tiles(int64_t B, int64_t C);
// d r / d b and dw_part[tiles][C]; dX (fp32 [B][n*C] = dP . Phi per stream)
// and s_tok (the r_h term's s per token) with dynamic H, both null with
// static H.
hipError_t launch_wgen_dx(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                          const float* w, const float* coef, int64_t coef_stride, const float* ep, const float* dX,
                          const float* s_tok, void* dres, void* dbr, float* dw_part, int tiles, int64_t B, int64_t C,
                          hipStream_t s);
// The projection backward over the pre / post rows (rows = 2n) without the
// stream rows: dPhi partials dphi_part[tiles][rows][n*C] (tiles from
// wgen_dphi_tiles), and d r / d b with dP . Phi folded over the streams
// (dw_part[tiles][C], tiles from wgen_fold_tiles).
int wgen_dphi_tiles(int64_t B, int64_t C);
hipError_t launch_wgen_dphi(int dt, int n, bool decay, const void* res, const void* br, const float* dP,
                            int dp_stride, int rows, float* dphi_part, int tiles, int64_t B, int64_t C,
                            hipStream_t s);
int wgen_fold_tiles(int64_t B, int64_t C);
hipError_t launch_wgen_dx_fold(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                               const float* w, const float* coef, int64_t coef_stride, const float* ep,
                               const float* dP, int dp_stride, int rows,
                               const float* s_tok, const float* phi_pre, const float* phi_post, void* dres,
                               void* dbr, float* dw_part, int tiles, int64_t B, int64_t C, hipStream_t s);
// X[B][n*C] in out_dt (kF32, or the storage dtype dt).
hipError_t launch_wgen_synth(int dt, int out_dt, int n, bool decay, const void* res, const void* br, void* X,
                             int64_t B, int64_t C, hipStream_t s);

// ---- compat.hip ------------------------------------------------------------
// The reference-shaped dynamic-H entries (mhc_layer_fwd_dynamic /
// mhc_layer_bwd_dynamic).  dst[0..2] = (a, b, c).
hipError_t launch_set_scalars(float* dst, float a, float b, float c, hipStream_t s);
// From x, the fp32 weight and the fused forward's per-token coefficients and
// r_h: rms [B], x_agg / y_norm [B, C] bf16, x_flat [B, n*C] bf16, h_pre /
// h_post [B, n], M [B, n, n], rms_h [B].
hipError_t launch_dyn_intermediates(int x_dtype, const void* x, const float* w32, const float* coef, const float* rh,
                                    int n, int64_t B, int64_t C, float eps, float* rms, void* x_agg, void* y_norm,
                                    void* x_flat, float* h_pre, float* h_post, float* M, float* rms_h,
                                    hipStream_t s);
// The inverse for the coefficients: coef [B, 2n+n^2] = (h_pre, h_post, M),
// rh [B] = rms_h.
hipError_t launch_dyn_saved_assemble(const float* h_pre, const float* h_post, const float* M, const float* rms_h,
                                     int n, int64_t B, float* coef, float* rh, hipStream_t s);

// ---- sinkhorn.hip ----------------------------------------------------------
hipError_t launch_sinkhorn_fwd(int n, const float* inp, float* out, int64_t batch, int iters, float eps,
                               hipStream_t s);
hipError_t launch_sinkhorn_bwd(int n, const float* grad_out, const float* inp, float* grad_inp, int64_t batch,
                               int iters, float eps, hipStream_t s);

}  // namespace mhc

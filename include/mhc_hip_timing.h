/*
 * mhc_hip_timing.h - per-kernel timing of the benchmark's build of the library
 * (libmhc_hip_timed.so, compiled with MHC_KERNEL_TIMING).  Not part of the
 * product library libmhc_hip.so, which keeps no timing state.
 *
 * When enabled, the timed build records a start/end hipEvent pair around each
 * of its main kernels on the stream it launches them on.  mhc_timing_query
 * synchronises the recorded events of `kernel` and returns the summed
 * duration (ms) and the launch count since the last reset.  No counterpart in
 * the reference (its benchmark times whole calls with NPU events,
 * benchmark.py:196-204).
 */
#ifndef MHC_HIP_TIMING_H_
#define MHC_HIP_TIMING_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int mhc_timing_enable(int enable);
int mhc_timing_reset(void);
int mhc_timing_query(const char* kernel, double* total_ms, int64_t* launches);

/* A/B of the projection's arithmetic (the benchmark build only): the same
 * out[b, o] = sum_k inp[b, k] weight[o, k] as mhc_fused_rmsnorm_matmul_fwd
 * (inp [batch, k] F32 or BF16, weight [out_dim <= 32, k] fp32, k % 32 == 0,
 * out [batch, out_dim] fp32), with the products on the VALU (fp32 FMAs, one
 * token per lane, weight rows through scalar loads) instead of bf16 MFMA.
 * Its main kernel times as "proj_valu" (the MFMA one as "proj").  No
 * counterpart in the reference: it measures the choice of MFMA for the
 * projection of fused_rmsnorm_matmul_fwd (bindings.cpp:480-528). */
size_t mhc_timing_proj_valu_workspace_size(int64_t batch, int64_t k, int32_t out_dim);
int mhc_timing_proj_valu(const void* inp, int32_t dtype, const float* weight, float* out, void* workspace,
                         size_t workspace_bytes, int64_t batch, int64_t k, int32_t out_dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MHC_HIP_TIMING_H_ */

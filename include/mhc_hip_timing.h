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

#ifdef __cplusplus
}
#endif

#endif /* MHC_HIP_TIMING_H_ */

// Row-kernel helpers shared by the fused layer kernels and the standalone
// stream/norm operators: a workgroup owns one token row at a time, each
// lane VPT chunks of WC channels (chunk q = k * blockDim.x + tid, channels
// q * WC ... q * WC + WC - 1) of each stream.
#pragma once

#include "mhc_device.h"

namespace mhc {

// ---------------------------------------------------------------------------
// This thread's VPT chunks of WC channels of each of the N streams of one
// token row starting at `base` (stream stride C).
// NTL selects non-temporal loads.  All streaming rows use them: a plain-load
// forward is faster in isolation but slows the following backward more than
// it gains (whole fwd+bwd step measured at n=4, C=4096).
// ---------------------------------------------------------------------------
template <typename T, int N, int VPT, int WC, bool NTL>
__device__ __forceinline__ void load_rows(const T* __restrict__ base, int C, float (&v)[N][VPT][WC]) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if (c0 < C) {
                if constexpr (NTL) {
                    load_run_nt<T, WC>(base + (int64_t)i * C + c0, v[i][k]);
                } else {
                    load_run<T, WC>(base + (int64_t)i * C + c0, v[i][k]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < WC; ++e) v[i][k][e] = 0.f;
            }
        }
    }
}

template <int VPT, int WC>
__device__ __forceinline__ void load_weight(const float* __restrict__ w, int C, float (&wv)[VPT][WC]) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) {
            load_run<float, WC>(w + c0, wv[k]);
        } else {
#pragma unroll
            for (int e = 0; e < WC; ++e) wv[k][e] = 0.f;
        }
    }
}

// Workgroup size bound: the prefetching variants hold two token rows and
// run with up to 256 lanes (512 VGPRs available); the others up to 512.
#define MHC_ROW_BOUNDS(PF) __attribute__((amdgpu_flat_work_group_size(1, (PF) ? 256 : 512)))

// Store one stream row chunk set (VPT chunks of WC channels).
template <typename T, int VPT, int WC, bool NT>
__device__ __forceinline__ void store_row1(T* __restrict__ base, int C, const float (&v)[VPT][WC]) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) {
            if constexpr (NT) {
                store_run_nt<T, WC>(base + c0, v[k]);
            } else {
                store_run<T, WC>(base + c0, v[k]);
            }
        }
    }
}

// Row state budget shared with choose_row_tiling(): n_arrays * VPT * W <= 128.
template <typename TX>
constexpr bool row_fits(int n_arrays, int vpt) {
    return n_arrays * vpt * VecIO<TX>::W <= 128;
}

}  // namespace mhc

// Batched Sinkhorn-Knopp forward / exact backward on [batch, n, n] fp32.
//
// Replaces sinkhorn_knopp_forward (sinkhorn_knopp.cpp:739, v3 path 625-665)
// and sinkhorn_knopp_backward (1904, N4 path 1608-1814).  One matrix per
// group of pow2ceil(n) lanes, one row per lane, all iterations in registers;
// column sums are lane-group butterflies.  The backward keeps the forward
// history (post-row-step rows and row sums) in registers and applies the
// exact adjoint (the reference's row step is approximate,
// sinkhorn_knopp.cpp:1773-1795).  Small n = 4 batches run one element per
// lane of a 16-lane DPP row instead (sk16_* in mhc_device.h); 8 < n <= 64
// runs the masked wide kernels (skw_*), whose backward recomputes the
// forward state per iteration instead of keeping a history.
#include "mhc_device.h"
#include "mhc_internal.h"

namespace mhc {

template <int N>
__device__ __forceinline__ void load_row(const float* p, float (&a)[N]) {
    if constexpr (N == 4) {
        const float4 q = *reinterpret_cast<const float4*>(p);
        a[0] = q.x; a[1] = q.y; a[2] = q.z; a[3] = q.w;
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) a[c] = p[c];
    }
}

template <int N>
__device__ __forceinline__ void store_row(float* p, const float (&a)[N]) {
    if constexpr (N == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(a[0], a[1], a[2], a[3]);
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) p[c] = a[c];
    }
}

template <int N>
__global__ __launch_bounds__(256) void sinkhorn_fwd_kernel(const float* __restrict__ inp, float* __restrict__ out,
                                                           int64_t batch, int iters, float eps) {
    constexpr int G = pow2ceil(N);
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = gid / G;
    const int r = (int)(gid % G);
    const bool ok = (m < batch) && (r < N);
    float a[N];
    if (ok) {
        load_row<N>(inp + m * N * N + r * N, a);
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) a[c] = 0.f;
    }
    sk_forward<N>(a, iters, eps, ok);
    if (ok) store_row<N>(out + m * N * N + r * N, a);
}

template <int N>
__global__ __launch_bounds__(256) void sinkhorn_bwd_kernel(const float* __restrict__ grad_out,
                                                           const float* __restrict__ inp,
                                                           float* __restrict__ grad_inp, int64_t batch, int iters,
                                                           float eps) {
    constexpr int G = pow2ceil(N);
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = gid / G;
    const int r = (int)(gid % G);
    const bool ok = (m < batch) && (r < N);
    float x0[N], g[N];
    if (ok) {
        load_row<N>(inp + m * N * N + r * N, x0);
        load_row<N>(grad_out + m * N * N + r * N, g);
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) { x0[c] = 0.f; g[c] = 0.f; }
    }
    sk_backward<N>(g, x0, iters, eps, ok);
    if (ok) store_row<N>(grad_inp + m * N * N + r * N, g);
}

// n = 4: one matrix per 16-lane DPP row, one element per lane (lane 4 r + c);
// the loads and stores are one contiguous float per lane.  The chain per
// matrix is about 4x shorter than with one row per lane but issues more
// instructions in total, so it is used for batches that leave the chip
// latency-bound; large batches (throughput-bound) keep one row per lane.
constexpr int64_t kSk16MaxBatch = 16384;
__global__ __launch_bounds__(256) void sinkhorn16_fwd_kernel(const float* __restrict__ inp, float* __restrict__ out,
                                                             int64_t batch, int iters, float eps) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool ok = gid < batch * 16;
    float a = ok ? inp[gid] : 0.f;
    sk16_forward(a, iters, eps);
    if (ok) out[gid] = a;
}

__global__ __launch_bounds__(256) void sinkhorn16_bwd_kernel(const float* __restrict__ grad_out,
                                                             const float* __restrict__ inp,
                                                             float* __restrict__ grad_inp, int64_t batch, int iters,
                                                             float eps) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool ok = gid < batch * 16;
    float g = ok ? grad_out[gid] : 0.f;
    const float x0 = ok ? inp[gid] : 0.f;
    sk16_backward(g, x0, iters, eps);
    if (ok) grad_inp[gid] = g;
}

// 8 < n <= 64: one matrix per group of NM = pow2ceil(n) lanes (16, 32 or
// 64), one row per lane, n taken at run time with the padded columns masked.
template <int NM>
__global__ __launch_bounds__(256) void sinkhorn_wide_fwd_kernel(const float* __restrict__ inp,
                                                                float* __restrict__ out, int n, int64_t batch,
                                                                int iters, float eps) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = gid / NM;
    const int r = (int)(gid % NM);
    const bool ok = (m < batch) && (r < n);
    const float* row = inp + (m * n + r) * n;
    float a[NM];
#pragma unroll
    for (int c = 0; c < NM; ++c) a[c] = (ok && c < n) ? row[c] : 0.f;
    skw_forward<NM>(a, n, iters, eps, ok);
    if (ok) {
        float* o = out + (m * n + r) * n;
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            if (c < n) o[c] = a[c];
        }
    }
}

template <int NM>
__global__ __launch_bounds__(256) void sinkhorn_wide_bwd_kernel(const float* __restrict__ grad_out,
                                                                const float* __restrict__ inp,
                                                                float* __restrict__ grad_inp, int n, int64_t batch,
                                                                int iters, float eps) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = gid / NM;
    const int r = (int)(gid % NM);
    const bool ok = (m < batch) && (r < n);
    const int64_t off = (m * n + r) * n;
    float x0[NM], g[NM];
#pragma unroll
    for (int c = 0; c < NM; ++c) {
        x0[c] = (ok && c < n) ? inp[off + c] : 0.f;
        g[c] = (ok && c < n) ? grad_out[off + c] : 0.f;
    }
    skw_backward<NM>(g, x0, n, iters, eps, ok);
    if (ok) {
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            if (c < n) grad_inp[off + c] = g[c];
        }
    }
}

#define MHC_SK_WIDE(n, ...)                                                   \
    if (n <= 16) {                                                            \
        constexpr int NM_ = 16; __VA_ARGS__;                                  \
    } else if (n <= 32) {                                                     \
        constexpr int NM_ = 32; __VA_ARGS__;                                  \
    } else if (n <= 64) {                                                     \
        constexpr int NM_ = 64; __VA_ARGS__;                                  \
    } else {                                                                  \
        return hipErrorInvalidValue;                                          \
    }

#define MHC_SK_DISPATCH(n, ...)                                   \
    switch (n) {                                                  \
        case 1: { constexpr int N_ = 1; __VA_ARGS__; break; }     \
        case 2: { constexpr int N_ = 2; __VA_ARGS__; break; }     \
        case 3: { constexpr int N_ = 3; __VA_ARGS__; break; }     \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }     \
        case 5: { constexpr int N_ = 5; __VA_ARGS__; break; }     \
        case 6: { constexpr int N_ = 6; __VA_ARGS__; break; }     \
        case 7: { constexpr int N_ = 7; __VA_ARGS__; break; }     \
        case 8: { constexpr int N_ = 8; __VA_ARGS__; break; }     \
        default: return hipErrorInvalidValue;                     \
    }

hipError_t launch_sinkhorn_fwd(int n, const float* inp, float* out, int64_t batch, int iters, float eps,
                               hipStream_t s) {
    if (batch == 0) return hipSuccess;
    const int G = pow2ceil(n);
    const int64_t threads = batch * G;
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    const int tok = timing_begin("sinkhorn_fwd", s);
    if (n == 4 && batch < kSk16MaxBatch) {
        MHC_LAUNCH_GGL(sinkhorn16_fwd_kernel, dim3((unsigned)((batch * 16 + 255) / 256)), dim3(256), 0, s, inp, out,
                           batch, iters, eps);
    } else if (n > 8) {
        MHC_SK_WIDE(n, MHC_LAUNCH_GGL((sinkhorn_wide_fwd_kernel<NM_>), dim3(blocks), dim3(256), 0, s, inp, out, n,
                                          batch, iters, eps));
    } else {
        MHC_SK_DISPATCH(n, MHC_LAUNCH_GGL((sinkhorn_fwd_kernel<N_>), dim3(blocks), dim3(256), 0, s, inp, out,
                                              batch, iters, eps));
    }
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_sinkhorn_bwd(int n, const float* grad_out, const float* inp, float* grad_inp, int64_t batch,
                               int iters, float eps, hipStream_t s) {
    if (batch == 0) return hipSuccess;
    const int G = pow2ceil(n);
    const int64_t threads = batch * G;
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    const int tok = timing_begin("sinkhorn_bwd", s);
    if (n == 4 && batch < kSk16MaxBatch) {
        MHC_LAUNCH_GGL(sinkhorn16_bwd_kernel, dim3((unsigned)((batch * 16 + 255) / 256)), dim3(256), 0, s,
                           grad_out, inp, grad_inp, batch, iters, eps);
    } else if (n > 8) {
        MHC_SK_WIDE(n, MHC_LAUNCH_GGL((sinkhorn_wide_bwd_kernel<NM_>), dim3(blocks), dim3(256), 0, s, grad_out,
                                          inp, grad_inp, n, batch, iters, eps));
    } else {
        MHC_SK_DISPATCH(n, MHC_LAUNCH_GGL((sinkhorn_bwd_kernel<N_>), dim3(blocks), dim3(256), 0, s, grad_out,
                                              inp, grad_inp, batch, iters, eps));
    }
    timing_end(tok, s);
    return hipGetLastError();
}

}  // namespace mhc

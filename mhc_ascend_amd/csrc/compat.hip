// Kernels behind the reference-shaped dynamic-H entries mhc_layer_fwd_dynamic
// / mhc_layer_bwd_dynamic (bindings.cpp:600-952).  The reference hands nine
// tensors from its forward to its backward; the fused path keeps one saved
// buffer instead.  These kernels translate between the two:
//   * dyn_intermediates_kernel derives the reference's tensors from the
//     fused forward's saved state and x (one extra pass over x);
//   * dyn_saved_assemble_kernel rebuilds the fused backward's saved state from
//     the reference's tensors plus a recomputed projection P (the reference
//     recomputes P in its backward too, bindings.cpp:764-766).
// Neither runs on the fused training path.
#include "mhc_device.h"
#include "mhc_internal.h"

namespace mhc {

namespace {

// The three alphas of a call given as floats (the reference's signature)
// written to device memory for the kernels, which read them as pointers.
// Three lanes, three vector stores; a kernel (not a memset or a host copy)
// so that the entry stays stream-ordered and capturable.
__global__ void set_scalars_kernel(float* __restrict__ dst, float a, float b, float c) {
    const int t = threadIdx.x;
    if (t < 3) dst[t] = t == 0 ? a : (t == 1 ? b : c);
}

template <typename T>
__device__ __forceinline__ float load_elem(const T* p);
template <>
__device__ __forceinline__ float load_elem<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_elem<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

constexpr int kInterThreads = 256;

// One token per workgroup (bindings.cpp:894-940):
//   x_flat = bf16(x)                       [B, nC]
//   x_agg[c] = sum_i h_pre[i] x[i][c]      (stored bf16)
//   rms = sqrt(mean_c x_agg^2 + eps)       [B]   (fp32, from the fp32 x_agg)
//   y_norm[c] = x_agg[c] / rms * w[c]      (stored bf16)
//   h_pre_act, h_post_act, M, rms_h        copied from the saved coefficients
// saved coef row of a token: (h_pre[n], h_post[n], M[n*n] row-major).
template <typename T>
__global__ __launch_bounds__(kInterThreads) void dyn_intermediates_kernel(
    const T* __restrict__ x, const float* __restrict__ w32, const float* __restrict__ coef,
    const float* __restrict__ rh, int n, int64_t C, float eps, float* __restrict__ rms, bf16_t* __restrict__ x_agg,
    bf16_t* __restrict__ y_norm, bf16_t* __restrict__ x_flat, float* __restrict__ h_pre, float* __restrict__ h_post,
    float* __restrict__ M, float* __restrict__ rms_h) {
    __shared__ float hp[32];
    __shared__ float red[kInterThreads / kWave];
    const int64_t tok = blockIdx.x;
    const int np = 2 * n + n * n;
    const float* cf = coef + tok * np;
    for (int o = threadIdx.x; o < np; o += blockDim.x) {
        const float v = cf[o];
        if (o < n) {
            hp[o] = v;
            h_pre[tok * n + o] = v;
        } else if (o < 2 * n) {
            h_post[tok * n + (o - n)] = v;
        } else {
            M[tok * n * n + (o - 2 * n)] = v;
        }
    }
    if (threadIdx.x == 0) rms_h[tok] = rh[tok];
    __syncthreads();

    const T* xr = x + tok * n * C;
    bf16_t* xf = x_flat + tok * n * C;
    float ss = 0.f;
    for (int64_t c = threadIdx.x; c < C; c += blockDim.x) {
        float a = 0.f;
        for (int i = 0; i < n; ++i) {
            const float v = load_elem<T>(xr + i * C + c);
            xf[i * C + c] = f32_to_bf16(v);
            a = fmaf(hp[i], v, a);
        }
        ss = fmaf(a, a, ss);
    }
    float v[1] = {ss};
    block_sum<1>(v, red);
    const float r = sqrtf(v[0] / (float)C + eps);
    if (threadIdx.x == 0) rms[tok] = r;
    const float inv = 1.f / r;
    for (int64_t c = threadIdx.x; c < C; c += blockDim.x) {
        float a = 0.f;
        for (int i = 0; i < n; ++i) a = fmaf(hp[i], load_elem<T>(xr + i * C + c), a);
        x_agg[tok * C + c] = f32_to_bf16(a);
        y_norm[tok * C + c] = f32_to_bf16(a * inv * w32[c]);
    }
}

// Per token: coef = (h_pre_act, h_post_act, M), rh = rms_h, and P from the
// projection's output rows p [B, np] (copied as is).  One lane per value.
__global__ __launch_bounds__(256) void dyn_saved_assemble_kernel(
    const float* __restrict__ h_pre, const float* __restrict__ h_post, const float* __restrict__ M,
    const float* __restrict__ rms_h, int n, int64_t B, float* __restrict__ coef, float* __restrict__ rh) {
    const int np = 2 * n + n * n;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * (np + 1)) return;
    const int64_t tok = i / (np + 1);
    const int o = (int)(i % (np + 1));
    if (o == np) {
        rh[tok] = rms_h[tok];
    } else {
        float v;
        if (o < n) v = h_pre[tok * n + o];
        else if (o < 2 * n) v = h_post[tok * n + (o - n)];
        else v = M[tok * n * n + (o - 2 * n)];
        coef[tok * np + o] = v;
    }
}

}  // namespace

hipError_t launch_set_scalars(float* dst, float a, float b, float c, hipStream_t s) {
    MHC_LAUNCH_GGL(set_scalars_kernel, dim3(1), dim3(64), 0, s, dst, a, b, c);
    return hipGetLastError();
}

hipError_t launch_dyn_intermediates(int x_dtype, const void* x, const float* w32, const float* coef, const float* rh,
                                    int n, int64_t B, int64_t C, float eps, float* rms, void* x_agg, void* y_norm,
                                    void* x_flat, float* h_pre, float* h_post, float* M, float* rms_h,
                                    hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (n > 32) return hipErrorInvalidValue;
    const dim3 grid((unsigned)B), block(kInterThreads);
    if (x_dtype == kBF16)
        MHC_LAUNCH_GGL(dyn_intermediates_kernel<bf16_t>, grid, block, 0, s, (const bf16_t*)x, w32, coef, rh, n, C,
                           eps, rms, (bf16_t*)x_agg, (bf16_t*)y_norm, (bf16_t*)x_flat, h_pre, h_post, M, rms_h);
    else
        MHC_LAUNCH_GGL(dyn_intermediates_kernel<float>, grid, block, 0, s, (const float*)x, w32, coef, rh, n, C,
                           eps, rms, (bf16_t*)x_agg, (bf16_t*)y_norm, (bf16_t*)x_flat, h_pre, h_post, M, rms_h);
    return hipGetLastError();
}

hipError_t launch_dyn_saved_assemble(const float* h_pre, const float* h_post, const float* M, const float* rms_h,
                                     int n, int64_t B, float* coef, float* rh, hipStream_t s) {
    if (B == 0) return hipSuccess;
    const int64_t total = B * (2 * n + n * n + 1);
    const unsigned blocks = (unsigned)((total + 255) / 256);
    MHC_LAUNCH_GGL(dyn_saved_assemble_kernel, dim3(blocks), dim3(256), 0, s, h_pre, h_post, M, rms_h, n, B,
                       coef, rh);
    return hipGetLastError();
}

}  // namespace mhc

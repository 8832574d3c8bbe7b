// Fused mHC layer kernels: one HBM pass per direction over the [B, n, C]
// residual streams.
//
// Forward (layer.py:142-170 composed from stream_ops.cpp:142-228,
// rmsnorm.cpp:170-178, stream_ops.cpp:403-525):
//     xa = sum_i h_pre[i] x_i;  r = sqrt(mean_c xa^2 + eps);  y = xa / r * w
//     out_i = sum_j M[i][j] x_j + h_post[i] y
// One workgroup per token; the token row stays in registers between the
// RMS reduction and the output, so x is read once and out written once.
//
// Backward (bindings.cpp:654-749 and the kernels it calls): with cotangent G,
//     gy = sum_i h_post[i] G_i
//     gxa = w gy / r - xa (sum_c gy w xa) / (C r^3)
//     dx_j = sum_i M[i][j] G_i + h_pre[j] gxa
//     dM[i][j] = sum_c G_i x_j,  dh_post[i] = sum_c G_i y,
//     dh_pre[j] = sum_c gxa x_j = (1/r) sum_c w gy x_j - (dot/(C r^3)) sum_c xa x_j,
//     dw[c] = sum_b gy xa / r.
// All row sums of a token are formed in ONE block reduction (the dh_pre
// identity above avoids a second pass over gxa).  Workgroups are persistent
// over tokens and keep dw and the scalar sums in registers; per-workgroup
// partials are reduced deterministically afterwards.
#include "mhc_device.h"
#include "mhc_internal.h"

namespace mhc {

template <int N> constexpr int coef_size() { return 2 * N + N * N; }

// ---------------------------------------------------------------------------
// Static coefficients: h_pre = sigmoid(H_pre), h_post = 2 sigmoid(H_post),
// M = SK(exp(H_res)) (layer.py:144-160), computed once per call.
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(64) void static_coef_kernel(const float* __restrict__ h_pre,
                                                         const float* __restrict__ h_post,
                                                         const float* __restrict__ h_res, float* __restrict__ coef,
                                                         int iters, float eps) {
    const int r = threadIdx.x;
    float a[N];
#pragma unroll
    for (int c = 0; c < N; ++c) a[c] = (r < N) ? expf(h_res[r * N + c]) : 0.f;
    sk_forward<N>(a, iters, eps);
    if (r < N) {
        coef[r] = sigmoidf(h_pre[r]);
        coef[N + r] = 2.f * sigmoidf(h_post[r]);
#pragma unroll
        for (int c = 0; c < N; ++c) coef[2 * N + r * N + c] = a[c];
    }
}

// ---------------------------------------------------------------------------
// Fused forward.  grid = B workgroups, block = tiling.threads.
// ---------------------------------------------------------------------------
template <typename TX, int N, int VPT>
__global__ __launch_bounds__(512) void layer_fwd_kernel(const TX* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ coef, int64_t coef_stride,
                                                         float* __restrict__ out, float* __restrict__ rms_out, int C,
                                                         float eps) {
    constexpr int WC = VecIO<TX>::W;
    constexpr int NC = coef_size<N>();
    __shared__ float red[8];
    const int64_t b = blockIdx.x;
    const float* cf = coef + b * coef_stride;
    float cfv[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) cfv[k] = cf[k];

    const TX* xb = x + b * (int64_t)N * C;
    float xv[N][VPT][WC];
    float xa[VPT][WC];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        const bool ok = c0 < C;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if (ok) {
                load_run<TX, WC>(xb + (int64_t)i * C + c0, xv[i][k]);
            } else {
#pragma unroll
                for (int e = 0; e < WC; ++e) xv[i][k][e] = 0.f;
            }
        }
#pragma unroll
        for (int e = 0; e < WC; ++e) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < N; ++i) s += cfv[i] * xv[i][k][e];
            xa[k][e] = s;
            ss += s * s;
        }
    }
    float v[1] = {ss};
    block_sum<1>(v, red);
    const float r = sqrtf(v[0] / (float)C + eps);
    const float inv = 1.f / r;

    float* ob = out + b * (int64_t)N * C;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) {
            float wv[WC];
            load_run<float, WC>(w + c0, wv);
            float y[WC];
#pragma unroll
            for (int e = 0; e < WC; ++e) y[e] = xa[k][e] * inv * wv[e];
#pragma unroll
            for (int i = 0; i < N; ++i) {
                float o[WC];
#pragma unroll
                for (int e = 0; e < WC; ++e) {
                    float s = cfv[N + i] * y[e];
#pragma unroll
                    for (int j = 0; j < N; ++j) s += cfv[2 * N + i * N + j] * xv[j][k][e];
                    o[e] = s;
                }
                store_run<float, WC>(ob + (int64_t)i * C + c0, o);
            }
        }
    }
    if (threadIdx.x == 0 && rms_out) rms_out[b] = r;
}

// ---------------------------------------------------------------------------
// Fused backward.  Persistent: grid <= B workgroups loop over tokens.
// Every token's row sums go to scal_out[b][NS + 2] = (dM[n*n],
// dh_post_act[n], dh_pre_act[n], 1/r, k2 = dot/(C r^3)); dw accumulates in
// registers per workgroup and is written to dw_part[blockIdx.x][C].
// MODE 0 (static H) also writes dx; MODE 1 (dynamic H) leaves dx to a later
// kernel that needs the per-token Sinkhorn backward first.
// ---------------------------------------------------------------------------
template <typename TX, int N, int VPT, int MODE>
__global__ __launch_bounds__(512) void layer_bwd_kernel(const float* __restrict__ g, const TX* __restrict__ x,
                                                        const float* __restrict__ w, const float* __restrict__ coef,
                                                        int64_t coef_stride, TX* __restrict__ dx,
                                                        float* __restrict__ dw_part, float* __restrict__ scal_out,
                                                        int64_t B, int C, float eps) {
    constexpr int WC = VecIO<TX>::W;
    constexpr int NC = coef_size<N>();
    constexpr int NS = N * N + 2 * N;              // dM, dh_post_act, dh_pre_act
    constexpr int NR = 2 + N * N + 3 * N;          // ss, dot, dM, t_i, u_j, v_j
    __shared__ float red[9 * NR];                   // 8 wave partials + totals
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    float* tot = red + 8 * NR;

    float wv[VPT][WC];
    float dwacc[VPT][WC];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) {
            load_run<float, WC>(w + c0, wv[k]);
        } else {
#pragma unroll
            for (int e = 0; e < WC; ++e) wv[k][e] = 0.f;
        }
#pragma unroll
        for (int e = 0; e < WC; ++e) dwacc[k][e] = 0.f;
    }

    for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
        const float* cf = coef + b * coef_stride;
        float cfv[NC];
#pragma unroll
        for (int k = 0; k < NC; ++k) cfv[k] = cf[k];

        const TX* xb = x + b * (int64_t)N * C;
        const float* gb = g + b * (int64_t)N * C;
        float xv[N][VPT][WC];
        float gv[N][VPT][WC];
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int c0 = (k * blockDim.x + threadIdx.x) * WC;
            const bool ok = c0 < C;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (ok) {
                    load_run<TX, WC>(xb + (int64_t)i * C + c0, xv[i][k]);
                    load_run<float, WC>(gb + (int64_t)i * C + c0, gv[i][k]);
                } else {
#pragma unroll
                    for (int e = 0; e < WC; ++e) { xv[i][k][e] = 0.f; gv[i][k][e] = 0.f; }
                }
            }
        }

        {
            float rv[NR];
#pragma unroll
            for (int k = 0; k < NR; ++k) rv[k] = 0.f;
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
#pragma unroll
                for (int e = 0; e < WC; ++e) {
                    float xa = 0.f, gy = 0.f;
#pragma unroll
                    for (int i = 0; i < N; ++i) {
                        xa += cfv[i] * xv[i][k][e];
                        gy += cfv[N + i] * gv[i][k][e];
                    }
                    const float wgy = wv[k][e] * gy;
                    const float wxa = wv[k][e] * xa;
                    rv[0] += xa * xa;
                    rv[1] += wgy * xa;
#pragma unroll
                    for (int i = 0; i < N; ++i) {
#pragma unroll
                        for (int j = 0; j < N; ++j) rv[2 + i * N + j] += gv[i][k][e] * xv[j][k][e];
                        rv[2 + N * N + i] += gv[i][k][e] * wxa;
                        rv[2 + N * N + N + i] += wgy * xv[i][k][e];
                        rv[2 + N * N + 2 * N + i] += xa * xv[i][k][e];
                    }
                }
            }
            wave_sum<NR>(rv);
            if (lane == 0) {
#pragma unroll
                for (int k = 0; k < NR; ++k) red[wave * NR + k] = rv[k];
            }
        }
        __syncthreads();
        if (threadIdx.x < NR) {
            float s = 0.f;
            for (int q = 0; q < nwaves; ++q) s += red[q * NR + threadIdx.x];
            tot[threadIdx.x] = s;
        }
        __syncthreads();
        const float r = sqrtf(tot[0] / (float)C + eps);
        const float inv = 1.f / r;
        const float k2 = tot[1] * inv * inv * inv / (float)C;

        if (threadIdx.x < NS + 2) {
            const int t = threadIdx.x;
            float v;
            if (t < N * N) {
                v = tot[2 + t];
            } else if (t < N * N + N) {
                v = tot[2 + t] * inv;                                   // dh_post_act = (sum G_i xa w) / r
            } else if (t < NS) {
                const int j = t - N * N - N;
                v = inv * tot[2 + N * N + N + j] - k2 * tot[2 + N * N + 2 * N + j];  // dh_pre_act
            } else {
                v = (t == NS) ? inv : k2;
            }
            scal_out[b * (NS + 2) + t] = v;
        }

#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int c0 = (k * blockDim.x + threadIdx.x) * WC;
            float gxa[WC];
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float xa = 0.f, gy = 0.f;
#pragma unroll
                for (int i = 0; i < N; ++i) {
                    xa += cfv[i] * xv[i][k][e];
                    gy += cfv[N + i] * gv[i][k][e];
                }
                gxa[e] = wv[k][e] * gy * inv - xa * k2;
                dwacc[k][e] += gy * xa * inv;
            }
            if (MODE == 0 && c0 < C) {
                TX* db = dx + b * (int64_t)N * C;
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    float d[WC];
#pragma unroll
                    for (int e = 0; e < WC; ++e) {
                        float s = cfv[j] * gxa[e];
#pragma unroll
                        for (int i = 0; i < N; ++i) s += cfv[2 * N + i * N + j] * gv[i][k][e];
                        d[e] = s;
                    }
                    store_run<TX, WC>(db + (int64_t)j * C + c0, d);
                }
            }
        }
    }

    float* dwp = dw_part + (int64_t)blockIdx.x * C;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) store_run<float, WC>(dwp + c0, dwacc[k]);
    }
}

// ---------------------------------------------------------------------------
// out[c] = sum_r part[r][c]   (fixed order -> deterministic)
// grid = ceil(cols / 64), block = 256: wave w sums rows w, w+4, ...
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void column_sum_kernel(const float* __restrict__ part, int rows, int64_t cols,
                                                         float* __restrict__ out) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (c < cols) {
        for (int r = wave; r < rows; r += 4) s += part[(int64_t)r * cols + c];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < cols) out[c] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

// ---------------------------------------------------------------------------
// Static parameter gradients: sum the per-token [dM, dh_post_act, dh_pre_act],
// apply the activation derivatives (ops.py:211, 279-281) and one Sinkhorn
// backward on the token-summed dM (SK is shared, so its VJP is linear in dM):
//     dH_pre = dh_pre_act h_pre (1 - h_pre)
//     dH_post = dh_post_act h_post (1 - h_post / 2)
//     dH_res = SK^T(dM) * exp(H_res)
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void static_finalize_kernel(const float* __restrict__ part, int rows,
                                                              const float* __restrict__ h_pre,
                                                              const float* __restrict__ h_post,
                                                              const float* __restrict__ h_res, float* d_h_pre,
                                                              float* d_h_post, float* d_h_res, int iters,
                                                              float eps) {
    constexpr int NS = N * N + 2 * N;
    __shared__ float red[4 * NS];
    float v[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) v[k] = 0.f;
    for (int r = threadIdx.x; r < rows; r += blockDim.x) {
#pragma unroll
        for (int k = 0; k < NS; ++k) v[k] += part[(int64_t)r * (NS + 2) + k];
    }
    block_sum<NS>(v, red);
    if (threadIdx.x < 64) {
        const int r = threadIdx.x;
        float e[N], gm[N];
#pragma unroll
        for (int c = 0; c < N; ++c) {
            e[c] = (r < N) ? expf(h_res[r * N + c]) : 0.f;
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < N; ++q) s = (r == q) ? v[q * N + c] : s;
            gm[c] = (r < N) ? s : 0.f;
        }
        sk_backward<N>(gm, e, iters, eps);
        if (r < N) {
#pragma unroll
            for (int c = 0; c < N; ++c) d_h_res[r * N + c] = gm[c] * e[c];
            float hp = 0.f, hq = 0.f, tp = 0.f, tq = 0.f;
#pragma unroll
            for (int q = 0; q < N; ++q) {
                hp = (r == q) ? v[N * N + N + q] : hp;
                hq = (r == q) ? v[N * N + q] : hq;
            }
            tp = sigmoidf(h_pre[r]);
            tq = 2.f * sigmoidf(h_post[r]);
            d_h_pre[r] = hp * tp * (1.f - tp);
            d_h_post[r] = hq * tq * (1.f - tq * 0.5f);
        }
    }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

#define MHC_DISPATCH_N(n, ...)                                   \
    switch (n) {                                                 \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }    \
        default: return hipErrorInvalidValue;                    \
    }

#define MHC_DISPATCH_VPT(v, ...)                                 \
    switch (v) {                                                 \
        case 1: { constexpr int V_ = 1; __VA_ARGS__; break; }    \
        case 2: { constexpr int V_ = 2; __VA_ARGS__; break; }    \
        case 4: { constexpr int V_ = 4; __VA_ARGS__; break; }    \
        case 8: { constexpr int V_ = 8; __VA_ARGS__; break; }    \
        default: return hipErrorInvalidValue;                    \
    }

// Row state budget shared with choose_row_tiling(): n_arrays * VPT * W <= 128.
template <typename TX>
constexpr bool row_fits(int n_arrays, int vpt) {
    return n_arrays * vpt * VecIO<TX>::W <= 128;
}

hipError_t launch_static_coef(int n, const float* h_pre, const float* h_post, const float* h_res, float* coef,
                              int iters, float sk_eps, hipStream_t s) {
    MHC_DISPATCH_N(n, hipLaunchKernelGGL((static_coef_kernel<N_>), dim3(1), dim3(64), 0, s, h_pre, h_post, h_res,
                                         coef, iters, sk_eps));
    return hipGetLastError();
}

hipError_t launch_layer_fwd(int x_dtype, int n, const void* x, const float* w, const float* coef,
                            int64_t coef_stride, float* out, float* rms_out, int64_t B, int64_t C, float eps,
                            hipStream_t s) {
    if (B == 0) return hipSuccess;
    const int wc = x_dtype == kBF16 ? 8 : 4;
    const RowTiling t = choose_row_tiling(C, wc, n);
    if (t.vpt <= 0) return hipErrorInvalidValue;
    const int tok = timing_begin("layer_fwd", s);
#define MHC_FWD_LAUNCH(TX_)                                                                                     \
    MHC_DISPATCH_N(n, MHC_DISPATCH_VPT(t.vpt, if constexpr (row_fits<TX_>(N_, V_)) {                              \
        hipLaunchKernelGGL((layer_fwd_kernel<TX_, N_, V_>), dim3(B), dim3(t.threads), 0, s, (const TX_*)x, w, coef, \
                           coef_stride, out, rms_out, (int)C, eps);                                                \
    } else { return hipErrorInvalidValue; }))
    if (x_dtype == kBF16) { MHC_FWD_LAUNCH(bf16_t); } else { MHC_FWD_LAUNCH(float); }
#undef MHC_FWD_LAUNCH
    timing_end(tok, s);
    return hipGetLastError();
}

int layer_bwd_grid(int x_dtype, int n, int64_t B, int64_t C) {
    const int wc = x_dtype == kBF16 ? 8 : 4;
    const RowTiling t = choose_row_tiling(C, wc, 2 * n);
    const int waves = (t.threads + 63) / 64;
    // Aim for ~8 resident waves per CU; the row state makes occupancy
    // register-bound, so more workgroups only add dw partials.
    int per_cu = waves >= 8 ? 1 : 8 / waves;
    int64_t g = (int64_t)device_cu_count() * per_cu;
    if (g > B) g = B;
    if (g < 1) g = 1;
    return (int)g;
}

hipError_t launch_layer_bwd(int x_dtype, int n, int mode, const float* g, const void* x, const float* w,
                            const float* coef, int64_t coef_stride, void* dx, float* dw_part, float* scal_out,
                            int grid, int64_t B, int64_t C, float eps, hipStream_t s) {
    const int wc = x_dtype == kBF16 ? 8 : 4;
    const RowTiling t = choose_row_tiling(C, wc, 2 * n);
    if (t.vpt <= 0) return hipErrorInvalidValue;
    const int tok = timing_begin(mode == 0 ? "layer_bwd" : "layer_bwd_reduce", s);
#define MHC_BWD_LAUNCH(TX_, MODE_)                                                                               \
    MHC_DISPATCH_N(n, MHC_DISPATCH_VPT(t.vpt, if constexpr (row_fits<TX_>(2 * N_, V_)) {                          \
        hipLaunchKernelGGL((layer_bwd_kernel<TX_, N_, V_, MODE_>), dim3(grid), dim3(t.threads), 0, s, g,          \
                           (const TX_*)x, w, coef, coef_stride, (TX_*)dx, dw_part, scal_out, B, (int)C, eps);      \
    } else { return hipErrorInvalidValue; }))
    if (x_dtype == kBF16) {
        if (mode == 0) { MHC_BWD_LAUNCH(bf16_t, 0); } else { MHC_BWD_LAUNCH(bf16_t, 1); }
    } else {
        if (mode == 0) { MHC_BWD_LAUNCH(float, 0); } else { MHC_BWD_LAUNCH(float, 1); }
    }
#undef MHC_BWD_LAUNCH
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_column_sum(const float* part, int rows, int64_t cols, float* out, hipStream_t s) {
    if (cols == 0) return hipSuccess;
    hipLaunchKernelGGL(column_sum_kernel, dim3((unsigned)((cols + 63) / 64)), dim3(256), 0, s, part, rows, cols, out);
    return hipGetLastError();
}

hipError_t launch_static_finalize(int n, const float* scal_part, int rows, const float* h_pre,
                                  const float* h_post, const float* h_res, float* d_h_pre, float* d_h_post,
                                  float* d_h_res, int iters, float sk_eps, hipStream_t s) {
    MHC_DISPATCH_N(n, hipLaunchKernelGGL((static_finalize_kernel<N_>), dim3(1), dim3(256), 0, s, scal_part, rows,
                                         h_pre, h_post, h_res, d_h_pre, d_h_post, d_h_res, iters, sk_eps));
    return hipGetLastError();
}

}  // namespace mhc

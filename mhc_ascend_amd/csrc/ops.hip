// Standalone stream / norm operators of the mHC API, one HBM pass each.
// Rows that are not a multiple of the 16-byte vector, too wide for the
// register rows, or n > 8 run the channel-loop variants of wide.hip.
//
// They replace the Ascend kernels bound at bindings.cpp:237-374 and
// 380-460 (rmsnorm.cpp, stream_ops.cpp) and compute_rms.cpp (bound at
// bindings.cpp:543-566).  A workgroup owns one token row at a time; row sums
// are DPP wave sums plus one LDS step.  Large tensors are fp32 or bf16
// (T); arithmetic and small outputs are fp32.  Per-token coefficient inputs
// (H, M) take a batch stride that may be 0 (one set shared by all tokens).
#include "mhc_device.h"
#include "mhc_internal.h"
#include "mhc_rows.h"

namespace mhc {

// ---------------------------------------------------------------------------
// RMSNorm (ops_pytorch_backward.py:78-91; rmsnorm.cpp:170-178 / 394-411)
//   y = x / r * w,  r = sqrt(mean(x^2) + eps)
//   dx = w g / r - x (sum_c g w x) / (C r^3),  dw = sum_rows g x / r
// ---------------------------------------------------------------------------
template <typename T, int VPT>
__global__ MHC_ROW_BOUNDS(false) void rmsnorm_fwd_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                         T* __restrict__ y, float* __restrict__ rms, int C,
                                                         float eps) {
    constexpr int WC = VecIO<T>::W;
    __shared__ float red[8];
    const int64_t b = blockIdx.x;
    float xv[1][VPT][WC];
    load_rows<T, 1, VPT, WC, true>(x + b * C, C, xv);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
#pragma unroll
        for (int e = 0; e < WC; ++e) ss += xv[0][k][e] * xv[0][k][e];
    }
    float v[1] = {ss};
    block_sum<1>(v, red);
    const float r = sqrtf(v[0] / (float)C + eps);
    const float inv = 1.f / r;
    float wv[VPT][WC];
    load_weight<VPT, WC>(w, C, wv);
    float out[VPT][WC];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
#pragma unroll
        for (int e = 0; e < WC; ++e) out[k][e] = xv[0][k][e] * inv * wv[k][e];
    }
    store_row1<T, VPT, WC, true>(y + b * C, C, out);
    if (threadIdx.x == 0) rms[b] = r;
}

template <typename T, int VPT>
__global__ MHC_ROW_BOUNDS(false) void rmsnorm_bwd_kernel(const T* __restrict__ g, const T* __restrict__ x,
                                                         const float* __restrict__ w, const float* __restrict__ rms,
                                                         T* __restrict__ gx, float* __restrict__ dw_part, int64_t B,
                                                         int C) {
    constexpr int WC = VecIO<T>::W;
    __shared__ float red[8];
    float wv[VPT][WC];
    load_weight<VPT, WC>(w, C, wv);
    float dwacc[VPT][WC];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
#pragma unroll
        for (int e = 0; e < WC; ++e) dwacc[k][e] = 0.f;
    }
    for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
        RawRows<T, 1, VPT, WC> xr, gr;
        float xv[1][VPT][WC], gv[1][VPT][WC];
        load_rows_raw<T, 1, VPT, WC, true>(x + b * C, C, xr);
        load_rows_raw<T, 1, VPT, WC, true>(g + b * C, C, gr);
        unpack_rows<T, 1, VPT, WC>(xr, C, xv);
        unpack_rows<T, 1, VPT, WC>(gr, C, gv);
        const float inv = 1.f / rms[b];
        float dot = 0.f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) dot += gv[0][k][e] * wv[k][e] * xv[0][k][e];
        }
        float v[1] = {dot};
        block_sum<1>(v, red);
        const float k2 = v[0] * inv * inv * inv / (float)C;
        float out[VPT][WC];
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                out[k][e] = wv[k][e] * gv[0][k][e] * inv - xv[0][k][e] * k2;
                dwacc[k][e] += gv[0][k][e] * xv[0][k][e] * inv;
            }
        }
        store_row1<T, VPT, WC, true>(gx + b * C, C, out);
    }
    store_row1<float, VPT, WC, false>(dw_part + (int64_t)blockIdx.x * C, C, dwacc);
}

// compute_rms (compute_rms.cpp:124; ops_pytorch_backward.py:65-75):
// rms[b] = sqrt(mean_k x[b,k]^2 + eps) over rows of K.
template <typename T, int VPT>
__global__ MHC_ROW_BOUNDS(false) void compute_rms_kernel(const T* __restrict__ x, float* __restrict__ rms, int K,
                                                         float eps) {
    constexpr int WC = VecIO<T>::W;
    __shared__ float red[8];
    const int64_t b = blockIdx.x;
    float xv[1][VPT][WC];
    load_rows<T, 1, VPT, WC, true>(x + b * K, K, xv);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
#pragma unroll
        for (int e = 0; e < WC; ++e) ss += xv[0][k][e] * xv[0][k][e];
    }
    float v[1] = {ss};
    block_sum<1>(v, red);
    if (threadIdx.x == 0) rms[b] = sqrtf(v[0] / (float)K + eps);
}

// ---------------------------------------------------------------------------
// stream_aggregate (ops_pytorch_backward.py:94-111; stream_ops.cpp:142-228,
// 700-816):  h = sigmoid(H), out = sum_i h_i x_i;
//   bwd: dx_i = g h_i, dh_act_i = sum_c g x_i, dH_i = dh_act_i h_i (1 - h_i)
// ---------------------------------------------------------------------------
// TPW tokens per workgroup as in aggregate_bwd_kernel (C2: 216-217 against
// 231-233 us with two).
template <typename T, int N, int VPT, int TPW>
__global__ MHC_ROW_BOUNDS(false) void aggregate_fwd_kernel(const T* __restrict__ x, const float* __restrict__ H,
                                                           int64_t h_stride, T* __restrict__ out,
                                                           float* __restrict__ h_act, int64_t B, int C) {
    constexpr int WC = VecIO<T>::W;
    const int64_t b0 = (int64_t)blockIdx.x * TPW;
    RawRows<T, N, VPT, WC> xr[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t)
        load_rows_raw_rs<T, N, VPT, WC, true>(token_rows_rsrc(x, b0 + t, B, N, C), C, xr[t]);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int64_t b = b0 + t;
        if (b >= B) break;  // the last workgroup's second token only
        float h[N];
#pragma unroll
        for (int i = 0; i < N; ++i) h[i] = sigmoidf(H[b * h_stride + i]);
        float xv[N][VPT][WC];
        unpack_rows<T, N, VPT, WC>(xr[t], C, xv);
        float o[VPT][WC];
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < N; ++i) s += h[i] * xv[i][k][e];
                o[k][e] = s;
            }
        }
        store_row1<T, VPT, WC, true>(out + b * C, C, o);
        if (threadIdx.x < N) h_act[b * N + threadIdx.x] = h[threadIdx.x];
    }
}

// TPW tokens per workgroup (1 or 2): with two, both tokens' rows are loaded
// up front, so the second token's loads run under the first one's sums,
// stores and barrier (C2 [16384, 4, 4096] fp32: 405-406 against 425-429 us).
// Rows go through buffer resources over one token each (token_rows_rsrc): a
// token past B reads zeros and stores nothing.
template <typename T, int N, int VPT, int TPW>
__global__ MHC_ROW_BOUNDS(false) void aggregate_bwd_kernel(const T* __restrict__ g, const T* __restrict__ x,
                                                           const float* __restrict__ h_act, int64_t h_stride,
                                                           T* __restrict__ gx, float* __restrict__ gh_act,
                                                           float* __restrict__ gh_raw, int64_t B, int C) {
    constexpr int WC = VecIO<T>::W;
    __shared__ float red[TPW][8 * N];
    const int64_t b0 = (int64_t)blockIdx.x * TPW;
    RawRows<T, 1, VPT, WC> gr[TPW];
    RawRows<T, N, VPT, WC> xr[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        load_rows_raw_rs<T, 1, VPT, WC, true>(token_rows_rsrc(g, b0 + t, B, 1, C), C, gr[t]);
        load_rows_raw_rs<T, N, VPT, WC, true>(token_rows_rsrc(x, b0 + t, B, N, C), C, xr[t]);
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int64_t b = b0 + t;
        if (b >= B) break;  // the last workgroup's second token only
        float h[N];
#pragma unroll
        for (int i = 0; i < N; ++i) h[i] = h_act[b * h_stride + i];
        float gv[1][VPT][WC], xv[N][VPT][WC];
        unpack_rows<T, 1, VPT, WC>(gr[t], C, gv);
        unpack_rows<T, N, VPT, WC>(xr[t], C, xv);
        float s[N];
#pragma unroll
        for (int i = 0; i < N; ++i) s[i] = 0.f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
#pragma unroll
                for (int i = 0; i < N; ++i) s[i] += gv[0][k][e] * xv[i][k][e];
            }
        }
        T* gb = gx + b * (int64_t)N * C;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            float d[VPT][WC];
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
#pragma unroll
                for (int e = 0; e < WC; ++e) d[k][e] = gv[0][k][e] * h[i];
            }
            store_row1<T, VPT, WC, true>(gb + (int64_t)i * C, C, d);
        }
        block_sum<N>(s, red[t]);
        if (threadIdx.x < N) {
            const int i = threadIdx.x;
            float si = 0.f, hi = 0.f;
#pragma unroll
            for (int q = 0; q < N; ++q) {
                si = (q == i) ? s[q] : si;
                hi = (q == i) ? h[q] : hi;
            }
            if (gh_act) gh_act[b * N + i] = si;
            if (gh_raw) gh_raw[b * N + i] = si * hi * (1.f - hi);
        }
    }
}

// ---------------------------------------------------------------------------
// stream_distribute_mix_add (ops_pytorch_backward.py:36-62; stream_ops.cpp
// 403-525, 960-1108):  h = 2 sigmoid(H), out_i = h_i y + sum_j M_ij x_j;
//   bwd: dx_j = sum_i M_ij g_i, dy = sum_i h_i g_i, dM_ij = sum_c g_i x_j,
//        dh_act_i = sum_c g_i y, dH_i = dh_act_i h_i (1 - h_i / 2)
// ---------------------------------------------------------------------------
template <typename T, int N, int VPT>
__global__ MHC_ROW_BOUNDS(false) void distribute_fwd_kernel(const T* __restrict__ y, const float* __restrict__ H,
                                                            int64_t h_stride, const float* __restrict__ M,
                                                            int64_t m_stride, const T* __restrict__ x,
                                                            float* __restrict__ out, float* __restrict__ h_act,
                                                            int C) {
    constexpr int WC = VecIO<T>::W;
    const int64_t b = blockIdx.x;
    float h[N], m[N * N];
#pragma unroll
    for (int i = 0; i < N; ++i) h[i] = 2.f * sigmoidf(H[b * h_stride + i]);
#pragma unroll
    for (int k = 0; k < N * N; ++k) m[k] = M[b * m_stride + k];
    RawRows<T, 1, VPT, WC> yr;
    RawRows<T, N, VPT, WC> xr;
    float yv[1][VPT][WC], xv[N][VPT][WC];
    load_rows_raw<T, 1, VPT, WC, true>(y + b * C, C, yr);
    load_rows_raw<T, N, VPT, WC, true>(x + b * (int64_t)N * C, C, xr);
    unpack_rows<T, 1, VPT, WC>(yr, C, yv);
    unpack_rows<T, N, VPT, WC>(xr, C, xv);
    float* ob = out + b * (int64_t)N * C;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        float o[VPT][WC];
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float s = h[i] * yv[0][k][e];
#pragma unroll
                for (int j = 0; j < N; ++j) s += m[i * N + j] * xv[j][k][e];
                o[k][e] = s;
            }
        }
        store_row1<float, VPT, WC, true>(ob + (int64_t)i * C, C, o);
    }
    if (threadIdx.x < N) {
        float hi = 0.f;
#pragma unroll
        for (int q = 0; q < N; ++q) hi = (q == (int)threadIdx.x) ? h[q] : hi;
        h_act[b * N + threadIdx.x] = hi;
    }
}

template <typename T, int N, int VPT>
__global__ MHC_ROW_BOUNDS(false) void distribute_bwd_kernel(
    const float* __restrict__ g, const T* __restrict__ x, const T* __restrict__ y, const float* __restrict__ M,
    int64_t m_stride, const float* __restrict__ h_act, int64_t h_stride, T* __restrict__ gx, T* __restrict__ gy,
    float* __restrict__ gM, float* __restrict__ gh_act, float* __restrict__ gh_raw, int C) {
    constexpr int WC = VecIO<T>::W;
    constexpr int NR = N * N + N;
    __shared__ float red[8 * NR];
    const int64_t b = blockIdx.x;
    float h[N], m[N * N];
#pragma unroll
    for (int i = 0; i < N; ++i) h[i] = h_act[b * h_stride + i];
#pragma unroll
    for (int k = 0; k < N * N; ++k) m[k] = M[b * m_stride + k];
    RawRows<float, N, VPT, WC> gr;
    RawRows<T, N, VPT, WC> xr;
    RawRows<T, 1, VPT, WC> yr;
    float gv[N][VPT][WC], xv[N][VPT][WC], yv[1][VPT][WC];
    load_rows_raw<float, N, VPT, WC, true>(g + b * (int64_t)N * C, C, gr);
    load_rows_raw<T, N, VPT, WC, true>(x + b * (int64_t)N * C, C, xr);
    load_rows_raw<T, 1, VPT, WC, true>(y + b * C, C, yr);
    unpack_rows<float, N, VPT, WC>(gr, C, gv);
    unpack_rows<T, N, VPT, WC>(xr, C, xv);
    unpack_rows<T, 1, VPT, WC>(yr, C, yv);
    float s[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) s[k] = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
#pragma unroll
        for (int e = 0; e < WC; ++e) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
#pragma unroll
                for (int j = 0; j < N; ++j) s[i * N + j] += gv[i][k][e] * xv[j][k][e];
                s[N * N + i] += gv[i][k][e] * yv[0][k][e];
            }
        }
    }
    T* gb = gx + b * (int64_t)N * C;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        float d[VPT][WC];
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float t = 0.f;
#pragma unroll
                for (int i = 0; i < N; ++i) t += m[i * N + j] * gv[i][k][e];
                d[k][e] = t;
            }
        }
        store_row1<T, VPT, WC, true>(gb + (int64_t)j * C, C, d);
    }
    {
        float d[VPT][WC];
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float t = 0.f;
#pragma unroll
                for (int i = 0; i < N; ++i) t += h[i] * gv[i][k][e];
                d[k][e] = t;
            }
        }
        store_row1<T, VPT, WC, true>(gy + b * C, C, d);
    }
    block_sum<NR>(s, red);
    if (threadIdx.x < NR) {
        const int t = threadIdx.x;
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < NR; ++q) v = (q == t) ? s[q] : v;
        if (t < N * N) {
            gM[b * N * N + t] = v;
        } else {
            const int i = t - N * N;
            float hi = 0.f;
#pragma unroll
            for (int q = 0; q < N; ++q) hi = (q == i) ? h[q] : hi;
            if (gh_act) gh_act[b * N + i] = v;
            if (gh_raw) gh_raw[b * N + i] = v * hi * (1.f - 0.5f * hi);
        }
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#define MHC_OPS_VPT(v, ARR, TX_, ...)                                                          \
    switch (v) {                                                                              \
        case 1: { constexpr int V_ = 1; if constexpr (row_fits<TX_>(ARR, 1)) { __VA_ARGS__; } else { return hipErrorInvalidValue; } break; } \
        case 2: { constexpr int V_ = 2; if constexpr (row_fits<TX_>(ARR, 2)) { __VA_ARGS__; } else { return hipErrorInvalidValue; } break; } \
        case 4: { constexpr int V_ = 4; if constexpr (row_fits<TX_>(ARR, 4)) { __VA_ARGS__; } else { return hipErrorInvalidValue; } break; } \
        case 8: { constexpr int V_ = 8; if constexpr (row_fits<TX_>(ARR, 8)) { __VA_ARGS__; } else { return hipErrorInvalidValue; } break; } \
        default: return hipErrorInvalidValue;                                                 \
    }

#define MHC_OPS_T(dt, ...)                                        \
    if (dt == kBF16) {                                            \
        using T_ = bf16_t;                                        \
        __VA_ARGS__;                                              \
    } else {                                                      \
        using T_ = float;                                         \
        __VA_ARGS__;                                              \
    }

hipError_t launch_rmsnorm_fwd(int dt, const void* x, const float* w, void* y, float* rms, int64_t B, int64_t C,
                              float eps, hipStream_t s) {
    if (B == 0) return hipSuccess;
    const RowTiling t = choose_row_tiling(C, dt == kBF16 ? 8 : 4, 1, 512);
    const int tok = timing_begin("rmsnorm_fwd", s);
    if (t.vpt <= 0) {
        // rows that are not a multiple of the vector (or too wide): channel loop
        const hipError_t e = launch_wide_rmsnorm_fwd(dt, x, w, y, rms, B, C, eps, s);
        timing_end(tok, s);
        return e;
    }
    MHC_OPS_T(dt, MHC_OPS_VPT(t.vpt, 1, T_, MHC_LAUNCH_GGL((rmsnorm_fwd_kernel<T_, V_>), dim3(B), dim3(t.threads),
                                                               0, s, (const T_*)x, w, (T_*)y, rms, (int)C, eps)));
    timing_end(tok, s);
    return hipGetLastError();
}

int rmsnorm_bwd_grid(int dt, int64_t B, int64_t C) {
    const RowTiling t = choose_row_tiling(C, dt == kBF16 ? 8 : 4, 2, 512);
    if (t.vpt <= 0) return wide_rmsnorm_bwd_grid(dt, B, C);
    int64_t g = (int64_t)device_cu_count() * ((t.threads <= 256) ? 4 : 2);
    if (g > B) g = B;
    return g < 1 ? 1 : (int)g;
}

hipError_t launch_rmsnorm_bwd(int dt, const void* g, const void* x, const float* w, const float* rms, void* gx,
                              float* dw_part, int grid, int64_t B, int64_t C, hipStream_t s) {
    const RowTiling t = choose_row_tiling(C, dt == kBF16 ? 8 : 4, 2, 512);
    const int tok = timing_begin("rmsnorm_bwd", s);
    if (t.vpt <= 0) {
        const hipError_t e = launch_wide_rmsnorm_bwd(dt, g, x, w, rms, gx, dw_part, grid, B, C, s);
        timing_end(tok, s);
        return e;
    }
    MHC_OPS_T(dt, MHC_OPS_VPT(t.vpt, 2, T_, MHC_LAUNCH_GGL((rmsnorm_bwd_kernel<T_, V_>), dim3(grid),
                                                               dim3(t.threads), 0, s, (const T_*)g, (const T_*)x, w,
                                                               rms, (T_*)gx, dw_part, B, (int)C)));
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_compute_rms(int dt, const void* x, float* rms, int64_t B, int64_t K, float eps, hipStream_t s) {
    if (B == 0) return hipSuccess;
    const RowTiling t = choose_row_tiling(K, dt == kBF16 ? 8 : 4, 1);
    if (t.vpt <= 0) return launch_wide_compute_rms(dt, x, rms, B, K, eps, s);
    MHC_OPS_T(dt, MHC_OPS_VPT(t.vpt, 1, T_, MHC_LAUNCH_GGL((compute_rms_kernel<T_, V_>), dim3(B),
                                                               dim3(t.threads), 0, s, (const T_*)x, rms, (int)K,
                                                               eps)));
    return hipGetLastError();
}

#define MHC_OPS_N(n, ...)                                        \
    switch (n) {                                                 \
        case 1: { constexpr int N_ = 1; __VA_ARGS__; break; }    \
        case 2: { constexpr int N_ = 2; __VA_ARGS__; break; }    \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }    \
        case 8: { constexpr int N_ = 8; __VA_ARGS__; break; }    \
        default: return hipErrorInvalidValue;                    \
    }

hipError_t launch_aggregate_fwd(int dt, int n, const void* x, const float* H, int64_t hs, void* out, float* h_act,
                                int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (generic_ops_n(n)) {
        const int tok = timing_begin("aggregate_fwd", s);
        const hipError_t e = launch_gen_aggregate_fwd(dt, n, x, H, hs, out, h_act, B, C, s);
        timing_end(tok, s);
        return e;
    }
    const RowTiling t = n > 8 ? RowTiling{0, 0} : choose_row_tiling(C, dt == kBF16 ? 8 : 4, n + 1, 512);
    const int tok = timing_begin("aggregate_fwd", s);
    if (t.vpt <= 0) {
        const hipError_t e = launch_wide_aggregate_fwd(dt, n, x, H, hs, out, h_act, B, C, s);
        timing_end(tok, s);
        return e;
    }
#define MHC_AGG_FWD(TPW_)                                                                               \
    MHC_LAUNCH_GGL((aggregate_fwd_kernel<T_, N_, V_, TPW_>), dim3((unsigned)((B + TPW_ - 1) / TPW_)),  \
                   dim3(t.threads), 0, s, (const T_*)x, H, hs, (T_*)out, h_act, B, (int)C)
    MHC_OPS_T(dt, MHC_OPS_N(n, MHC_OPS_VPT(t.vpt, N_ + 1, T_, {
        if constexpr (row_fits<T_>(2 * (N_ + 1), V_)) {
            MHC_AGG_FWD(2);
        } else {
            MHC_AGG_FWD(1);
        }
    })));
#undef MHC_AGG_FWD
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_aggregate_bwd(int dt, int n, const void* g, const void* x, const float* h_act, int64_t hs,
                                void* gx, float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (generic_ops_n(n)) {
        const int tok = timing_begin("aggregate_bwd", s);
        const hipError_t e = launch_gen_aggregate_bwd(dt, n, g, x, h_act, hs, gx, gh_act, gh_raw, B, C, s);
        timing_end(tok, s);
        return e;
    }
    const RowTiling t = n > 8 ? RowTiling{0, 0} : choose_row_tiling(C, dt == kBF16 ? 8 : 4, n + 1, 512);
    const int tok = timing_begin("aggregate_bwd", s);
    if (t.vpt <= 0) {
        const hipError_t e = launch_wide_aggregate_bwd(dt, n, g, x, h_act, hs, gx, gh_act, gh_raw, B, C, s);
        timing_end(tok, s);
        return e;
    }
    // two tokens per workgroup where both tokens' rows fit the row budget
#define MHC_AGG_BWD(TPW_)                                                                                   \
    MHC_LAUNCH_GGL((aggregate_bwd_kernel<T_, N_, V_, TPW_>), dim3((unsigned)((B + TPW_ - 1) / TPW_)),      \
                   dim3(t.threads), 0, s, (const T_*)g, (const T_*)x, h_act, hs, (T_*)gx, gh_act, gh_raw, B, \
                   (int)C)
    MHC_OPS_T(dt, MHC_OPS_N(n, MHC_OPS_VPT(t.vpt, N_ + 1, T_, {
        if constexpr (row_fits<T_>(2 * (N_ + 1), V_)) {
            MHC_AGG_BWD(2);
        } else {
            MHC_AGG_BWD(1);
        }
    })));
#undef MHC_AGG_BWD
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_distribute_fwd(int dt, int n, const void* y, const float* H, int64_t hs, const float* M,
                                 int64_t ms, const void* x, float* out, float* h_act, int64_t B, int64_t C,
                                 hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (generic_ops_n(n)) return launch_gen_distribute_fwd(dt, n, y, H, hs, M, ms, x, out, h_act, B, C, s);
    const RowTiling t = n > 8 ? RowTiling{0, 0} : choose_row_tiling(C, dt == kBF16 ? 8 : 4, n + 1, 512);
    const int tok = timing_begin("distribute_fwd", s);
    if (t.vpt <= 0) {
        const hipError_t e = launch_wide_distribute_fwd(dt, n, y, H, hs, M, ms, x, out, h_act, B, C, s);
        timing_end(tok, s);
        return e;
    }
    MHC_OPS_T(dt, MHC_OPS_N(n, MHC_OPS_VPT(t.vpt, N_ + 1, T_, MHC_LAUNCH_GGL((distribute_fwd_kernel<T_, N_, V_>),
                                                                                 dim3(B), dim3(t.threads), 0, s,
                                                                                 (const T_*)y, H, hs, M, ms,
                                                                                 (const T_*)x, out, h_act, (int)C))));
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_distribute_bwd(int dt, int n, const float* g, const void* x, const void* y, const float* M,
                                 int64_t ms, const float* h_act, int64_t hs, void* gx, void* gy, float* gM,
                                 float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (generic_ops_n(n))
        return launch_gen_distribute_bwd(dt, n, g, x, y, M, ms, h_act, hs, gx, gy, gM, gh_act, gh_raw, B, C, s);
    // the block hands one of the n*n + n row sums to each thread
    const RowTiling t =
        n > 8 ? RowTiling{0, 0} : with_min_threads(choose_row_tiling(C, dt == kBF16 ? 8 : 4, 2 * n + 1), n * n + n);
    const int tok = timing_begin("distribute_bwd", s);
    if (t.vpt <= 0) {
        const hipError_t e =
            launch_wide_distribute_bwd(dt, n, g, x, y, M, ms, h_act, hs, gx, gy, gM, gh_act, gh_raw, B, C, s);
        timing_end(tok, s);
        return e;
    }
    MHC_OPS_T(dt, MHC_OPS_N(n, MHC_OPS_VPT(t.vpt, 2 * N_ + 1, T_,
                                           MHC_LAUNCH_GGL((distribute_bwd_kernel<T_, N_, V_>), dim3(B),
                                                              dim3(t.threads), 0, s, g, (const T_*)x, (const T_*)y, M,
                                                              ms, h_act, hs, (T_*)gx, (T_*)gy, gM, gh_act, gh_raw,
                                                              (int)C))));
    timing_end(tok, s);
    return hipGetLastError();
}

}  // namespace mhc

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
#include "mhc_rows.h"

namespace mhc {

template <int N> constexpr int coef_size() { return 2 * N + N * N; }

// ---------------------------------------------------------------------------
// Static coefficients: h_pre = sigmoid(H_pre), h_post = 2 sigmoid(H_post),
// M = SK(exp(H_res)) (layer.py:144-160), computed once per call, plus the
// RMSNorm weight converted to fp32.  saved = [coef (2n+n^2) | pad | w32 (C)]
// with w32 at saved_w_offset(n) floats.
// ---------------------------------------------------------------------------
template <int N, typename TW>
__global__ __launch_bounds__(256) void static_coef_kernel(const float* __restrict__ h_pre,
                                                          const float* __restrict__ h_post,
                                                          const float* __restrict__ h_res,
                                                          const TW* __restrict__ weight, int C,
                                                          float* __restrict__ saved, int w_off, int iters,
                                                          float eps) {
    if (blockIdx.x > 0) {
        // weight -> fp32, 8 elements per lane, one pass
        const int c0 = ((blockIdx.x - 1) * blockDim.x + threadIdx.x) * 8;
        if (c0 + 8 <= C) {
            float v[8];
            load_run<TW, 8>(weight + c0, v);
            store_run<float, 8>(saved + w_off + c0, v);
        } else {
            for (int c = c0; c < C; ++c) saved[w_off + c] = VecIO<TW>::scalar(weight + c);
        }
        return;
    }
    const int r = threadIdx.x;
    if (r < N) {
        saved[r] = sigmoidf(h_pre[r]);
        saved[N + r] = 2.f * sigmoidf(h_post[r]);
    }
    if constexpr (N == skb::kN) {
        // the whole workgroup on the one 32 x 32 matrix (the finalize's
        // adjoint recomputes it with the same code)
        __shared__ float part[skb::kPartFloats];
        const int i = skb::row(), c0 = skb::col0();
        float a[skb::kV];
#pragma unroll
        for (int k = 0; k < skb::kV; ++k) a[k] = expf(h_res[i * N + c0 + k]);
        skb::forward(a, iters, eps, part);
#pragma unroll
        for (int k = 0; k < skb::kV; ++k) saved[2 * N + i * N + c0 + k] = a[k];
        return;
    }
    if (r >= kWave) return;
    if constexpr (N == 4) {
        // the shared M = SK(exp(H_res)): one element per lane of lanes 0..15
        // (the finalize's adjoint recomputes it with the same code)
        float a = r < 16 ? expf(h_res[r]) : 0.f;
        sk16_forward(a, iters, eps);
        if (r < 16) saved[2 * N + r] = a;
    } else if constexpr (N == skw16::kN) {
        // the 16 x 16 matrix on wave 0, four elements per lane (the
        // finalize's adjoint recomputes it with the same code)
        const int i = skw16::row(), c0 = skw16::col0();
        float a[skw16::kV];
#pragma unroll
        for (int k = 0; k < skw16::kV; ++k) a[k] = expf(h_res[i * N + c0 + k]);
        skw16::forward(a, iters, eps);
#pragma unroll
        for (int k = 0; k < skw16::kV; ++k) saved[2 * N + i * N + c0 + k] = a[k];
    } else {
        float a[N];
#pragma unroll
        for (int c = 0; c < N; ++c) a[c] = (r < N) ? expf(h_res[r * N + c]) : 0.f;
        sk_forward<N>(a, iters, eps, r < N);
        if (r < N) {
#pragma unroll
            for (int c = 0; c < N; ++c) saved[2 * N + r * N + c] = a[c];
        }
    }
}

// ---------------------------------------------------------------------------
// Fused forward, one token per workgroup (grid = tokens): the row loads of
// the next workgroups on a CU overlap this one's reduction and stores, which
// measured faster than persistent workgroups with a register prefetch for
// this pass (C4 bf16 147 -> 136 us; fp32 equal).
// ---------------------------------------------------------------------------
template <typename TX, typename TO, int N, int VPT>
__device__ __forceinline__ void fwd_token(int64_t b, const float* __restrict__ coef, int64_t coef_stride,
                                          const float (&wv)[VPT][kLayerWC],
                                          const float (&xv)[N][VPT][kLayerWC], TO* __restrict__ out,
                                          float* __restrict__ rms_out, int C, float eps, float* red) {
    constexpr int WC = kLayerWC;
    constexpr int NC = coef_size<N>();
    const float* cf = coef + b * coef_stride;
    float cfv[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) cfv[k] = cf[k];
    float xa[VPT][WC];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
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
    // stores through a resource over the token's output rows, out-of-range
    // offsets past the row end (no store behind a branch)
    const buf_rsrc_t ors = make_buf_rsrc(out + b * (int64_t)N * C, (uint32_t)((int64_t)N * C * (int64_t)sizeof(TO)));
    static_assert(WC == 4, "4-channel chunks: one 16-byte (fp32) or 8-byte (bf16) store");
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        const uint32_t o0 = c0 < C ? (uint32_t)c0 * (uint32_t)sizeof(TO) : kBufOff;
        float y[WC];
#pragma unroll
        for (int e = 0; e < WC; ++e) y[e] = xa[k][e] * inv * wv[k][e];
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
            const uint32_t off = o0 + (uint32_t)(i * C * (int)sizeof(TO));
            if constexpr (sizeof(TO) == 4) {
                buf_st16<true>(ors, off, 0u, make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]),
                                                        __float_as_uint(o[2]), __float_as_uint(o[3])));
            } else {
                buf_st8<true>(ors, off, 0u, make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])));
            }
        }
    }
    if (rms_out) {
        const buf_rsrc_t rrs = make_buf_rsrc(rms_out + b, 4u);
        buf_st4(rrs, threadIdx.x == 0 ? 0u : kBufOff, 0u, r);
    }
}

template <typename TX, typename TO, int N, int VPT>
__global__ MHC_ROW_BOUNDS(false) void layer_fwd_kernel(const TX* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ coef, int64_t coef_stride,
                                                       TO* __restrict__ out, float* __restrict__ rms_out, int64_t B,
                                                       int C, float eps) {
    constexpr int WC = kLayerWC;
    __shared__ float red[8];
    const int64_t b = blockIdx.x;
    if (b >= B) return;
    RawRows<TX, N, VPT, WC> xr;
    load_rows_raw<TX, N, VPT, WC, true>(x + b * (int64_t)N * C, C, xr);
    float wv[VPT][WC];
    load_weight<VPT, WC>(w, C, wv);
    float xv[N][VPT][WC];
    unpack_rows<TX, N, VPT, WC>(xr, C, xv);
    fwd_token<TX, TO, N, VPT>(b, coef, coef_stride, wv, xv, out, rms_out, C, eps, red);
}

// ---------------------------------------------------------------------------
// Static forward in ONE launch: every workgroup forms the shared coefficients
// h_pre = sigmoid(H_pre), h_post = 2 sigmoid(H_post), M = SK(exp(H_res)) in
// its first wave (the same code as static_coef_kernel, so every workgroup
// gets identical values) while its row loads are in flight, and reads the
// RMSNorm weight in its own dtype.  Workgroup 0 also writes the backward's
// saved state ([coef | pad | w32]).  One launch instead of two (n <= 8).
// ---------------------------------------------------------------------------
// Lanes of the first wave; each value goes to cf (LDS) and, when `save` is
// not null, to the saved state.
template <int N>
__device__ __forceinline__ void static_coefs_wave(const float* __restrict__ h_pre, const float* __restrict__ h_post,
                                                  const float* __restrict__ h_res, int iters, float eps,
                                                  float* __restrict__ cf, float* __restrict__ save) {
    const int r = threadIdx.x;
    auto put = [&](int i, float v) {
        cf[i] = v;
        if (save) save[i] = v;
    };
    if (r < N) {
        put(r, sigmoidf(h_pre[r]));
        put(N + r, 2.f * sigmoidf(h_post[r]));
    }
    if constexpr (N == 4) {
        float a = r < 16 ? expf(h_res[r]) : 0.f;
        sk16_forward(a, iters, eps);
        if (r < 16) put(2 * N + r, a);
    } else {
        float a[N];
#pragma unroll
        for (int c = 0; c < N; ++c) a[c] = (r < N) ? expf(h_res[r * N + c]) : 0.f;
        sk_forward<N>(a, iters, eps, r < N);
        if (r < N) {
#pragma unroll
            for (int c = 0; c < N; ++c) put(2 * N + r * N + c, a[c]);
        }
    }
}

template <typename TX, typename TW, int N, int VPT>
__global__ MHC_ROW_BOUNDS(false) void layer_static_fwd_kernel(const TX* __restrict__ x, const TW* __restrict__ weight,
                                                              const float* __restrict__ h_pre,
                                                              const float* __restrict__ h_post,
                                                              const float* __restrict__ h_res,
                                                              float* __restrict__ saved, int w_off, int iters,
                                                              float sk_eps, float* __restrict__ out,
                                                              float* __restrict__ rms_out, int64_t B, int C,
                                                              float eps) {
    (void)B;  // the grid is one workgroup per token
    constexpr int WC = kLayerWC;
    constexpr int NC = coef_size<N>();
    __shared__ float red[8];
    __shared__ float cf[NC];
    const int64_t b = blockIdx.x;
    RawRows<TX, N, VPT, WC> xr;
    load_rows_raw<TX, N, VPT, WC, true>(x + b * (int64_t)N * C, C, xr);
    if (threadIdx.x < kWave) static_coefs_wave<N>(h_pre, h_post, h_res, iters, sk_eps, cf, b == 0 ? saved : nullptr);
    float wv[VPT][WC];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
#pragma unroll
        for (int e = 0; e < WC; ++e) wv[k][e] = c0 < C ? VecIO<TW>::scalar(weight + c0 + e) : 0.f;
        if (b == 0 && c0 < C) store_run<float, WC>(saved + w_off + c0, wv[k]);
    }
    __syncthreads();
    float xv[N][VPT][WC];
    unpack_rows<TX, N, VPT, WC>(xr, C, xv);
    fwd_token<TX, float, N, VPT>(b, cf, 0, wv, xv, out, rms_out, C, eps, red);
}

// ---------------------------------------------------------------------------
// Fused backward.  Persistent workgroups stride over tokens (optionally with
// the two-buffer prefetch of the forward).  Per token the block forms
// (dM[n*n], dh_post_act[n], dh_pre_act[n], 1/r, k2 = dot/(C r^3)).  MODE 0
// (static H) writes dx and sums the first n*n+2n of those over its tokens
// (thread t keeps entry t in one register) into scal_out[blockIdx.x][n*n+2n];
// MODE 1 (dynamic H) writes them per token to scal_out[b][n*n+2n+2]; its dx
// holds the stream terms only (sum_i M_ij G_i + h_pre_j gxa), and a later
// kernel adds the terms that need the per-token Sinkhorn backward first (the
// projection and r_h terms).  dw accumulates in registers and goes to
// dw_part[blockIdx.x][C].
// ---------------------------------------------------------------------------
template <typename TX, int N, int VPT, int MODE>
__device__ __forceinline__ void bwd_token(int64_t b, const float* __restrict__ coef, int64_t coef_stride,
                                          const float (&wv)[VPT][kLayerWC],
                                          const float (&xv)[N][VPT][kLayerWC],
                                          const float (&gv)[N][VPT][kLayerWC],
                                          float (&dwacc)[VPT][kLayerWC], float& sacc, TX* __restrict__ dx,
                                          float* __restrict__ scal_out, int32_t* __restrict__ dx_scale, int C,
                                          float eps, float* red) {
    constexpr int WC = kLayerWC;
    constexpr int NC = coef_size<N>();
    constexpr int NS = N * N + 2 * N;
    constexpr int NR = 2 + N * N + 3 * N;  // ss, dot, dM, t_i, u_j, v_j
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    float* tot = red + 8 * NR;
    const float* cf = coef + b * coef_stride;
    float cfv[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) cfv[k] = cf[k];
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
        wave_sum_last<NR>(rv);
        if (lane == kWave - 1) {
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

    // Global stores of this routine go through resources with out-of-range
    // offsets for lanes that store nothing: no store sits behind a branch
    // (the caller's prefetch of the next token keeps exact wait counts).
    float v = 0.f;
    if (threadIdx.x < NS + 2) {
        const int t = threadIdx.x;
        if (t < N * N) {
            v = tot[2 + t];
        } else if (t < N * N + N) {
            v = tot[2 + t] * inv;  // dh_post_act = (sum G_i xa w) / r
        } else if (t < NS) {
            const int j = t - N * N - N;
            v = inv * tot[2 + N * N + N + j] - k2 * tot[2 + N * N + 2 * N + j];  // dh_pre_act
        } else {
            v = (t == NS) ? inv : k2;
        }
        if (MODE == 0) sacc += v;
    }
    if constexpr (MODE != 0) {
        const buf_rsrc_t srs = make_buf_rsrc(scal_out + b * (NS + 2), (uint32_t)((NS + 2) * 4));
        buf_st4(srs, threadIdx.x < NS + 2 ? (uint32_t)threadIdx.x * 4u : kBufOff, 0u, v);
    }

    if constexpr (MODE == 1 && sizeof(TX) == 2) {
        // The dynamic backward's stream part with bf16 x: the projection
        // kernel adds its terms and rounds the sum once, so this part travels
        // as fp16 against a power-of-two scale (part_pack4), one scale
        // exponent per half wave of this token: dx_scale[b][threadIdx.x / 32].
        float a[N][VPT][WC];
        float m = 0.f;  // largest |value|: fmaxf drops NaN, keeps +Inf
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
                const float gxa = wv[k][e] * gy * inv - xa * k2;
                dwacc[k][e] += gy * xa * inv;
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    float s = cfv[j] * gxa;
#pragma unroll
                    for (int i = 0; i < N; ++i) s += cfv[2 * N + i * N + j] * gv[i][k][e];
                    a[j][k][e] = s;
                    m = fmaxf(m, fabsf(s));
                }
            }
        }
        m = half_wave_max_nonneg(m);
        if (__ballot(!(m < INFINITY))) {
            // an infinite value in this wave: the scale comes from the finite
            // values only (the whole wave takes this branch)
            m = 0.f;
#pragma unroll
            for (int k = 0; k < VPT; ++k)
#pragma unroll
                for (int e = 0; e < WC; ++e)
#pragma unroll
                    for (int j = 0; j < N; ++j) {
                        const float v = fabsf(a[j][k][e]);
                        m = v < INFINITY ? fmaxf(m, v) : m;
                    }
            m = half_wave_max_nonneg(m);
        }
        const int ks = part_scale_exp(m);
        const buf_rsrc_t drs = make_buf_rsrc(dx + b * (int64_t)N * C, (uint32_t)((int64_t)N * C * 2));
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int c0 = (k * blockDim.x + threadIdx.x) * WC;
            const uint32_t o0 = c0 < C ? (uint32_t)c0 * 2u : kBufOff;
#pragma unroll
            for (int j = 0; j < N; ++j) buf_st8<true>(drs, o0 + (uint32_t)(j * C * 2), 0u, part_pack4(a[j][k], ks));
        }
        const int ng = blockDim.x / 32;
        const buf_rsrc_t qrs = make_buf_rsrc(dx_scale + b * ng, (uint32_t)(ng * 4));
        buf_st4(qrs, (threadIdx.x & 31) == 0 ? (uint32_t)(threadIdx.x / 32) * 4u : kBufOff, 0u, __int_as_float(ks));
    } else {
        const buf_rsrc_t drs = make_buf_rsrc(dx + b * (int64_t)N * C, (uint32_t)((int64_t)N * C * (int64_t)sizeof(TX)));
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
            const uint32_t o0 = c0 < C ? (uint32_t)c0 * (uint32_t)sizeof(TX) : kBufOff;
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
                const uint32_t o = o0 + (uint32_t)(j * C * (int)sizeof(TX));
                static_assert(WC == 4, "4-channel chunks: one 16-byte (fp32) or 8-byte (bf16) store");
                if constexpr (sizeof(TX) == 4) {
                    buf_st16<true>(drs, o, 0u, make_uint4(__float_as_uint(d[0]), __float_as_uint(d[1]),
                                                          __float_as_uint(d[2]), __float_as_uint(d[3])));
                } else {
                    buf_st8<true>(drs, o, 0u, make_uint2(pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3])));
                }
            }
        }
    }
}

template <typename TX, int N, int VPT, int MODE, bool PF>
__global__ MHC_ROW_BOUNDS(PF) void layer_bwd_kernel(const float* __restrict__ g, const TX* __restrict__ x,
                                                    const float* __restrict__ w, const float* __restrict__ coef,
                                                    int64_t coef_stride, TX* __restrict__ dx,
                                                    float* __restrict__ dw_part, float* __restrict__ scal_out,
                                                    int32_t* __restrict__ dx_scale, int64_t B, int C, float eps) {
    constexpr int WC = kLayerWC;
    constexpr int NS = N * N + 2 * N;
    constexpr int NR = 2 + N * N + 3 * N;
    __shared__ float red[9 * NR];  // 8 wave partials + totals
    float wv[VPT][WC];
    load_weight<VPT, WC>(w, C, wv);
    float dwacc[VPT][WC];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
#pragma unroll
        for (int e = 0; e < WC; ++e) dwacc[k][e] = 0.f;
    }
    float sacc = 0.f;
    const int64_t G = gridDim.x;
    const int64_t NCs = (int64_t)N * C;
    int64_t b = blockIdx.x;
    if constexpr (PF) {
        // token rows stay raw (unconverted words) until their token is processed
        RawRows<TX, N, VPT, WC> xA, xB;
        RawRows<float, N, VPT, WC> gA, gB;
        float xv[N][VPT][WC], gv[N][VPT][WC];
        // every row load goes through a per-token resource (0 bytes past the
        // last token), so the prefetch is unconditional
        load_rows_raw_rs<TX, N, VPT, WC, true>(token_rows_rsrc(x, b, B, N, C), C, xA);
        load_rows_raw_rs<float, N, VPT, WC, true>(token_rows_rsrc(g, b, B, N, C), C, gA);
        while (b < B) {
            const int64_t b1 = b + G;
            load_rows_raw_rs<TX, N, VPT, WC, true>(token_rows_rsrc(x, b1, B, N, C), C, xB);
            load_rows_raw_rs<float, N, VPT, WC, true>(token_rows_rsrc(g, b1, B, N, C), C, gB);
            unpack_rows<TX, N, VPT, WC>(xA, C, xv);
            unpack_rows<float, N, VPT, WC>(gA, C, gv);
            bwd_token<TX, N, VPT, MODE>(b, coef, coef_stride, wv, xv, gv, dwacc, sacc, dx, scal_out, dx_scale, C, eps,
                                       red);
            if (b1 >= B) break;
            const int64_t b2 = b1 + G;
            load_rows_raw_rs<TX, N, VPT, WC, true>(token_rows_rsrc(x, b2, B, N, C), C, xA);
            load_rows_raw_rs<float, N, VPT, WC, true>(token_rows_rsrc(g, b2, B, N, C), C, gA);
            unpack_rows<TX, N, VPT, WC>(xB, C, xv);
            unpack_rows<float, N, VPT, WC>(gB, C, gv);
            bwd_token<TX, N, VPT, MODE>(b1, coef, coef_stride, wv, xv, gv, dwacc, sacc, dx, scal_out, dx_scale, C, eps,
                                       red);
            b = b2;
        }
    } else {
        for (; b < B; b += G) {
            RawRows<TX, N, VPT, WC> xr;
            RawRows<float, N, VPT, WC> gr;
            float xv[N][VPT][WC], gv[N][VPT][WC];
            load_rows_raw<TX, N, VPT, WC, true>(x + b * NCs, C, xr);
            load_rows_raw<float, N, VPT, WC, true>(g + b * NCs, C, gr);
            unpack_rows<TX, N, VPT, WC>(xr, C, xv);
            unpack_rows<float, N, VPT, WC>(gr, C, gv);
            bwd_token<TX, N, VPT, MODE>(b, coef, coef_stride, wv, xv, gv, dwacc, sacc, dx, scal_out, dx_scale, C, eps,
                                       red);
        }
    }

    float* dwp = dw_part + (int64_t)blockIdx.x * C;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) store_run<float, WC>(dwp + c0, dwacc[k]);
    }
    if (MODE == 0 && threadIdx.x < NS) scal_out[(int64_t)blockIdx.x * NS + threadIdx.x] = sacc;
}

// Several deterministic column sums in one launch (ColSumJob in
// mhc_internal.h): each job takes its own run of workgroups and sums as
// layer_finalize_kernel's column blocks do (`phases` row phases of
// 256 / phases columns, each phase over every phases-th row in order, the
// phases added in order); columns below `split` go to `out` (fp32 or bf16),
// the rest to `out2` (fp32).
__global__ __launch_bounds__(256) void multi_column_sum_kernel(ColSumJobs jobs) {
    __shared__ float cred[256];
    int bid = (int)blockIdx.x;
    int q = 0;
    while (q + 1 < jobs.count && bid >= jobs.j[q].blocks) {
        bid -= jobs.j[q].blocks;
        ++q;
    }
    const ColSumJob jb = jobs.j[q];
    const int phases = jb.phases;
    const int cpb = 256 / phases;
    const int cl = threadIdx.x % cpb;
    const int ph = threadIdx.x / cpb;
    const int64_t c = (int64_t)bid * cpb + cl;
    const float* part = jb.part;
    const int64_t cols = jb.cols;
    float s = 0.f;
    if (c < cols) {
        int r = ph;
        for (; r + 7 * phases < jb.rows; r += 8 * phases) {
            float a[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) a[u] = part[(int64_t)(r + u * phases) * cols + c];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += a[u];
        }
        for (; r < jb.rows; r += phases) s += part[(int64_t)r * cols + c];
    }
    float t = s;
    if (phases > 1) {
        cred[threadIdx.x] = s;
        __syncthreads();
        t = 0.f;
        for (int k = 0; k < phases; ++k) t += cred[k * cpb + cl];
    }
    if (ph == 0 && c < cols) {
        if (c < jb.split) {
            if (jb.out_bf16) static_cast<bf16_t*>(jb.out)[c] = f32_to_bf16(t);
            else static_cast<float*>(jb.out)[c] = t;
        } else {
            jb.out2[c - jb.split] = t;
        }
    }
}

// ---------------------------------------------------------------------------
// Deterministic column sums of per-workgroup partials part[rows][cols]:
// stage 1 (grid = col tiles of 256 x rsplit row groups) writes
// stage[rsplit][cols]; the finalize kernel sums the rsplit rows.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void column_partial_kernel(const float* __restrict__ part, int rows,
                                                             int64_t cols, float* __restrict__ stage) {
    __shared__ float4 red[4][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * 256 + lane * 4;
    const int r0 = (int)((int64_t)rows * blockIdx.y / gridDim.y);
    const int r1 = (int)((int64_t)rows * (blockIdx.y + 1) / gridDim.y);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c < cols) {
        int r = r0 + wave;
        // 8 independent loads in flight per step; fixed summation order
        for (; r + 28 < r1; r += 32) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const float4*>(part + (int64_t)(r + 4 * u) * cols + c);
#pragma unroll
            for (int u = 0; u < 8; ++u) { s.x += v[u].x; s.y += v[u].y; s.z += v[u].z; s.w += v[u].w; }
        }
        for (; r < r1; r += 4) {
            const float4 v = *reinterpret_cast<const float4*>(part + (int64_t)r * cols + c);
            s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
        }
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < cols) {
        float4 t = red[0][lane];
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            t.x += red[q][lane].x; t.y += red[q][lane].y; t.z += red[q][lane].z; t.w += red[q][lane].w;
        }
        *reinterpret_cast<float4*>(stage + (int64_t)blockIdx.y * cols + c) = t;
    }
}

// Same sums with one column per lane, for column counts that are not a
// multiple of 4 (rows are then not 16-byte aligned).
__global__ __launch_bounds__(256) void column_partial1_kernel(const float* __restrict__ part, int rows,
                                                              int64_t cols, float* __restrict__ stage) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    const int r0 = (int)((int64_t)rows * blockIdx.y / gridDim.y);
    const int r1 = (int)((int64_t)rows * (blockIdx.y + 1) / gridDim.y);
    float s = 0.f;
    for (int r = r0; r < r1; ++r) s += part[(int64_t)r * cols + c];
    stage[(int64_t)blockIdx.y * cols + c] = s;
}

// The first blocks finish the column sums of stage[rsplit][cols]
// (per-workgroup partials, or their first-pass sums when there are many)
// and store them in the weight's dtype: 256 lanes per block as `phases` row
// phases (1, 2 or 4, from the row count) x 256/phases columns, fixed
// summation order.  With N > 0 the last block also forms the static
// parameter gradients from the per-workgroup sums of
// [dM, dh_post_act, dh_pre_act]: the activation derivatives (ops.py:172,
// 240-242) and ONE Sinkhorn backward on the token-summed dM (M is shared, so
// its VJP is linear in dM):
//     dH_pre = dh_pre_act h_pre (1 - h_pre)
//     dH_post = dh_post_act h_post (1 - h_post / 2)
//     dH_res = SK^T(dM) * exp(H_res)
// For n = 4 the Sinkhorn recompute and adjoint run one element per lane of a
// 16-lane row, as the forward's coefficient kernel computes M.
constexpr int kColSplit = 16;   // row groups of the first pass when rows are many
constexpr int kDirectRows = 512;  // partial rows the finalize sums directly

template <int N, typename TW>
__global__ __launch_bounds__(256) void layer_finalize_kernel(
    const float* __restrict__ stage, int rsplit, int64_t cols, TW* __restrict__ dw,
    const float* __restrict__ scal_part, int rows, const float* __restrict__ h_pre,
    const float* __restrict__ h_post, const float* __restrict__ h_res, float* __restrict__ d_h_pre,
    float* __restrict__ d_h_post, float* __restrict__ d_h_res, int iters, float eps, int phases) {
    // column blocks: 256 lanes = `phases` row phases x (256 / phases) columns
    const int cpb = 256 / phases;
    const int col_blocks = (int)((cols + cpb - 1) / cpb);
    if ((int)blockIdx.x < col_blocks) {
        __shared__ float cred[256];
        const int cl = threadIdx.x % cpb;
        const int ph = threadIdx.x / cpb;
        const int64_t c = (int64_t)blockIdx.x * cpb + cl;
        float s = 0.f;
        if (c < cols) {
            // 8 loads in flight per step, fixed summation order
            int r = ph;
            for (; r + 7 * phases < rsplit; r += 8 * phases) {
                float a[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) a[u] = stage[(int64_t)(r + u * phases) * cols + c];
#pragma unroll
                for (int u = 0; u < 8; ++u) s += a[u];
            }
            for (; r < rsplit; r += phases) s += stage[(int64_t)r * cols + c];
        }
        if (phases == 1) {
            if (c < cols) VecIO<TW>::put(dw + c, s);
            return;
        }
        cred[threadIdx.x] = s;
        __syncthreads();
        if (ph == 0 && c < cols) {
            float t = 0.f;
            for (int k = 0; k < phases; ++k) t += cred[k * cpb + cl];
            VecIO<TW>::put(dw + c, t);
        }
        return;
    }
    if constexpr (N > 0) {
        constexpr int NS = N * N + 2 * N;
        __shared__ float red[4 * NS];
        float v[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) v[k] = 0.f;
        for (int r = threadIdx.x; r < rows; r += blockDim.x) {
#pragma unroll
            for (int k = 0; k < NS; ++k) v[k] += scal_part[(int64_t)r * NS + k];
        }
        block_sum<NS>(v, red);
        if constexpr (N == 4) {
            if (threadIdx.x < kWave) {
                // one element per lane of lanes 0..15, as the forward computed M
                const int l = threadIdx.x;
                const float e = l < 16 ? expf(h_res[l]) : 0.f;
                float g = 0.f;
#pragma unroll
                for (int q = 0; q < 16; ++q) g = (l == q) ? v[q] : g;
                sk16_backward(g, e, iters, eps);
                if (l < 16) d_h_res[l] = g * e;
            }
        } else if (threadIdx.x < kWave) {
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
            sk_backward<N>(gm, e, iters, eps, r < N);
            if (r < N) {
#pragma unroll
                for (int c = 0; c < N; ++c) d_h_res[r * N + c] = gm[c] * e[c];
            }
        }
        if (threadIdx.x < N) {
            const int r = threadIdx.x;
            float hp = 0.f, hq = 0.f;
#pragma unroll
            for (int q = 0; q < N; ++q) {
                hp = (r == q) ? v[N * N + N + q] : hp;
                hq = (r == q) ? v[N * N + q] : hq;
            }
            const float tp = sigmoidf(h_pre[r]);
            const float tq = 2.f * sigmoidf(h_post[r]);
            d_h_pre[r] = hp * tp * (1.f - tp);
            d_h_post[r] = hq * tq * (1.f - tq * 0.5f);
        }
    }
}

template <typename TW>
__global__ __launch_bounds__(256) void weight_f32_kernel(const TW* __restrict__ w, int64_t C, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < C) out[i] = VecIO<TW>::scalar(w + i);
}

__global__ __launch_bounds__(256) void cast_bf16_kernel(const float* __restrict__ in, int64_t n,
                                                        bf16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(in[i]);
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

// p0[0, n0) and p1[0, n1) = s - s with s = c[0] + .. + c[nc - 1]: +0 while
// the carrier sum is finite, NaN once it is not (no fast-math, so s - s is
// not folded).  For gradients that vanish by construction but would be
// non-finite on non-finite inputs, with a gradient sum over the same tokens
// as the carrier.
__global__ __launch_bounds__(256) void fill_zero_carry_kernel(float* __restrict__ p0, int64_t n0,
                                                              float* __restrict__ p1, int64_t n1,
                                                              const float* __restrict__ c, int nc) {
    float s = 0.f;
    for (int k = 0; k < nc; ++k) s += c[k];
    const float z = s - s;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n0) {
        p0[i] = z;
    } else if (i - n0 < n1) {
        p1[i - n0] = z;
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
hipError_t launch_weight_f32(const void* w, int w_dtype, int64_t C, float* out, hipStream_t s) {
    if (C <= 0) return hipSuccess;
    const unsigned blocks = (unsigned)((C + 255) / 256);
    if (w_dtype == kBF16) {
        MHC_LAUNCH_GGL(weight_f32_kernel<bf16_t>, dim3(blocks), dim3(256), 0, s, (const bf16_t*)w, C, out);
    } else {
        MHC_LAUNCH_GGL(weight_f32_kernel<float>, dim3(blocks), dim3(256), 0, s, (const float*)w, C, out);
    }
    return hipGetLastError();
}

hipError_t launch_cast_bf16(const float* in, int64_t n, void* out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    MHC_LAUNCH_GGL(cast_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, n, (bf16_t*)out);
    return hipGetLastError();
}

hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    MHC_LAUNCH_GGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

hipError_t launch_fill_zero_carry(float* p0, int64_t n0, float* p1, int64_t n1, const float* c, int nc,
                                  hipStream_t s) {
    if (n0 < 0 || n1 < 0) return hipErrorInvalidValue;
    const int64_t n = n0 + n1;
    if (n == 0) return hipSuccess;
    MHC_LAUNCH_GGL(fill_zero_carry_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p0, n0, p1, n1, c,
                   nc);
    return hipGetLastError();
}

#define MHC_DISPATCH_N(n, ...)                                   \
    switch (n) {                                                 \
        case 2: { constexpr int N_ = 2; __VA_ARGS__; break; }    \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }    \
        case 8: { constexpr int N_ = 8; __VA_ARGS__; break; }    \
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

int saved_w_offset(int n) { return ((2 * n + n * n + 63) / 64) * 64; }

#define MHC_COEF_N(n, ...)                                       \
    switch (n) {                                                 \
        case 2: { constexpr int N_ = 2; __VA_ARGS__; break; }    \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }    \
        case 8: { constexpr int N_ = 8; __VA_ARGS__; break; }    \
        case 16: { constexpr int N_ = 16; __VA_ARGS__; break; }  \
        case 32: { constexpr int N_ = 32; __VA_ARGS__; break; }  \
        default: return hipErrorInvalidValue;                    \
    }

hipError_t launch_static_coef(int n, const float* h_pre, const float* h_post, const float* h_res,
                              const void* weight, int w_dtype, int64_t C, float* saved, int iters, float sk_eps,
                              hipStream_t s) {
    if (generic_layer_n(n))
        return launch_gen_static_coef(n, h_pre, h_post, h_res, weight, w_dtype, C, saved, iters, sk_eps, s);
    const int off = saved_w_offset(n);
    const unsigned blocks = 1 + (unsigned)((C + 2047) / 2048);
    if (w_dtype == kBF16) {
        MHC_COEF_N(n, MHC_LAUNCH_GGL((static_coef_kernel<N_, bf16_t>), dim3(blocks), dim3(256), 0, s,
                                         h_pre, h_post, h_res, (const bf16_t*)weight, (int)C, saved, off, iters,
                                         sk_eps));
    } else {
        MHC_COEF_N(n, MHC_LAUNCH_GGL((static_coef_kernel<N_, float>), dim3(blocks), dim3(256), 0, s,
                                         h_pre, h_post, h_res, (const float*)weight, (int)C, saved, off, iters,
                                         sk_eps));
    }
    return hipGetLastError();
}
#undef MHC_COEF_N

// ---------------------------------------------------------------------------
// Persistent row kernels: pick the instantiation, size the grid from its
// occupancy (resident workgroups per CU x CUs, capped by the token count).
// ---------------------------------------------------------------------------
#define MHC_PICK_VPT(v, ...)                                     \
    switch (v) {                                                 \
        case 1: { constexpr int V_ = 1; __VA_ARGS__; break; }    \
        case 2: { constexpr int V_ = 2; __VA_ARGS__; break; }    \
        case 4: { constexpr int V_ = 4; __VA_ARGS__; break; }    \
        case 8: { constexpr int V_ = 8; __VA_ARGS__; break; }    \
        default: break;                                          \
    }

template <typename TX, typename TO, int N, int V>
static const void* fwd_fn() {
    if constexpr (layer_row_fits(N, V)) return reinterpret_cast<const void*>(&layer_fwd_kernel<TX, TO, N, V>);
    return nullptr;
}

template <typename TX, int N, int V, int MODE, bool PF>
static const void* bwd_fn() {
    if constexpr (layer_row_fits(2 * N, V)) return reinterpret_cast<const void*>(&layer_bwd_kernel<TX, N, V, MODE, PF>);
    return nullptr;
}

static const void* pick_fwd(int x_dtype, int out_dtype, int n, int vpt) {
    const void* fn = nullptr;
#define MHC_FWD_TO(TX_, N_)                                                      \
    if (out_dtype == kBF16) {                                                    \
        MHC_PICK_VPT(vpt, fn = fwd_fn<TX_, bf16_t, N_, V_>());                   \
    } else {                                                                     \
        MHC_PICK_VPT(vpt, fn = fwd_fn<TX_, float, N_, V_>());                    \
    }
#define MHC_FWD_N(N_)                                                            \
    if (x_dtype == kBF16) {                                                      \
        MHC_FWD_TO(bf16_t, N_)                                                   \
    } else {                                                                     \
        MHC_FWD_TO(float, N_)                                                    \
    }
    switch (n) {
        case 2: { MHC_FWD_N(2); break; }
        case 4: { MHC_FWD_N(4); break; }
        case 8: { MHC_FWD_N(8); break; }
        default: break;
    }
#undef MHC_FWD_N
#undef MHC_FWD_TO
    return fn;
}

static const void* pick_bwd(int x_dtype, int n, int vpt, int mode, bool pf) {
    const void* fn = nullptr;
#define MHC_BWD_FN(TX_, N_)                                                                                     \
    MHC_PICK_VPT(vpt, fn = mode == 0 ? (pf ? bwd_fn<TX_, N_, V_, 0, true>() : bwd_fn<TX_, N_, V_, 0, false>())   \
                                     : (pf ? bwd_fn<TX_, N_, V_, 1, true>() : bwd_fn<TX_, N_, V_, 1, false>()))
    const bool bf = x_dtype == kBF16;
    switch (n) {
        case 2: { if (bf) { MHC_BWD_FN(bf16_t, 2); } else { MHC_BWD_FN(float, 2); } break; }
        case 4: { if (bf) { MHC_BWD_FN(bf16_t, 4); } else { MHC_BWD_FN(float, 4); } break; }
        case 8: { if (bf) { MHC_BWD_FN(bf16_t, 8); } else { MHC_BWD_FN(float, 8); } break; }
        default: break;
    }
#undef MHC_BWD_FN
    return fn;
}

static int persistent_grid(const void* fn, int threads, int64_t B) {
    int per_cu = 0;
    if (fn == nullptr || hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess ||
        per_cu < 1) {
        (void)hipGetLastError();
        per_cu = 1;
    }
    int64_t g = (int64_t)device_cu_count() * per_cu;
    if (g > B) g = B;
    if (g < 1) g = 1;
    return (int)g;
}

// Backward workgroups of <= 256 lanes run the two-buffer prefetch variant.
static bool use_prefetch(const RowTiling& t) { return t.threads <= 256; }

// The register-row kernels take n <= 8 and a multiple of the 4-channel
// chunk that fits their row state; everything else runs the channel-loop
// kernels of wide.hip.
static RowTiling fwd_tiling(int64_t C, int n) {
    if (n > 8 || generic_layer_n(n)) return RowTiling{0, 0};
    return choose_row_tiling(C, kLayerWC, n, 512);
}

bool layer_fwd_is_wide(int n, int64_t C) { return fwd_tiling(C, n).vpt <= 0; }

hipError_t launch_layer_fwd(int x_dtype, int n, const void* x, const float* w, const float* coef,
                            int64_t coef_stride, void* out, int out_dtype, float* rms_out, int64_t B, int64_t C,
                            float eps, hipStream_t s, int64_t rms_scratch) {
    if (B == 0) return hipSuccess;
    if (generic_layer_n(n))
        return launch_gen_layer_fwd(x_dtype, out_dtype, n, x, w, coef, coef_stride, out, rms_out, B, C, eps, s);
    const RowTiling t = fwd_tiling(C, n);
    if (t.vpt <= 0)
        return launch_wide_fwd(x_dtype, out_dtype, n, x, w, coef, coef_stride, out, rms_out, B, C, eps, s, rms_scratch);
    const void* fn = pick_fwd(x_dtype, out_dtype, n, t.vpt);
    if (!fn) return hipErrorInvalidValue;
    if (B > 0x7fffffff) return hipErrorInvalidValue;  // grid x limit
    const unsigned grid = (unsigned)B;  // one token per workgroup
    int Ci = (int)C;
    void* args[] = {(void*)&x, (void*)&w, (void*)&coef, (void*)&coef_stride, (void*)&out, (void*)&rms_out,
                    (void*)&B, (void*)&Ci, (void*)&eps};
    const int tok = timing_begin("layer_fwd", s);
    hipError_t e = mhc_launch_kernel(fn, dim3(grid), dim3(t.threads), args, 0, s);
    timing_end(tok, s);
    return e != hipSuccess ? e : hipGetLastError();
}

template <typename TX, typename TW, int N, int V>
static const void* static_fwd_fn() {
    if constexpr (layer_row_fits(N, V))
        return reinterpret_cast<const void*>(&layer_static_fwd_kernel<TX, TW, N, V>);
    return nullptr;
}

bool layer_static_fwd_fused(int n, int64_t C) { return n <= 8 && fwd_tiling(C, n).vpt > 0; }

hipError_t launch_layer_static_fwd(int x_dtype, int n, const void* x, const void* weight, int w_dtype,
                                   const float* h_pre, const float* h_post, const float* h_res, float* saved,
                                   int iters, float sk_eps, float* out, float* rms_out, int64_t B, int64_t C,
                                   float eps, hipStream_t s) {
    const RowTiling t = fwd_tiling(C, n);
    if (t.vpt <= 0 || n > 8) return hipErrorInvalidValue;
    if (B == 0) {
        // no tokens: the saved state alone (the backward still needs it)
        return launch_static_coef(n, h_pre, h_post, h_res, weight, w_dtype, C, saved, iters, sk_eps, s);
    }
    if (B > 0x7fffffff) return hipErrorInvalidValue;  // grid x limit
    const void* fn = nullptr;
#define MHC_SF_TW(TX_, N_)                                                                \
    if (w_dtype == kBF16) {                                                               \
        MHC_PICK_VPT(t.vpt, fn = static_fwd_fn<TX_, bf16_t, N_, V_>());                   \
    } else {                                                                              \
        MHC_PICK_VPT(t.vpt, fn = static_fwd_fn<TX_, float, N_, V_>());                    \
    }
#define MHC_SF_N(N_)                                                                      \
    if (x_dtype == kBF16) {                                                               \
        MHC_SF_TW(bf16_t, N_)                                                             \
    } else {                                                                              \
        MHC_SF_TW(float, N_)                                                              \
    }
    switch (n) {
        case 2: { MHC_SF_N(2); break; }
        case 4: { MHC_SF_N(4); break; }
        case 8: { MHC_SF_N(8); break; }
        default: break;
    }
#undef MHC_SF_N
#undef MHC_SF_TW
    if (!fn) return hipErrorInvalidValue;
    int Ci = (int)C;
    int w_off = saved_w_offset(n);
    void* args[] = {(void*)&x, (void*)&weight, (void*)&h_pre, (void*)&h_post, (void*)&h_res, (void*)&saved,
                    (void*)&w_off, (void*)&iters, (void*)&sk_eps, (void*)&out, (void*)&rms_out, (void*)&B,
                    (void*)&Ci, (void*)&eps};
    const int tok = timing_begin("layer_fwd", s);
    hipError_t e = mhc_launch_kernel(fn, dim3((unsigned)B), dim3(t.threads), args, 0, s);
    timing_end(tok, s);
    return e != hipSuccess ? e : hipGetLastError();
}

// The backward hands one of its 2 + n^2 + 3n row sums to each thread.  Both
// storage dtypes run 256-lane workgroups with the two-token prefetch (C4
// MODE 1: 213 -> 182 us against 512 lanes with one token in registers, once
// the prefetch was unconditional; with the prefetch behind a branch the
// 512-lane form had been the faster one).
static RowTiling bwd_tiling(int64_t C, int n, int x_dtype = kF32) {
    (void)x_dtype;
    if (n > 8 || generic_layer_n(n)) return RowTiling{0, 0};
    return with_min_threads(choose_row_tiling(C, kLayerWC, 2 * n, 256), 2 + n * n + 3 * n);
}

bool layer_bwd_is_wide(int n, int64_t C) { return bwd_tiling(C, n).vpt <= 0; }

int layer_bwd_part_groups(int x_dtype, int n, int64_t C) {
    const RowTiling t = bwd_tiling(C, n, x_dtype);
    return t.vpt > 0 ? t.threads / 32 : 0;
}

int layer_bwd_grid(int x_dtype, int n, int64_t B, int64_t C) {
    if (generic_layer_n(n)) return gen_layer_bwd_grid(B);
    const RowTiling t = bwd_tiling(C, n, x_dtype);
    if (t.vpt <= 0) return wide_bwd_grid(x_dtype, n, B, C);
    return persistent_grid(pick_bwd(x_dtype, n, t.vpt, 0, use_prefetch(t)), t.threads, B);
}

size_t layer_bwd_scratch_bytes(int x_dtype, int n, int64_t B, int64_t C) {
    if (generic_layer_n(n)) return gen_layer_bwd_scratch_bytes(B, C);
    return bwd_tiling(C, n, x_dtype).vpt <= 0 ? wide_bwd_scratch_bytes(n, B, C) : 0;
}

hipError_t launch_layer_bwd(int x_dtype, int n, int mode, const float* g, const void* x, const float* w,
                            const float* coef, int64_t coef_stride, void* dx, float* dw_part, float* scal_out,
                            int grid, int64_t B, int64_t C, float eps, float* scratch, hipStream_t s,
                            int32_t* dx_scale) {
    if (generic_layer_n(n)) {
        // the generic kernels write a full-precision stream part only for
        // fp32 x; the dynamic entries send bf16 x through fp32 accumulation
        if (mode == 1 && x_dtype == kBF16) return hipErrorInvalidValue;
        return launch_gen_layer_bwd(x_dtype, n, mode, g, x, w, coef, coef_stride, dx, dw_part, scal_out, grid, B, C,
                                    eps, scratch, s);
    }
    const RowTiling t = bwd_tiling(C, n, x_dtype);
    if (t.vpt <= 0) {
        // the channel-loop kernels write a bf16 stream part; the dynamic
        // entries send bf16 x there through fp32 accumulation instead
        if (mode == 1 && x_dtype == kBF16) return hipErrorInvalidValue;
        return launch_wide_bwd(x_dtype, n, mode, g, x, w, coef, coef_stride, dx, dw_part, scal_out, grid, B, C, eps,
                               scratch, s);
    }
    if (mode == 1 && x_dtype == kBF16 && (dx_scale == nullptr || C % kPartGroup != 0)) return hipErrorInvalidValue;
    const void* fn = pick_bwd(x_dtype, n, t.vpt, mode, use_prefetch(t));
    if (!fn) return hipErrorInvalidValue;
    int Ci = (int)C;
    void* args[] = {(void*)&g, (void*)&x, (void*)&w, (void*)&coef, (void*)&coef_stride, (void*)&dx,
                    (void*)&dw_part, (void*)&scal_out, (void*)&dx_scale, (void*)&B, (void*)&Ci, (void*)&eps};
    const int tok = timing_begin(mode == 0 ? "layer_bwd" : "layer_bwd_reduce", s);
    hipError_t e = mhc_launch_kernel(fn, dim3(grid), dim3(t.threads), args, 0, s);
    timing_end(tok, s);
    return e != hipSuccess ? e : hipGetLastError();
}

hipError_t launch_column_partial(const float* part, int rows, int64_t cols, float* stage, int rsplit,
                                 hipStream_t s) {
    if (cols == 0) return hipSuccess;
    if (cols % 4 != 0) {
        MHC_LAUNCH_GGL(column_partial1_kernel, dim3((unsigned)((cols + 255) / 256), rsplit), dim3(256), 0, s, part,
                           rows, cols, stage);
    } else {
        MHC_LAUNCH_GGL(column_partial_kernel, dim3((unsigned)((cols + 255) / 256), rsplit), dim3(256), 0, s, part,
                           rows, cols, stage);
    }
    return hipGetLastError();
}

bool column_sums_direct(int rows) { return rows >= 1 && rows <= kDirectRows; }

hipError_t launch_multi_column_sum(ColSumJobs jobs, hipStream_t s) {
    if (jobs.count < 1 || jobs.count > kMaxColSumJobs) return hipErrorInvalidValue;
    int64_t blocks = 0;
    for (int q = 0; q < jobs.count; ++q) {
        ColSumJob& jb = jobs.j[q];
        if (!column_sums_direct(jb.rows) || jb.cols < 1 || jb.split < 0 || jb.split > jb.cols ||
            (jb.split < jb.cols && !jb.out2))
            return hipErrorInvalidValue;
        // as launch_layer_finalize; narrow jobs take more phases (shorter chains)
        jb.phases = jb.cols <= 32 ? 16 : (jb.rows <= 16 ? 1 : (jb.rows <= 64 ? 2 : 4));
        const int cpb = 256 / jb.phases;
        jb.blocks = (int)((jb.cols + cpb - 1) / cpb);
        blocks += jb.blocks;
    }
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    MHC_LAUNCH_GGL(multi_column_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, s, jobs);
    return hipGetLastError();
}

hipError_t launch_layer_finalize(int n, int w_dtype, const float* stage, int rsplit, int64_t cols, void* dw,
                                 const float* scal_part, int rows, const float* h_pre, const float* h_post,
                                 const float* h_res, float* d_h_pre, float* d_h_post, float* d_h_res, int iters,
                                 float sk_eps, hipStream_t s) {
    // row phases per 256-lane column block: one for a few partial rows (each
    // lane sums its column), more for many rows; the static scalar block
    // (n > 0) runs with the same 256 lanes
    const int phases = rsplit <= 16 ? 1 : (rsplit <= 64 ? 2 : 4);
    const int64_t cpb = 256 / phases;
    const unsigned col_blocks = (unsigned)((cols + cpb - 1) / cpb);
    const unsigned blocks = col_blocks + (n > 0 ? 1 : 0);
    if (blocks == 0) return hipSuccess;
    const unsigned threads = 256;
#define MHC_FIN_LAUNCH(N_, TW_)                                                                                  \
    MHC_LAUNCH_GGL((layer_finalize_kernel<N_, TW_>), dim3(blocks), dim3(threads), 0, s, stage, rsplit, cols,  \
                       (TW_*)dw, scal_part, rows, h_pre, h_post, h_res, d_h_pre, d_h_post, d_h_res, iters, sk_eps, \
                       phases)
    if (n == 0) {
        if (w_dtype == kBF16) { MHC_FIN_LAUNCH(0, bf16_t); } else { MHC_FIN_LAUNCH(0, float); }
    } else {
        if (w_dtype == kBF16) {
            MHC_DISPATCH_N(n, MHC_FIN_LAUNCH(N_, bf16_t));
        } else {
            MHC_DISPATCH_N(n, MHC_FIN_LAUNCH(N_, float));
        }
    }
#undef MHC_FIN_LAUNCH
    return hipGetLastError();
}

size_t column_sums_stage_floats(int64_t cols) { return (size_t)kColSplit * (size_t)cols; }

hipError_t launch_column_finalize(int n, int w_dtype, const float* part, int rows, int64_t cols, float* stage,
                                  void* dw, const float* scal_part, int scal_rows, const float* h_pre,
                                  const float* h_post, const float* h_res, float* d_h_pre, float* d_h_post,
                                  float* d_h_res, int iters, float sk_eps, hipStream_t s, float* sk_hist) {
    if (n > 0 && generic_layer_n(n)) {
        hipError_t e = launch_column_finalize(0, w_dtype, part, rows, cols, stage, dw, nullptr, 0, nullptr, nullptr,
                                              nullptr, nullptr, nullptr, nullptr, 0, 0.f, s);
        if (e != hipSuccess) return e;
        return launch_gen_static_finalize(n, scal_part, scal_rows, h_pre, h_post, h_res, d_h_pre, d_h_post, d_h_res,
                                          iters, sk_eps, s, sk_hist, sk_hist ? kStaticSkHistBytes : 0);
    }
    if (n > 8) {
        // the static scalar gradients of wide n have their own kernel
        hipError_t e = launch_column_finalize(0, w_dtype, part, rows, cols, stage, dw, nullptr, 0, nullptr, nullptr,
                                              nullptr, nullptr, nullptr, nullptr, 0, 0.f, s);
        if (e != hipSuccess) return e;
        return launch_wide_static_finalize(n, scal_part, scal_rows, h_pre, h_post, h_res, d_h_pre, d_h_post, d_h_res,
                                           iters, sk_eps, sk_hist, sk_hist ? kStaticSkHistBytes : 0, s);
    }
    if (rows <= kDirectRows)
        return launch_layer_finalize(n, w_dtype, part, rows, cols, dw, scal_part, scal_rows, h_pre, h_post, h_res,
                                     d_h_pre, d_h_post, d_h_res, iters, sk_eps, s);
    hipError_t e = launch_column_partial(part, rows, cols, stage, kColSplit, s);
    if (e != hipSuccess) return e;
    return launch_layer_finalize(n, w_dtype, stage, kColSplit, cols, dw, scal_part, scal_rows, h_pre, h_post, h_res,
                                 d_h_pre, d_h_post, d_h_res, iters, sk_eps, s);
}

}  // namespace mhc

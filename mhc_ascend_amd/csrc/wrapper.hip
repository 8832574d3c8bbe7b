// MHCResidualWrapper fused on gfx950 (layer.py:269-322).
//
// The wrapper turns (residual r, branch b) [tokens, C] into n layer streams
//     X_0 = r,  X_1 = b,  X_i = r * 0.1^(i-1) rounded to the storage dtype
//     ('decay', layer.py:306-308) or X_i = 0 ('zero'),
// runs the mHC layer on X [tokens, n, C] and returns the mean over streams.
// Here X never exists in memory: every kernel rebuilds the stream values of
// the channels it holds from r and b, in registers.  The stream mean folds
// into the layer's output:
//     mean_i out_i = sum_j cm_j X_j + hs * y,   cm_j = (1/n) sum_i M_ij,
//                                               hs = (1/n) sum_i h_post_i.
// Backward, with G the cotangent of the mean (every stream receives G / n):
//     gy = hs G,  gxa = w gy / r_rms - xa k2,  dX_j = cm_j G + h_pre_j gxa
//     d r = dX_0 + sum_{i>=2} 0.1^(i-1) dX_i,  d b = dX_1
// plus, for dynamic H, the projection and r_h terms (s X_j + dP . Phi_j).
//
// Kernels:
//   wrap_fwd_kernel       row pass: xa, RMSNorm, the stream mean (fp32 out)
//   wrap_bwd_kernel       static-H row pass: all row sums of a token
//                         (per-workgroup sums) and d r / d b
//   wrap_bwd_red_kernel   dynamic-H backward pass 1: the row sums of each
//                         token (one wave per token), reading only
//   wrap_proj_kernel      P = X_flat . Phi^T split-K on bf16 MFMA, reading r
//                         and b once per channel for all n streams
//   wrap_proj_bwd_kernel  dynamic-H backward pass 2: d r, d b = stream parts
//                         + s X + dP . Phi (Phi folded over the
//                         residual-derived streams), dw and dPhi partials
#include <type_traits>

#include "mhc_device.h"
#include "mhc_internal.h"
#include "mhc_rows.h"

namespace mhc {

// 0.1^e in double, as Python's 0.1 ** e for the small e used here
// (layer.py:308 multiplies by that double; the product is formed in fp32).
constexpr double pow01(int e) { return e <= 0 ? 1.0 : 0.1 * pow01(e - 1); }

template <int I>
constexpr float decay_mult() { return (float)pow01(I - 1); }

// Round to the storage dtype (the synthesised stream is a tensor of it).
template <typename TX>
__device__ __forceinline__ float round_store(float v) {
    if constexpr (sizeof(TX) == 2) {
        return bf16_to_f32(f32_to_bf16(v));
    } else {
        return v;
    }
}

// Stream I of the synthesised row at one element.
template <typename TX, int I, bool DECAY>
__device__ __forceinline__ float wrap_stream(float r, float b) {
    if constexpr (I == 0) {
        return r;
    } else if constexpr (I == 1) {
        return b;
    } else if constexpr (DECAY) {
        constexpr float m = decay_mult<I>();
        return round_store<TX>(r * m);
    } else {
        return 0.f;
    }
}

template <typename TX, int N, bool DECAY>
__device__ __forceinline__ void wrap_streams(float r, float b, float (&x)[N]) {
    x[0] = r;
    if constexpr (N > 1) x[1] = b;
    if constexpr (N > 2) x[2] = wrap_stream<TX, 2, DECAY>(r, b);
    if constexpr (N > 3) x[3] = wrap_stream<TX, 3, DECAY>(r, b);
    static_assert(N <= 4, "wrapper kernels are instantiated for n <= 4");
}

// d r contribution weight of stream j (0 for the branch and for zero streams)
template <int J, bool DECAY>
__device__ __forceinline__ float res_weight() {
    constexpr float w = J == 0 ? 1.f : (J == 1 ? 0.f : (DECAY ? decay_mult<J>() : 0.f));
    return w;
}

template <int N> constexpr int wcoef_size() { return 2 * N + N * N; }

// ---------------------------------------------------------------------------
// Forward row pass.
// ---------------------------------------------------------------------------
template <typename TX, int N, int VPT, bool DECAY>
__device__ __forceinline__ void wrap_fwd_token(int64_t b, const float* __restrict__ coef, int64_t coef_stride,
                                               const float (&wv)[VPT][kLayerWC], const float (&rv)[1][VPT][kLayerWC],
                                               const float (&bv)[1][VPT][kLayerWC], float* __restrict__ out, int C,
                                               float eps, float* red) {
    constexpr int WC = kLayerWC;
    const float* cf = coef + b * coef_stride;
    float hp[N], cm[N], hs = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        hp[j] = cf[j];
        hs += cf[N + j];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) s += cf[2 * N + i * N + j];
        cm[j] = s * (1.f / N);
    }
    hs *= 1.f / N;
    float xa[VPT][WC];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
#pragma unroll
        for (int e = 0; e < WC; ++e) {
            float x[N];
            wrap_streams<TX, N, DECAY>(rv[0][k][e], bv[0][k][e], x);
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < N; ++j) s += hp[j] * x[j];
            xa[k][e] = s;
            ss += s * s;
        }
    }
    float v[1] = {ss};
    block_sum<1>(v, red);
    const float inv = 1.f / sqrtf(v[0] / (float)C + eps);
    float* ob = out + b * (int64_t)C;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) {
            float o[WC];
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float x[N];
                wrap_streams<TX, N, DECAY>(rv[0][k][e], bv[0][k][e], x);
                float s = hs * (xa[k][e] * inv * wv[k][e]);
#pragma unroll
                for (int j = 0; j < N; ++j) s += cm[j] * x[j];
                o[e] = s;
            }
            store_run_nt<float, WC>(ob + c0, o);
        }
    }
}

// One token per workgroup (grid = tokens): the row loads of the next
// workgroups on the CU overlap this one's reduction, which measured faster
// than persistent workgroups with a register prefetch for this pass.
template <typename TX, int N, int VPT, bool DECAY>
__global__ MHC_ROW_BOUNDS(false) void wrap_fwd_kernel(const TX* __restrict__ res, const TX* __restrict__ br,
                                                      const float* __restrict__ w, const float* __restrict__ coef,
                                                      int64_t coef_stride, float* __restrict__ out, int64_t B, int C,
                                                      float eps) {
    constexpr int WC = kLayerWC;
    __shared__ float red[8];
    const int64_t b = blockIdx.x;
    if (b >= B) return;
    RawRows<TX, 1, VPT, WC> rA, bA;
    load_rows_raw<TX, 1, VPT, WC, true>(res + b * C, C, rA);
    load_rows_raw<TX, 1, VPT, WC, true>(br + b * C, C, bA);
    float wv[VPT][WC];
    load_weight<VPT, WC>(w, C, wv);
    float rv[1][VPT][WC], bv[1][VPT][WC];
    unpack_rows<TX, 1, VPT, WC>(rA, C, rv);
    unpack_rows<TX, 1, VPT, WC>(bA, C, bv);
    wrap_fwd_token<TX, N, VPT, DECAY>(b, coef, coef_stride, wv, rv, bv, out, C, eps, red);
}

// One token per wave, bf16 storage, C = 256 KQ: the row's 4-channel chunks
// (lane l takes chunks l, l + 64, ..., KQ of them) stay in registers as
// packed words, the row sum is a wave sum (no barrier), and the weight is
// staged once per workgroup in LDS.  The second pass rebuilds the streams
// from the packed words (kept from being hoisted by an empty asm that
// "changes" them) rather than holding the row's fp32 values.  Rows that are
// not whole rounds of 64 chunks run wrap_fwd_kernel: masking the last round
// took the register count from 141 to about 200 at KQ = 28.
template <int KQ, bool DECAY>
__global__ __launch_bounds__(256) void wrap_fwd_wave_kernel(const bf16_t* __restrict__ res, const bf16_t* __restrict__ br,
                                                            const float* __restrict__ w, const float* __restrict__ coef,
                                                            int64_t coef_stride, float* __restrict__ out, int64_t B,
                                                            int C, float eps) {
    constexpr int N = 4;
    extern __shared__ __align__(16) float wl[];  // C floats
    for (int i = threadIdx.x; i < C; i += blockDim.x) wl[i] = w[i];
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t b = (int64_t)blockIdx.x * (blockDim.x / kWave) + (int64_t)wave_uniform(threadIdx.x / kWave);
    if (b >= B) return;
    uint32_t rw[KQ][2], bw[KQ][2];
    const bf16_t* rb = res + b * (int64_t)C;
    const bf16_t* bb = br + b * (int64_t)C;
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
        const int c0 = (k * kWave + lane) * 4;
        const uint2 a = ld8_nt(rb + c0), c = ld8_nt(bb + c0);
        rw[k][0] = a.x; rw[k][1] = a.y;
        bw[k][0] = c.x; bw[k][1] = c.y;
    }
    const float* cf = coef + b * coef_stride;
    float hp[N], cm[N], hs = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        hp[j] = cf[j];
        hs += cf[N + j];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) s += cf[2 * N + i * N + j];
        cm[j] = s * (1.f / N);
    }
    hs *= 1.f / N;
    auto unpack = [&](int k, int e, float& r, float& bv) __attribute__((always_inline)) {
        const uint32_t wr = rw[k][e >> 1], wb = bw[k][e >> 1];
        r = __uint_as_float((e & 1) ? (wr & 0xffff0000u) : (wr << 16));
        bv = __uint_as_float((e & 1) ? (wb & 0xffff0000u) : (wb << 16));
    };
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float r, bv, x[N];
            unpack(k, e, r, bv);
            wrap_streams<bf16_t, N, DECAY>(r, bv, x);
            float xa = 0.f;
#pragma unroll
            for (int j = 0; j < N; ++j) xa += hp[j] * x[j];
            ss += xa * xa;
        }
    }
    ss = group_sum<kWave>(ss);
    const float inv = 1.f / sqrtf(ss / (float)C + eps);
    const float hsi = hs * inv;
#pragma unroll
    for (int k = 0; k < KQ; ++k) asm volatile("" : "+v"(rw[k][0]), "+v"(rw[k][1]), "+v"(bw[k][0]), "+v"(bw[k][1]));
    float* ob = out + b * (int64_t)C;
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
        const int q = k * kWave + lane;
        const float4 wq = *reinterpret_cast<const float4*>(&wl[q * 4]);
        const float wv[4] = {wq.x, wq.y, wq.z, wq.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float r, bv, x[N];
            unpack(k, e, r, bv);
            wrap_streams<bf16_t, N, DECAY>(r, bv, x);
            float xa = 0.f, s = 0.f;
#pragma unroll
            for (int j = 0; j < N; ++j) {
                xa += hp[j] * x[j];
                s += cm[j] * x[j];
            }
            o[e] = s + hsi * (xa * wv[e]);
        }
        st16_nt(ob + q * 4, make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                       __float_as_uint(o[3])));
    }
}

// ---------------------------------------------------------------------------
// Backward row pass.  Per token the block forms, in one reduction,
//   ss = sum xa^2, gwx = sum G w xa, u_j = sum G X_j, v_j = sum G w X_j,
//   z_j = sum xa X_j
// and from them the scalars of the layer backward in its layout
// (dM[n*n], dh_post_act[n], dh_pre_act[n], 1/r, k2):
//   dM_ij = u_j / n,  dh_post_act_i = gwx / (n r),
//   dh_pre_act_j = hs v_j / r - k2 z_j,  k2 = hs gwx / (C r^3).
// The first n*n+2n are summed per workgroup (static H, shared M); d r / d b
// get the stream terms, which are the whole gradient with static H.
// ---------------------------------------------------------------------------
template <typename TX, int N, int VPT, bool DECAY>
__device__ __forceinline__ void wrap_bwd_token(int64_t b, const float* __restrict__ coef, int64_t coef_stride,
                                               const float (&wv)[VPT][kLayerWC], const float (&gv)[1][VPT][kLayerWC],
                                               const float (&rv)[1][VPT][kLayerWC],
                                               const float (&bv)[1][VPT][kLayerWC], float (&dwacc)[VPT][kLayerWC],
                                               float& sacc, TX* __restrict__ dres, TX* __restrict__ dbr, int C,
                                               float eps, float* red) {
    constexpr int WC = kLayerWC;
    constexpr int NS = N * N + 2 * N;
    constexpr int NR = 2 + 3 * N;  // ss, gwx, u_j, v_j, z_j
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    float* tot = red + 8 * NR;
    const float* cf = coef + b * coef_stride;
    float hp[N], cm[N], hs = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        hp[j] = cf[j];
        hs += cf[N + j];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) s += cf[2 * N + i * N + j];
        cm[j] = s * (1.f / N);
    }
    hs *= 1.f / N;
    {
        float rsum[NR];
#pragma unroll
        for (int q = 0; q < NR; ++q) rsum[q] = 0.f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float x[N];
                wrap_streams<TX, N, DECAY>(rv[0][k][e], bv[0][k][e], x);
                float xa = 0.f;
#pragma unroll
                for (int j = 0; j < N; ++j) xa += hp[j] * x[j];
                const float g = gv[0][k][e];
                const float wg = wv[k][e] * g;
                rsum[0] += xa * xa;
                rsum[1] += wg * xa;
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    rsum[2 + j] += g * x[j];
                    rsum[2 + N + j] += wg * x[j];
                    rsum[2 + 2 * N + j] += xa * x[j];
                }
            }
        }
        wave_sum_last<NR>(rsum);
        if (lane == kWave - 1) {
#pragma unroll
            for (int q = 0; q < NR; ++q) red[wave * NR + q] = rsum[q];
        }
    }
    __syncthreads();
    if (threadIdx.x < NR) {
        float s = 0.f;
        for (int q = 0; q < nwaves; ++q) s += red[q * NR + threadIdx.x];
        tot[threadIdx.x] = s;
    }
    __syncthreads();
    const float inv = 1.f / sqrtf(tot[0] / (float)C + eps);
    const float gwx = tot[1];
    const float k2 = hs * gwx * inv * inv * inv / (float)C;

    if (threadIdx.x < NS) {
        const int t = threadIdx.x;
        float v;
        if (t < N * N) {
            v = tot[2 + t % N] * (1.f / N);  // dM_ij = u_j / n
        } else if (t < N * N + N) {
            v = gwx * inv * (1.f / N);  // dh_post_act_i
        } else {
            const int j = t - N * N - N;
            v = hs * inv * tot[2 + N + j] - k2 * tot[2 + 2 * N + j];  // dh_pre_act_j
        }
        sacc += v;
    }

    // stores through row resources, out-of-range offsets past the row end:
    // none behind a branch (the caller's prefetch keeps exact wait counts)
    const buf_rsrc_t drs = make_buf_rsrc(dres + b * (int64_t)C, (uint32_t)((int64_t)C * (int64_t)sizeof(TX)));
    const buf_rsrc_t dbs = make_buf_rsrc(dbr + b * (int64_t)C, (uint32_t)((int64_t)C * (int64_t)sizeof(TX)));
    static_assert(kLayerWC == 4, "4-channel chunks: one 16-byte (fp32) or 8-byte (bf16) store");
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        float dr[WC], db[WC];
#pragma unroll
        for (int e = 0; e < WC; ++e) {
            float x[N];
            wrap_streams<TX, N, DECAY>(rv[0][k][e], bv[0][k][e], x);
            float xa = 0.f;
#pragma unroll
            for (int j = 0; j < N; ++j) xa += hp[j] * x[j];
            const float g = gv[0][k][e];
            const float gy = hs * g;
            const float gxa = wv[k][e] * gy * inv - xa * k2;
            dwacc[k][e] += gy * xa * inv;
            float a = 0.f;
            if constexpr (N > 0) a += cm[0] * g + hp[0] * gxa;
            if constexpr (N > 2) a += res_weight<2, DECAY>() * (cm[2] * g + hp[2] * gxa);
            if constexpr (N > 3) a += res_weight<3, DECAY>() * (cm[3] * g + hp[3] * gxa);
            dr[e] = a;
            db[e] = (N > 1) ? cm[N > 1 ? 1 : 0] * g + hp[N > 1 ? 1 : 0] * gxa : 0.f;
        }
        const uint32_t o = c0 < C ? (uint32_t)c0 * (uint32_t)sizeof(TX) : kBufOff;
        if constexpr (sizeof(TX) == 4) {
            buf_st16<true>(drs, o, 0u, make_uint4(__float_as_uint(dr[0]), __float_as_uint(dr[1]), __float_as_uint(dr[2]),
                                                  __float_as_uint(dr[3])));
            buf_st16<true>(dbs, o, 0u, make_uint4(__float_as_uint(db[0]), __float_as_uint(db[1]), __float_as_uint(db[2]),
                                                  __float_as_uint(db[3])));
        } else {
            buf_st8<true>(drs, o, 0u, make_uint2(pack_bf16x2(dr[0], dr[1]), pack_bf16x2(dr[2], dr[3])));
            buf_st8<true>(dbs, o, 0u, make_uint2(pack_bf16x2(db[0], db[1]), pack_bf16x2(db[2], db[3])));
        }
    }
}

template <typename TX, int N, int VPT, bool PF, bool DECAY>
__device__ __forceinline__ void wrap_bwd_rows(const float* __restrict__ g, const TX* __restrict__ res,
                                              const TX* __restrict__ br, const float* __restrict__ w,
                                              const float* __restrict__ coef, int64_t coef_stride,
                                              TX* __restrict__ dres, TX* __restrict__ dbr,
                                              float* __restrict__ dw_part, float* __restrict__ scal_out, int64_t B,
                                              int C, float eps) {
    constexpr int WC = kLayerWC;
    constexpr int NS = N * N + 2 * N;
    constexpr int NR = 2 + 3 * N;
    __shared__ float red[9 * NR];
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
    int64_t b = blockIdx.x;
    RawRows<float, 1, VPT, WC> gA, gB;
    RawRows<TX, 1, VPT, WC> rA, bA, rB, bB;
    float gv[1][VPT][WC], rv[1][VPT][WC], bv[1][VPT][WC];
    if constexpr (PF) {
        // row loads through per-token resources (0 bytes past the last
        // token): the prefetch of the next token is unconditional, which
        // keeps the compiler's wait before the current token partial
        load_rows_raw_rs<float, 1, VPT, WC, true>(token_rows_rsrc(g, b, B, 1, C), C, gA);
        load_rows_raw_rs<TX, 1, VPT, WC, true>(token_rows_rsrc(res, b, B, 1, C), C, rA);
        load_rows_raw_rs<TX, 1, VPT, WC, true>(token_rows_rsrc(br, b, B, 1, C), C, bA);
        while (b < B) {
            const int64_t b1 = b + G;
            load_rows_raw_rs<float, 1, VPT, WC, true>(token_rows_rsrc(g, b1, B, 1, C), C, gB);
            load_rows_raw_rs<TX, 1, VPT, WC, true>(token_rows_rsrc(res, b1, B, 1, C), C, rB);
            load_rows_raw_rs<TX, 1, VPT, WC, true>(token_rows_rsrc(br, b1, B, 1, C), C, bB);
            unpack_rows<float, 1, VPT, WC>(gA, C, gv);
            unpack_rows<TX, 1, VPT, WC>(rA, C, rv);
            unpack_rows<TX, 1, VPT, WC>(bA, C, bv);
            wrap_bwd_token<TX, N, VPT, DECAY>(b, coef, coef_stride, wv, gv, rv, bv, dwacc, sacc, dres, dbr, C, eps,
                                              red);
            if (b1 >= B) break;
            const int64_t b2 = b1 + G;
            load_rows_raw_rs<float, 1, VPT, WC, true>(token_rows_rsrc(g, b2, B, 1, C), C, gA);
            load_rows_raw_rs<TX, 1, VPT, WC, true>(token_rows_rsrc(res, b2, B, 1, C), C, rA);
            load_rows_raw_rs<TX, 1, VPT, WC, true>(token_rows_rsrc(br, b2, B, 1, C), C, bA);
            unpack_rows<float, 1, VPT, WC>(gB, C, gv);
            unpack_rows<TX, 1, VPT, WC>(rB, C, rv);
            unpack_rows<TX, 1, VPT, WC>(bB, C, bv);
            wrap_bwd_token<TX, N, VPT, DECAY>(b1, coef, coef_stride, wv, gv, rv, bv, dwacc, sacc, dres, dbr, C, eps,
                                              red);
            b = b2;
        }
    } else {
        for (; b < B; b += G) {
            load_rows_raw<float, 1, VPT, WC, true>(g + b * C, C, gA);
            load_rows_raw<TX, 1, VPT, WC, true>(res + b * C, C, rA);
            load_rows_raw<TX, 1, VPT, WC, true>(br + b * C, C, bA);
            unpack_rows<float, 1, VPT, WC>(gA, C, gv);
            unpack_rows<TX, 1, VPT, WC>(rA, C, rv);
            unpack_rows<TX, 1, VPT, WC>(bA, C, bv);
            wrap_bwd_token<TX, N, VPT, DECAY>(b, coef, coef_stride, wv, gv, rv, bv, dwacc, sacc, dres, dbr, C, eps,
                                              red);
        }
    }
    float* dwp = dw_part + (int64_t)blockIdx.x * C;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int c0 = (k * blockDim.x + threadIdx.x) * WC;
        if (c0 < C) store_run<float, WC>(dwp + c0, dwacc[k]);
    }
    if (threadIdx.x < NS) scal_out[(int64_t)blockIdx.x * NS + threadIdx.x] = sacc;
}

// Workgroups of more than 256 lanes hold one token at a time.
template <typename TX, int N, int VPT, bool DECAY>
__global__ MHC_ROW_BOUNDS(false) __attribute__((amdgpu_waves_per_eu(4))) void wrap_bwd_kernel(
    const float* __restrict__ g, const TX* __restrict__ res, const TX* __restrict__ br, const float* __restrict__ w,
    const float* __restrict__ coef, int64_t coef_stride, TX* __restrict__ dres, TX* __restrict__ dbr,
    float* __restrict__ dw_part, float* __restrict__ scal_out, int64_t B, int C, float eps) {
    wrap_bwd_rows<TX, N, VPT, false, DECAY>(g, res, br, w, coef, coef_stride, dres, dbr, dw_part, scal_out, B, C, eps);
}

// Up to 256 lanes: two tokens in flight (register prefetch).
template <typename TX, int N, int VPT, bool DECAY>
__global__ MHC_ROW_BOUNDS(true) void wrap_bwd_pf_kernel(
    const float* __restrict__ g, const TX* __restrict__ res, const TX* __restrict__ br, const float* __restrict__ w,
    const float* __restrict__ coef, int64_t coef_stride, TX* __restrict__ dres, TX* __restrict__ dbr,
    float* __restrict__ dw_part, float* __restrict__ scal_out, int64_t B, int C, float eps) {
    wrap_bwd_rows<TX, N, VPT, true, DECAY>(g, res, br, w, coef, coef_stride, dres, dbr, dw_part, scal_out, B, C, eps);
}

// ---------------------------------------------------------------------------
// Dynamic-H backward, pass 1: the row sums of each token and nothing else.
// One wave per token streams G, r and b in 4-channel chunks (lane l takes
// chunks l, l + 64, ...; kRedChunks of them in flight per lane), forms the
// sums of wrap_bwd_token
//   ss = sum xa^2, gwx = sum G w xa, u_j = sum G X_j, v_j = sum G w X_j,
//   z_j = sum xa X_j,
// adds them over the wave (fixed order) and writes the per-token scalars in
// the layout of the coefficient backward (dM[n*n], dh_post_act[n],
// dh_pre_act[n], 1/r, k2) to scal_out[b][n*n+2n+2], and the per-token
// factors of the stream parts to ep_out[b][kWrapEp]: with w_j the d r weight
// of stream j, cm_j = (1/n) sum_i M_ij and hs = (1/n) sum_i h_post_i,
//   (A_r, B_r, A_b, B_b) = (sum_j w_j cm_j, sum_j w_j h_pre_j, cm_1, h_pre_1),
// d r = A_r G + B_r gxa + ... and d b = A_b G + B_b gxa + ... with
// gxa = (hs/r) w G - k2 xa; the record holds the factors of G, w G and xa:
//   A_r, B_r hs/r, A_b, B_b hs/r, h_pre_0..3, hs/r, -B_r k2, -B_b k2, 0
// (the last slot is free for s).  The stream parts of d r / d b and dw are formed
// by the projection backward, which reads G once more: that read costs less
// than writing the stream parts here and reading
// them back there, and this pass then only reads.
// ---------------------------------------------------------------------------
constexpr int kRedChunks = 4;

template <typename TX, int N, bool DECAY>
__global__ __launch_bounds__(256) void wrap_bwd_red_kernel(const float* __restrict__ g, const TX* __restrict__ res,
                                                           const TX* __restrict__ br, const float* __restrict__ w,
                                                           const float* __restrict__ coef, int64_t coef_stride,
                                                           float* __restrict__ scal_out, float* __restrict__ ep_out,
                                                           int64_t B, int C, float eps) {
    constexpr int NS = N * N + 2 * N;
    constexpr int NR = 2 + 3 * N;
    constexpr int U = kRedChunks;
    constexpr int XW = (int)sizeof(TX);  // 32-bit words of one 4-channel chunk of r or b
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t b = (int64_t)blockIdx.x * (blockDim.x / kWave) + (int64_t)wave_uniform(threadIdx.x / kWave);
    if (b >= B) return;
    const float* cf = coef + b * coef_stride;
    float hp[N], cm[N], hs = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        hp[j] = cf[j];
        hs += cf[N + j];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) s += cf[2 * N + i * N + j];
        cm[j] = s * (1.f / N);
    }
    hs *= 1.f / N;
    float rs[NR];
#pragma unroll
    for (int q = 0; q < NR; ++q) rs[q] = 0.f;
    const float* gb = g + b * (int64_t)C;
    const TX* rb = res + b * (int64_t)C;
    const TX* bb = br + b * (int64_t)C;
    const int nq = C / 4;
    for (int q0 = 0; q0 < nq; q0 += U * kWave) {
        // all loads of the U chunks first (chunks past the row read chunk 0)
        uint4 graw[U], wraw[U];
        uint32_t rraw[U][XW], braw[U][XW];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + u * kWave + lane;
            const int c0 = (q < nq ? q : 0) * 4;
            graw[u] = ld16_nt(gb + c0);
            wraw[u] = *reinterpret_cast<const uint4*>(w + c0);
            if constexpr (XW == 2) {
                const uint2 a = ld8_nt(rb + c0), c = ld8_nt(bb + c0);
                rraw[u][0] = a.x; rraw[u][1] = a.y;
                braw[u][0] = c.x; braw[u][1] = c.y;
            } else {
                const uint4 a = ld16_nt(rb + c0), c = ld16_nt(bb + c0);
                rraw[u][0] = a.x; rraw[u][1] = a.y; rraw[u][2] = a.z; rraw[u][3] = a.w;
                braw[u][0] = c.x; braw[u][1] = c.y; braw[u][2] = c.z; braw[u][3] = c.w;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (q0 + u * kWave + lane >= nq) continue;
            const float gv[4] = {__uint_as_float(graw[u].x), __uint_as_float(graw[u].y), __uint_as_float(graw[u].z),
                                 __uint_as_float(graw[u].w)};
            const float wv[4] = {__uint_as_float(wraw[u].x), __uint_as_float(wraw[u].y), __uint_as_float(wraw[u].z),
                                 __uint_as_float(wraw[u].w)};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float r, bv;
                if constexpr (XW == 2) {
                    const uint32_t wr = rraw[u][e >> 1], wb = braw[u][e >> 1];
                    r = __uint_as_float((e & 1) ? (wr & 0xffff0000u) : (wr << 16));
                    bv = __uint_as_float((e & 1) ? (wb & 0xffff0000u) : (wb << 16));
                } else {
                    r = __uint_as_float(rraw[u][e]);
                    bv = __uint_as_float(braw[u][e]);
                }
                float x[N];
                wrap_streams<TX, N, DECAY>(r, bv, x);
                float xa = 0.f;
#pragma unroll
                for (int j = 0; j < N; ++j) xa += hp[j] * x[j];
                const float gg = gv[e];
                const float wg = wv[e] * gg;
                rs[0] += xa * xa;
                rs[1] += wg * xa;
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    rs[2 + j] += gg * x[j];
                    rs[2 + N + j] += wg * x[j];
                    rs[2 + 2 * N + j] += xa * x[j];
                }
            }
        }
    }
    wave_sum<NR>(rs);
    const float inv = 1.f / sqrtf(rs[0] / (float)C + eps);
    const float gwx = rs[1];
    const float k2 = hs * gwx * inv * inv * inv / (float)C;
    float v[NS + 2];
#pragma unroll
    for (int t = 0; t < NS + 2; ++t) {
        if (t < N * N) {
            v[t] = rs[2 + t % N] * (1.f / N);  // dM_ij = u_j / n
        } else if (t < N * N + N) {
            v[t] = gwx * inv * (1.f / N);  // dh_post_act_i
        } else if (t < NS) {
            const int j = t - N * N - N;
            v[t] = hs * inv * rs[2 + N + j] - k2 * rs[2 + 2 * N + j];  // dh_pre_act_j
        } else {
            v[t] = (t == NS) ? inv : k2;
        }
    }
    float* so = scal_out + b * (NS + 2);
#pragma unroll
    for (int t = 0; t < NS + 2; ++t) {
        if (lane == t) so[t] = v[t];
    }
    float ep[kWrapEp];
#pragma unroll
    for (int t = 0; t < kWrapEp; ++t) ep[t] = 0.f;
    float a_r = cm[0], b_r = hp[0], a_b = 0.f, b_b = 0.f;
    if constexpr (N > 2) {
        a_r += res_weight<2, DECAY>() * cm[2];
        b_r += res_weight<2, DECAY>() * hp[2];
    }
    if constexpr (N > 3) {
        a_r += res_weight<3, DECAY>() * cm[3];
        b_r += res_weight<3, DECAY>() * hp[3];
    }
    if constexpr (N > 1) {
        a_b = cm[1];
        b_b = hp[1];
    }
    const float hsi = hs * inv;
    ep[0] = a_r;
    ep[1] = b_r * hsi;
    ep[2] = a_b;
    ep[3] = b_b * hsi;
#pragma unroll
    for (int j = 0; j < N; ++j) ep[4 + j] = hp[j];
    ep[8] = hsi;
    ep[9] = -b_r * k2;
    ep[10] = -b_b * k2;
    float* eo = ep_out + b * kWrapEp;
#pragma unroll
    for (int t = 0; t < kWrapEp; ++t) {
        if (lane == t) eo[t] = ep[t];
    }
}

// ---------------------------------------------------------------------------
// Projection of the synthesised row: P[b][o] = sum_j sum_c X_j[b][c]
// Phi[o][j*C + c], and sum_j sum_c X_j^2, on bf16 MFMA 16x16x32.  Workgroup =
// TB = 16*MT tokens x one channel range, walked in stages of 128 channels:
// the residual and branch pieces of a stage are loaded as whole 256-byte row
// slices and staged in LDS; wave w takes the 32-channel step w of the stage,
// forms the stream operands of its rows in registers and runs them against
// the Phi fragments at k = j*C + c (1 KB contiguous loads in the fragment
// order of phi_split_kernel).  bf16 storage: every stream is exact in bf16,
// so P = X.(hi + mid + lo) (three MFMAs per stream and N-tile; two, hi and
// mid, for the decay streams, whose lo term is below 2^-17 of a term at
// most 0.1 of the residual's), and sum X^2 runs on packed pairs.  fp32
// storage: X is split into hi/mid/lo too and the six products down to 2^-16
// relative weight are kept, as in proj_mfma_kernel.  p_part[ks][B][32],
// ss_part[ks][B].
// Pipeline per stage s: the r/b pieces of s+1 load while s computes; the Phi
// fragments of streams {0,1} and {2,3} reload right after their MFMAs, so
// each half's next fragments load behind the other half's work.  Blocks
// start at different stages by XCD: concurrent XCDs read different columns,
// and the blocks of one XCD share a small window of Phi in its L2.
// ---------------------------------------------------------------------------
typedef __bf16 wbf16x8_t __attribute__((ext_vector_type(8)));
typedef float wf32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int wu32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ wf32x4_t wmfma16x16x32(wu32x4_t a, wu32x4_t b, wf32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(wbf16x8_t, a), __builtin_bit_cast(wbf16x8_t, b),
                                                   c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t wpack(float lo, float hi) { return pack_bf16x2(lo, hi); }

__device__ __forceinline__ void wsplit3(float v, float& h, float& m, float& l) {
    h = bf16_to_f32(f32_to_bf16(v));
    const float r = v - h;
    m = bf16_to_f32(f32_to_bf16(r));
    l = r - m;
}

__device__ __forceinline__ wu32x4_t wop(const uint4& q) { return wu32x4_t{q.x, q.y, q.z, q.w}; }

template <typename TX> constexpr int wproj_mt() { return sizeof(TX) == 2 ? 4 : 2; }

typedef __bf16 wbf16x2_t __attribute__((ext_vector_type(2)));

// ss + a.x^2 + a.y^2 for a packed bf16 pair (v_dot2c_f32_bf16; the squares
// of bf16 values are exact in fp32)
__device__ __forceinline__ float wsq2(uint32_t a, float ss) {
    const wbf16x2_t v = __builtin_bit_cast(wbf16x2_t, a);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, ss, false);
}

// Phi planes a stream's products use: bf16 storage keeps hi and mid only for
// the decay streams (j >= 2: X_j <= 0.1 |r|), whose lo term is below 2^-17
// of an already small term.
template <typename TX, int J> constexpr int wproj_planes() { return (sizeof(TX) == 2 && J >= 2) ? 2 : 3; }

// Stream J's MFMA products for one M-tile: r/b hold the tile row's 8
// channels (raw 16-byte pieces and their values), g the stream's Phi
// fragments (plane p, N-tile nt at index 2p + nt).  bf16 storage: the stream
// operand is the stored bf16 pair (r and b as loaded; the decay streams
// packed from r * 0.1^(j-1) by the round-to-nearest-even conversion that
// stores them), and sum X^2 runs on packed pairs.
template <typename TX, int J, bool DECAY>
__device__ __forceinline__ void wproj_stream(const uint4 (&rw)[sizeof(TX) / 2], const uint4 (&bw)[sizeof(TX) / 2],
                                             const float (&r)[8], const float (&b)[8], const uint4* g,
                                             wf32x4_t (&acc)[2], float& ss) {
    if constexpr (sizeof(TX) == 2) {
        wu32x4_t a;
        if constexpr (J == 0) {
            a = wop(rw[0]);
        } else if constexpr (J == 1) {
            a = wop(bw[0]);
        } else {
            constexpr float m = decay_mult<J>();
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] = DECAY ? wpack(r[2 * e] * m, r[2 * e + 1] * m) : 0u;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = wsq2(a[e], ss);
        // g[2 p + nt]: plane p of output tile nt, where tile 1 (rows
        // 16..23) holds [hi | mid] at p = 0 and [lo | 0] at p = 1
        // (wrap_phi_pack_kernel), so its last plane is not there
        constexpr int PL = wproj_planes<TX, J>();
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
            for (int p = 0; p < PL - nt; ++p) acc[nt] = wmfma16x16x32(a, wop(g[2 * p + nt]), acc[nt]);
        }
    } else {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            x[e] = wrap_stream<TX, J, DECAY>(r[e], b[e]);
            ss += x[e] * x[e];
        }
        wu32x4_t ah, am, al;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float h0, m0, l0, h1, m1, l1;
            wsplit3(x[2 * e], h0, m0, l0);
            wsplit3(x[2 * e + 1], h1, m1, l1);
            ah[e] = wpack(h0, h1);
            am[e] = wpack(m0, m1);
            al[e] = wpack(l0, l1);
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            acc[nt] = wmfma16x16x32(ah, wop(g[0 + nt]), acc[nt]);
            acc[nt] = wmfma16x16x32(ah, wop(g[2 + nt]), acc[nt]);
            acc[nt] = wmfma16x16x32(am, wop(g[0 + nt]), acc[nt]);
            acc[nt] = wmfma16x16x32(ah, wop(g[4 + nt]), acc[nt]);
            acc[nt] = wmfma16x16x32(am, wop(g[2 + nt]), acc[nt]);
            acc[nt] = wmfma16x16x32(al, wop(g[0 + nt]), acc[nt]);
        }
    }
}

template <typename TX, int N, bool DECAY>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void wrap_proj_kernel(
    const TX* __restrict__ res, const TX* __restrict__ br, const uint4* __restrict__ phif,
    float* __restrict__ p_part, float* __restrict__ ss_part, int64_t B, int C, int64_t cchunk) {
    constexpr int MT = wproj_mt<TX>();
    constexpr int TB = 16 * MT;
    constexpr int KP = 32;  // padded projection rows
    constexpr int KS = 128;
    constexpr int EPV = 16 / (int)sizeof(TX);
    constexpr int VPR = KS / EPV;
    constexpr int RPP = 256 / VPR;
    constexpr int PASSES = TB / RPP;
    constexpr int PITCH = KS * (int)sizeof(TX) + 16;
    constexpr int XW = sizeof(TX) / 2;
    constexpr int NSTR = DECAY ? N : (N < 2 ? N : 2);  // streams with nonzero values
    constexpr int NHA = NSTR < 2 ? NSTR : 2;           // streams of the first Phi half
    constexpr int NHB = NSTR - NHA;
    constexpr int PLB = wproj_planes<TX, 2>();  // planes of the decay streams
    constexpr bool PK = sizeof(TX) == 2;               // packed rows 16..23 (five Phi slots)
    static_assert(N == 4, "wrapper projection is instantiated for n = 4");
    static_assert(PASSES * RPP == TB, "stage rows");
    static_assert(3 * 9 * MT * 64 * 4 <= 2 * 2 * TB * PITCH, "epilogue reuses the stage buffers");
    __shared__ __align__(16) char xs[2][2][TB * PITCH];  // [buf][r | b]

    const int lane = threadIdx.x & 63;
    const int wave = (int)wave_uniform(threadIdx.x >> 6);
    const int row = lane & 15;
    const int kg = lane >> 4;
    const int64_t K = (int64_t)N * C;
    const int64_t ksteps = K / 32;
    const int64_t tok0 = (int64_t)blockIdx.x * TB;
    const int64_t cb = (int64_t)blockIdx.y * cchunk;
    const int64_t ce = (cb + cchunk < C) ? cb + cchunk : C;
    const int64_t nst = ce > cb ? (ce - cb + KS - 1) / KS : 0;

    wf32x4_t acc[MT][2];
    float ss[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        acc[mt][0] = wf32x4_t{0.f, 0.f, 0.f, 0.f};
        acc[mt][1] = wf32x4_t{0.f, 0.f, 0.f, 0.f};
        ss[mt] = 0.f;
    }
    // rows of this block past the batch read zeros (resource range); the
    // whole offset is per lane, so a column past C in the last row does too
    const int64_t rows = (B - tok0 < TB) ? B - tok0 : TB;
    const uint32_t xbytes = (uint32_t)(rows * C * (int64_t)sizeof(TX));
    const buf_rsrc_t rrs = make_buf_rsrc(res + tok0 * C, xbytes);
    const buf_rsrc_t brs = make_buf_rsrc(br + tok0 * C, xbytes);
    const buf_rsrc_t prs = make_buf_rsrc(phif, (uint32_t)((PK ? 5 : 6) * ksteps * 64 * 16));
    const int lrow = threadIdx.x / VPR;
    const int lvec = threadIdx.x % VPR;
    const uint32_t xoff = (uint32_t)(((int64_t)lrow * C + lvec * EPV) * (int64_t)sizeof(TX));
    const uint32_t xpass = (uint32_t)((int64_t)RPP * C * (int64_t)sizeof(TX));
    // start stage by XCD (workgroups go round-robin over the 8 XCDs)
    const int64_t xcd = ((int64_t)blockIdx.x + (int64_t)blockIdx.y * gridDim.x) % 8;
    const int64_t rot = nst > 0 ? (xcd * nst) / 8 : 0;
    auto srot = [&](int64_t st) __attribute__((always_inline)) {
        const int64_t r = st + rot;
        return r < nst ? r : r - nst;
    };
    auto clampst = [&](int64_t st) __attribute__((always_inline)) { return st < nst ? st : (int64_t)0; };

    uint4 F[2][PASSES];
    uint4 GA[6 * (NHA > 0 ? NHA : 1)];
    uint4 GB[6 * (NHB > 0 ? NHB : 1)];
    // Lanes whose 8 channels lie past the chunk end load from kBufOff (zeros),
    // so the commit stores the loaded words as they are: a mask applied at
    // the commit was moved by the compiler to just after the loads, and each
    // stage then waited for its own prefetch in the middle of its MFMAs.
    auto fetch_x = [&](int64_t st) __attribute__((always_inline)) {
        const int64_t c0 = cb + srot(st) * KS;
        const uint32_t base =
            c0 + lvec * EPV < ce ? xoff + (uint32_t)(c0 * (int64_t)sizeof(TX)) : kBufOff;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            F[0][p] = buf_ld16<true, true>(rrs, base + p * xpass, 0u);
            F[1][p] = buf_ld16<true, true>(brs, base + p * xpass, 0u);
        }
    };
    // Phi fragments of streams j0 .. j0+nj-1 at this wave's 32 channels of
    // stage st (clamped to the last k step: past ce the operands are zero);
    // pl planes each, at slot 2p + nt (phi_split_kernel's planes; bf16
    // storage: wrap_phi_pack_kernel's five slots, tile 1 one plane short).
    auto fetch_phi = [&](uint4* g, int j0, int nj, int pl, int64_t st) __attribute__((always_inline)) {
        const int64_t c0 = cb + srot(st) * KS + wave * 32;
#pragma unroll
        for (int jj = 0; jj < nj; ++jj) {
            int64_t kstep = ((int64_t)(j0 + jj) * C + c0) / 32;
            kstep = kstep < ksteps ? kstep : ksteps - 1;
            const uint32_t so = (uint32_t)(kstep * 64 * 16);
#pragma unroll
            for (int q = 0; q < 2 * pl - (PK ? 1 : 0); ++q)
                g[6 * jj + q] = buf_ld16<false>(prs, (uint32_t)((q * ksteps * 64 + lane) * 16), so);
        }
    };
    auto commit = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int p = 0; p < PASSES; ++p)
                *reinterpret_cast<uint4*>(&xs[buf][a][(lrow + p * RPP) * PITCH + lvec * 16]) = F[a][p];
        }
    };
    // MFMAs of streams J0 (and J0 + 1 when two) against fragments g
    auto compute_half = [&](int buf, const uint4* g, auto j0c, auto njc) __attribute__((always_inline)) {
        constexpr int J0 = decltype(j0c)::value;
        constexpr int NJ = decltype(njc)::value;
        const int off = row * PITCH + (wave * 32 + kg * 8) * (int)sizeof(TX);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            uint4 rw[XW], bw[XW];
#pragma unroll
            for (int q = 0; q < XW; ++q) {
                rw[q] = *reinterpret_cast<const uint4*>(&xs[buf][0][off + mt * 16 * PITCH + 16 * q]);
                bw[q] = *reinterpret_cast<const uint4*>(&xs[buf][1][off + mt * 16 * PITCH + 16 * q]);
            }
            float r[8], b[8];
#pragma unroll
            for (int q = 0; q < XW; ++q) {
                const uint32_t rr[4] = {rw[q].x, rw[q].y, rw[q].z, rw[q].w};
                const uint32_t bb[4] = {bw[q].x, bw[q].y, bw[q].z, bw[q].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (sizeof(TX) == 2) {
                        r[2 * e] = __uint_as_float(rr[e] << 16);
                        r[2 * e + 1] = __uint_as_float(rr[e] & 0xffff0000u);
                        b[2 * e] = __uint_as_float(bb[e] << 16);
                        b[2 * e + 1] = __uint_as_float(bb[e] & 0xffff0000u);
                    } else {
                        r[4 * q + e] = __uint_as_float(rr[e]);
                        b[4 * q + e] = __uint_as_float(bb[e]);
                    }
                }
            }
            if constexpr (NJ > 0) wproj_stream<TX, J0, DECAY>(rw, bw, r, b, g, acc[mt], ss[mt]);
            if constexpr (NJ > 1) wproj_stream<TX, J0 + 1, DECAY>(rw, bw, r, b, g + 6, acc[mt], ss[mt]);
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I2 = std::integral_constant<int, 2>;
    using IHA = std::integral_constant<int, NHA>;
    using IHB = std::integral_constant<int, NHB>;

    if (nst > 0) {
        fetch_x(0);
        fetch_phi(GA, 0, NHA, 3, 0);
        if constexpr (NHB > 0) fetch_phi(GB, 2, NHB, PLB, 0);
        commit(0);
        __syncthreads();
        for (int64_t st = 0; st < nst; ++st) {
            const int buf = (int)(st & 1);
            fetch_x(clampst(st + 1));
            __builtin_amdgcn_sched_barrier(0);
            compute_half(buf, GA, I0{}, IHA{});
            fetch_phi(GA, 0, NHA, 3, clampst(st + 1));
            if constexpr (NHB > 0) {
                compute_half(buf, GB, I2{}, IHB{});
                fetch_phi(GB, 2, NHB, PLB, clampst(st + 1));
            }
            commit(buf ^ 1);
            __syncthreads();
        }
    }
    __syncthreads();  // the stage buffers become the cross-wave reduction area
    float (*red)[9 * MT][64] = reinterpret_cast<float (*)[9 * MT][64]>(&xs[0][0][0]);

    // waves 1..3 hand their partials to wave 0 through LDS
    if (wave > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave - 1][(mt * 2 + nt) * 4 + i][lane] = acc[mt][nt][i];
            }
            red[wave - 1][8 * MT + mt][lane] = ss[mt];
        }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll 1
    for (int q = 0; q < 3; ++q) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mt][nt][i] += red[q][(mt * 2 + nt) * 4 + i][lane];
            }
            ss[mt] += red[q][8 * MT + mt][lane];
        }
    }
    float* pp = p_part + (int64_t)blockIdx.y * B * KP;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if constexpr (PK) {
            // packed tile: row 16 + c = column c (hi, lo) + column c + 8 (mid);
            // rows 24..31 are zero
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = acc[mt][1][i] + __shfl_xor(acc[mt][1][i], 8);
                acc[mt][1][i] = row < 8 ? v : 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t tok = tok0 + mt * 16 + kg * 4 + i;
            if (tok < B) {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) pp[tok * KP + nt * 16 + row] = acc[mt][nt][i];
            }
        }
        float s2 = ss[mt];
        s2 = xor32_add(xor16_add(s2));
        const int64_t tok = tok0 + mt * 16 + row;
        if (kg == 0 && tok < B) ss_part[(int64_t)blockIdx.y * B + tok] = s2;
    }
}

// Phi of the n = 4 wrapper (24 rows) as the bf16 MFMA B fragments of
// wrap_proj_kernel's bf16-storage path: five slots per 32-wide k step ks,
//   phif[(q * (K / 32) + ks) * 64 + lane]  (8 bf16, 16 bytes),
// k = 32 ks + 8 (lane / 16) .. + 7, c = lane % 16, slot q = 2 p + nt as in
// phi_split_kernel for tile 0 (rows 0..15), while tile 1 (rows 16..23,
// half empty) takes two slots instead of three:
//   q = 0, 2, 4: hi, mid, lo of row c
//   q = 1:       hi of row 16 + c (c < 8), mid of row 16 + c - 8 (c >= 8)
//   q = 3:       lo of row 16 + c (c < 8), zero (c >= 8)
// One MFMA over slot 1 leaves the hi and mid products of rows 16..23 in
// columns c and c + 8, which the kernel adds once at the end.
__global__ __launch_bounds__(256) void wrap_phi_pack_kernel(const float* __restrict__ pre,
                                                            const float* __restrict__ post,
                                                            const float* __restrict__ res, int64_t K,
                                                            uint4* __restrict__ phif) {
    const int64_t ksteps = K / 32;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < ksteps * 64;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i & 63);
        const int64_t ks = i >> 6;
        const int c = lane & 15;
        const int64_t k = ks * 32 + 8 * (lane >> 4);
        float v0[8], v1[8];
        load_run<float, 8>(phi_row(pre, post, res, 4, c, K) + k, v0);
        load_run<float, 8>(phi_row(pre, post, res, 4, 16 + (c & 7), K) + k, v1);
        uint32_t w[5][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float h0, m0, l0, h1, m1, l1;
            wsplit3(v0[2 * e], h0, m0, l0);
            wsplit3(v0[2 * e + 1], h1, m1, l1);
            w[0][e] = wpack(h0, h1);
            w[2][e] = wpack(m0, m1);
            w[4][e] = wpack(l0, l1);
            wsplit3(v1[2 * e], h0, m0, l0);
            wsplit3(v1[2 * e + 1], h1, m1, l1);
            w[1][e] = c < 8 ? wpack(h0, h1) : wpack(m0, m1);
            w[3][e] = c < 8 ? wpack(l0, l1) : 0u;
        }
#pragma unroll
        for (int q = 0; q < 5; ++q) phif[(q * ksteps + ks) * 64 + lane] = make_uint4(w[q][0], w[q][1], w[q][2], w[q][3]);
    }
}

// ---------------------------------------------------------------------------
// Projection backward of the wrapper, dynamic H, pass 2, over channels c
// (bf16 MFMA 16x16x32 with hi/lo split fp32 operands, as
// proj_bwd_mfma_kernel):
//   d r[b][c] = sum_j w_j dX_j + s[b] sum_j w_j X_j + sum_o dP[b][o] Phi_r[o][c]
//   d b[b][c] = dX_1           + s[b] X_1           + sum_o dP[b][o] Phi[o][C + c]
//   dX_j = cm_j G + h_pre_j gxa,  gxa = w gy / r - xa k2,  gy = hs G
//   dPhi_part[tile][o][j*C + c] = sum_{b in tile} dP[b][o] X_j[b][c]
//   dw_part[tile][c] = sum_{b in tile} gy xa / r
// with w_j the d r weight of stream j (1, 0, 0.1, 0.01, ...), Phi_r =
// sum_j w_j Phi_j (the residual-derived streams share one dx_proj chain) and
// the per-token factors of wrap_bwd_red_kernel (sum_j w_j dX_j = A_r G +
// B_r gxa, dX_1 = A_b G + B_b gxa).
// Every term is summed in fp32 and d r / d b are rounded once to the storage
// dtype.  Workgroup = 8 waves x 16 columns; stages of 32 tokens with r, b
// and G staged in LDS (three stages in flight in registers); results go
// through one LDS tile per output and leave with coalesced 16-byte stores.
//
// RES = false: the H_res rows of dP are zero (every stream receives G / n
// through the stream mean, so dM is constant down each column, and the
// Sinkhorn pass, which ends with a column normalisation, maps it to zero:
// wrap_res_grad_vanishes in abi.hip).  Only the 2N pre / post rows are
// carried, and their hi / lo halves share one MFMA:
//   dPhi: A rows 0..7 = dP_hi^T, rows 8..15 = dP_lo^T over the stage's
//         tokens; dPhi[o] = D[o] + D[o + 8] (one 16x16x32 MFMA per stream
//         instead of four);
//   dx:   k = 0..7 Phi_hi x dP_hi, 8..15 Phi_lo x dP_hi, 16..23 Phi_hi x
//         dP_lo, 24..31 zero (one MFMA per output and token half instead of
//         three).
// dphi_part then holds 2N rows per tile.
// ---------------------------------------------------------------------------
typedef __bf16 wbf16x8b_t __attribute__((ext_vector_type(8)));

// Workgroup of the projection backward: 8 waves x 16 channels, one per CU at
// two waves per SIMD of registers.  A stage's row pieces are 256 bytes of
// r and b and 512 of G per token; against 4-wave workgroups over 64 channels
// (three per CU) the kernel went from 4.8-5.2 to 4.7 ms at C5.  The loads
// and stores of this shape alone, with no compute, take 4.36-4.42 ms at C5
// (5.1-5.2 TB/s for 8 bytes read and 4 written per element).
constexpr int kWpbThreads = 512;
constexpr int kWpbCols = kWpbThreads / 64 * 16;
// Waves per SIMD the register allocation targets: two (one 8-wave workgroup
// per CU either way), so three stages of rows and records fit in registers.
template <typename TX> constexpr int kWpbWaves() { return 2; }

template <typename TX> constexpr int wpb_pitch() { return kWpbCols * (int)sizeof(TX) + 8; }
constexpr int kWDpPitch = 40;

__device__ __forceinline__ void wsplit_pack8(const float (&v)[8], wu32x4_t& hi, wu32x4_t& lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float h0 = bf16_to_f32(f32_to_bf16(v[2 * e]));
        const float h1 = bf16_to_f32(f32_to_bf16(v[2 * e + 1]));
        hi[e] = wpack(h0, h1);
        lo[e] = wpack(v[2 * e] - h0, v[2 * e + 1] - h1);
    }
}

template <typename TX>
__device__ __forceinline__ void wlds_get4(const char* p, float (&v)[4]) {
    const uint2* q = reinterpret_cast<const uint2*>(p);
    if constexpr (sizeof(TX) == 2) {
        const uint2 w = q[0];
        v[0] = __uint_as_float(w.x << 16); v[1] = __uint_as_float(w.x & 0xffff0000u);
        v[2] = __uint_as_float(w.y << 16); v[3] = __uint_as_float(w.y & 0xffff0000u);
    } else {
        const uint2 a = q[0], b = q[1];
        v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
        v[2] = __uint_as_float(b.x); v[3] = __uint_as_float(b.y);
    }
}
template <typename TX>
__device__ __forceinline__ void wlds_put4(char* p, const float (&v)[4]) {
    uint2* q = reinterpret_cast<uint2*>(p);
    if constexpr (sizeof(TX) == 2) {
        q[0] = make_uint2(wpack(v[0], v[1]), wpack(v[2], v[3]));
    } else {
        q[0] = make_uint2(__float_as_uint(v[0]), __float_as_uint(v[1]));
        q[1] = make_uint2(__float_as_uint(v[2]), __float_as_uint(v[3]));
    }
}

template <typename TX, int N, bool DECAY, bool RES>
__global__ __launch_bounds__(kWpbThreads) __attribute__((amdgpu_waves_per_eu(kWpbWaves<TX>()))) void wrap_proj_bwd_kernel(
    const float* __restrict__ g, const TX* __restrict__ res, const TX* __restrict__ br, const float* __restrict__ w,
    const float* __restrict__ ep, const float* __restrict__ dP, const float* __restrict__ s_tok,
    const float* __restrict__ phi_pre, const float* __restrict__ phi_post, const float* __restrict__ phi_res,
    TX* __restrict__ dres, TX* __restrict__ dbr, float* __restrict__ dw_part, float* __restrict__ dphi_part,
    int64_t B, int C, int64_t tile) {
    constexpr int NP = 2 * N + N * N;
    constexpr int NPO = RES ? NP : 2 * N;  // rows of dphi_part
    static_assert(NP <= 32, "projection rows must fit one 32-row tile");
    static_assert(RES || 2 * N <= 8, "packed pre / post rows: at most 8");
    static_assert(N <= 4 && kWrapEp == 12, "factor record: 4 + 4 h_pre + hs/r, 2 xa factors, s");
    constexpr int NSTR = DECAY ? N : (N < 2 ? N : 2);  // streams with nonzero values
    constexpr int TB = 32;
    constexpr int NT = kWpbThreads;
    constexpr int CB = kWpbCols;
    constexpr int EPV = 16 / sizeof(TX);
    constexpr int VPR = CB / EPV;      // 16-byte vectors per r / b tile row
    constexpr int RPP = NT / VPR;
    constexpr int PASSES = TB / RPP;
    constexpr int GVPR = CB / 4;       // 16-byte vectors per G tile row
    constexpr int GRPP = NT / GVPR;
    constexpr int GPASSES = TB / GRPP;
    constexpr int PITCH = wpb_pitch<TX>();
    constexpr int GPITCH = CB * 4 + 16;
    static_assert(PASSES * RPP == TB && GPASSES * GRPP == TB, "stage rows");
    // One copy of each stage tile: a stage is committed after the barrier that
    // ends the compute of the previous one.  out_lds holds the results of the
    // stage being stored while the next stage is committed.
    __shared__ __align__(16) char rb_lds[2][TB * PITCH];  // [r | b]
    __shared__ __align__(16) char g_lds[TB * GPITCH];
    __shared__ __align__(16) char out_lds[2][TB * PITCH];  // [d r | d b]
    __shared__ __align__(16) bf16_t dps_lds[4][32 * kWDpPitch];
    __shared__ __align__(16) float ep_lds[TB][kWrapEp];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int64_t K = (int64_t)N * C;
    const int64_t cb0 = (int64_t)blockIdx.x * CB;
    const int wc0 = wave * 16;
    const bool wave_on = cb0 + wc0 < C;  // C % 16 == 0

    const int lrow = tid / VPR;
    const int lvec = tid % VPR;
    const int64_t lcol = cb0 + (int64_t)lvec * EPV;
    const bool lcol_ok = lcol < C;
    const int grow = tid / GVPR;
    const int gvec = tid % GVPR;
    const int64_t gcol = cb0 + (int64_t)gvec * 4;
    const bool gcol_ok = gcol < C;
    const bool dp_loader = tid < 256;
    const int dtk = (tid & 255) >> 3;
    const int dpo = (tid & 7) * 4;
    // factor loaders: lane tid < 3 TB takes piece tid % 3 of token tid / 3;
    // piece 2 also carries s into the last slot
    const bool ep_loader = tid < 3 * TB;
    const int etk = tid / 3;
    const int epc = tid % 3;

    // dx_proj A operands: Phi_r^T and Phi_1^T at column wc0 + lr, o = 8 lg + e
    // (RES = false: o = e, the hi, lo, hi and zero k-blocks by lg)
    wu32x4_t prh, prl, pbh, pbl;
    float wv[4];
    {
        const int64_t c = cb0 + wc0 + lr;
        float vr[8], vb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int o = RES ? 8 * lg + e : e;
            float r = 0.f, b = 0.f;
            if (wave_on && o < NP) {
                const float* rowp = phi_row(phi_pre, phi_post, phi_res, N, o, K);
                r = rowp[c];
                if constexpr (N > 1) b = rowp[C + c];
                if constexpr (N > 2) r += res_weight<2, DECAY>() * rowp[2 * (int64_t)C + c];
                if constexpr (N > 3) r += res_weight<3, DECAY>() * rowp[3 * (int64_t)C + c];
            }
            vr[e] = r;
            vb[e] = b;
        }
        wsplit_pack8(vr, prh, prl);
        wsplit_pack8(vb, pbh, pbl);
        if constexpr (!RES) {
            const wu32x4_t z = wu32x4_t{0u, 0u, 0u, 0u};
            prh = lg == 1 ? prl : (lg == 3 ? z : prh);
            pbh = lg == 1 ? pbl : (lg == 3 ? z : pbh);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[i] = wave_on ? w[cb0 + wc0 + 4 * lg + i] : 0.f;
    }
    wf32x4_t accP[NSTR][2];
#pragma unroll
    for (int j = 0; j < NSTR; ++j) {
        accP[j][0] = wf32x4_t{0.f, 0.f, 0.f, 0.f};
        accP[j][1] = wf32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    float dwacc[4] = {0.f, 0.f, 0.f, 0.f};

    const int64_t t_begin = (int64_t)blockIdx.y * tile;
    const int64_t t_end = (t_begin + tile < B) ? t_begin + tile : B;
    const int64_t nrows = t_end > t_begin ? t_end - t_begin : 0;

    // Every global access goes through a buffer resource over this block's
    // rows [t_begin, t_end) (under 2 GiB each: wrap_proj_bwd_tiles): rows
    // past t_end and lanes with nothing to load read zeros, and such stores
    // are dropped, so no access sits behind a branch and the compiler's
    // wait counts stay exact across the prefetch.  Offsets are bytes.
    const uint32_t xrow = (uint32_t)C * (uint32_t)sizeof(TX);
    const buf_rsrc_t rs_r = make_buf_rsrc(res + t_begin * C, (uint32_t)(nrows * xrow));
    const buf_rsrc_t rs_b = make_buf_rsrc(br + t_begin * C, (uint32_t)(nrows * xrow));
    const buf_rsrc_t rs_g = make_buf_rsrc(g + t_begin * C, (uint32_t)(nrows * C * 4));
    const buf_rsrc_t rs_dr = make_buf_rsrc(dres + t_begin * C, (uint32_t)(nrows * xrow));
    const buf_rsrc_t rs_db = make_buf_rsrc(dbr + t_begin * C, (uint32_t)(nrows * xrow));
    const buf_rsrc_t rs_p = make_buf_rsrc(dP + t_begin * 32, (uint32_t)(nrows * 128));
    const buf_rsrc_t rs_e = make_buf_rsrc(ep + t_begin * kWrapEp, (uint32_t)(nrows * kWrapEp * 4));
    const buf_rsrc_t rs_s = make_buf_rsrc(s_tok + t_begin, (uint32_t)(nrows * 4));
    // stage-relative lane offsets (kBufOff: nothing to access)
    const uint32_t xo = lcol_ok ? (uint32_t)lrow * xrow + (uint32_t)(lcol * (int64_t)sizeof(TX)) : kBufOff;
    const uint32_t go = gcol_ok ? ((uint32_t)grow * (uint32_t)C + (uint32_t)gcol) * 4u : kBufOff;
    const uint32_t po = dp_loader ? (uint32_t)(dtk * 32 + dpo) * 4u : kBufOff;
    const uint32_t eo = ep_loader ? (uint32_t)(etk * kWrapEp + 4 * epc) * 4u : kBufOff;
    const uint32_t so = (ep_loader && epc == 2) ? (uint32_t)etk * 4u : kBufOff;

    // A stage's row tiles and per-token records are fetched three stages
    // ahead, into one of three register sets, so two stages stay in flight
    // while one is committed.
    struct Fetched {
        uint4 v[2][PASSES];
        uint4 gq[GPASSES];
        uint4 e, dp;
        uint32_t s;
    };
    Fetched f0, f1, f2;
    // the stage of rows rel .. rel + TB - 1 (relative to t_begin)
    auto fetch = [&](Fetched& f, uint32_t rel) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const uint32_t off = xo + (rel + p * RPP) * xrow;
            f.v[0][p] = buf_ld16<true>(rs_r, off, 0u);
            f.v[1][p] = buf_ld16<true>(rs_b, off, 0u);
        }
#pragma unroll
        for (int p = 0; p < GPASSES; ++p)
            f.gq[p] = buf_ld16<true>(rs_g, go + (rel + p * GRPP) * (uint32_t)C * 4u, 0u);
    };
    auto fetch_small = [&](Fetched& sm, uint32_t rel) __attribute__((always_inline)) {
        sm.dp = buf_ld16<false>(rs_p, po + rel * 128u, 0u);
        sm.e = buf_ld16<false>(rs_e, eo + rel * (uint32_t)(kWrapEp * 4), 0u);
        sm.s = buf_ld4(rs_s, so + rel * 4u, 0u);
    };
    auto commit = [&](const Fetched& f) __attribute__((always_inline)) {
        const Fetched& sm = f;
        // The small records are consumed behind branches below; an empty use
        // of their registers here makes every lane wait for them in straight-
        // line code, so the compiler's wait counts do not carry them as
        // possibly in flight past the branches.
        asm volatile("" ::"v"(sm.dp.x), "v"(sm.dp.y), "v"(sm.dp.z), "v"(sm.dp.w), "v"(sm.e.x), "v"(sm.e.y),
                     "v"(sm.e.z), "v"(sm.e.w), "v"(sm.s));
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int row = lrow + p * RPP;
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                const uint4 v = f.v[a][p];
                uint2* pw = reinterpret_cast<uint2*>(&rb_lds[a][row * PITCH + lvec * 16]);
                pw[0] = make_uint2(v.x, v.y);
                pw[1] = make_uint2(v.z, v.w);
            }
        }
#pragma unroll
        for (int p = 0; p < GPASSES; ++p)
            *reinterpret_cast<uint4*>(&g_lds[(grow + p * GRPP) * GPITCH + gvec * 16]) = f.gq[p];
        if constexpr (!RES) {
            // token-major B rows [hi 0..7 | hi 0..7 | lo 0..7 | 0] in
            // dps_lds[0], o-major A rows [hi 0..7 ; lo 0..7] in dps_lds[2]
            if (dp_loader && dpo < 2 * N) {
                const uint32_t dw4[4] = {sm.dp.x, sm.dp.y, sm.dp.z, sm.dp.w};
                float hi[4], lo[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float v = __uint_as_float(dw4[q]);
                    hi[q] = bf16_to_f32(f32_to_bf16(v));
                    lo[q] = v - hi[q];
                }
                const uint2 h2 = make_uint2(wpack(hi[0], hi[1]), wpack(hi[2], hi[3]));
                *reinterpret_cast<uint2*>(&dps_lds[0][dtk * kWDpPitch + dpo]) = h2;
                *reinterpret_cast<uint2*>(&dps_lds[0][dtk * kWDpPitch + 8 + dpo]) = h2;
                *reinterpret_cast<uint2*>(&dps_lds[0][dtk * kWDpPitch + 16 + dpo]) =
                    make_uint2(wpack(lo[0], lo[1]), wpack(lo[2], lo[3]));
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    dps_lds[2][(dpo + q) * kWDpPitch + dtk] = f32_to_bf16(hi[q]);
                    dps_lds[2][(8 + dpo + q) * kWDpPitch + dtk] = f32_to_bf16(lo[q]);
                }
            }
        } else if (dp_loader) {
            const uint32_t dw4[4] = {sm.dp.x, sm.dp.y, sm.dp.z, sm.dp.w};
            float hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float v = dpo + q < NP ? __uint_as_float(dw4[q]) : 0.f;
                hi[q] = bf16_to_f32(f32_to_bf16(v));
                lo[q] = v - hi[q];
            }
            *reinterpret_cast<uint2*>(&dps_lds[0][dtk * kWDpPitch + dpo]) =
                make_uint2(wpack(hi[0], hi[1]), wpack(hi[2], hi[3]));
            *reinterpret_cast<uint2*>(&dps_lds[1][dtk * kWDpPitch + dpo]) =
                make_uint2(wpack(lo[0], lo[1]), wpack(lo[2], lo[3]));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                dps_lds[2][(dpo + q) * kWDpPitch + dtk] = f32_to_bf16(hi[q]);
                dps_lds[3][(dpo + q) * kWDpPitch + dtk] = f32_to_bf16(lo[q]);
            }
        }
        if (ep_loader)
            *reinterpret_cast<uint4*>(&ep_lds[etk][4 * epc]) =
                make_uint4(sm.e.x, sm.e.y, sm.e.z, epc == 2 ? sm.s : sm.e.w);
    };
    auto read16 = [&](const bf16_t* p) __attribute__((always_inline)) -> wu32x4_t {
        const uint4 q = *reinterpret_cast<const uint4*>(p);
        return wu32x4_t{q.x, q.y, q.z, q.w};
    };
    auto compute = [&]() __attribute__((always_inline)) {
        if (!wave_on) return;
        const char* rt = rb_lds[0];
        const char* bt = rb_lds[1];
        const char* gt = g_lds;
        // dPhi: B operands x_j over tokens 8 lg .. + 7 at column wc0 + lr
        wu32x4_t xh[NSTR], xl[NSTR];
        if constexpr (sizeof(TX) == 2) {
            // bf16 pairs of tokens (e, e + 1) at column c straight from the
            // raw halves; the decay streams rounded pairwise by one conversion
            const int c = wc0 + lr;
            uint32_t rr[8], bb[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int t = 8 * lg + e;
                rr[e] = *reinterpret_cast<const uint16_t*>(rt + t * PITCH + c * 2);
                bb[e] = *reinterpret_cast<const uint16_t*>(bt + t * PITCH + c * 2);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xh[0][e] = rr[2 * e] | (rr[2 * e + 1] << 16);
                if constexpr (NSTR > 1) xh[1][e] = bb[2 * e] | (bb[2 * e + 1] << 16);
                if constexpr (NSTR > 2) {
                    const float r0 = __uint_as_float(rr[2 * e] << 16), r1 = __uint_as_float(rr[2 * e + 1] << 16);
                    constexpr float m2 = decay_mult<2>();
                    xh[2][e] = wpack(r0 * m2, r1 * m2);
                    if constexpr (NSTR > 3) {
                        constexpr float m3 = decay_mult<3>();
                        xh[3][e] = wpack(r0 * m3, r1 * m3);
                    }
                }
            }
        } else {
            const int c = wc0 + lr;
            float xs[NSTR][8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int t = 8 * lg + e;
                const float r = VecIO<TX>::scalar(reinterpret_cast<const TX*>(rt + t * PITCH) + c);
                const float b = VecIO<TX>::scalar(reinterpret_cast<const TX*>(bt + t * PITCH) + c);
                float x[N];
                wrap_streams<TX, N, DECAY>(r, b, x);
#pragma unroll
                for (int j = 0; j < NSTR; ++j) xs[j][e] = x[j];
            }
#pragma unroll
            for (int j = 0; j < NSTR; ++j) wsplit_pack8(xs[j], xh[j], xl[j]);
        }
        if constexpr (!RES) {
            // rows lr < 8: dP_hi, else dP_lo (fp32 x: dP_hi x_lo into the hi rows)
            const wu32x4_t a = read16(&dps_lds[2][lr * kWDpPitch + 8 * lg]);
#pragma unroll
            for (int j = 0; j < NSTR; ++j) {
                accP[j][0] = wmfma16x16x32(a, xh[j], accP[j][0]);
                if constexpr (sizeof(TX) == 4) {
                    const wu32x4_t z = wu32x4_t{0u, 0u, 0u, 0u};
                    accP[j][0] = wmfma16x16x32(lr < 8 ? a : z, xl[j], accP[j][0]);
                }
            }
        } else {
#pragma unroll
            for (int ot = 0; ot < 2; ++ot) {
                const wu32x4_t ah = read16(&dps_lds[2][(16 * ot + lr) * kWDpPitch + 8 * lg]);
                const wu32x4_t al = read16(&dps_lds[3][(16 * ot + lr) * kWDpPitch + 8 * lg]);
#pragma unroll
                for (int j = 0; j < NSTR; ++j) {
                    accP[j][ot] = wmfma16x16x32(ah, xh[j], accP[j][ot]);
                    accP[j][ot] = wmfma16x16x32(al, xh[j], accP[j][ot]);
                    if constexpr (sizeof(TX) == 4) accP[j][ot] = wmfma16x16x32(ah, xl[j], accP[j][ot]);
                }
            }
        }
        // dx_proj^T for d r and d b: D[column wc0 + 4 lg + i][token 16 tt + lr],
        // then the stream parts and s X of the same four channels
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 16 * tt + lr;
            const wu32x4_t bh = read16(&dps_lds[0][t * kWDpPitch + 8 * lg]);
            wf32x4_t pr = wf32x4_t{0.f, 0.f, 0.f, 0.f}, pb = pr;
            pr = wmfma16x16x32(prh, bh, pr);
            pb = wmfma16x16x32(pbh, bh, pb);
            if constexpr (RES) {
                const wu32x4_t bl = read16(&dps_lds[1][t * kWDpPitch + 8 * lg]);
                pr = wmfma16x16x32(prl, bh, pr);
                pr = wmfma16x16x32(prh, bl, pr);
                pb = wmfma16x16x32(pbl, bh, pb);
                pb = wmfma16x16x32(pbh, bl, pb);
            }
            const float4 e0 = *reinterpret_cast<const float4*>(&ep_lds[t][0]);
            const float4 e1 = *reinterpret_cast<const float4*>(&ep_lds[t][4]);
            const float4 e2 = *reinterpret_cast<const float4*>(&ep_lds[t][8]);
            // d r = (A_r + B_r (hs/r) w) G - B_r k2 xa + s sx + dx_proj, d b alike
            const float a_r = e0.x, brh = e0.y, a_b = e0.z, bbh = e0.w;
            const float hp[4] = {e1.x, e1.y, e1.z, e1.w};
            const float hsi = e2.x, kr = e2.y, kb = e2.z, st = e2.w;
            const int col = wc0 + 4 * lg;
            const int boff = t * PITCH + col * (int)sizeof(TX);  // 8-byte aligned
            float rv[4], bv[4];
            wlds_get4<TX>(rt + boff, rv);
            wlds_get4<TX>(bt + boff, bv);
            const float4 gq = *reinterpret_cast<const float4*>(gt + t * GPITCH + col * 4);
            const float gv[4] = {gq.x, gq.y, gq.z, gq.w};
            float drv[4], dbv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x[N];
                wrap_streams<TX, N, DECAY>(rv[i], bv[i], x);
                float xa = 0.f;
#pragma unroll
                for (int j = 0; j < N; ++j) xa += hp[j] * x[j];
                float sx = x[0];
                if constexpr (N > 2) sx += res_weight<2, DECAY>() * x[2];
                if constexpr (N > 3) sx += res_weight<3, DECAY>() * x[3];
                const float gg = gv[i];
                dwacc[i] = fmaf(hsi, gg * xa, dwacc[i]);
                drv[i] = fmaf(st, sx, fmaf(kr, xa, fmaf(fmaf(brh, wv[i], a_r), gg, pr[i])));
                dbv[i] = (N > 1) ? fmaf(st, x[N > 1 ? 1 : 0], fmaf(kb, xa, fmaf(fmaf(bbh, wv[i], a_b), gg, pb[i]))) : pb[i];
            }
            wlds_put4<TX>(out_lds[0] + boff, drv);
            wlds_put4<TX>(out_lds[1] + boff, dbv);
        }
    };
    auto store = [&](uint32_t rel) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int row = lrow + p * RPP;
            const uint32_t off = xo + (rel + p * RPP) * xrow;
            const uint2* pr = reinterpret_cast<const uint2*>(&out_lds[0][row * PITCH + lvec * 16]);
            const uint2* pb = reinterpret_cast<const uint2*>(&out_lds[1][row * PITCH + lvec * 16]);
            const uint2 r0 = pr[0], r1 = pr[1], b0 = pb[0], b1 = pb[1];
            buf_st16<true>(rs_dr, off, 0u, make_uint4(r0.x, r0.y, r1.x, r1.y));
            buf_st16<true>(rs_db, off, 0u, make_uint4(b0.x, b0.y, b1.x, b1.y));
        }
    };

    // Two register sets: stage i+2 is fetched while stage i computes
    // (fetches and commits past the last row read zeros).
    auto step = [&](uint32_t r, Fetched& fc, Fetched& fp) __attribute__((always_inline)) {
        // stage r is in LDS, fc holds stage r + TB, fp is free
        fetch_small(fp, r + 3 * TB);
        fetch(fp, r + 3 * TB);
        compute();
        __syncthreads();
        store(r);
        commit(fc);
        __syncthreads();
    };
    const uint32_t nr = (uint32_t)nrows;
    if constexpr (!RES) {
        // k = 24..31 of the token-major dP rows stay zero
        if (tid < TB * 8) dps_lds[0][(tid >> 3) * kWDpPitch + 24 + (tid & 7)] = 0;
    }
    fetch_small(f0, 0u);
    fetch(f0, 0u);
    commit(f0);
    fetch_small(f1, TB);
    fetch(f1, TB);
    fetch_small(f2, 2 * TB);
    fetch(f2, 2 * TB);
    __syncthreads();
    // Whole triples of stages: stages past the last row read only zeros, add
    // zeros and store nothing.  An exit between them would leave a path
    // (seen by the compiler, never taken) from a stage back to the loop head
    // with its fetch outstanding, and the wait counts would then hold every
    // loop head until that fetch had landed.
    for (uint32_t r0 = 0; r0 < nr; r0 += 3 * TB) {
        step(r0, f1, f0);
        step(r0 + TB, f2, f1);
        step(r0 + 2 * TB, f0, f2);
    }
    if (!wave_on) return;
    // dw partial: dwacc[i] sums this lane's tokens at channel wc0 + 4 lg + i;
    // the 16 lanes lr of a row hold the block's other tokens
#pragma unroll
    for (int i = 0; i < 4; ++i) dwacc[i] = group_sum<16>(dwacc[i]);
    if (lr == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dw_part[(int64_t)blockIdx.y * C + cb0 + wc0 + 4 * lg + i] = dwacc[i];
    }
    // dPhi partial: accP[j][ot] register i holds o = 16 ot + 4 lg + i at channel wc0 + lr of stream j
    // (RES = false: row 4 lg + i of the packed tile, o = 4 lg + i for lg < 2
    // plus its lo half in lane + 32)
    float* out = dphi_part + (int64_t)blockIdx.y * NPO * K;
    if constexpr (!RES) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = (j < NSTR) ? xor32_add(accP[j < NSTR ? j : 0][0][i]) : 0.f;
                const int o = 4 * lg + i;
                if (lg < 2 && o < NPO) out[(int64_t)o * K + (int64_t)j * C + cb0 + wc0 + lr] = v;
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < N; ++j) {
#pragma unroll
        for (int ot = 0; ot < 2; ++ot) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = 16 * ot + 4 * lg + i;
                if (o < NP)
                    out[(int64_t)o * K + (int64_t)j * C + cb0 + wc0 + lr] = (j < NSTR) ? accP[j < NSTR ? j : 0][ot][i] : 0.f;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#define MHC_WRAP_PICK_VPT(v, ...)                                \
    switch (v) {                                                 \
        case 1: { constexpr int V_ = 1; __VA_ARGS__; break; }    \
        case 2: { constexpr int V_ = 2; __VA_ARGS__; break; }    \
        case 4: { constexpr int V_ = 4; __VA_ARGS__; break; }    \
        case 8: { constexpr int V_ = 8; __VA_ARGS__; break; }    \
        default: break;                                          \
    }

// live row arrays per thread: forward r, b (raw words and values); backward g, r, b
static constexpr int kWrapFwdArrays = 2;
static constexpr int kWrapBwdArrays = 3;

template <typename TX, int V, bool DECAY>
static const void* wrap_fwd_fn() {
    if constexpr (layer_row_fits(kWrapFwdArrays * 2, V)) return reinterpret_cast<const void*>(&wrap_fwd_kernel<TX, 4, V, DECAY>);
    return nullptr;
}

template <typename TX, int V, bool PF, bool DECAY>
static const void* wrap_bwd_fn() {
    if constexpr (layer_row_fits(kWrapBwdArrays * 2, V))
        return PF ? reinterpret_cast<const void*>(&wrap_bwd_pf_kernel<TX, 4, V, DECAY>)
                  : reinterpret_cast<const void*>(&wrap_bwd_kernel<TX, 4, V, DECAY>);
    return nullptr;
}

static int wrap_grid(const void* fn, int threads, int64_t B) {
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

static const void* pick_wrap_fwd(int dt, int vpt, bool decay) {
    const void* fn = nullptr;
#define MHC_WF(TX_) \
    MHC_WRAP_PICK_VPT(vpt, fn = decay ? wrap_fwd_fn<TX_, V_, true>() : wrap_fwd_fn<TX_, V_, false>())
    if (dt == kBF16) {
        MHC_WF(bf16_t);
    } else {
        MHC_WF(float);
    }
#undef MHC_WF
    return fn;
}

static const void* pick_wrap_bwd(int dt, int vpt, bool pf, bool decay) {
    const void* fn = nullptr;
#define MHC_WB(TX_)                                                                                    \
    MHC_WRAP_PICK_VPT(vpt, fn = pf ? (decay ? wrap_bwd_fn<TX_, V_, true, true>()                       \
                                            : wrap_bwd_fn<TX_, V_, true, false>())                     \
                                   : (decay ? wrap_bwd_fn<TX_, V_, false, true>()                      \
                                            : wrap_bwd_fn<TX_, V_, false, false>()))
    if (dt == kBF16) {
        MHC_WB(bf16_t);
    } else {
        MHC_WB(float);
    }
#undef MHC_WB
    return fn;
}

static bool wrap_prefetch(const RowTiling& t) { return t.threads <= 256; }

// Chunks per lane of the one-token-per-wave forward (bf16 rows of
// C = 256 KQ, KQ = 4, 8, ..., 32), 0 where the workgroup-per-token kernel runs.
static int wrap_fwd_wave_kq(int dt, int64_t C) {
    if (dt != kBF16 || C % 1024 != 0 || C > 8192) return 0;
    return (int)(C / 256);
}

hipError_t launch_wrap_fwd(int dt, int n, bool decay, const void* res, const void* br, const float* w,
                           const float* coef, int64_t coef_stride, float* out, int64_t B, int64_t C, float eps,
                           hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (n != 4) return hipErrorInvalidValue;
    if (const int kq = wrap_fwd_wave_kq(dt, C)) {
        const int64_t blocks = (B + 3) / 4;  // one token per wave
        if (blocks > 0x7fffffff) return hipErrorInvalidValue;
        const void* fn = nullptr;
#define MHC_WFW(KQ_) fn = decay ? reinterpret_cast<const void*>(&wrap_fwd_wave_kernel<KQ_, true>) \
                                : reinterpret_cast<const void*>(&wrap_fwd_wave_kernel<KQ_, false>)
        switch (kq) {
            case 4: MHC_WFW(4); break;
            case 8: MHC_WFW(8); break;
            case 12: MHC_WFW(12); break;
            case 16: MHC_WFW(16); break;
            case 20: MHC_WFW(20); break;
            case 24: MHC_WFW(24); break;
            case 28: MHC_WFW(28); break;
            default: MHC_WFW(32); break;
        }
#undef MHC_WFW
        int Ci = (int)C;
        void* args[] = {(void*)&res, (void*)&br, (void*)&w, (void*)&coef, (void*)&coef_stride, (void*)&out,
                        (void*)&B, (void*)&Ci, (void*)&eps};
        const int tok = timing_begin("wrap_fwd", s);
        hipError_t e = mhc_launch_kernel(fn, dim3((unsigned)blocks), dim3(256), args, (size_t)C * 4, s);
        timing_end(tok, s);
        return e != hipSuccess ? e : hipGetLastError();
    }
    const RowTiling t = choose_row_tiling(C, kLayerWC, kWrapFwdArrays * 2, 512);
    if (t.vpt <= 0) return hipErrorInvalidValue;
    const void* fn = pick_wrap_fwd(dt, t.vpt, decay);
    if (!fn) return hipErrorInvalidValue;
    if (B > 0x7fffffff) return hipErrorInvalidValue;  // grid x limit
    const unsigned grid = (unsigned)B;  // one token per workgroup
    int Ci = (int)C;
    void* args[] = {(void*)&res, (void*)&br, (void*)&w, (void*)&coef, (void*)&coef_stride, (void*)&out, (void*)&B,
                    (void*)&Ci, (void*)&eps};
    const int tok = timing_begin("wrap_fwd", s);
    hipError_t e = mhc_launch_kernel(fn, dim3(grid), dim3(t.threads), args, 0, s);
    timing_end(tok, s);
    return e != hipSuccess ? e : hipGetLastError();
}

int wrap_bwd_grid(int dt, int n, bool decay, int64_t B, int64_t C) {
    (void)n;
    const RowTiling t = choose_row_tiling(C, kLayerWC, kWrapBwdArrays * 2);
    if (t.vpt <= 0) return 1;
    return wrap_grid(pick_wrap_bwd(dt, t.vpt, wrap_prefetch(t), decay), t.threads, B);
}

hipError_t launch_wrap_bwd(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                           const float* w, const float* coef, int64_t coef_stride, void* dres, void* dbr,
                           float* dw_part, float* scal_out, int grid, int64_t B, int64_t C, float eps,
                           hipStream_t s) {
    if (n != 4) return hipErrorInvalidValue;
    const RowTiling t = choose_row_tiling(C, kLayerWC, kWrapBwdArrays * 2);
    if (t.vpt <= 0) return hipErrorInvalidValue;
    const void* fn = pick_wrap_bwd(dt, t.vpt, wrap_prefetch(t), decay);
    if (!fn) return hipErrorInvalidValue;
    int Ci = (int)C;
    void* args[] = {(void*)&g, (void*)&res, (void*)&br, (void*)&w, (void*)&coef, (void*)&coef_stride, (void*)&dres,
                    (void*)&dbr, (void*)&dw_part, (void*)&scal_out, (void*)&B, (void*)&Ci, (void*)&eps};
    const int tok = timing_begin("wrap_bwd", s);
    hipError_t e = mhc_launch_kernel(fn, dim3(grid), dim3(t.threads), args, 0, s);
    timing_end(tok, s);
    return e != hipSuccess ? e : hipGetLastError();
}

int wrap_proj_csplit(int64_t B, int64_t C) {
    const int64_t mblocks = (B + 63) / 64;
    int64_t ks = (2 * (int64_t)device_cu_count() + mblocks - 1) / mblocks;
    const int64_t kmax = C / 256;
    if (ks > kmax) ks = kmax;
    if (ks < 1) ks = 1;
    return (int)ks;
}

hipError_t launch_wrap_phi_planes(int dt, int n, const float* phi_pre, const float* phi_post, const float* phi_res,
                                  int64_t C, bf16_raw_t* phib, hipStream_t s) {
    if (n != 4 || C % 32 != 0) return hipErrorInvalidValue;
    const int64_t K = 4 * C;
    if (dt != kBF16) return launch_phi_split(phi_pre, phi_post, phi_res, n, 2 * n + n * n, K, phib, s);
    int64_t blocks = (K / 32 * 64 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    MHC_LAUNCH_GGL(wrap_phi_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, s, phi_pre, phi_post, phi_res, K,
                   reinterpret_cast<uint4*>(phib));
    return hipGetLastError();
}

hipError_t launch_wrap_proj(int dt, int n, bool decay, const void* res, const void* br, const bf16_raw_t* phib,
                            float* p_part, float* ss_part, int64_t B, int64_t C, int ks, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (n != 4 || C % 32 != 0) return hipErrorInvalidValue;
    if (C > (int64_t(1) << 20)) return hipErrorInvalidValue;  // 32-bit buffer offsets
    int64_t cchunk = (C + ks - 1) / ks;
    cchunk = ((cchunk + 127) / 128) * 128;
    const uint4* phif = reinterpret_cast<const uint4*>(phib);
    const int tok = timing_begin("wrap_proj", s);
#define MHC_WP(TX_, D_)                                                                                          \
    MHC_LAUNCH_GGL((wrap_proj_kernel<TX_, 4, D_>),                                                           \
                       dim3((unsigned)((B + 16 * wproj_mt<TX_>() - 1) / (16 * wproj_mt<TX_>())), (unsigned)ks),   \
                       dim3(256), 0, s, (const TX_*)res, (const TX_*)br, phif, p_part, ss_part, B, (int)C, cchunk)
    if (dt == kBF16) {
        if (decay) { MHC_WP(bf16_t, true); } else { MHC_WP(bf16_t, false); }
    } else {
        if (decay) { MHC_WP(float, true); } else { MHC_WP(float, false); }
    }
#undef MHC_WP
    timing_end(tok, s);
    return hipGetLastError();
}

// Token tiles: column blocks x tiles fill two rounds of resident workgroups
// (rounded down, so a last partial round is nearly full rather than leaving
// most CUs idle while it runs), at least one, and enough that a tile's rows
// of G, plus the three stages the pipeline reads past its end, stay under
// 2 GiB (the kernel's buffer resources and offsets).  Tiles are whole
// triples of 32-token stages; the pipeline reads up to six stages past the
// end.
static int64_t wrap_proj_bwd_max_tile(int64_t C) { return ((int64_t(1) << 31) - 1) / (C * 4) - 6 * 32; }

int wrap_proj_bwd_tiles(int dt, int64_t B, int64_t C) {
    const int64_t gx = (C + kWpbCols - 1) / kWpbCols;
    const void* fn = dt == kBF16 ? reinterpret_cast<const void*>(&wrap_proj_bwd_kernel<bf16_t, 4, true, true>)
                                 : reinterpret_cast<const void*>(&wrap_proj_bwd_kernel<float, 4, true, true>);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kWpbThreads, 0) != hipSuccess || per_cu < 1) {
        (void)hipGetLastError();
        per_cu = 1;
    }
    int64_t tiles = 2 * (int64_t)device_cu_count() * per_cu / gx;
    const int64_t blocks = (B + 31) / 32;
    if (tiles > blocks) tiles = blocks;
    if (tiles < 1) tiles = 1;
    const int64_t mt = wrap_proj_bwd_max_tile(C) / 96 * 96;
    if (mt >= 96 && (B + tiles - 1) / tiles > mt) tiles = (B + mt - 1) / mt;
    return (int)tiles;
}

hipError_t launch_wrap_proj_bwd(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                                const float* w, const float* ep, const float* dP, const float* s_tok,
                                const float* phi_pre, const float* phi_post, const float* phi_res, void* dres,
                                void* dbr, float* dw_part, float* dphi_part, int tiles, int64_t B, int64_t C,
                                bool res_rows, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (n != 4 || C % 32 != 0 || tiles < 1) return hipErrorInvalidValue;
    int64_t tile = (B + tiles - 1) / tiles;
    tile = ((tile + 95) / 96) * 96;
    if (tile > wrap_proj_bwd_max_tile(C)) return hipErrorInvalidValue;  // offsets past 2 GiB
    const dim3 grid((unsigned)((C + kWpbCols - 1) / kWpbCols), (unsigned)tiles);
    const int tok = timing_begin("wrap_proj_bwd", s);
#define MHC_WPB1(TX_, D_, R_)                                                                                     \
    MHC_LAUNCH_GGL((wrap_proj_bwd_kernel<TX_, 4, D_, R_>), grid, dim3(kWpbThreads), 0, s, g, (const TX_*)res,    \
                       (const TX_*)br, w, ep, dP, s_tok, phi_pre, phi_post, phi_res, (TX_*)dres, (TX_*)dbr, dw_part, \
                       dphi_part, B, (int)C, tile)
#define MHC_WPB(TX_, D_)                                   \
    if (res_rows) { MHC_WPB1(TX_, D_, true); } else { MHC_WPB1(TX_, D_, false); }
    if (dt == kBF16) {
        if (decay) { MHC_WPB(bf16_t, true); } else { MHC_WPB(bf16_t, false); }
    } else {
        if (decay) { MHC_WPB(float, true); } else { MHC_WPB(float, false); }
    }
#undef MHC_WPB
#undef MHC_WPB1
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_wrap_bwd_red(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                               const float* w, const float* coef, int64_t coef_stride, float* scal_out,
                               float* ep_out, int64_t B, int64_t C, float eps, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (n != 4 || C % 4 != 0) return hipErrorInvalidValue;
    const int64_t blocks = (B + 3) / 4;  // one token per wave, four waves per workgroup
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const int tok = timing_begin("wrap_bwd_reduce", s);
#define MHC_WR(TX_, D_)                                                                                        \
    MHC_LAUNCH_GGL((wrap_bwd_red_kernel<TX_, 4, D_>), dim3((unsigned)blocks), dim3(256), 0, s, g,             \
                       (const TX_*)res, (const TX_*)br, w, coef, coef_stride, scal_out, ep_out, B, (int)C, eps)
    if (dt == kBF16) {
        if (decay) { MHC_WR(bf16_t, true); } else { MHC_WR(bf16_t, false); }
    } else {
        if (decay) { MHC_WR(float, true); } else { MHC_WR(float, false); }
    }
#undef MHC_WR
    timing_end(tok, s);
    return hipGetLastError();
}

}  // namespace mhc

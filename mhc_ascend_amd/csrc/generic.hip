// Kernels for expansion rates with no compiled instantiation: any n in
// 1..64 outside {2, 4, 8, 16, 32} for the layer, outside {1, 2, 4, 8, 16, 32}
// for the stream operators.  The reference takes n at run time up to
// MAX_EXPANSION_RATE = 64 (mhc_types.h:68, stream_ops.cpp:198-208,
// sinkhorn_knopp.cpp:575-617); here the rates the paper uses
// (benchmark.py:302-310) and their powers of two keep their fixed-n kernels
// and every other n runs these, with n as an argument.
//
// Layout of the work (one token per workgroup of 256 lanes, n read at run
// time, per-lane arrays sized by a compile-time capacity NM in {16, 32, 64}
// so that nothing is indexed at run time in registers):
//   * stream mixing out_i = a_i + sum_j A_ij x_j over a channel chunk: the
//     chunk's n input rows are staged in LDS ([n][64] floats), wave q of the
//     workgroup forms outputs i = q, q + 4, ... for the chunk's 64 channels
//     with the matrix row held as a wave-uniform LDS broadcast;
//   * per-stream channel sums: one stream at a time, lane partials reduced
//     within the wave, the four waves' totals added in order in LDS;
//   * the n x n Gram matrix sum_c g_i x_j (dM): fp32 MFMA over zero-padded
//     stream blocks of 16 or 32 (gen_gram_kernel);
//   * Sinkhorn-Knopp and its exact adjoint: one row per lane in a group of
//     NM lanes (skw_* in mhc_device.h); the static H_res at n <= 16 on one
//     wave, four elements per lane (skw16::forward_n / backward_n), and at
//     n in 17..31 on the whole workgroup (skb::forward_n / backward_n).
// Every reduction has a fixed order, so the results are deterministic.
//
// Math (layer.py:142-170, ops_pytorch_backward.py:9-150), per token with
// coefficients (h_pre[n], h_post[n], M[n][n]):
//   xa = sum_j h_pre_j x_j,  r = sqrt(mean_c xa^2 + eps),  y = xa / r * w
//   out_i = h_post_i y + sum_j M_ij x_j
// and for the cotangent g: gy = sum_i h_post_i g_i, k2 = sum(w gy xa)/(C r^3),
//   gxa = w gy / r - xa k2,  dx_j = h_pre_j gxa + sum_i M_ij g_i,
//   dw += gy xa / r,  dh_post_i = sum(g_i xa w) / r,
//   dh_pre_j = sum(w gy x_j) / r - k2 sum(xa x_j),  dM_ij = sum g_i x_j.
#include "mhc_device.h"
#include "mhc_internal.h"

namespace mhc {

constexpr int kGenThreads = 256;
constexpr int kGenWaves = kGenThreads / kWave;
constexpr int kGenChunk = 64;  // channels per LDS chunk of the mixing loops
static_assert(kGenThreads == skb::kThreads, "the static Sinkhorn at n in 17..31 takes the whole workgroup");

bool generic_layer_n(int n) {
    return n >= 1 && n <= kGenMaxN && !(n == 2 || n == 4 || n == 8 || n == 16 || n == 32);
}
bool generic_ops_n(int n) {
    return n >= 1 && n <= kGenMaxN && !(n == 1 || n == 2 || n == 4 || n == 8 || n == 16 || n == 32);
}

#define MHC_GEN_NM(n, ...)                     \
    if ((n) <= 16) {                           \
        constexpr int NM_ = 16; __VA_ARGS__;   \
    } else if ((n) <= 32) {                    \
        constexpr int NM_ = 32; __VA_ARGS__;   \
    } else {                                   \
        constexpr int NM_ = 64; __VA_ARGS__;   \
    }

// Block totals of two per-thread values (all threads receive them).
__device__ __forceinline__ void gen_block_total2(float& a, float& b, float* red) {
    float v[2] = {a, b};
    block_sum<2>(v, red);
    a = v[0];
    b = v[1];
}

// Wave total of v added into acc[wave] (LDS, one slot per wave), for the
// per-stream sums: the caller adds the kGenWaves slots in order after a
// barrier.
__device__ __forceinline__ void gen_wave_partial(float v, float* slots) {
    float t[1] = {v};
    wave_sum_last<1>(t);
    if ((threadIdx.x & (kWave - 1)) == kWave - 1) slots[threadIdx.x / kWave] = t[0];
}

// ---------------------------------------------------------------------------
// Static coefficients (layer.py:146-160): h_pre = sigmoid(H_pre), h_post =
// 2 sigmoid(H_post), M = SK(exp(H_res)) once, into saved[0 .. 2n + n^2), and
// the fp32 copy of the RMSNorm weight at saved[w_off ..].  Workgroup 0 forms
// the coefficients (n <= 16: four elements of M per lane of wave 0; n in
// 17..31: the whole workgroup; else a row per lane of wave 0); the others copy
// 2048-channel pieces of the weight.
// ---------------------------------------------------------------------------
template <int NM, typename TW>
__global__ __launch_bounds__(kGenThreads) void gen_static_coef_kernel(
    const float* __restrict__ h_pre, const float* __restrict__ h_post, const float* __restrict__ h_res,
    const TW* __restrict__ w, int C, float* __restrict__ saved, int w_off, int n, int iters, float eps) {
    if (blockIdx.x > 0) {
        const int c0 = (int)(blockIdx.x - 1) * 2048;
        for (int c = c0 + (int)threadIdx.x; c < C && c < c0 + 2048; c += kGenThreads)
            saved[w_off + c] = VecIO<TW>::scalar(w + c);
        return;
    }
    if constexpr (NM == skb::kN) {
        // n in 17..31: the zero-padded 32 x 32 matrix on the whole workgroup
        // (the finalize's adjoint recomputes it with the same code)
        if ((int)threadIdx.x < n) {
            saved[threadIdx.x] = sigmoidf(h_pre[threadIdx.x]);
            saved[n + threadIdx.x] = 2.f * sigmoidf(h_post[threadIdx.x]);
        }
        __shared__ float part[skb::kPartFloats];
        const int i = skb::row(), c0 = skb::col0();
        float a[skb::kV];
#pragma unroll
        for (int k = 0; k < skb::kV; ++k) a[k] = (i < n && c0 + k < n) ? expf(h_res[i * n + c0 + k]) : 0.f;
        skb::forward_n(a, n, iters, eps, part);
#pragma unroll
        for (int k = 0; k < skb::kV; ++k) {
            if (i < n && c0 + k < n) saved[2 * n + i * n + c0 + k] = a[k];
        }
        return;
    }
    if (threadIdx.x >= kWave) return;
    const int r = threadIdx.x;
    const bool active = r < n;
    if (active) {
        saved[r] = sigmoidf(h_pre[r]);
        saved[n + r] = 2.f * sigmoidf(h_post[r]);
    }
    if constexpr (NM == skw16::kN) {
        // the zero-padded 16 x 16 matrix on the wave, four elements per lane
        // (the finalize's adjoint recomputes it with the same code)
        const int i = skw16::row(), c0 = skw16::col0();
        float a[skw16::kV];
#pragma unroll
        for (int k = 0; k < skw16::kV; ++k) a[k] = (i < n && c0 + k < n) ? expf(h_res[i * n + c0 + k]) : 0.f;
        skw16::forward_n(a, n, iters, eps);
#pragma unroll
        for (int k = 0; k < skw16::kV; ++k) {
            if (i < n && c0 + k < n) saved[2 * n + i * n + c0 + k] = a[k];
        }
        return;
    }
    float e[NM];
#pragma unroll
    for (int c = 0; c < NM; ++c) e[c] = (active && c < n) ? expf(h_res[r * n + c]) : 0.f;
    skw_forward<NM>(e, n, iters, eps, active);
    if (active) {
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            if (c < n) saved[2 * n + r * n + c] = e[c];
        }
    }
}

// ---------------------------------------------------------------------------
// Coefficients of token b into LDS: hp[NM], hq[NM] and the mixing matrix
// with rows of NM floats, zero beyond n: TR = false mr[i][j] = M_ij (rows i:
// the forward's out_i = sum_j M_ij x_j reads row i ... as mr[j][i]: see the
// callers), TR = true mr[j][i] = M_ij.
// ---------------------------------------------------------------------------
template <int NM, bool TR>
__device__ __forceinline__ void gen_load_coef(const float* __restrict__ cf, int n, float* hp, float* hq, float* mr) {
    for (int t = threadIdx.x; t < NM; t += kGenThreads) {
        hp[t] = t < n ? cf[t] : 0.f;
        hq[t] = t < n ? cf[n + t] : 0.f;
    }
    for (int t = threadIdx.x; t < NM * NM; t += kGenThreads) {
        const int a = t / NM, bcol = t % NM;
        float v = 0.f;
        if (a < n && bcol < n) v = TR ? cf[2 * n + bcol * n + a] : cf[2 * n + a * n + bcol];
        mr[t] = v;
    }
}

// ---------------------------------------------------------------------------
// Layer forward, one token per workgroup.  Pass 1: r from sum_c xa^2 (the
// row read once).  Pass 2, per 64-channel chunk: the n rows of the chunk in
// LDS, wave q forms out_i for i = q, q + 4, ... (the row read again, from
// cache).  mt[j][i] = M_ij, so wave q's matrix reads at (j, q + 4u) are
// wave-uniform.  out in TO; rms_out[b] = r when not null.
// ---------------------------------------------------------------------------
template <typename TX, typename TO, int NM>
__global__ __launch_bounds__(kGenThreads) void gen_fwd_kernel(const TX* __restrict__ x, const float* __restrict__ w,
                                                              const float* __restrict__ coef, int64_t coef_stride,
                                                              TO* __restrict__ out, float* __restrict__ rms_out,
                                                              int n, int C, float eps) {
    constexpr int U = NM / kGenWaves;  // outputs per lane and chunk
    __shared__ float xs[NM][kGenChunk];
    __shared__ float mt[NM * NM];
    __shared__ float hp[NM], hq[NM];
    __shared__ float red[2 * kGenWaves];
    const int64_t b = blockIdx.x;
    gen_load_coef<NM, true>(coef + b * coef_stride, n, hp, hq, mt);
    __syncthreads();
    const TX* xb = x + b * (int64_t)n * C;
    float ss = 0.f, unused = 0.f;
    for (int c = threadIdx.x; c < C; c += kGenThreads) {
        float xa = 0.f;
        for (int j = 0; j < n; ++j) xa += hp[j] * VecIO<TX>::scalar(xb + (int64_t)j * C + c);
        ss += xa * xa;
    }
    gen_block_total2(ss, unused, red);
    const float r = sqrtf(ss / (float)C + eps);
    const float inv = 1.f / r;
    if (rms_out && threadIdx.x == 0) rms_out[b] = r;
    const int cl = threadIdx.x % kGenChunk;
    const int q = threadIdx.x / kGenChunk;
    TO* ob = out + b * (int64_t)n * C;
    for (int c0 = 0; c0 < C; c0 += kGenChunk) {
        for (int t = threadIdx.x; t < n * kGenChunk; t += kGenThreads) {
            const int j = t / kGenChunk, c = c0 + t % kGenChunk;
            xs[j][t % kGenChunk] = c < C ? VecIO<TX>::scalar(xb + (int64_t)j * C + c) : 0.f;
        }
        __syncthreads();
        float acc[U], xa = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = 0.f;
        for (int j = 0; j < n; ++j) {
            const float xj = xs[j][cl];
            xa += hp[j] * xj;
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u] += mt[j * NM + q + kGenWaves * u] * xj;
        }
        const int c = c0 + cl;
        if (c < C) {
            const float y = xa * inv * w[c];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = q + kGenWaves * u;
                if (i < n) VecIO<TO>::put(ob + (int64_t)i * C + c, acc[u] + hq[i] * y);
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Layer backward without dM (gen_gram_kernel forms it), persistent
// workgroups over tokens b = blockIdx.x + k gridDim.x.  Per token:
//   A: xa and gy per channel into this workgroup's row of `rows`
//      ([grid][2][C] floats), sum xa^2 and sum w gy xa -> r, k2;
//   B: per stream s: sum g_s xa w, sum w gy x_s, sum xa x_s (wave partials
//      in LDS, added in order) -> dh_post_act, dh_pre_act;
//   C: per 64-channel chunk, the n cotangent rows in LDS: dx_j = h_pre_j gxa
//      + sum_i M_ij g_i (wave q forms j = q, q + 4, ...), dw_part row +=
//      gy xa / r (each channel owned by one lane of wave 0 for every token).
// MODE 0 (static): scal_out[blockIdx.x][n^2 + 2n] gets the workgroup's sums
// of dh_post_act, dh_pre_act at offset n^2.  MODE 1 (dynamic): per token
// scal_out[b][n^2 + 2n + 2] gets dh_post_act, dh_pre_act, 1/r, k2.
// ---------------------------------------------------------------------------
template <typename TX, int NM, int MODE>
__global__ __launch_bounds__(kGenThreads) void gen_bwd_kernel(
    const float* __restrict__ g, const TX* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ coef, int64_t coef_stride, TX* __restrict__ dx, float* __restrict__ dw_part,
    float* __restrict__ scal_out, float* __restrict__ rows, int64_t B, int n, int C, float eps) {
    constexpr int U = NM / kGenWaves;
    __shared__ float gs[NM][kGenChunk];
    __shared__ float mr[NM * NM];
    __shared__ float hp[NM], hq[NM];
    __shared__ float red[2 * kGenWaves];
    __shared__ float sred[3][NM][kGenWaves];
    __shared__ float acc_s[2 * NM];
    const int NS = n * n + 2 * n;
    float* dwr = dw_part + (int64_t)blockIdx.x * C;
    float* xar = rows + (int64_t)blockIdx.x * 2 * C;
    float* gyr = xar + C;
    for (int c = threadIdx.x; c < C; c += kGenThreads) dwr[c] = 0.f;
    for (int t = threadIdx.x; t < 2 * NM; t += kGenThreads) acc_s[t] = 0.f;
    const int cl = threadIdx.x % kGenChunk;
    const int q = threadIdx.x / kGenChunk;
    const int wave = threadIdx.x / kWave;
    for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
        __syncthreads();  // the previous token's LDS reads are done
        gen_load_coef<NM, false>(coef + b * coef_stride, n, hp, hq, mr);
        __syncthreads();
        const float* gb = g + b * (int64_t)n * C;
        const TX* xb = x + b * (int64_t)n * C;
        // A
        float s1 = 0.f, s2 = 0.f;
        for (int c = threadIdx.x; c < C; c += kGenThreads) {
            float xa = 0.f, gy = 0.f;
            for (int j = 0; j < n; ++j) {
                xa += hp[j] * VecIO<TX>::scalar(xb + (int64_t)j * C + c);
                gy += hq[j] * gb[(int64_t)j * C + c];
            }
            xar[c] = xa;
            gyr[c] = gy;
            s1 += xa * xa;
            s2 += w[c] * gy * xa;
        }
        gen_block_total2(s1, s2, red);
        const float inv = 1.f / sqrtf(s1 / (float)C + eps);
        const float k2 = s2 * inv * inv * inv / (float)C;
        // B (each lane reads back the xa / gy it wrote in A)
        for (int s = 0; s < n; ++s) {
            float a1 = 0.f, a2 = 0.f, a3 = 0.f;
            for (int c = threadIdx.x; c < C; c += kGenThreads) {
                const float xa = xar[c], wgy = w[c] * gyr[c];
                const float xv = VecIO<TX>::scalar(xb + (int64_t)s * C + c);
                a1 += gb[(int64_t)s * C + c] * xa * w[c];
                a2 += wgy * xv;
                a3 += xa * xv;
            }
            gen_wave_partial(a1, sred[0][s]);
            gen_wave_partial(a2, sred[1][s]);
            gen_wave_partial(a3, sred[2][s]);
        }
        __syncthreads();
        if ((int)threadIdx.x < 2 * n) {
            const int t = threadIdx.x;
            const int s = t < n ? t : t - n;
            float v[3];
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                float tot = 0.f;
#pragma unroll
                for (int q2 = 0; q2 < kGenWaves; ++q2) tot += sred[k][s][q2];
                v[k] = tot;
            }
            // [dh_post_act (n), dh_pre_act (n)]
            const float val = t < n ? v[0] * inv : v[1] * inv - k2 * v[2];
            if constexpr (MODE == 0) {
                acc_s[t] += val;
            } else {
                float* so = scal_out + b * (int64_t)(NS + 2);
                so[n * n + t] = val;
                if (t == 0) {
                    so[NS] = inv;
                    so[NS + 1] = k2;
                }
            }
        }
        // C
        TX* db = dx + b * (int64_t)n * C;
        for (int c0 = 0; c0 < C; c0 += kGenChunk) {
            __syncthreads();
            for (int t = threadIdx.x; t < n * kGenChunk; t += kGenThreads) {
                const int i = t / kGenChunk, c = c0 + t % kGenChunk;
                gs[i][t % kGenChunk] = c < C ? gb[(int64_t)i * C + c] : 0.f;
            }
            __syncthreads();
            float acc[U];
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u] = 0.f;
            for (int i = 0; i < n; ++i) {
                const float gi = gs[i][cl];
#pragma unroll
                for (int u = 0; u < U; ++u) acc[u] += mr[i * NM + q + kGenWaves * u] * gi;
            }
            const int c = c0 + cl;
            if (c < C) {
                const float xa = xar[c], gy = gyr[c], wc = w[c];
                const float gxa = wc * gy * inv - xa * k2;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int j = q + kGenWaves * u;
                    if (j < n) VecIO<TX>::put(db + (int64_t)j * C + c, hp[j] * gxa + acc[u]);
                }
                if (wave == 0) dwr[c] += gy * xa * inv;
            }
        }
    }
    if constexpr (MODE == 0) {
        __syncthreads();
        float* so = scal_out + (int64_t)blockIdx.x * NS;
        if ((int)threadIdx.x < 2 * n) so[n * n + threadIdx.x] = acc_s[threadIdx.x];
    }
}

// ---------------------------------------------------------------------------
// dM_ij = sum_c g_i x_j per token on fp32 MFMA, the streams zero-padded to
// blocks of NB = 16 (v_mfma_f32_16x16x4f32) or 32 (v_mfma_f32_32x32x2f32):
// blockIdx.y selects the block (i0, j0) of rows and columns.  Lane l loads
// 16 consecutive channels of stream i0 + l % NB of g (A operand) and of
// stream j0 + l % NB of x (B operand); the k slots of one MFMA are the
// lane groups l / NB, so a wave step covers 16 * (64 / NB) channels.  The
// four waves take alternate steps and add their accumulators in LDS.
// MODE 0: the workgroup's sum over tokens b = blockIdx.x + k gridDim.x into
// out[blockIdx.x * ostride + i * n + j]; MODE 1: per token into
// out[b * ostride + i * n + j].
// ---------------------------------------------------------------------------
typedef float gen_f32x16_t __attribute__((ext_vector_type(16)));
typedef float gen_f32x4_t __attribute__((ext_vector_type(4)));

template <int NB> struct GenGram;
template <> struct GenGram<32> {
    using acc_t = gen_f32x16_t;
    static constexpr int R = 16;
    __device__ __forceinline__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    __device__ __forceinline__ static int row(int l, int r) { return 8 * (r / 4) + 4 * (l / 32) + (r % 4); }
    __device__ __forceinline__ static int col(int l) { return l % 32; }
};
template <> struct GenGram<16> {
    using acc_t = gen_f32x4_t;
    static constexpr int R = 4;
    __device__ __forceinline__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    __device__ __forceinline__ static int row(int l, int r) { return 4 * (l / 16) + r; }
    __device__ __forceinline__ static int col(int l) { return l % 16; }
};

template <typename T>
__device__ __forceinline__ void gen_load16(const T* __restrict__ row, bool on, int c, int C, float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = (on && c + k < C) ? VecIO<T>::scalar(row + c + k) : 0.f;
}

template <typename TX, int NB, int MODE>
__global__ __launch_bounds__(kGenThreads) void gen_gram_kernel(const float* __restrict__ g, const TX* __restrict__ x,
                                                               float* __restrict__ out, int64_t B, int n, int C,
                                                               int64_t ostride) {
    using M = GenGram<NB>;
    using acc_t = typename M::acc_t;
    constexpr int KQ = kWave / NB;
    constexpr int SC = 16 * KQ;
    __shared__ float red[kGenWaves - 1][M::R][kWave];
    const int nb = (n + NB - 1) / NB;
    const int i0 = (int)(blockIdx.y / nb) * NB, j0 = (int)(blockIdx.y % nb) * NB;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int li = lane % NB, h = lane / NB;
    const bool on_g = i0 + li < n, on_x = j0 + li < n;
    const int nsteps = (C + SC - 1) / SC;
    const int64_t nC = (int64_t)n * C;
    acc_t acc = {};
    auto flush = [&](float* o) __attribute__((always_inline)) {
        if (wave > 0) {
#pragma unroll
            for (int r = 0; r < M::R; ++r) red[wave - 1][r][lane] = acc[r];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < M::R; ++r) {
                float v = acc[r];
#pragma unroll
                for (int q = 0; q < kGenWaves - 1; ++q) v += red[q][r][lane];
                const int i = i0 + M::row(lane, r), j = j0 + M::col(lane);
                if (i < n && j < n) o[i * n + j] = v;
            }
        }
        __syncthreads();
    };
    for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
        if (MODE == 1) acc = acc_t{};
        const float* gr = g + b * nC + (int64_t)(on_g ? i0 + li : 0) * C;
        const TX* xr = x + b * nC + (int64_t)(on_x ? j0 + li : 0) * C;
        for (int st = wave; st < nsteps; st += kGenWaves) {
            float ga[16], xa[16];
            gen_load16<float>(gr, on_g, st * SC + 16 * h, C, ga);
            gen_load16<TX>(xr, on_x, st * SC + 16 * h, C, xa);
#pragma unroll
            for (int k = 0; k < 16; ++k) acc = M::step(ga[k], xa[k], acc);
        }
        if (MODE == 1) flush(out + b * ostride);
    }
    if (MODE == 0) flush(out + (int64_t)blockIdx.x * ostride);
}

// ---------------------------------------------------------------------------
// Static parameter gradients from the per-workgroup sums scal_part[rows][n^2
// + 2n] = [dM, dh_post_act, dh_pre_act] (layer.hip's finalize, generic n):
// column totals in LDS (fixed order), then dH_pre = dh_pre_act h_pre (1 -
// h_pre), dH_post = dh_post_act h_post (1 - h_post / 2) and dH_res =
// SK^T(dM) * exp(H_res): for n <= 16 (iters <= skw16::kTMax) on wave 0,
// four elements per lane, for n in 17..31 (iters <= skb::kTMax) on the
// whole workgroup, zero-padded to 32 x 32; otherwise the adjoint one row per
// lane of wave 0
// (with hist, skw_hist_floats(kWave, n, iters) floats, the iterations' state
// in memory; without, recomputed per iteration).
// ---------------------------------------------------------------------------
template <int NM>
__global__ __launch_bounds__(kGenThreads) void gen_static_finalize_kernel(
    const float* __restrict__ scal_part, int rows, const float* __restrict__ h_pre, const float* __restrict__ h_post,
    const float* __restrict__ h_res, float* __restrict__ d_h_pre, float* __restrict__ d_h_post,
    float* __restrict__ d_h_res, int n, int iters, float eps, float* __restrict__ hist) {
    __shared__ float tot[NM * NM + 2 * NM];
    const int NS = n * n + 2 * n;
    // column totals in row order; each lane's next RB rows are loaded
    // together so that their latencies overlap
    constexpr int RB = 8;
    for (int k = threadIdx.x; k < NS; k += kGenThreads) {
        float s = 0.f;
        int r = 0;
        for (; r + RB <= rows; r += RB) {
            float v[RB];
#pragma unroll
            for (int j = 0; j < RB; ++j) v[j] = scal_part[(int64_t)(r + j) * NS + k];
#pragma unroll
            for (int j = 0; j < RB; ++j) s += v[j];
        }
        for (; r < rows; ++r) s += scal_part[(int64_t)r * NS + k];
        tot[k] = s;
    }
    __syncthreads();
    const bool one_wave = NM == skw16::kN && iters <= skw16::kTMax;
    const bool whole_wg = NM == skb::kN && iters <= skb::kTMax;
    if constexpr (NM == skb::kN) {
        if (whole_wg) {
            // n in 17..31: the zero-padded 32 x 32 matrix on the whole
            // workgroup (every thread takes part in its barriers)
            __shared__ float part[skb::kPartFloats];
            __shared__ float hc[skb::kHistFloats];
            const int i = skb::row(), c0 = skb::col0();
            float e[skb::kV], gm[skb::kV];
#pragma unroll
            for (int k = 0; k < skb::kV; ++k) {
                const bool on = i < n && c0 + k < n;
                e[k] = on ? expf(h_res[i * n + c0 + k]) : 0.f;
                gm[k] = on ? tot[i * n + c0 + k] : 0.f;
            }
            skb::backward_n(gm, e, n, iters, eps, part, hc);
#pragma unroll
            for (int k = 0; k < skb::kV; ++k) {
                if (i < n && c0 + k < n) d_h_res[i * n + c0 + k] = gm[k] * e[k];
            }
        }
    }
    if (one_wave && threadIdx.x < kWave) {
        // n <= 16: the zero-padded 16 x 16 matrix on wave 0, four elements
        // per lane, each iteration's state in registers
        const int i = skw16::row(), c0 = skw16::col0();
        float e[skw16::kV], gm[skw16::kV];
#pragma unroll
        for (int k = 0; k < skw16::kV; ++k) {
            const bool on = i < n && c0 + k < n;
            e[k] = on ? expf(h_res[i * n + c0 + k]) : 0.f;
            gm[k] = on ? tot[i * n + c0 + k] : 0.f;
        }
        skw16::backward_n(gm, e, n, iters, eps);
#pragma unroll
        for (int k = 0; k < skw16::kV; ++k) {
            if (i < n && c0 + k < n) d_h_res[i * n + c0 + k] = gm[k] * e[k];
        }
    }
    if (!one_wave && !whole_wg && threadIdx.x < kWave) {
        const int r = threadIdx.x;
        const bool active = r < n;
        float e[NM], gm[NM];
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            e[c] = (active && c < n) ? expf(h_res[r * n + c]) : 0.f;
            gm[c] = (active && c < n) ? tot[r * n + c] : 0.f;
        }
        if (hist) {
            skw_backward_mem<NM>(gm, e, n, iters, eps, active, hist, r, kWave);
        } else {
            skw_backward<NM>(gm, e, n, iters, eps, active);
        }
        if (active) {
#pragma unroll
            for (int c = 0; c < NM; ++c) {
                if (c < n) d_h_res[r * n + c] = gm[c] * e[c];
            }
        }
    }
    if ((int)threadIdx.x < n) {
        const int r = threadIdx.x;
        const float tp = sigmoidf(h_pre[r]);
        const float tq = 2.f * sigmoidf(h_post[r]);
        d_h_pre[r] = tot[n * n + n + r] * tp * (1.f - tp);
        d_h_post[r] = tot[n * n + r] * tq * (1.f - tq * 0.5f);
    }
}

// ---------------------------------------------------------------------------
// Standalone stream operators (ops.py:143-265, bindings.cpp:307-460) for
// generic n, one token per workgroup.
// ---------------------------------------------------------------------------
// out[c] = sum_i sigmoid(H_i) x_i[c]; h_act[b][i] = sigmoid(H_i)
template <typename T>
__global__ __launch_bounds__(kGenThreads) void gen_aggregate_fwd_kernel(const T* __restrict__ x,
                                                                        const float* __restrict__ H,
                                                                        int64_t h_stride, T* __restrict__ out,
                                                                        float* __restrict__ h_act, int n, int C) {
    __shared__ float h[kGenMaxN];
    const int64_t b = blockIdx.x;
    if ((int)threadIdx.x < n) {
        const float v = sigmoidf(H[b * h_stride + threadIdx.x]);
        h[threadIdx.x] = v;
        h_act[b * n + threadIdx.x] = v;
    }
    __syncthreads();
    const T* xb = x + b * (int64_t)n * C;
    for (int c = threadIdx.x; c < C; c += kGenThreads) {
        float s = 0.f;
        for (int i = 0; i < n; ++i) s += h[i] * VecIO<T>::scalar(xb + (int64_t)i * C + c);
        VecIO<T>::put(out + b * C + c, s);
    }
}

// gx_i[c] = g[c] h_i; gh_act_i = sum_c g x_i, gh_raw_i = gh_act_i h_i (1 - h_i)
template <typename T>
__global__ __launch_bounds__(kGenThreads) void gen_aggregate_bwd_kernel(
    const T* __restrict__ g, const T* __restrict__ x, const float* __restrict__ h_act, int64_t h_stride,
    T* __restrict__ gx, float* __restrict__ gh_act, float* __restrict__ gh_raw, int n, int C) {
    __shared__ float sred[kGenMaxN][kGenWaves];
    const int64_t b = blockIdx.x;
    const T* xb = x + b * (int64_t)n * C;
    T* gb = gx + b * (int64_t)n * C;
    for (int i = 0; i < n; ++i) {
        const float hi = h_act[b * h_stride + i];
        float a = 0.f;
        for (int c = threadIdx.x; c < C; c += kGenThreads) {
            const float gv = VecIO<T>::scalar(g + b * C + c);
            a += gv * VecIO<T>::scalar(xb + (int64_t)i * C + c);
            VecIO<T>::put(gb + (int64_t)i * C + c, gv * hi);
        }
        gen_wave_partial(a, sred[i]);
    }
    __syncthreads();
    if ((int)threadIdx.x < n) {
        const int i = threadIdx.x;
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < kGenWaves; ++q) t += sred[i][q];
        const float hi = h_act[b * h_stride + i];
        if (gh_act) gh_act[b * n + i] = t;
        if (gh_raw) gh_raw[b * n + i] = t * hi * (1.f - hi);
    }
}

// out_i[c] = h_i y[c] + sum_j M_ij x_j[c] (fp32), h = 2 sigmoid(H)
template <typename T, int NM>
__global__ __launch_bounds__(kGenThreads) void gen_distribute_fwd_kernel(
    const T* __restrict__ y, const float* __restrict__ H, int64_t h_stride, const float* __restrict__ M,
    int64_t m_stride, const T* __restrict__ x, float* __restrict__ out, float* __restrict__ h_act, int n, int C) {
    constexpr int U = NM / kGenWaves;
    __shared__ float xs[NM][kGenChunk];
    __shared__ float mt[NM * NM];
    __shared__ float h[NM];
    const int64_t b = blockIdx.x;
    for (int t = threadIdx.x; t < NM; t += kGenThreads) {
        const float v = t < n ? 2.f * sigmoidf(H[b * h_stride + t]) : 0.f;
        h[t] = v;
        if (t < n) h_act[b * n + t] = v;
    }
    const float* mb = M + b * m_stride;
    for (int t = threadIdx.x; t < NM * NM; t += kGenThreads) {
        const int j = t / NM, i = t % NM;
        mt[t] = (i < n && j < n) ? mb[i * n + j] : 0.f;
    }
    const T* xb = x + b * (int64_t)n * C;
    float* ob = out + b * (int64_t)n * C;
    const int cl = threadIdx.x % kGenChunk;
    const int q = threadIdx.x / kGenChunk;
    for (int c0 = 0; c0 < C; c0 += kGenChunk) {
        __syncthreads();
        for (int t = threadIdx.x; t < n * kGenChunk; t += kGenThreads) {
            const int j = t / kGenChunk, c = c0 + t % kGenChunk;
            xs[j][t % kGenChunk] = c < C ? VecIO<T>::scalar(xb + (int64_t)j * C + c) : 0.f;
        }
        __syncthreads();
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = 0.f;
        for (int j = 0; j < n; ++j) {
            const float xj = xs[j][cl];
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u] += mt[j * NM + q + kGenWaves * u] * xj;
        }
        const int c = c0 + cl;
        if (c < C) {
            const float yv = VecIO<T>::scalar(y + b * C + c);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = q + kGenWaves * u;
                if (i < n) ob[(int64_t)i * C + c] = acc[u] + h[i] * yv;
            }
        }
    }
}

// gy[c] = sum_i h_i g_i[c], gx_j[c] = sum_i M_ij g_i[c], gh_act_i = sum_c g_i
// y, gh_raw_i = gh_act_i h_i (1 - h_i / 2); gM from gen_gram_kernel.
template <typename T, int NM>
__global__ __launch_bounds__(kGenThreads) void gen_distribute_bwd_kernel(
    const float* __restrict__ g, const T* __restrict__ y, const float* __restrict__ M, int64_t m_stride,
    const float* __restrict__ h_act, int64_t h_stride, T* __restrict__ gx, T* __restrict__ gy,
    float* __restrict__ gh_act, float* __restrict__ gh_raw, int n, int C) {
    constexpr int U = NM / kGenWaves;
    __shared__ float gsh[NM][kGenChunk];
    __shared__ float mr[NM * NM];
    __shared__ float h[NM];
    __shared__ float sred[NM][kGenWaves];
    const int64_t b = blockIdx.x;
    for (int t = threadIdx.x; t < NM; t += kGenThreads) h[t] = t < n ? h_act[b * h_stride + t] : 0.f;
    const float* mb = M + b * m_stride;
    for (int t = threadIdx.x; t < NM * NM; t += kGenThreads) {
        const int i = t / NM, j = t % NM;
        mr[t] = (i < n && j < n) ? mb[i * n + j] : 0.f;
    }
    const float* gb = g + b * (int64_t)n * C;
    // gh_act: per stream, sum_c g_i y
    for (int i = 0; i < n; ++i) {
        float a = 0.f;
        for (int c = threadIdx.x; c < C; c += kGenThreads)
            a += gb[(int64_t)i * C + c] * VecIO<T>::scalar(y + b * C + c);
        gen_wave_partial(a, sred[i]);
    }
    T* gxb = gx + b * (int64_t)n * C;
    const int cl = threadIdx.x % kGenChunk;
    const int q = threadIdx.x / kGenChunk;
    for (int c0 = 0; c0 < C; c0 += kGenChunk) {
        __syncthreads();
        for (int t = threadIdx.x; t < n * kGenChunk; t += kGenThreads) {
            const int i = t / kGenChunk, c = c0 + t % kGenChunk;
            gsh[i][t % kGenChunk] = c < C ? gb[(int64_t)i * C + c] : 0.f;
        }
        __syncthreads();
        float acc[U], dy = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = 0.f;
        for (int i = 0; i < n; ++i) {
            const float gi = gsh[i][cl];
            dy += h[i] * gi;
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u] += mr[i * NM + q + kGenWaves * u] * gi;
        }
        const int c = c0 + cl;
        if (c < C) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = q + kGenWaves * u;
                if (j < n) VecIO<T>::put(gxb + (int64_t)j * C + c, acc[u]);
            }
            if (q == 0) VecIO<T>::put(gy + b * C + c, dy);
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < n) {
        const int i = threadIdx.x;
        float t = 0.f;
#pragma unroll
        for (int q2 = 0; q2 < kGenWaves; ++q2) t += sred[i][q2];
        if (gh_act) gh_act[b * n + i] = t;
        if (gh_raw) gh_raw[b * n + i] = t * h[i] * (1.f - 0.5f * h[i]);
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static bool gen_grid_ok(int64_t B) { return B >= 0 && B <= 0x7fffffff; }

hipError_t launch_gen_static_coef(int n, const float* h_pre, const float* h_post, const float* h_res,
                                  const void* weight, int w_dtype, int64_t C, float* saved, int iters, float sk_eps,
                                  hipStream_t s) {
    if (!generic_layer_n(n) || C < 1 || C > 0x7fffffff) return hipErrorInvalidValue;
    const unsigned blocks = 1 + (unsigned)((C + 2047) / 2048);
    const int off = saved_w_offset(n);
    if (w_dtype == kBF16) {
        MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_static_coef_kernel<NM_, bf16_t>), dim3(blocks), dim3(kGenThreads), 0, s,
                                     h_pre, h_post, h_res, (const bf16_t*)weight, (int)C, saved, off, n, iters,
                                     sk_eps));
    } else {
        MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_static_coef_kernel<NM_, float>), dim3(blocks), dim3(kGenThreads), 0, s,
                                     h_pre, h_post, h_res, (const float*)weight, (int)C, saved, off, n, iters,
                                     sk_eps));
    }
    return hipGetLastError();
}

hipError_t launch_gen_layer_fwd(int x_dtype, int out_dtype, int n, const void* x, const float* w, const float* coef,
                                int64_t coef_stride, void* out, float* rms_out, int64_t B, int64_t C, float eps,
                                hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!generic_layer_n(n) || !gen_grid_ok(B) || C < 1 || C > 0x7fffffff) return hipErrorInvalidValue;
    const int Ci = (int)C;
    const int tok = timing_begin("layer_fwd", s);
#define MHC_GEN_FWD(TX_, TO_)                                                                                   \
    MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_fwd_kernel<TX_, TO_, NM_>), dim3((unsigned)B), dim3(kGenThreads), 0, s,   \
                                 (const TX_*)x, w, coef, coef_stride, (TO_*)out, rms_out, n, Ci, eps))
    if (x_dtype == kBF16) {
        if (out_dtype == kBF16) { MHC_GEN_FWD(bf16_t, bf16_t); } else { MHC_GEN_FWD(bf16_t, float); }
    } else {
        if (out_dtype == kBF16) { MHC_GEN_FWD(float, bf16_t); } else { MHC_GEN_FWD(float, float); }
    }
#undef MHC_GEN_FWD
    timing_end(tok, s);
    return hipGetLastError();
}

int gen_layer_bwd_grid(int64_t B) {
    int64_t g = 2 * (int64_t)device_cu_count();
    if (g > B) g = B;
    return (int)(g < 1 ? 1 : g);
}

size_t gen_layer_bwd_scratch_bytes(int64_t B, int64_t C) {
    return (size_t)gen_layer_bwd_grid(B) * 2 * (size_t)C * sizeof(float);
}

// Gram launches: blocks of 16 for n <= 16, else 32 (two per side above 32).
template <typename TX, int MODE>
static hipError_t gen_gram(const float* g, const TX* x, float* out, int grid, int64_t B, int n, int C, int64_t ostride,
                           hipStream_t s) {
    if (n <= 16) {
        MHC_LAUNCH_GGL((gen_gram_kernel<TX, 16, MODE>), dim3((unsigned)grid, 1), dim3(kGenThreads), 0, s, g, x, out,
                           B, n, C, ostride);
    } else {
        const int nb = (n + 31) / 32;
        MHC_LAUNCH_GGL((gen_gram_kernel<TX, 32, MODE>), dim3((unsigned)grid, (unsigned)(nb * nb)), dim3(kGenThreads),
                           0, s, g, x, out, B, n, C, ostride);
    }
    return hipGetLastError();
}

hipError_t launch_gen_layer_bwd(int x_dtype, int n, int mode, const float* g, const void* x, const float* w,
                                const float* coef, int64_t coef_stride, void* dx, float* dw_part, float* scal_out,
                                int grid, int64_t B, int64_t C, float eps, float* scratch, hipStream_t s) {
    if (!generic_layer_n(n) || (mode != 0 && mode != 1) || C < 1 || C > 0x7fffffff || grid < 1) return hipErrorInvalidValue;
    if (B == 0) return hipSuccess;
    if (grid != gen_layer_bwd_grid(B) || scratch == nullptr) return hipErrorInvalidValue;
    const int Ci = (int)C;
    const int NS = n * n + 2 * n;
    const int tok = timing_begin(mode == 0 ? "layer_bwd" : "layer_bwd_reduce", s);
#define MHC_GEN_BWD(TX_, M_)                                                                                       \
    MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_bwd_kernel<TX_, NM_, M_>), dim3((unsigned)grid), dim3(kGenThreads), 0, s, g, \
                                 (const TX_*)x, w, coef, coef_stride, (TX_*)dx, dw_part, scal_out, scratch, B, n,  \
                                 Ci, eps))
    hipError_t e;
    if (x_dtype == kBF16) {
        if (mode == 0) { MHC_GEN_BWD(bf16_t, 0); } else { MHC_GEN_BWD(bf16_t, 1); }
        e = hipGetLastError();
        if (e == hipSuccess)
            e = mode == 0 ? gen_gram<bf16_t, 0>(g, (const bf16_t*)x, scal_out, grid, B, n, Ci, NS, s)
                          : gen_gram<bf16_t, 1>(g, (const bf16_t*)x, scal_out, grid, B, n, Ci, NS + 2, s);
    } else {
        if (mode == 0) { MHC_GEN_BWD(float, 0); } else { MHC_GEN_BWD(float, 1); }
        e = hipGetLastError();
        if (e == hipSuccess)
            e = mode == 0 ? gen_gram<float, 0>(g, (const float*)x, scal_out, grid, B, n, Ci, NS, s)
                          : gen_gram<float, 1>(g, (const float*)x, scal_out, grid, B, n, Ci, NS + 2, s);
    }
#undef MHC_GEN_BWD
    timing_end(tok, s);
    return e;
}

hipError_t launch_gen_static_finalize(int n, const float* scal_part, int rows, const float* h_pre,
                                      const float* h_post, const float* h_res, float* d_h_pre, float* d_h_post,
                                      float* d_h_res, int iters, float sk_eps, hipStream_t s, float* hist,
                                      size_t hist_bytes) {
    if (!generic_layer_n(n) || rows < 1) return hipErrorInvalidValue;
    // the history when it fits, else the recomputing adjoint
    if ((size_t)skw_hist_floats(kWave, n, iters) * sizeof(float) > hist_bytes) hist = nullptr;
    MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_static_finalize_kernel<NM_>), dim3(1), dim3(kGenThreads), 0, s, scal_part, rows,
                                 h_pre, h_post, h_res, d_h_pre, d_h_post, d_h_res, n, iters, sk_eps, hist));
    return hipGetLastError();
}

hipError_t launch_gen_aggregate_fwd(int dt, int n, const void* x, const float* H, int64_t hs, void* out,
                                    float* h_act, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!generic_ops_n(n) || !gen_grid_ok(B) || C > 0x7fffffff) return hipErrorInvalidValue;
    if (dt == kBF16) {
        MHC_LAUNCH_GGL(gen_aggregate_fwd_kernel<bf16_t>, dim3((unsigned)B), dim3(kGenThreads), 0, s, (const bf16_t*)x,
                           H, hs, (bf16_t*)out, h_act, n, (int)C);
    } else {
        MHC_LAUNCH_GGL(gen_aggregate_fwd_kernel<float>, dim3((unsigned)B), dim3(kGenThreads), 0, s, (const float*)x,
                           H, hs, (float*)out, h_act, n, (int)C);
    }
    return hipGetLastError();
}

hipError_t launch_gen_aggregate_bwd(int dt, int n, const void* g, const void* x, const float* h_act, int64_t hs,
                                    void* gx, float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!generic_ops_n(n) || !gen_grid_ok(B) || C > 0x7fffffff) return hipErrorInvalidValue;
    if (dt == kBF16) {
        MHC_LAUNCH_GGL(gen_aggregate_bwd_kernel<bf16_t>, dim3((unsigned)B), dim3(kGenThreads), 0, s, (const bf16_t*)g,
                           (const bf16_t*)x, h_act, hs, (bf16_t*)gx, gh_act, gh_raw, n, (int)C);
    } else {
        MHC_LAUNCH_GGL(gen_aggregate_bwd_kernel<float>, dim3((unsigned)B), dim3(kGenThreads), 0, s, (const float*)g,
                           (const float*)x, h_act, hs, (float*)gx, gh_act, gh_raw, n, (int)C);
    }
    return hipGetLastError();
}

hipError_t launch_gen_distribute_fwd(int dt, int n, const void* y, const float* H, int64_t hs, const float* M,
                                     int64_t ms, const void* x, float* out, float* h_act, int64_t B, int64_t C,
                                     hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!generic_ops_n(n) || !gen_grid_ok(B) || C > 0x7fffffff) return hipErrorInvalidValue;
    if (dt == kBF16) {
        MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_distribute_fwd_kernel<bf16_t, NM_>), dim3((unsigned)B), dim3(kGenThreads),
                                     0, s, (const bf16_t*)y, H, hs, M, ms, (const bf16_t*)x, out, h_act, n, (int)C));
    } else {
        MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_distribute_fwd_kernel<float, NM_>), dim3((unsigned)B), dim3(kGenThreads),
                                     0, s, (const float*)y, H, hs, M, ms, (const float*)x, out, h_act, n, (int)C));
    }
    return hipGetLastError();
}

hipError_t launch_gen_distribute_bwd(int dt, int n, const float* g, const void* x, const void* y, const float* M,
                                     int64_t ms, const float* h_act, int64_t hs, void* gx, void* gy, float* gM,
                                     float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!generic_ops_n(n) || !gen_grid_ok(B) || C > 0x7fffffff) return hipErrorInvalidValue;
    const int grid = (int)B;
    hipError_t e;
    if (dt == kBF16) {
        MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_distribute_bwd_kernel<bf16_t, NM_>), dim3((unsigned)B), dim3(kGenThreads),
                                     0, s, g, (const bf16_t*)y, M, ms, h_act, hs, (bf16_t*)gx, (bf16_t*)gy, gh_act,
                                     gh_raw, n, (int)C));
        e = hipGetLastError();
        if (e == hipSuccess) e = gen_gram<bf16_t, 1>(g, (const bf16_t*)x, gM, grid, B, n, (int)C, (int64_t)n * n, s);
    } else {
        MHC_GEN_NM(n, MHC_LAUNCH_GGL((gen_distribute_bwd_kernel<float, NM_>), dim3((unsigned)B), dim3(kGenThreads),
                                     0, s, g, (const float*)y, M, ms, h_act, hs, (float*)gx, (float*)gy, gh_act,
                                     gh_raw, n, (int)C));
        e = hipGetLastError();
        if (e == hipSuccess) e = gen_gram<float, 1>(g, (const float*)x, gM, grid, B, n, (int)C, (int64_t)n * n, s);
    }
    return e;
}

#undef MHC_GEN_NM

}  // namespace mhc

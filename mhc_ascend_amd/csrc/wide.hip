// Channel-loop ("wide") row kernels of the mHC layer: one lane per channel,
// and each token row is walked twice - once for its row sums, once (reading
// it again, from cache) for the outputs - instead of being held in
// registers.  They serve what the register-resident kernels of layer.hip
// cannot hold: expansion rates above 8 (the paper's n = 32 configurations,
// benchmark.py:307-309) and, at any n, hidden sizes that are not a multiple
// of the 4-channel chunk (the reference pads those rows, stream_ops.cpp:66-68)
// or too wide for the register rows.  Loads and stores are element-wise, so
// no alignment is assumed.
//
// Math (layer.py:142-170, ops_pytorch_backward.py:9-150), per token b with
// coefficients cf = (h_pre[n], h_post[n], M[n][n]):
//   xa = sum_j h_pre_j x_j,  r = sqrt(mean_c xa^2 + eps),  y = xa / r * w
//   out_i = h_post_i y + sum_j M_ij x_j
// Backward for cotangent g: gy = sum_i h_post_i g_i, k2 = sum(w gy xa)/(C r^3),
//   gxa = w gy / r - xa k2,  dx_j = h_pre_j gxa + sum_i M_ij g_i,
//   dw += gy xa / r,  dh_post_i = sum(g_i xa w) / r,
//   dh_pre_j = sum(w gy x_j) / r - k2 sum(xa x_j),  dM_ij = sum g_i x_j.
// dM (n^2 row sums) is formed in the row pass for n <= 8 and by the Gram
// kernel below for larger n.
#include "mhc_device.h"
#include "mhc_internal.h"

namespace mhc {

constexpr int kWideThreads = 256;
constexpr int kWideFwdThreads = 1024;  // the forward: one token per workgroup, 1-2 channels per lane

template <typename T>
__device__ __forceinline__ float ld_elem_nt(const T* p) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_nontemporal_load(p);
    } else {
        return bf16_to_f32(__builtin_nontemporal_load(p));
    }
}

template <typename T>
__device__ __forceinline__ void st_elem_nt(T* p, float v) {
    if constexpr (sizeof(T) == 4) {
        __builtin_nontemporal_store(v, p);
    } else {
        __builtin_nontemporal_store(f32_to_bf16(v), p);
    }
}

// Block totals of NV per-thread values into tot[NV] (LDS; every thread may
// read them after the call).  red holds NV * (blockDim.x / 64) floats.
template <int NV>
__device__ __forceinline__ void wide_block_total(float (&v)[NV], float* red, float* tot) {
    wave_sum_last<NV>(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    if (lane == kWave - 1) {
#pragma unroll
        for (int k = 0; k < NV; ++k) red[wave * NV + k] = v[k];
    }
    __syncthreads();
    for (int k = threadIdx.x; k < NV; k += blockDim.x) {
        float s = 0.f;
        for (int q = 0; q < nwaves; ++q) s += red[q * NV + k];
        tot[k] = s;
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Forward: one token per workgroup of 1024 lanes (one or two channels per
// lane at the paper widths), so the row sum of xa^2 is one round of 2 N
// loads per lane in flight and the output pass re-reads the row from cache
// (wide_fwd_kernel).  With fewer tokens than two workgroups per CU the
// output pass instead runs over token x 256-channel chunks
// (wide_fwd_out_kernel), after the row sums: one token per workgroup into the
// caller's rms (wide_fwd_rms_kernel), or, when the caller lends scratch of
// at least tokens x chunks floats, token x chunk partials
// (wide_fwd_part_kernel) that each output workgroup sums in a fixed order.
// out in TO (fp32, or bf16 for the forward-only entry); rms_out[b] = r when
// rms_out is the caller's output.
// ---------------------------------------------------------------------------
// Row sum of xa^2 over the token's C channels and r = sqrt(mean + eps),
// block-wide (all threads get r).  cf: the token's coefficients (global).
template <typename TX, int N>
__device__ __forceinline__ float wide_fwd_rowsum(const TX* __restrict__ xb, const float* __restrict__ cf, int C,
                                                 float eps, float* red, float* tot) {
    float ss[1] = {0.f};
    const int step = 2 * (int)blockDim.x;
    int c = threadIdx.x;
    for (; c + (int)blockDim.x < C; c += step) {
        float xa0 = 0.f, xa1 = 0.f;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            xa0 += cf[j] * VecIO<TX>::scalar(xb + (int64_t)j * C + c);
            xa1 += cf[j] * VecIO<TX>::scalar(xb + (int64_t)j * C + c + blockDim.x);
        }
        ss[0] += xa0 * xa0;
        ss[0] += xa1 * xa1;
    }
    if (c < C) {
        float xa = 0.f;
#pragma unroll
        for (int j = 0; j < N; ++j) xa += cf[j] * VecIO<TX>::scalar(xb + (int64_t)j * C + c);
        ss[0] += xa * xa;
    }
    wide_block_total<1>(ss, red, tot);
    return sqrtf(tot[0] / (float)C + eps);
}

// The N output rows of channel c: out_i = h_post_i y + sum_j M_ij x_j with
// y = xa w_c / r; cfs = [h_pre | h_post | M] in LDS.
template <typename TX, typename TO, int N>
__device__ __forceinline__ void wide_fwd_channel(const TX* __restrict__ xb, const float* cfs, float inv,
                                                 const float* __restrict__ w, TO* __restrict__ ob, int c, int C) {
    float xv[N];
#pragma unroll
    for (int j = 0; j < N; ++j) xv[j] = ld_elem_nt(xb + (int64_t)j * C + c);
    float xa = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) xa += cfs[j] * xv[j];
    const float y = xa * inv * w[c];
#pragma unroll 4
    for (int i = 0; i < N; ++i) {
        float s = cfs[N + i] * y;
#pragma unroll
        for (int j = 0; j < N; ++j) s += cfs[2 * N + i * N + j] * xv[j];
        st_elem_nt(ob + (int64_t)i * C + c, s);
    }
}

// ---------------------------------------------------------------------------
// Forward: one token per workgroup of 1024 lanes (one or two channels per
// lane at the paper widths), so the row sum of xa^2 is one round of 2 N
// loads per lane in flight and the output pass re-reads the row from cache.
// (Splitting a token's channels over 256-lane workgroups, each redoing the
// row sum, measured slower at 32-128 tokens: the n = 32, C = 1280 eval
// forward took 0.076 against 0.058 ms at 32 tokens.)  out in TO (fp32, or
// bf16 for the forward-only entry); rms_out[b] = r when not null.
// ---------------------------------------------------------------------------
template <typename TX, typename TO, int N>
__global__ __launch_bounds__(kWideFwdThreads) void wide_fwd_kernel(const TX* __restrict__ x, const float* __restrict__ w,
                                                                   const float* __restrict__ coef, int64_t coef_stride,
                                                                   TO* __restrict__ out, float* __restrict__ rms_out,
                                                                   int64_t B, int C, float eps) {
    constexpr int NC = 2 * N + N * N;
    __shared__ float red[kWideFwdThreads / kWave];
    __shared__ float tot[1];
    __shared__ float cfs[NC];
    const int64_t b = blockIdx.x;
    if (b >= B) return;
    const float* cf = coef + b * coef_stride;
    // the coefficients go to LDS for the output pass (read there, all lanes
    // one address, instead of one dependent scalar load round per output row)
    for (int k = threadIdx.x; k < NC; k += blockDim.x) cfs[k] = cf[k];
    const TX* xb = x + b * (int64_t)N * C;
    const float r = wide_fwd_rowsum<TX, N>(xb, cf, C, eps, red, tot);
    const float inv = 1.f / r;
    TO* ob = out + b * (int64_t)N * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) wide_fwd_channel<TX, TO, N>(xb, cfs, inv, w, ob, c, C);
    if (threadIdx.x == 0 && rms_out) rms_out[b] = r;
}

// Few tokens (fewer than two workgroups per CU): the 1024-lane form leaves
// most CUs idle while its output pass (N rows of N + 1 FMAs per channel)
// runs VALU-bound on one CU per token (n = 32, C = 1280, 32 tokens: 32
// workgroups on 32 of 256 CUs).  Then the row sums run one token per
// workgroup into rms_out (wide_fwd_rms_kernel), and the output pass runs
// over token x 256-channel chunks (wide_fwd_out_kernel), both with the
// arithmetic of wide_fwd_kernel (same r, same per-channel outputs).
template <typename TX, int N>
__global__ __launch_bounds__(kWideFwdThreads) void wide_fwd_rms_kernel(const TX* __restrict__ x,
                                                                       const float* __restrict__ coef,
                                                                       int64_t coef_stride,
                                                                       float* __restrict__ rms_out, int64_t B, int C,
                                                                       float eps) {
    __shared__ float red[kWideFwdThreads / kWave];
    __shared__ float tot[1];
    const int64_t b = blockIdx.x;
    if (b >= B) return;
    const float r = wide_fwd_rowsum<TX, N>(x + b * (int64_t)N * C, coef + b * coef_stride, C, eps, red, tot);
    if (threadIdx.x == 0) rms_out[b] = r;
}

constexpr int kWideFwdChunk = 256;

// Row-sum partials of one 256-channel chunk (for callers whose r is only an
// intermediate): part[b * gridDim.x + chunk] = the chunk's sum of xa^2, in
// fixed-order wave and block sums.
template <typename TX, int N>
__global__ __launch_bounds__(kWideFwdChunk) void wide_fwd_part_kernel(const TX* __restrict__ x,
                                                                      const float* __restrict__ coef,
                                                                      int64_t coef_stride, float* __restrict__ part,
                                                                      int64_t B, int C) {
    __shared__ float red[kWideFwdChunk / kWave];
    __shared__ float tot[1];
    const int64_t b = blockIdx.y;
    if (b >= B) return;
    const float* cf = coef + b * coef_stride;
    const TX* xb = x + b * (int64_t)N * C;
    const int c = (int)blockIdx.x * kWideFwdChunk + (int)threadIdx.x;
    float ss[1] = {0.f};
    if (c < C) {
        float xa = 0.f;
#pragma unroll
        for (int j = 0; j < N; ++j) xa += cf[j] * VecIO<TX>::scalar(xb + (int64_t)j * C + c);
        ss[0] = xa * xa;
    }
    wide_block_total<1>(ss, red, tot);
    if (threadIdx.x == 0) part[b * (int64_t)gridDim.x + blockIdx.x] = tot[0];
}

template <typename TX, typename TO, int N>
__global__ __launch_bounds__(kWideFwdChunk) void wide_fwd_out_kernel(const TX* __restrict__ x,
                                                                     const float* __restrict__ w,
                                                                     const float* __restrict__ coef,
                                                                     int64_t coef_stride, TO* __restrict__ out,
                                                                     const float* __restrict__ rms, int S, int64_t B,
                                                                     int C, float eps) {
    constexpr int NC = 2 * N + N * N;
    __shared__ float cfs[NC];
    const int64_t b = blockIdx.y;
    if (b >= B) return;
    const float* cf = coef + b * coef_stride;
    for (int k = threadIdx.x; k < NC; k += blockDim.x) cfs[k] = cf[k];
    __syncthreads();
    // r of the token: rms[b], or (S > 0) from its S chunk partials rms[b S ..]
    float r;
    if (S > 0) {
        float t = 0.f;
        for (int q = 0; q < S; ++q) t += rms[b * S + q];
        r = sqrtf(t / (float)C + eps);
    } else {
        r = rms[b];
    }
    const float inv = 1.f / r;
    const int c = (int)blockIdx.x * kWideFwdChunk + (int)threadIdx.x;
    if (c < C) wide_fwd_channel<TX, TO, N>(x + b * (int64_t)N * C, cfs, inv, w, out + b * (int64_t)N * C, c, C);
}

// ---------------------------------------------------------------------------
// Backward pieces shared by the persistent and the chunked kernels.
// Row sums per channel (NR of them): ss, dot, t_i, u_j, v_j (, dM_ij).
// Per-token scalar entries (layout [dM | dh_post | dh_pre | 1/r | k2]) from
// the row totals; dx of one channel (returns its dw term gy xa / r).
// ---------------------------------------------------------------------------
template <int N, bool DM> constexpr int wide_nr() { return 2 + 3 * N + (DM ? N * N : 0); }

template <typename TX, int N, bool DM>
__device__ __forceinline__ void wide_bwd_accum(const float* __restrict__ cf, const TX* __restrict__ xb,
                                               const float* __restrict__ gb, const float* __restrict__ w, int c,
                                               int C, float (&rv)[wide_nr<N, DM>()]) {
    float xv[N], gv[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
        xv[j] = VecIO<TX>::scalar(xb + (int64_t)j * C + c);
        gv[j] = gb[(int64_t)j * C + c];
    }
    float xa = 0.f, gy = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        xa += cf[j] * xv[j];
        gy += cf[N + j] * gv[j];
    }
    const float wc = w[c];
    const float wgy = wc * gy, wxa = wc * xa;
    rv[0] += xa * xa;
    rv[1] += wgy * xa;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        rv[2 + i] += gv[i] * wxa;
        rv[2 + N + i] += wgy * xv[i];
        rv[2 + 2 * N + i] += xa * xv[i];
    }
    if constexpr (DM) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
#pragma unroll
            for (int j = 0; j < N; ++j) rv[2 + 3 * N + i * N + j] += gv[i] * xv[j];
        }
    }
}

template <int N>
__device__ __forceinline__ float wide_bwd_scalar(const float* tot, int t, float inv, float k2) {
    constexpr int NS = N * N + 2 * N;
    if (t < N * N) return tot[2 + 3 * N + t];
    if (t < N * N + N) return tot[2 + t - N * N] * inv;  // dh_post_act
    if (t < NS) {
        const int j = t - N * N - N;
        return inv * tot[2 + N + j] - k2 * tot[2 + 2 * N + j];  // dh_pre_act
    }
    return t == NS ? inv : k2;
}

template <typename TX, int N>
__device__ __forceinline__ float wide_bwd_dx(const float* __restrict__ cf, const TX* __restrict__ xb,
                                             const float* __restrict__ gb, const float* __restrict__ w,
                                             TX* __restrict__ db, int c, int C, float inv, float k2) {
    float xv[N], gv[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
        xv[j] = ld_elem_nt(xb + (int64_t)j * C + c);
        gv[j] = ld_elem_nt(gb + (int64_t)j * C + c);
    }
    float xa = 0.f, gy = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        xa += cf[j] * xv[j];
        gy += cf[N + j] * gv[j];
    }
    const float gxa = w[c] * gy * inv - xa * k2;
#pragma unroll 4
    for (int j = 0; j < N; ++j) {
        float s = cf[j] * gxa;
#pragma unroll
        for (int i = 0; i < N; ++i) s += cf[2 * N + i * N + j] * gv[i];
        st_elem_nt(db + (int64_t)j * C + c, s);
    }
    return gy * xa * inv;
}

// ---------------------------------------------------------------------------
// Backward.  Persistent workgroups stride over tokens; the workgroup's dw
// partial lives in LDS (dynamic shared memory, C floats, each entry owned by
// the lane that owns the channel) and goes to dw_part[blockIdx.x][C] at the
// end.  Per-token scalars: MODE 0 sums them per workgroup into
// scal_out[blockIdx.x][NS], MODE 1 writes them per token into
// scal_out[b][NS + 2].  With DM false the dM entries are left to
// stream_gram_kernel.
// ---------------------------------------------------------------------------
template <typename TX, int N, int MODE, bool DM>
__global__ __launch_bounds__(kWideThreads) void wide_bwd_kernel(const float* __restrict__ g, const TX* __restrict__ x,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ coef, int64_t coef_stride,
                                                                TX* __restrict__ dx, float* __restrict__ dw_part,
                                                                float* __restrict__ scal_out, int64_t B, int C,
                                                                float eps) {
    extern __shared__ float dws[];
    constexpr int NS = N * N + 2 * N;
    constexpr int NR = wide_nr<N, DM>();
    // scalar entries this kernel writes: E0 .. NS + 1, one per lane
    constexpr int E0 = DM ? 0 : N * N;
    constexpr int NE = NS + 2 - E0;
    static_assert(NE <= kWideThreads, "one scalar entry per lane");
    __shared__ float red[(kWideThreads / kWave) * NR];
    __shared__ float tot[NR];
    const int tid = threadIdx.x;
    for (int c = tid; c < C; c += blockDim.x) dws[c] = 0.f;
    float sacc = 0.f;
    const int64_t NCs = (int64_t)N * C;
    __shared__ float cfs[2 * N + N * N];
    for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
        const float* cf = coef + b * coef_stride;
        const TX* xb = x + b * NCs;
        const float* gb = g + b * NCs;
        for (int k = tid; k < 2 * N + N * N; k += blockDim.x) cfs[k] = cf[k];
        float rv[NR];
#pragma unroll
        for (int k = 0; k < NR; ++k) rv[k] = 0.f;
        for (int c = tid; c < C; c += blockDim.x) wide_bwd_accum<TX, N, DM>(cf, xb, gb, w, c, C, rv);
        wide_block_total<NR>(rv, red, tot);
        const float r = sqrtf(tot[0] / (float)C + eps);
        const float inv = 1.f / r;
        const float k2 = tot[1] * inv * inv * inv / (float)C;
        if (tid < NE) {
            const int t = E0 + tid;
            const float v = wide_bwd_scalar<N>(tot, t, inv, k2);
            if (MODE == 0) {
                sacc += v;
            } else {
                scal_out[b * (NS + 2) + t] = v;
            }
        }
        TX* db = dx + b * NCs;
        for (int c = tid; c < C; c += blockDim.x) dws[c] += wide_bwd_dx<TX, N>(cfs, xb, gb, w, db, c, C, inv, k2);
        __syncthreads();  // cfs is restaged for the next token
    }
    float* dwp = dw_part + (int64_t)blockIdx.x * C;
    for (int c = tid; c < C; c += blockDim.x) dwp[c] = dws[c];
    if (MODE == 0 && tid < NE && E0 + tid < NS) scal_out[(int64_t)blockIdx.x * NS + E0 + tid] = sacc;
}

// ---------------------------------------------------------------------------
// Backward over channel chunks, for fewer tokens than fill the chip:
// workgroup (b, s) of grid B x S takes token b's channel chunk s.  The first
// kernel stores the chunk's row sums in part[b][s][NR]; the second adds a
// token's S partials in chunk order, forms the per-token scalars (chunk 0
// stores them: MODE 1 per token as wide_bwd_kernel, MODE 0 as row b of
// scal_out[B][NS]) and the chunk's dx and dw terms (row b of dw_part[B][C]).
// Same outputs as wide_bwd_kernel with one token per workgroup.
// ---------------------------------------------------------------------------
template <typename TX, int N, bool DM>
__global__ __launch_bounds__(kWideThreads) void wide_bwd_sums_kernel(const float* __restrict__ g,
                                                                     const TX* __restrict__ x,
                                                                     const float* __restrict__ w,
                                                                     const float* __restrict__ coef,
                                                                     int64_t coef_stride, float* __restrict__ part,
                                                                     int64_t B, int C, int S, int chunk) {
    constexpr int NR = wide_nr<N, DM>();
    __shared__ float red[(kWideThreads / kWave) * NR];
    __shared__ float tot[NR];
    const int64_t b = blockIdx.x / S;
    const int sc = (int)(blockIdx.x % S);
    if (b >= B) return;
    const int64_t NCs = (int64_t)N * C;
    const float* cf = coef + b * coef_stride;
    const TX* xb = x + b * NCs;
    const float* gb = g + b * NCs;
    float rv[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) rv[k] = 0.f;
    const int c_end = (sc + 1) * chunk < C ? (sc + 1) * chunk : C;
    for (int c = sc * chunk + (int)threadIdx.x; c < c_end; c += blockDim.x)
        wide_bwd_accum<TX, N, DM>(cf, xb, gb, w, c, C, rv);
    wide_block_total<NR>(rv, red, tot);
    for (int k = threadIdx.x; k < NR; k += blockDim.x) part[((int64_t)blockIdx.x) * NR + k] = tot[k];
}

template <typename TX, int N, int MODE, bool DM>
__global__ __launch_bounds__(kWideThreads) void wide_bwd_out_kernel(
    const float* __restrict__ g, const TX* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ coef, int64_t coef_stride, TX* __restrict__ dx, float* __restrict__ dw_part,
    float* __restrict__ scal_out, const float* __restrict__ part, int64_t B, int C, float eps, int S, int chunk) {
    constexpr int NS = N * N + 2 * N;
    constexpr int NR = wide_nr<N, DM>();
    constexpr int E0 = DM ? 0 : N * N;
    constexpr int NE = NS + 2 - E0;
    static_assert(NE <= kWideThreads && NR <= kWideThreads, "one entry per lane");
    __shared__ float tot[NR];
    __shared__ float cfs[2 * N + N * N];
    const int64_t b = blockIdx.x / S;
    const int sc = (int)(blockIdx.x % S);
    if (b >= B) return;
    const int tid = threadIdx.x;
    for (int k = tid; k < 2 * N + N * N; k += blockDim.x) cfs[k] = coef[b * coef_stride + k];
    if (tid < NR) {
        const float* pb = part + b * S * NR + tid;
        float v = 0.f;
        for (int q = 0; q < S; ++q) v += pb[(int64_t)q * NR];
        tot[tid] = v;
    }
    __syncthreads();
    const float r = sqrtf(tot[0] / (float)C + eps);
    const float inv = 1.f / r;
    const float k2 = tot[1] * inv * inv * inv / (float)C;
    if (sc == 0 && tid < NE) {
        const int t = E0 + tid;
        const float v = wide_bwd_scalar<N>(tot, t, inv, k2);
        if (MODE == 1) {
            scal_out[b * (NS + 2) + t] = v;
        } else if (t < NS) {
            scal_out[b * NS + t] = v;
        }
    }
    const int64_t NCs = (int64_t)N * C;
    const TX* xb = x + b * NCs;
    const float* gb = g + b * NCs;
    TX* db = dx + b * NCs;
    float* dwp = dw_part + b * C;
    const int c_end = (sc + 1) * chunk < C ? (sc + 1) * chunk : C;
    for (int c = sc * chunk + tid; c < c_end; c += blockDim.x)
        dwp[c] = wide_bwd_dx<TX, N>(cfs, xb, gb, w, db, c, C, inv, k2);
}

// ---------------------------------------------------------------------------
// dM_ij = sum_c g_i x_j of each token (n = 16, 32) on the fp32 matrix cores:
// v_mfma_f32_32x32x2_f32 (n = 32) or v_mfma_f32_16x16x4_f32 (n = 16) with
// A = g (row i = stream i), B = x^T and k = channel.  Lane l holds stream
// i = l % n in k slot h = l / n (KQ = 64 / n slots).  A step of a wave loads
// 16 consecutive channels of g_i and x_i at c0 + 16 h (16 KQ channels per
// step) and issues 16 MFMAs, product q taking channel c0 + 16 h + q in slot
// h; steps go round-robin to the 4 waves, the next one in flight while the
// current one is on the matrix cores.  The waves' partial matrices are
// added through LDS in wave order.  MODE 0 sums the workgroup's tokens
// (strided over the grid, as wide_bwd_kernel's) into
// scal_out[blockIdx.x][0 .. n^2); MODE 1 stores each token's dM at
// scal_out[b * ostride + 0 .. n^2).  VEC: 16-byte loads (C % 8 == 0 and
// aligned rows), else element loads.
// ---------------------------------------------------------------------------
typedef float gram_f32x16_t __attribute__((ext_vector_type(16)));
typedef float gram_f32x4_t __attribute__((ext_vector_type(4)));

template <int N> struct GramMfma;
template <> struct GramMfma<32> {
    using acc_t = gram_f32x16_t;
    static constexpr int R = 16;  // accumulator registers per lane
    __device__ __forceinline__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    // element (row, col) of D held in register r of lane l
    __device__ __forceinline__ static int row(int l, int r) { return 8 * (r / 4) + 4 * (l / 32) + (r % 4); }
    __device__ __forceinline__ static int col(int l) { return l % 32; }
};
template <> struct GramMfma<16> {
    using acc_t = gram_f32x4_t;
    static constexpr int R = 4;
    __device__ __forceinline__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    __device__ __forceinline__ static int row(int l, int r) { return 4 * (l / 16) + r; }
    __device__ __forceinline__ static int col(int l) { return l % 16; }
};

// 16 consecutive channels c .. c + 15 of one row as floats; channels past C
// read zero.  VEC: C % 8 == 0 and 16-byte aligned rows, so each 16-byte
// piece is wholly inside or outside the row.
template <typename T, bool VEC>
__device__ __forceinline__ void gram_load16(const T* __restrict__ row, int c, int C, float (&v)[16]) {
    if constexpr (VEC) {
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
                if (c + 4 * u < C) q = *reinterpret_cast<const float4*>(row + c + 4 * u);
                v[4 * u] = q.x;
                v[4 * u + 1] = q.y;
                v[4 * u + 2] = q.z;
                v[4 * u + 3] = q.w;
            }
        } else {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                uint4 q = make_uint4(0u, 0u, 0u, 0u);
                if (c + 8 * u < C) q = *reinterpret_cast<const uint4*>(row + c + 8 * u);
                const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[8 * u + 2 * e] = __uint_as_float(wv[e] << 16);
                    v[8 * u + 2 * e + 1] = __uint_as_float(wv[e] & 0xffff0000u);
                }
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = (c + q < C) ? VecIO<T>::scalar(row + c + q) : 0.f;
    }
}

template <typename TX, int N, int MODE, bool VEC>
__global__ __launch_bounds__(kWideThreads) void stream_gram_kernel(const float* __restrict__ g,
                                                                  const TX* __restrict__ x,
                                                                  float* __restrict__ scal_out, int64_t B, int C,
                                                                  int64_t ostride) {
    using M = GramMfma<N>;
    using acc_t = typename M::acc_t;
    constexpr int KQ = kWave / N;       // k slots per MFMA
    constexpr int SC = 16 * KQ;         // channels per wave step
    constexpr int NW = kWideThreads / kWave;
    constexpr int NS = N * N + 2 * N;
    __shared__ float red[NW - 1][M::R][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int i = lane % N, h = lane / N;
    const int nsteps = (C + SC - 1) / SC;
    const int64_t NCs = (int64_t)N * C;
    acc_t acc = {};
    for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
        if (MODE == 1) acc = acc_t{};
        const float* gr = g + b * NCs + (int64_t)i * C;
        const TX* xr = x + b * NCs + (int64_t)i * C;
        float ga[16], xa[16];
        int st = wave;
        if (st < nsteps) {
            gram_load16<float, VEC>(gr, st * SC + 16 * h, C, ga);
            gram_load16<TX, VEC>(xr, st * SC + 16 * h, C, xa);
        }
        for (; st < nsteps; st += NW) {
            float gn[16], xn[16];
            const int nx = st + NW;
            if (nx < nsteps) {
                gram_load16<float, VEC>(gr, nx * SC + 16 * h, C, gn);
                gram_load16<TX, VEC>(xr, nx * SC + 16 * h, C, xn);
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) acc = M::step(ga[q], xa[q], acc);
            if (nx < nsteps) {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    ga[q] = gn[q];
                    xa[q] = xn[q];
                }
            }
        }
        if (MODE == 1) {
            if (wave > 0) {
#pragma unroll
                for (int r = 0; r < M::R; ++r) red[wave - 1][r][lane] = acc[r];
            }
            __syncthreads();
            if (wave == 0) {
                float* o = scal_out + b * ostride;
#pragma unroll
                for (int r = 0; r < M::R; ++r) {
                    float v = acc[r];
#pragma unroll
                    for (int q = 0; q < NW - 1; ++q) v += red[q][r][lane];
                    o[M::row(lane, r) * N + M::col(lane)] = v;
                }
            }
            __syncthreads();
        }
    }
    if (MODE == 0) {
        if (wave > 0) {
#pragma unroll
            for (int r = 0; r < M::R; ++r) red[wave - 1][r][lane] = acc[r];
        }
        __syncthreads();
        if (wave == 0) {
            float* o = scal_out + (int64_t)blockIdx.x * NS;
#pragma unroll
            for (int r = 0; r < M::R; ++r) {
                float v = acc[r];
#pragma unroll
                for (int q = 0; q < NW - 1; ++q) v += red[q][r][lane];
                o[M::row(lane, r) * N + M::col(lane)] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Static parameter gradients for n >= 16 from the per-workgroup sums
// scal_part[rows][n^2 + 2n]: column totals in LDS, then (as layer.hip's
// finalize) dH_pre = dh_pre_act h_pre (1 - h_pre), dH_post = dh_post_act
// h_post (1 - h_post / 2) and dH_res = SK^T(dM) * exp(H_res), the Sinkhorn
// adjoint on the whole workgroup for n = 32 (iters <= skb::kTMax, state in
// registers), on wave 0 for n = 16 (iters <= skw16::kTMax, state in
// registers), otherwise one row per lane of the first n lanes with its
// per-iteration state in hist (iters * (n + 1) * n floats) or, without hist,
// recomputed.
// ---------------------------------------------------------------------------
constexpr int kStaticFinalizeThreads = skb::kThreads;

template <int N>
__global__ __launch_bounds__(kStaticFinalizeThreads) void wide_static_finalize_kernel(
    const float* __restrict__ scal_part, int rows, const float* __restrict__ h_pre, const float* __restrict__ h_post,
    const float* __restrict__ h_res, float* __restrict__ d_h_pre, float* __restrict__ d_h_post,
    float* __restrict__ d_h_res, int iters, float eps, float* __restrict__ hist) {
    constexpr int NS = N * N + 2 * N;
    constexpr int KPT = (NS + kStaticFinalizeThreads - 1) / kStaticFinalizeThreads;
    constexpr int RB = 4;  // rows loaded per round trip
    __shared__ float tot[NS];
    {
        // column sums of the partial rows, in row order; each lane's columns
        // and RB rows are loaded together
        float acc[KPT];
#pragma unroll
        for (int q = 0; q < KPT; ++q) acc[q] = 0.f;
        for (int r0 = 0; r0 < rows; r0 += RB) {
            float v[RB][KPT];
#pragma unroll
            for (int j = 0; j < RB; ++j) {
#pragma unroll
                for (int q = 0; q < KPT; ++q) {
                    const int k = threadIdx.x + q * kStaticFinalizeThreads;
                    v[j][q] = (r0 + j < rows && k < NS) ? scal_part[(int64_t)(r0 + j) * NS + k] : 0.f;
                }
            }
#pragma unroll
            for (int j = 0; j < RB; ++j) {
#pragma unroll
                for (int q = 0; q < KPT; ++q) {
                    if (r0 + j < rows) acc[q] += v[j][q];
                }
            }
        }
#pragma unroll
        for (int q = 0; q < KPT; ++q) {
            const int k = threadIdx.x + q * kStaticFinalizeThreads;
            if (k < NS) tot[k] = acc[q];
        }
    }
    __syncthreads();
    if constexpr (N == skb::kN) {
        if (iters <= skb::kTMax) {
            __shared__ float part[skb::kPartFloats];
            __shared__ float hc[skb::kHistFloats];
            const int i = skb::row(), c0 = skb::col0();
            float e[skb::kV], gm[skb::kV];
#pragma unroll
            for (int k = 0; k < skb::kV; ++k) {
                e[k] = expf(h_res[i * N + c0 + k]);
                gm[k] = tot[i * N + c0 + k];
            }
            skb::backward(gm, e, iters, eps, part, hc);
#pragma unroll
            for (int k = 0; k < skb::kV; ++k) d_h_res[i * N + c0 + k] = gm[k] * e[k];
        }
    }
    if constexpr (N == skw16::kN) {
        if (iters <= skw16::kTMax && threadIdx.x < kWave) {
            // wave 0 on the 16 x 16 matrix, four elements per lane
            const int i = skw16::row(), c0 = skw16::col0();
            float e[skw16::kV], gm[skw16::kV];
#pragma unroll
            for (int k = 0; k < skw16::kV; ++k) {
                e[k] = expf(h_res[i * N + c0 + k]);
                gm[k] = tot[i * N + c0 + k];
            }
            skw16::backward(gm, e, iters, eps);
#pragma unroll
            for (int k = 0; k < skw16::kV; ++k) d_h_res[i * N + c0 + k] = gm[k] * e[k];
        }
    }
    const bool lane_rows = (N == skb::kN && iters > skb::kTMax) || (N == skw16::kN && iters > skw16::kTMax) ||
                           (N != skb::kN && N != skw16::kN);
    if (threadIdx.x < N && lane_rows) {
        const int r = threadIdx.x;
        float e[N], gm[N];
#pragma unroll
        for (int c = 0; c < N; ++c) {
            e[c] = expf(h_res[r * N + c]);
            gm[c] = tot[r * N + c];
        }
        if (hist) {
            sk_backward_mem<N>(gm, e, iters, eps, true, hist, r);
        } else {
            sk_backward<N>(gm, e, iters, eps, true);
        }
#pragma unroll
        for (int c = 0; c < N; ++c) d_h_res[r * N + c] = gm[c] * e[c];
    }
    if (threadIdx.x < N) {
        const int r = threadIdx.x;
        const float tp = sigmoidf(h_pre[r]);
        const float tq = 2.f * sigmoidf(h_post[r]);
        d_h_pre[r] = tot[N * N + N + r] * tp * (1.f - tp);
        d_h_post[r] = tot[N * N + r] * tq * (1.f - tq * 0.5f);
    }
}

// ---------------------------------------------------------------------------
// Standalone operators on rows of any width and n in {1, 2, 4, 8, 16, 32}
// (the formulas of ops.hip; bindings.cpp:237-374, 380-460, 543-566).  One
// token row per workgroup (the RMSNorm backward: persistent, dw in LDS).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kWideThreads) void wide_rmsnorm_fwd_kernel(const T* __restrict__ x,
                                                                        const float* __restrict__ w,
                                                                        T* __restrict__ y, float* __restrict__ rms,
                                                                        int C, float eps) {
    __shared__ float red[kWideThreads / kWave];
    __shared__ float tot[1];
    const int64_t b = blockIdx.x;
    const T* xb = x + b * C;
    float ss[1] = {0.f};
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        const float v = VecIO<T>::scalar(xb + c);
        ss[0] += v * v;
    }
    wide_block_total<1>(ss, red, tot);
    const float r = sqrtf(tot[0] / (float)C + eps);
    const float inv = 1.f / r;
    for (int c = threadIdx.x; c < C; c += blockDim.x) st_elem_nt(y + b * C + c, ld_elem_nt(xb + c) * inv * w[c]);
    if (threadIdx.x == 0) rms[b] = r;
}

template <typename T>
__global__ __launch_bounds__(kWideThreads) void wide_rmsnorm_bwd_kernel(const T* __restrict__ g,
                                                                        const T* __restrict__ x,
                                                                        const float* __restrict__ w,
                                                                        const float* __restrict__ rms,
                                                                        T* __restrict__ gx,
                                                                        float* __restrict__ dw_part, int64_t B,
                                                                        int C) {
    extern __shared__ float dws[];
    __shared__ float red[kWideThreads / kWave];
    __shared__ float tot[1];
    for (int c = threadIdx.x; c < C; c += blockDim.x) dws[c] = 0.f;
    for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
        const T* xb = x + b * C;
        const T* gb = g + b * C;
        const float inv = 1.f / rms[b];
        float dot[1] = {0.f};
        for (int c = threadIdx.x; c < C; c += blockDim.x)
            dot[0] += VecIO<T>::scalar(gb + c) * w[c] * VecIO<T>::scalar(xb + c);
        wide_block_total<1>(dot, red, tot);
        const float k2 = tot[0] * inv * inv * inv / (float)C;
        for (int c = threadIdx.x; c < C; c += blockDim.x) {
            const float gv = ld_elem_nt(gb + c), xv = ld_elem_nt(xb + c);
            st_elem_nt(gx + b * C + c, w[c] * gv * inv - xv * k2);
            dws[c] += gv * xv * inv;
        }
    }
    for (int c = threadIdx.x; c < C; c += blockDim.x) dw_part[(int64_t)blockIdx.x * C + c] = dws[c];
}

template <typename T>
__global__ __launch_bounds__(kWideThreads) void wide_compute_rms_kernel(const T* __restrict__ x,
                                                                        float* __restrict__ rms, int64_t K,
                                                                        float eps) {
    __shared__ float red[kWideThreads / kWave];
    __shared__ float tot[1];
    const int64_t b = blockIdx.x;
    float ss[1] = {0.f};
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
        const float v = ld_elem_nt(x + b * K + k);
        ss[0] += v * v;
    }
    wide_block_total<1>(ss, red, tot);
    if (threadIdx.x == 0) rms[b] = sqrtf(tot[0] / (float)K + eps);
}

template <typename T, int N>
__global__ __launch_bounds__(kWideThreads) void wide_aggregate_fwd_kernel(const T* __restrict__ x,
                                                                          const float* __restrict__ H,
                                                                          int64_t h_stride, T* __restrict__ out,
                                                                          float* __restrict__ h_act, int C) {
    const int64_t b = blockIdx.x;
    float h[N];
#pragma unroll
    for (int i = 0; i < N; ++i) h[i] = sigmoidf(H[b * h_stride + i]);
    const T* xb = x + b * (int64_t)N * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) s += h[i] * ld_elem_nt(xb + (int64_t)i * C + c);
        st_elem_nt(out + b * C + c, s);
    }
    if (threadIdx.x < N) {
        float hi = 0.f;
#pragma unroll
        for (int q = 0; q < N; ++q) hi = (q == (int)threadIdx.x) ? h[q] : hi;
        h_act[b * N + threadIdx.x] = hi;
    }
}

template <typename T, int N>
__global__ __launch_bounds__(kWideThreads) void wide_aggregate_bwd_kernel(
    const T* __restrict__ g, const T* __restrict__ x, const float* __restrict__ h_act, int64_t h_stride,
    T* __restrict__ gx, float* __restrict__ gh_act, float* __restrict__ gh_raw, int C) {
    __shared__ float red[(kWideThreads / kWave) * N];
    __shared__ float tot[N];
    const int64_t b = blockIdx.x;
    float h[N], sv[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        h[i] = h_act[b * h_stride + i];
        sv[i] = 0.f;
    }
    const T* xb = x + b * (int64_t)N * C;
    T* gb = gx + b * (int64_t)N * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        const float gv = ld_elem_nt(g + b * C + c);
#pragma unroll
        for (int i = 0; i < N; ++i) {
            sv[i] += gv * ld_elem_nt(xb + (int64_t)i * C + c);
            st_elem_nt(gb + (int64_t)i * C + c, gv * h[i]);
        }
    }
    wide_block_total<N>(sv, red, tot);
    if (threadIdx.x < N) {
        const int i = threadIdx.x;
        const float hi = h_act[b * h_stride + i];
        if (gh_act) gh_act[b * N + i] = tot[i];
        if (gh_raw) gh_raw[b * N + i] = tot[i] * hi * (1.f - hi);
    }
}

template <typename T, int N>
__global__ __launch_bounds__(kWideThreads) void wide_distribute_fwd_kernel(
    const T* __restrict__ y, const float* __restrict__ H, int64_t h_stride, const float* __restrict__ M,
    int64_t m_stride, const T* __restrict__ x, float* __restrict__ out, float* __restrict__ h_act, int C) {
    const int64_t b = blockIdx.x;
    float h[N];
#pragma unroll
    for (int i = 0; i < N; ++i) h[i] = 2.f * sigmoidf(H[b * h_stride + i]);
    const float* mb = M + b * m_stride;
    const T* xb = x + b * (int64_t)N * C;
    float* ob = out + b * (int64_t)N * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        float xv[N];
#pragma unroll
        for (int j = 0; j < N; ++j) xv[j] = ld_elem_nt(xb + (int64_t)j * C + c);
        const float yv = ld_elem_nt(y + b * C + c);
        for (int i = 0; i < N; ++i) {
            float s = h[i] * yv;
#pragma unroll
            for (int j = 0; j < N; ++j) s += mb[i * N + j] * xv[j];
            st_elem_nt(ob + (int64_t)i * C + c, s);
        }
    }
    if (threadIdx.x < N) {
        float hi = 0.f;
#pragma unroll
        for (int q = 0; q < N; ++q) hi = (q == (int)threadIdx.x) ? h[q] : hi;
        h_act[b * N + threadIdx.x] = hi;
    }
}

// dM in the row sums for n <= 8 (DM); for n >= 16 stream_gram_kernel writes it.
template <typename T, int N, bool DM>
__global__ __launch_bounds__(kWideThreads) void wide_distribute_bwd_kernel(
    const float* __restrict__ g, const T* __restrict__ x, const T* __restrict__ y, const float* __restrict__ M,
    int64_t m_stride, const float* __restrict__ h_act, int64_t h_stride, T* __restrict__ gx, T* __restrict__ gy,
    float* __restrict__ gM, float* __restrict__ gh_act, float* __restrict__ gh_raw, int C) {
    constexpr int NR = N + (DM ? N * N : 0);  // dh_act_i (, dM_ij)
    __shared__ float red[(kWideThreads / kWave) * NR];
    __shared__ float tot[NR];
    const int64_t b = blockIdx.x;
    float h[N], sv[NR];
#pragma unroll
    for (int i = 0; i < N; ++i) h[i] = h_act[b * h_stride + i];
#pragma unroll
    for (int k = 0; k < NR; ++k) sv[k] = 0.f;
    const float* mb = M + b * m_stride;
    const float* gb = g + b * (int64_t)N * C;
    const T* xb = x + b * (int64_t)N * C;
    T* dxb = gx + b * (int64_t)N * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        float gv[N];
#pragma unroll
        for (int i = 0; i < N; ++i) gv[i] = ld_elem_nt(gb + (int64_t)i * C + c);
        const float yv = ld_elem_nt(y + b * C + c);
        float dy = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            sv[i] += gv[i] * yv;
            dy += h[i] * gv[i];
        }
        st_elem_nt(gy + b * C + c, dy);
        if constexpr (DM) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const float xj = ld_elem_nt(xb + (int64_t)j * C + c);
#pragma unroll
                for (int i = 0; i < N; ++i) sv[N + i * N + j] += gv[i] * xj;
            }
        }
        for (int j = 0; j < N; ++j) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < N; ++i) t += mb[i * N + j] * gv[i];
            st_elem_nt(dxb + (int64_t)j * C + c, t);
        }
    }
    wide_block_total<NR>(sv, red, tot);
    for (int t = threadIdx.x; t < NR; t += blockDim.x) {
        if (t < N) {
            const float hi = h_act[b * h_stride + t];
            if (gh_act) gh_act[b * N + t] = tot[t];
            if (gh_raw) gh_raw[b * N + t] = tot[t] * hi * (1.f - 0.5f * hi);
        } else {
            gM[b * N * N + (t - N)] = tot[t];
        }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
#define MHC_WIDE_N(n, ...)                                        \
    switch (n) {                                                  \
        case 2: { constexpr int N_ = 2; __VA_ARGS__; break; }     \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }     \
        case 8: { constexpr int N_ = 8; __VA_ARGS__; break; }     \
        case 16: { constexpr int N_ = 16; __VA_ARGS__; break; }   \
        case 32: { constexpr int N_ = 32; __VA_ARGS__; break; }   \
        default: return hipErrorInvalidValue;                     \
    }

bool wide_supported(int n, int64_t C) {
    return (n == 2 || n == 4 || n == 8 || n == 16 || n == 32) && C >= 1 && C <= kWideMaxC;
}

hipError_t launch_wide_fwd(int x_dtype, int out_dtype, int n, const void* x, const float* w, const float* coef,
                           int64_t coef_stride, void* out, float* rms_out, int64_t B, int64_t C, float eps,
                           hipStream_t s, int64_t rms_scratch) {
    if (B == 0) return hipSuccess;
    if (!wide_supported(n, C) || B > 0x7fffffff) return hipErrorInvalidValue;
    const int Ci = (int)C;
    const dim3 grid((unsigned)B), block(kWideFwdThreads);
    // token x channel-chunk output pass when the row sums have somewhere to go
    // (rms_out) and the tokens alone would leave CUs idle
    const int64_t chunks = (C + kWideFwdChunk - 1) / kWideFwdChunk;
    const bool split = rms_out != nullptr && chunks >= 2 && B < 2 * (int64_t)device_cu_count();
    // rms_out as scratch of rms_scratch floats (r not needed by the caller):
    // the row sums too run over token x chunk workgroups, into B * chunks partials
    const bool parts = split && rms_scratch >= B * chunks;
    const int S = parts ? (int)chunks : 0;
    const dim3 ogrid((unsigned)chunks, (unsigned)B), oblock(kWideFwdChunk);
    const int tok = timing_begin("layer_fwd", s);
#define MHC_WIDE_FWD(TX_, TO_)                                                                                      \
    MHC_WIDE_N(n, if (split) {                                                                                      \
        if (parts) {                                                                                                \
            MHC_LAUNCH_GGL((wide_fwd_part_kernel<TX_, N_>), ogrid, oblock, 0, s, (const TX_*)x, coef,          \
                               coef_stride, rms_out, B, Ci);                                                        \
        } else {                                                                                                    \
            MHC_LAUNCH_GGL((wide_fwd_rms_kernel<TX_, N_>), grid, block, 0, s, (const TX_*)x, coef, coef_stride,\
                               rms_out, B, Ci, eps);                                                                \
        }                                                                                                           \
        MHC_LAUNCH_GGL((wide_fwd_out_kernel<TX_, TO_, N_>), ogrid, oblock, 0, s, (const TX_*)x, w, coef,       \
                           coef_stride, (TO_*)out, (const float*)rms_out, S, B, Ci, eps);                          \
    } else {                                                                                                        \
        MHC_LAUNCH_GGL((wide_fwd_kernel<TX_, TO_, N_>), grid, block, 0, s, (const TX_*)x, w, coef, coef_stride, \
                           (TO_*)out, rms_out, B, Ci, eps);                                                         \
    })
    if (x_dtype == kBF16) {
        if (out_dtype == kBF16) { MHC_WIDE_FWD(bf16_t, bf16_t); } else { MHC_WIDE_FWD(bf16_t, float); }
    } else {
        if (out_dtype == kBF16) { MHC_WIDE_FWD(float, bf16_t); } else { MHC_WIDE_FWD(float, float); }
    }
#undef MHC_WIDE_FWD
    timing_end(tok, s);
    return hipGetLastError();
}

template <typename TX, int N, int MODE>
static const void* wide_bwd_fn() {
    return reinterpret_cast<const void*>(&wide_bwd_kernel<TX, N, MODE, (N <= 8)>);
}

// Channel chunks of the backward: one chunk of kWideThreads channels per
// workgroup (one channel per lane) when there are fewer tokens than two
// workgroups per CU, used only when a token splits into at least two chunks
// (then the partial rows are one per token).
static int wide_bwd_chunks(int64_t B, int64_t C) {
    if (B >= 2 * (int64_t)device_cu_count()) return 1;
    const int64_t S = (C + kWideThreads - 1) / kWideThreads;
    return (int)(S < 1 ? 1 : S);
}

size_t wide_bwd_scratch_bytes(int n, int64_t B, int64_t C) {
    if (!wide_supported(n, C) || B <= 0) return 0;
    const int S = wide_bwd_chunks(B, C);
    if (S < 2) return 0;
    const int nr = 2 + 3 * n + (n <= 8 ? n * n : 0);
    return (size_t)B * S * nr * sizeof(float);
}

int wide_bwd_grid(int x_dtype, int n, int64_t B, int64_t C) {
    if (!wide_supported(n, C) || B <= 0) return 1;
    if (wide_bwd_chunks(B, C) >= 2) return (int)B;
    const void* fn = nullptr;
    auto pick = [&]() -> hipError_t {
        if (x_dtype == kBF16) {
            MHC_WIDE_N(n, fn = wide_bwd_fn<bf16_t, N_, 0>());
        } else {
            MHC_WIDE_N(n, fn = wide_bwd_fn<float, N_, 0>());
        }
        return hipSuccess;
    };
    if (pick() != hipSuccess || !fn) return 1;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kWideThreads, (size_t)C * sizeof(float)) !=
            hipSuccess ||
        per_cu < 1) {
        (void)hipGetLastError();
        per_cu = 1;
    }
    int64_t grid = (int64_t)device_cu_count() * per_cu;
    if (grid > B) grid = B;
    return (int)(grid < 1 ? 1 : grid);
}

hipError_t launch_wide_bwd(int x_dtype, int n, int mode, const float* g, const void* x, const float* w,
                           const float* coef, int64_t coef_stride, void* dx, float* dw_part, float* scal_out, int grid,
                           int64_t B, int64_t C, float eps, float* scratch, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!wide_supported(n, C) || grid < 1 || (mode != 0 && mode != 1)) return hipErrorInvalidValue;
    const int Ci = (int)C;
    const int S = wide_bwd_chunks(B, C);
    const int tok = timing_begin(mode == 0 ? "layer_bwd" : "layer_bwd_reduce", s);
    if (S >= 2) {
        // chunked: the partial rows are one per token
        if (!scratch || grid != B) return hipErrorInvalidValue;
        const int chunk = (int)((C + S - 1) / S);
        const dim3 cgrid((unsigned)(B * S));
#define MHC_WIDE_BWD2(TX_, M_)                                                                                     \
    MHC_WIDE_N(n, {                                                                                                 \
        MHC_LAUNCH_GGL((wide_bwd_sums_kernel<TX_, N_, (N_ <= 8)>), cgrid, dim3(kWideThreads), 0, s, g,          \
                           (const TX_*)x, w, coef, coef_stride, scratch, B, Ci, S, chunk);                          \
        MHC_LAUNCH_GGL((wide_bwd_out_kernel<TX_, N_, M_, (N_ <= 8)>), cgrid, dim3(kWideThreads), 0, s, g,       \
                           (const TX_*)x, w, coef, coef_stride, (TX_*)dx, dw_part, scal_out, scratch, B, Ci, eps,  \
                           S, chunk);                                                                               \
    })
        if (x_dtype == kBF16) {
            if (mode == 0) { MHC_WIDE_BWD2(bf16_t, 0); } else { MHC_WIDE_BWD2(bf16_t, 1); }
        } else {
            if (mode == 0) { MHC_WIDE_BWD2(float, 0); } else { MHC_WIDE_BWD2(float, 1); }
        }
#undef MHC_WIDE_BWD2
    } else {
        const size_t lds = (size_t)C * sizeof(float);
#define MHC_WIDE_BWD(TX_, M_)                                                                                      \
    MHC_WIDE_N(n, MHC_LAUNCH_GGL((wide_bwd_kernel<TX_, N_, M_, (N_ <= 8)>), dim3(grid), dim3(kWideThreads), lds, \
                                     s, g, (const TX_*)x, w, coef, coef_stride, (TX_*)dx, dw_part, scal_out, B, Ci,  \
                                     eps))
        if (x_dtype == kBF16) {
            if (mode == 0) { MHC_WIDE_BWD(bf16_t, 0); } else { MHC_WIDE_BWD(bf16_t, 1); }
        } else {
            if (mode == 0) { MHC_WIDE_BWD(float, 0); } else { MHC_WIDE_BWD(float, 1); }
        }
#undef MHC_WIDE_BWD
    }
    hipError_t e = hipGetLastError();
    timing_end(tok, s);
    if (e != hipSuccess || n <= 8) return e;
    // dM for n >= 16: same grid in MODE 0 (its rows of scal_out), one
    // workgroup per token in MODE 1
    const dim3 ggrid(mode == 0 ? (unsigned)grid : (unsigned)(B < 65536 ? B : 65536));
    const bool vec = C % 8 == 0 && ((uintptr_t)g % 16) == 0 && ((uintptr_t)x % 16) == 0;
#define MHC_GRAM(TX_, M_)                                                                                         \
    if (n == 16) {                                                                                                \
        if (vec) {                                                                                                \
            MHC_LAUNCH_GGL((stream_gram_kernel<TX_, 16, M_, true>), ggrid, dim3(kWideThreads), 0, s, g,       \
                               (const TX_*)x, scal_out, B, Ci, (int64_t)(16 * 16 + 2 * 16 + 2));                 \
        } else {                                                                                                  \
            MHC_LAUNCH_GGL((stream_gram_kernel<TX_, 16, M_, false>), ggrid, dim3(kWideThreads), 0, s, g,      \
                               (const TX_*)x, scal_out, B, Ci, (int64_t)(16 * 16 + 2 * 16 + 2));                 \
        }                                                                                                         \
    } else {                                                                                                      \
        if (vec) {                                                                                                \
            MHC_LAUNCH_GGL((stream_gram_kernel<TX_, 32, M_, true>), ggrid, dim3(kWideThreads), 0, s, g,       \
                               (const TX_*)x, scal_out, B, Ci, (int64_t)(32 * 32 + 2 * 32 + 2));                 \
        } else {                                                                                                  \
            MHC_LAUNCH_GGL((stream_gram_kernel<TX_, 32, M_, false>), ggrid, dim3(kWideThreads), 0, s, g,      \
                               (const TX_*)x, scal_out, B, Ci, (int64_t)(32 * 32 + 2 * 32 + 2));                 \
        }                                                                                                         \
    }
    const int tg = timing_begin("stream_gram", s);
    if (x_dtype == kBF16) {
        if (mode == 0) { MHC_GRAM(bf16_t, 0); } else { MHC_GRAM(bf16_t, 1); }
    } else {
        if (mode == 0) { MHC_GRAM(float, 0); } else { MHC_GRAM(float, 1); }
    }
#undef MHC_GRAM
    timing_end(tg, s);
    return hipGetLastError();
}

#define MHC_WIDE_OPS_N(n, ...)                                    \
    switch (n) {                                                  \
        case 1: { constexpr int N_ = 1; __VA_ARGS__; break; }     \
        case 2: { constexpr int N_ = 2; __VA_ARGS__; break; }     \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }     \
        case 8: { constexpr int N_ = 8; __VA_ARGS__; break; }     \
        case 16: { constexpr int N_ = 16; __VA_ARGS__; break; }   \
        case 32: { constexpr int N_ = 32; __VA_ARGS__; break; }   \
        default: return hipErrorInvalidValue;                     \
    }
#define MHC_WIDE_T(dt, ...)                                       \
    if (dt == kBF16) {                                            \
        using T_ = bf16_t;                                        \
        __VA_ARGS__;                                              \
    } else {                                                      \
        using T_ = float;                                         \
        __VA_ARGS__;                                              \
    }

static bool grid_ok(int64_t B) { return B > 0 && B <= 0x7fffffff; }

hipError_t launch_wide_rmsnorm_fwd(int dt, const void* x, const float* w, void* y, float* rms, int64_t B, int64_t C,
                                   float eps, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!grid_ok(B) || C < 1 || C > 0x7fffffff) return hipErrorInvalidValue;
    MHC_WIDE_T(dt, MHC_LAUNCH_GGL((wide_rmsnorm_fwd_kernel<T_>), dim3((unsigned)B), dim3(kWideThreads), 0, s,
                                      (const T_*)x, w, (T_*)y, rms, (int)C, eps));
    return hipGetLastError();
}

int wide_rmsnorm_bwd_grid(int dt, int64_t B, int64_t C) {
    if (B <= 0 || C < 1 || C > kWideMaxC) return 1;
    const void* fn = dt == kBF16 ? reinterpret_cast<const void*>(&wide_rmsnorm_bwd_kernel<bf16_t>)
                                 : reinterpret_cast<const void*>(&wide_rmsnorm_bwd_kernel<float>);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kWideThreads, (size_t)C * sizeof(float)) !=
            hipSuccess ||
        per_cu < 1) {
        (void)hipGetLastError();
        per_cu = 1;
    }
    int64_t grid = (int64_t)device_cu_count() * per_cu;
    if (grid > B) grid = B;
    return (int)(grid < 1 ? 1 : grid);
}

hipError_t launch_wide_rmsnorm_bwd(int dt, const void* g, const void* x, const float* w, const float* rms, void* gx,
                                   float* dw_part, int grid, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (grid < 1 || C < 1 || C > kWideMaxC) return hipErrorInvalidValue;
    MHC_WIDE_T(dt, MHC_LAUNCH_GGL((wide_rmsnorm_bwd_kernel<T_>), dim3(grid), dim3(kWideThreads),
                                      (size_t)C * sizeof(float), s, (const T_*)g, (const T_*)x, w, rms, (T_*)gx,
                                      dw_part, B, (int)C));
    return hipGetLastError();
}

hipError_t launch_wide_compute_rms(int dt, const void* x, float* rms, int64_t B, int64_t K, float eps,
                                   hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!grid_ok(B) || K < 1) return hipErrorInvalidValue;
    MHC_WIDE_T(dt, MHC_LAUNCH_GGL((wide_compute_rms_kernel<T_>), dim3((unsigned)B), dim3(kWideThreads), 0, s,
                                      (const T_*)x, rms, K, eps));
    return hipGetLastError();
}

hipError_t launch_wide_aggregate_fwd(int dt, int n, const void* x, const float* H, int64_t hs, void* out,
                                     float* h_act, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!grid_ok(B) || C < 1 || C > 0x7fffffff) return hipErrorInvalidValue;
    MHC_WIDE_T(dt, MHC_WIDE_OPS_N(n, MHC_LAUNCH_GGL((wide_aggregate_fwd_kernel<T_, N_>), dim3((unsigned)B),
                                                        dim3(kWideThreads), 0, s, (const T_*)x, H, hs, (T_*)out,
                                                        h_act, (int)C)));
    return hipGetLastError();
}

hipError_t launch_wide_aggregate_bwd(int dt, int n, const void* g, const void* x, const float* h_act, int64_t hs,
                                     void* gx, float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!grid_ok(B) || C < 1 || C > 0x7fffffff) return hipErrorInvalidValue;
    MHC_WIDE_T(dt, MHC_WIDE_OPS_N(n, MHC_LAUNCH_GGL((wide_aggregate_bwd_kernel<T_, N_>), dim3((unsigned)B),
                                                        dim3(kWideThreads), 0, s, (const T_*)g, (const T_*)x, h_act,
                                                        hs, (T_*)gx, gh_act, gh_raw, (int)C)));
    return hipGetLastError();
}

hipError_t launch_wide_distribute_fwd(int dt, int n, const void* y, const float* H, int64_t hs, const float* M,
                                      int64_t ms, const void* x, float* out, float* h_act, int64_t B, int64_t C,
                                      hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!grid_ok(B) || C < 1 || C > 0x7fffffff) return hipErrorInvalidValue;
    MHC_WIDE_T(dt, MHC_WIDE_OPS_N(n, MHC_LAUNCH_GGL((wide_distribute_fwd_kernel<T_, N_>), dim3((unsigned)B),
                                                        dim3(kWideThreads), 0, s, (const T_*)y, H, hs, M, ms,
                                                        (const T_*)x, out, h_act, (int)C)));
    return hipGetLastError();
}

hipError_t launch_wide_distribute_bwd(int dt, int n, const float* g, const void* x, const void* y, const float* M,
                                      int64_t ms, const float* h_act, int64_t hs, void* gx, void* gy, float* gM,
                                      float* gh_act, float* gh_raw, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!grid_ok(B) || C < 1 || C > 0x7fffffff) return hipErrorInvalidValue;
    MHC_WIDE_T(dt, MHC_WIDE_OPS_N(n, MHC_LAUNCH_GGL((wide_distribute_bwd_kernel<T_, N_, (N_ <= 8)>),
                                                        dim3((unsigned)B), dim3(kWideThreads), 0, s, g,
                                                        (const T_*)x, (const T_*)y, M, ms, h_act, hs, (T_*)gx,
                                                        (T_*)gy, gM, gh_act, gh_raw, (int)C)));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || n <= 8) return e;
    const dim3 ggrid((unsigned)(B < 65536 ? B : 65536));
    const bool vec = C % 8 == 0 && ((uintptr_t)g % 16) == 0 && ((uintptr_t)x % 16) == 0;
    MHC_WIDE_T(dt, if (n == 16) {
        if (vec) {
            MHC_LAUNCH_GGL((stream_gram_kernel<T_, 16, 1, true>), ggrid, dim3(kWideThreads), 0, s, g,
                               (const T_*)x, gM, B, (int)C, (int64_t)(16 * 16));
        } else {
            MHC_LAUNCH_GGL((stream_gram_kernel<T_, 16, 1, false>), ggrid, dim3(kWideThreads), 0, s, g,
                               (const T_*)x, gM, B, (int)C, (int64_t)(16 * 16));
        }
    } else {
        if (vec) {
            MHC_LAUNCH_GGL((stream_gram_kernel<T_, 32, 1, true>), ggrid, dim3(kWideThreads), 0, s, g,
                               (const T_*)x, gM, B, (int)C, (int64_t)(32 * 32));
        } else {
            MHC_LAUNCH_GGL((stream_gram_kernel<T_, 32, 1, false>), ggrid, dim3(kWideThreads), 0, s, g,
                               (const T_*)x, gM, B, (int)C, (int64_t)(32 * 32));
        }
    });
    return hipGetLastError();
}

hipError_t launch_wide_static_finalize(int n, const float* scal_part, int rows, const float* h_pre,
                                       const float* h_post, const float* h_res, float* d_h_pre, float* d_h_post,
                                       float* d_h_res, int iters, float sk_eps, float* hist, size_t hist_bytes,
                                       hipStream_t s) {
    // the history when it fits, else the recomputing adjoint
    if ((size_t)(iters > 0 ? iters : 0) * (n + 1) * n * sizeof(float) > hist_bytes) hist = nullptr;
    if (n == 16) {
        MHC_LAUNCH_GGL((wide_static_finalize_kernel<16>), dim3(1), dim3(kStaticFinalizeThreads), 0, s, scal_part, rows, h_pre, h_post,
                           h_res, d_h_pre, d_h_post, d_h_res, iters, sk_eps, hist);
    } else if (n == 32) {
        MHC_LAUNCH_GGL((wide_static_finalize_kernel<32>), dim3(1), dim3(kStaticFinalizeThreads), 0, s, scal_part, rows, h_pre, h_post,
                           h_res, d_h_pre, d_h_post, d_h_res, iters, sk_eps, hist);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mhc

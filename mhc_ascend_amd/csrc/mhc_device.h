// Device-side building blocks shared by the mHC kernels (gfx950, wave64).
//
//  * 16-byte vector loads/stores of fp32 (4 lanes of data) and bf16 (8).
//  * bf16 <-> fp32 conversion (round-to-nearest-even on the way down).
//  * Wave and block sum reductions of several values at once.
//  * Sigmoid and the register-resident Sinkhorn-Knopp forward/backward on
//    small n x n matrices, one matrix per group of G = pow2ceil(n) lanes,
//    one matrix row per lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {

typedef uint16_t bf16_t;

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16; NaN stays a quiet NaN.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<bf16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
}

// ---------------------------------------------------------------------------
// Element I/O.  VecIO<T>::W elements make one 16-byte access.
// ---------------------------------------------------------------------------
template <typename T> struct VecIO;

template <> struct VecIO<float> {
    static constexpr int W = 4;
    __device__ __forceinline__ static void load(const float* p, float (&v)[4]) {
        float4 q = *reinterpret_cast<const float4*>(p);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
    __device__ __forceinline__ static void store(float* p, const float (&v)[4]) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __device__ __forceinline__ static float scalar(const float* p) { return *p; }
    __device__ __forceinline__ static void put(float* p, float v) { *p = v; }
};

template <> struct VecIO<bf16_t> {
    static constexpr int W = 8;
    __device__ __forceinline__ static void load(const bf16_t* p, float (&v)[8]) {
        uint4 q = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    __device__ __forceinline__ static void store(bf16_t* p, const float (&v)[8]) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = static_cast<uint32_t>(f32_to_bf16(v[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(v[2 * i + 1])) << 16);
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    __device__ __forceinline__ static float scalar(const bf16_t* p) { return bf16_to_f32(*p); }
    __device__ __forceinline__ static void put(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

// Load/store W_OUT-wide runs of element type T from/to a float array by
// splitting into 16-byte pieces (W_OUT must be a multiple of VecIO<T>::W,
// or VecIO<T>::W a multiple of W_OUT with a scalar fallback).
template <typename T, int WN>
__device__ __forceinline__ void load_run(const T* p, float (&v)[WN]) {
    constexpr int W = VecIO<T>::W;
    if constexpr (WN % W == 0) {
#pragma unroll
        for (int s = 0; s < WN / W; ++s) {
            float t[W];
            VecIO<T>::load(p + s * W, t);
#pragma unroll
            for (int e = 0; e < W; ++e) v[s * W + e] = t[e];
        }
    } else if constexpr (WN == 4 && W == 8) {
        uint2 q = *reinterpret_cast<const uint2*>(p);
        v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
        v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
    } else {
#pragma unroll
        for (int e = 0; e < WN; ++e) v[e] = VecIO<T>::scalar(p + e);
    }
}

template <typename T, int WN>
__device__ __forceinline__ void store_run(T* p, const float (&v)[WN]) {
    constexpr int W = VecIO<T>::W;
    if constexpr (WN % W == 0) {
#pragma unroll
        for (int s = 0; s < WN / W; ++s) {
            float t[W];
#pragma unroll
            for (int e = 0; e < W; ++e) t[e] = v[s * W + e];
            VecIO<T>::store(p + s * W, t);
        }
    } else if constexpr (WN == 4 && W == 8) {
        uint2 q;
        q.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
        q.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
        *reinterpret_cast<uint2*>(p) = q;
    } else {
#pragma unroll
        for (int e = 0; e < WN; ++e) VecIO<T>::put(p + e, v[e]);
    }
}

// ---------------------------------------------------------------------------
// Reductions
// ---------------------------------------------------------------------------
template <int NV>
__device__ __forceinline__ void wave_sum(float (&v)[NV]) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] += __shfl_xor(v[i], off, kWave);
    }
}

// Sum NV values over the whole block; every thread receives the totals.
// `lds` must hold NV * (blockDim.x / 64) floats.  Contains two barriers, so
// back-to-back calls may reuse the same `lds`.
template <int NV>
__device__ __forceinline__ void block_sum(float (&v)[NV], float* lds) {
    wave_sum<NV>(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < NV; ++i) lds[wave * NV + i] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float s = 0.f;
        for (int w = 0; w < nwaves; ++w) s += lds[w * NV + i];
        v[i] = s;
    }
    __syncthreads();
}

// Sum over the aligned group of G lanes containing this lane (G a power of
// two dividing 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

constexpr int pow2ceil(int n) { return n <= 1 ? 1 : 2 * pow2ceil((n + 1) / 2); }

// ---------------------------------------------------------------------------
// Sinkhorn-Knopp on an N x N matrix held one row per lane in a group of
// G = pow2ceil(N) lanes (lanes r >= N hold zero rows and stay zero).
// Forward (ops_pytorch_backward.py:9-33): T times, A = X/(rowsum+eps),
// Y = A/(colsum+eps).  All divisions are IEEE.
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void sk_row_step(float (&a)[N], float eps, float& rs) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < N; ++c) s += a[c];
    rs = s + eps;
#pragma unroll
    for (int c = 0; c < N; ++c) a[c] = a[c] / rs;
}

template <int N>
__device__ __forceinline__ void sk_col_step(float (&a)[N], float eps) {
    constexpr int G = pow2ceil(N);
#pragma unroll
    for (int c = 0; c < N; ++c) {
        const float cs = group_sum<G>(a[c]) + eps;
        a[c] = a[c] / cs;
    }
}

template <int N>
__device__ __forceinline__ void sk_forward(float (&a)[N], int iters, float eps) {
    for (int t = 0; t < iters; ++t) {
        float rs;
        sk_row_step<N>(a, eps, rs);
        sk_col_step<N>(a, eps);
    }
}

// Register budget for the per-iteration history of the backward pass.
template <int N> struct SkHist { static constexpr int TMAX = (N <= 4) ? 32 : (N <= 8 ? 12 : 0); };

// Exact adjoint of sk_forward (lane holds row r of grad_out in `g`, row r of
// the forward input in `x0`; on return `g` holds row r of grad_inp).
//   column step: dA[r][c] = (dY[r][c] - sum_r' dY[r'][c] Y[r'][c]) / cs[c]
//   row step:    dX[r][c] = (dA[r][c] - sum_c' dA[r][c'] A[r][c']) / rs[r]
// For iters <= TMAX the post-row-step rows A_t and row sums rs_t of every
// iteration stay in registers; otherwise each iteration's state is
// recomputed from x0 (O(iters^2) work, no history).
template <int N>
__device__ __forceinline__ void sk_adjoint_step(float (&g)[N], const float (&A)[N], float rs, float eps) {
    constexpr int G = pow2ceil(N);
    float dA[N];
#pragma unroll
    for (int c = 0; c < N; ++c) {
        const float cs = group_sum<G>(A[c]) + eps;
        const float y = A[c] / cs;
        const float dot = group_sum<G>(g[c] * y);
        dA[c] = (g[c] - dot) / cs;
    }
    float rdot = 0.f;
#pragma unroll
    for (int c = 0; c < N; ++c) rdot += dA[c] * A[c];
#pragma unroll
    for (int c = 0; c < N; ++c) g[c] = (dA[c] - rdot) / rs;
}

template <int N>
__device__ __forceinline__ void sk_backward(float (&g)[N], const float (&x0)[N], int iters, float eps) {
    constexpr int TMAX = SkHist<N>::TMAX;
    if (TMAX > 0 && iters <= TMAX) {
        float hA[TMAX > 0 ? TMAX : 1][N];
        float hrs[TMAX > 0 ? TMAX : 1];
        float a[N];
#pragma unroll
        for (int c = 0; c < N; ++c) a[c] = x0[c];
#pragma unroll
        for (int t = 0; t < TMAX; ++t) {
            if (t < iters) {
                sk_row_step<N>(a, eps, hrs[t]);
#pragma unroll
                for (int c = 0; c < N; ++c) hA[t][c] = a[c];
                sk_col_step<N>(a, eps);
            }
        }
#pragma unroll
        for (int t = TMAX - 1; t >= 0; --t) {
            if (t < iters) sk_adjoint_step<N>(g, hA[t], hrs[t], eps);
        }
    } else {
        for (int t = iters - 1; t >= 0; --t) {
            float a[N];
#pragma unroll
            for (int c = 0; c < N; ++c) a[c] = x0[c];
            float rs = 0.f;
            for (int s = 0; s <= t; ++s) {
                sk_row_step<N>(a, eps, rs);
                if (s < t) sk_col_step<N>(a, eps);
            }
            sk_adjoint_step<N>(g, a, rs, eps);
        }
    }
}

}  // namespace mhc

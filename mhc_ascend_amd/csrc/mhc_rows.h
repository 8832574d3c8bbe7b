// Row-kernel helpers shared by the fused layer kernels and the standalone
// stream/norm operators: a workgroup owns one token row at a time, each
// lane VPT chunks of WC channels (chunk q = k * blockDim.x + tid, channels
// q * WC ... q * WC + WC - 1) of each stream.
#pragma once

#include "mhc_device.h"
#include "mhc_internal.h"

namespace mhc {

// ---------------------------------------------------------------------------
// This thread's VPT chunks of WC channels of each of the N streams of one
// token row starting at `base` (stream stride C).
// NTL selects non-temporal loads.  All streaming rows use them: a plain-load
// forward is faster in isolation but slows the following backward more than
// it gains (whole fwd+bwd step measured at n=4, C=4096).
// ---------------------------------------------------------------------------
//
// Loads are split in two steps.  load_rows_raw issues the 16-byte loads into
// raw 32-bit words and converts nothing; unpack_rows turns the words into
// fp32.  Keeping the conversion out of the load (and out of its bounds-check
// branch) lets every load of a row - and of the next token's row in the
// prefetching kernels - be in flight together: a bf16 unpack next to its load
// makes the compiler wait for that one load before issuing the next.
// ---------------------------------------------------------------------------
template <typename T, int WC>
struct RawChunk {
    static_assert((WC * sizeof(T)) % 16 == 0 || WC * sizeof(T) == 8, "row chunks are 8 bytes or 16-byte pieces");
    static constexpr int kWords = WC * (int)sizeof(T) / 4;
};

template <typename T, int N, int VPT, int WC>
using RawRows = uint32_t[N][VPT][RawChunk<T, WC>::kWords];

template <typename T, int N, int VPT, int WC, bool NTL>
__device__ __forceinline__ void load_rows_raw(const T* __restrict__ base, int C, RawRows<T, N, VPT, WC>& r) {
    constexpr int W = RawChunk<T, WC>::kWords;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        // Chunks past the row end load channel 0 instead (always in bounds)
        // and are zeroed by unpack_rows: no branch around the load.
        int c0 = (k * blockDim.x + threadIdx.x) * WC;
        c0 = c0 < C ? c0 : 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const char* p = reinterpret_cast<const char*>(base + (int64_t)i * C + c0);
            if constexpr (W == 2) {
                const uint2 q = NTL ? ld8_nt(p) : *reinterpret_cast<const uint2*>(p);
                r[i][k][0] = q.x;
                r[i][k][1] = q.y;
            } else {
#pragma unroll
                for (int s = 0; s < W / 4; ++s) {
                    const uint4 q = NTL ? ld16_nt(p + 16 * s) : *reinterpret_cast<const uint4*>(p + 16 * s);
                    r[i][k][4 * s] = q.x;
                    r[i][k][4 * s + 1] = q.y;
                    r[i][k][4 * s + 2] = q.z;
                    r[i][k][4 * s + 3] = q.w;
                }
            }
        }
    }
}

// The same loads through a buffer resource over one token's N rows (N * C
// elements; a resource of 0 bytes for a token past the end reads zeros
// without touching memory).  No load sits behind a branch, so a prefetch of
// the next token can be issued unconditionally and the compiler's wait
// counts stay exact (a conditional prefetch made it wait for every
// outstanding load, the prefetch included, before using the current row).
template <typename T, int N, int VPT, int WC, bool NTL>
__device__ __forceinline__ void load_rows_raw_rs(buf_rsrc_t rs, int C, RawRows<T, N, VPT, WC>& r) {
    constexpr int W = RawChunk<T, WC>::kWords;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        int c0 = (k * blockDim.x + threadIdx.x) * WC;
        c0 = c0 < C ? c0 : 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const uint32_t off = (uint32_t)(((int64_t)i * C + c0) * (int64_t)sizeof(T));
            if constexpr (W == 2) {
                const uint2 q = buf_ld8<NTL>(rs, off, 0u);
                r[i][k][0] = q.x;
                r[i][k][1] = q.y;
            } else {
#pragma unroll
                for (int s = 0; s < W / 4; ++s) {
                    const uint4 q = buf_ld16<NTL>(rs, off + 16 * s, 0u);
                    r[i][k][4 * s] = q.x;
                    r[i][k][4 * s + 1] = q.y;
                    r[i][k][4 * s + 2] = q.z;
                    r[i][k][4 * s + 3] = q.w;
                }
            }
        }
    }
}

// Resource over token b's N rows of C elements of a [B, N, C] array (0 bytes
// for b >= B); the rows are under 2 GiB (the register rows hold them).
template <typename T>
__device__ __forceinline__ buf_rsrc_t token_rows_rsrc(const T* base, int64_t b, int64_t B, int N, int C) {
    const int64_t bb = b < B ? b : 0;
    return make_buf_rsrc(base + bb * (int64_t)N * C, b < B ? (uint32_t)((int64_t)N * C * (int64_t)sizeof(T)) : 0u);
}

template <typename T, int N, int VPT, int WC>
__device__ __forceinline__ void unpack_rows(const RawRows<T, N, VPT, WC>& r, int C, float (&v)[N][VPT][WC]) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const bool ok = (int)((k * blockDim.x + threadIdx.x) * WC) < C;
#pragma unroll
        for (int i = 0; i < N; ++i) {
#pragma unroll
            for (int e = 0; e < WC; ++e) {
                float f;
                if constexpr (sizeof(T) == 4) {
                    f = __uint_as_float(r[i][k][e]);
                } else {
                    const uint32_t w = r[i][k][e >> 1];
                    f = __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
                }
                v[i][k][e] = ok ? f : 0.f;
            }
        }
    }
}

// Both steps at once, for rows used right away.  Call sites that load several
// arrays issue all load_rows_raw first and unpack afterwards.
template <typename T, int N, int VPT, int WC, bool NTL>
__device__ __forceinline__ void load_rows(const T* __restrict__ base, int C, float (&v)[N][VPT][WC]) {
    RawRows<T, N, VPT, WC> r;
    load_rows_raw<T, N, VPT, WC, NTL>(base, C, r);
    unpack_rows<T, N, VPT, WC>(r, C, v);
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

// Row state budget shared with choose_row_tiling(): n_arrays * VPT * W <= 136
// floats per thread (128 plus the one row of the distribute backward's
// y at n = 8 in bf16: 2n + 1 = 17 rows of 8 channels).
template <typename TX>
constexpr bool row_fits(int n_arrays, int vpt) {
    return n_arrays * vpt * VecIO<TX>::W <= kRowStateBudget;
}

// Channels per lane chunk in the fused layer kernels, for both storage
// dtypes.  They mix fp32 arrays (cotangent, output) with the x storage type;
// four channels make every fp32 access a contiguous 16-byte piece per lane
// and every bf16 access an 8-byte one, so each wave instruction covers one
// contiguous span.  (Eight bf16 channels per lane would split each fp32
// access into two 16-byte pieces at a 32-byte lane stride.)
constexpr int kLayerWC = 4;

constexpr bool layer_row_fits(int n_arrays, int vpt) { return n_arrays * vpt * kLayerWC <= kRowStateBudget; }

}  // namespace mhc

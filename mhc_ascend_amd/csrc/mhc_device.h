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

// fp32 -> bf16, round to nearest even, NaN stays a quiet NaN: gfx950's
// v_cvt_pk_bf16_f32 (bit-identical to the rounding-bias formulation
// u + 0x7fff + ((u >> 16) & 1) for every non-NaN input; checked on the GPU
// over 4M inputs including ties, denormals, overflow and infinities).
typedef __bf16 hw_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float hw_f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// Two fp32 -> two bf16 in one word (lo in bits 0-15): one instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(hw_f32x2_t{lo, hi}, hw_bf16x2_t));
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
        for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    __device__ __forceinline__ static float scalar(const bf16_t* p) { return bf16_to_f32(*p); }
    __device__ __forceinline__ static void put(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

// Non-temporal 16- and 8-byte accesses (the `nt` bit: streaming data that
// will not be re-read soon).  Each is one vector access: per-component
// non-temporal stores get merged into a wide store without the bit.
typedef unsigned int nt_u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int nt_u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld16_nt(const void* p) {
    const nt_u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4_t*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
    __builtin_nontemporal_store(nt_u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_u32x4_t*>(p));
}

// Raw buffer loads: a scalar resource over [base, base + bytes) plus a 32-bit
// per-lane offset and a wave-uniform scalar offset, so a load needs no 64-bit
// address arithmetic in vector registers.  A load whose per-lane offset is at
// or past `bytes` returns zeros (the hardware range check), which masks rows
// past the end of a block without a branch.  Word 3 = 0x00020000 is the raw
// (untyped, 32-bit data format) descriptor of the gfx9 family.
typedef __amdgpu_buffer_rsrc_t buf_rsrc_t;

__device__ __forceinline__ buf_rsrc_t make_buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// cache-policy operand: 2 = nt (streaming), 0 = default.  PIN sets the
// compiler-only volatile bit (bit 31): the load stays where it is written, so
// a prefetch is not sunk towards its use (the hardware still runs it
// asynchronously; the wait comes only at the first use).
template <bool NT, bool PIN = false>
__device__ __forceinline__ uint4 buf_ld16(buf_rsrc_t r, uint32_t voff, uint32_t soff) {
    constexpr int aux = (NT ? 2 : 0) | (PIN ? (int)0x80000000u : 0);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, aux);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

template <bool NT>
__device__ __forceinline__ uint2 buf_ld8(buf_rsrc_t r, uint32_t voff, uint32_t soff) {
    constexpr int aux = NT ? 2 : 0;
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, aux);
    return make_uint2(v[0], v[1]);
}

template <bool PIN = false>
__device__ __forceinline__ uint32_t buf_ld4(buf_rsrc_t r, uint32_t voff, uint32_t soff) {
    constexpr int aux = PIN ? (int)0x80000000u : 0;
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, aux);
}

// Raw buffer store: a lane whose offset is at or past the resource's size
// stores nothing (the same range check), so partial tiles need no branch
// around the store.  NT sets the streaming cache policy.
template <bool NT>
__device__ __forceinline__ void buf_st16(buf_rsrc_t r, uint32_t voff, uint32_t soff, uint4 v) {
    constexpr int aux = NT ? 2 : 0;
    typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(u32x4v_t{v.x, v.y, v.z, v.w}, r, (int)voff, (int)soff, aux);
}

template <bool NT>
__device__ __forceinline__ void buf_st8(buf_rsrc_t r, uint32_t voff, uint32_t soff, uint2 v) {
    constexpr int aux = NT ? 2 : 0;
    typedef unsigned int u32x2v_t __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(u32x2v_t{v.x, v.y}, r, (int)voff, (int)soff, aux);
}

__device__ __forceinline__ void buf_st4(buf_rsrc_t r, uint32_t voff, uint32_t soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)voff, (int)soff, 0);
}

// A per-lane buffer offset that fails the range check of any resource under
// 2 GiB, also after adding a stage offset that keeps real offsets under
// 2 GiB (the sum stays below 2^32: no wrap into range).
constexpr uint32_t kBufOff = 0x80000000u;

__device__ __forceinline__ uint32_t wave_uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ uint2 ld8_nt(const void* p) {
    const nt_u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x2_t*>(p));
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ void st8_nt(void* p, uint2 v) {
    __builtin_nontemporal_store(nt_u32x2_t{v.x, v.y}, reinterpret_cast<nt_u32x2_t*>(p));
}

// Streaming (non-temporal) runs of WN elements: whole 16-byte pieces, or one
// 8-byte piece (four bf16).
template <typename T, int WN>
__device__ __forceinline__ void load_run_nt(const T* p, float (&v)[WN]) {
    constexpr int PER = 16 / sizeof(T);
    if constexpr (sizeof(T) == 2 && WN == 4) {
        const uint2 q = ld8_nt(p);
        v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
        v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
        return;
    }
    static_assert(WN % PER == 0 || (sizeof(T) == 2 && WN == 4), "non-temporal runs are 16-byte pieces");
#pragma unroll
    for (int s = 0; s < WN / PER; ++s) {
        const uint4 q = ld16_nt(p + s * PER);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[s * PER + e] = __uint_as_float(w[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[s * PER + 2 * e] = __uint_as_float(w[e] << 16);
                v[s * PER + 2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
            }
        }
    }
}

template <typename T, int WN>
__device__ __forceinline__ void store_run_nt(T* p, const float (&v)[WN]) {
    constexpr int PER = 16 / sizeof(T);
    if constexpr (sizeof(T) == 2 && WN == 4) {
        st8_nt(p, make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])));
        return;
    }
    static_assert(WN % PER == 0 || (sizeof(T) == 2 && WN == 4), "non-temporal runs are 16-byte pieces");
#pragma unroll
    for (int s = 0; s < WN / PER; ++s) {
        uint32_t w[4];
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(v[s * PER + e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(v[s * PER + 2 * e], v[s * PER + 2 * e + 1]);
        }
        st16_nt(p + s * PER, make_uint4(w[0], w[1], w[2], w[3]));
    }
}

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
        *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else {
#pragma unroll
        for (int e = 0; e < WN; ++e) VecIO<T>::put(p + e, v[e]);
    }
}

// ---------------------------------------------------------------------------
// Reductions.  Cross-lane steps inside 16-lane rows use DPP (quad_perm,
// row_half_mirror, row_mirror); rows are combined with row_bcast15/31 (all
// GFX9-family DPP controls, available on gfx950).
// ---------------------------------------------------------------------------
namespace dpp {
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141; // lane i <- lane 7-i within 8
constexpr int kRowMirror = 0x140;     // lane i <- lane 15-i within 16
constexpr int kRowBcast15 = 0x142;    // lane 15 of row r -> row r+1
constexpr int kRowBcast31 = 0x143;    // lane 31 -> rows 2, 3
constexpr int kRowRor4 = 0x124;       // lane i <- lane (i - 4) mod 16 within 16
constexpr int kRowRor8 = 0x128;       // lane i <- lane (i - 8) mod 16 within 16

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
}  // namespace dpp

// v + v[lane ^ 16] and v + v[lane ^ 32] with the gfx950 lane-swap VALU ops
// instead of an LDS permute.  v_permlane16_swap(v, v) returns
// {rows (0, 0, 2, 2), rows (1, 1, 3, 3)} of v (a row is 16 lanes),
// v_permlane32_swap(v, v) returns {halves (0, 0), halves (1, 1)}, so the sum
// of the pair is the partner sum in every lane; the two operands are added
// in the same order in both lanes of a pair (IEEE addition commutes, so this
// is bit-identical to v + shuffle).  The whole pair must be active.
__device__ __forceinline__ float xor16_add(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xor32_add(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Sum over the aligned group of G lanes containing this lane (G a power of
// two dividing 64); every lane of the group receives the group total.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp::mov<dpp::kQuadXor1>(v);
    if constexpr (G >= 4) v += dpp::mov<dpp::kQuadXor2>(v);
    if constexpr (G >= 8) v += dpp::mov<dpp::kRowHalfMirror>(v);
    if constexpr (G >= 16) v += dpp::mov<dpp::kRowMirror>(v);
    if constexpr (G >= 32) v = xor16_add(v);
    if constexpr (G >= 64) v = xor32_add(v);
    return v;
}

// Wave total of NV values; valid in lane 63 only.
template <int NV>
__device__ __forceinline__ void wave_sum_last(float (&v)[NV]) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float x = v[i];
        x += dpp::mov<dpp::kQuadXor1>(x);
        x += dpp::mov<dpp::kQuadXor2>(x);
        x += dpp::mov<dpp::kRowHalfMirror>(x);
        x += dpp::mov<dpp::kRowMirror>(x);
        x += dpp::mov<dpp::kRowBcast15, 0xA>(x);
        x += dpp::mov<dpp::kRowBcast31, 0xC>(x);
        v[i] = x;
    }
}

// Wave total of NV values in every lane.
template <int NV>
__device__ __forceinline__ void wave_sum(float (&v)[NV]) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = group_sum<kWave>(v[i]);
}

// Sum NV values over the whole block; every thread receives the totals.
// `lds` must hold NV * (blockDim.x / 64) floats.  Contains two barriers, so
// back-to-back calls may reuse the same `lds`.
template <int NV>
__device__ __forceinline__ void block_sum(float (&v)[NV], float* lds) {
    wave_sum_last<NV>(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    if (lane == kWave - 1) {
#pragma unroll
        for (int i = 0; i < NV; ++i) lds[wave * NV + i] = v[i];
    }
    __syncthreads();
    // A wave's NV totals are read together (independent loads), so the second
    // level costs one LDS round trip per wave rather than one per value and
    // wave; the summation order (waves in order from 0) is unchanged.
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = 0.f;
    for (int w = 0; w < nwaves; ++w) {
        float t[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) t[i] = lds[w * NV + i];
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] += t[i];
    }
    __syncthreads();
}

// Maximum of a non-negative value over the aligned 32 lanes (half wave)
// containing this lane; every lane of the half receives it.  Row maxima by
// DPP, then rows (0, 1) and (2, 3) through v_permlane16_swap.  The whole
// wave must be active.
__device__ __forceinline__ float half_wave_max_nonneg(float x) {
    x = fmaxf(x, dpp::mov<dpp::kQuadXor1>(x));
    x = fmaxf(x, dpp::mov<dpp::kQuadXor2>(x));
    x = fmaxf(x, dpp::mov<dpp::kRowHalfMirror>(x));
    x = fmaxf(x, dpp::mov<dpp::kRowMirror>(x));
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// ---------------------------------------------------------------------------
// Half-precision transport of an fp32 row part between two kernels.
//
// Where a gradient is formed in two kernels (a row pass writes one part, a
// later kernel adds the rest and rounds the sum once to bf16), the first part
// travels through HBM in the 2 bytes per element the bf16 result occupies:
// as fp16 values of v * 2^-k, with one power-of-two scale 2^k per group.  k
// comes from the group's largest finite |value| m so that m * 2^-k lies in
// [2^14, 2^15) (k = 0 for m = 0).  Scaling by a power of two is exact (the
// ldexp on either side), and fp16 keeps 11 significant bits over its normal
// range, so every element of magnitude at least 2^-28 m comes back with a
// relative error of at most 2^-11 (one fp16 half-ulp, an eighth of the bf16
// half-ulp of the final rounding); smaller elements come back within 2^-39 m.
// NaN and +-Inf take no part in m and travel as fp16 NaN and +-Inf.  A group
// is one half wave's elements of a token row: every lane's 4-channel chunks
// (all streams, all chunks k) of lanes 32h .. 32h + 31, whose channels are
// the 128-channel ranges c / 128 = k * H + h (H = row-kernel lanes / 32), so
// the row kernel finds m with one half-wave reduction and a 128-column block
// of the row maps to one group.
// ---------------------------------------------------------------------------
constexpr int kPartGroup = 128;  // channels of one half wave's 4-channel chunks

typedef _Float16 part_h2_t __attribute__((ext_vector_type(2)));

// Scale exponent k of a group whose largest finite |value| is m >= 0.
__device__ __forceinline__ int part_scale_exp(float m) {
    return m > 0.f ? __builtin_amdgcn_frexp_expf(m) - 15 : 0;
}

// Four values -> four fp16 of v * 2^-k in 8 bytes (element 0 in the low half
// of .x), rounded to nearest even.
__device__ __forceinline__ uint2 part_pack4(const float (&v)[4], int k) {
    const part_h2_t a = {(_Float16)__builtin_ldexpf(v[0], -k), (_Float16)__builtin_ldexpf(v[1], -k)};
    const part_h2_t b = {(_Float16)__builtin_ldexpf(v[2], -k), (_Float16)__builtin_ldexpf(v[3], -k)};
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

__device__ __forceinline__ void part_unpack4(uint2 w, int k, float (&v)[4]) {
    const part_h2_t a = __builtin_bit_cast(part_h2_t, w.x);
    const part_h2_t b = __builtin_bit_cast(part_h2_t, w.y);
    v[0] = __builtin_ldexpf((float)a[0], k);
    v[1] = __builtin_ldexpf((float)a[1], k);
    v[2] = __builtin_ldexpf((float)b[0], k);
    v[3] = __builtin_ldexpf((float)b[1], k);
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

// Row o of the concatenated dynamic-H projection [pre; post; res] (ops.py:416-418):
// rows < n from `pre`, the next n from `post`, the rest from `res`; K = n * C.
__device__ __forceinline__ const float* phi_row(const float* pre, const float* post, const float* res, int n, int o,
                                                int64_t K) {
    if (o < n) return pre + (int64_t)o * K;
    if (o < 2 * n) return post + (int64_t)(o - n) * K;
    return res + (int64_t)(o - 2 * n) * K;
}

constexpr int pow2ceil(int n) { return n <= 1 ? 1 : 2 * pow2ceil((n + 1) / 2); }

// 1/d from the hardware reciprocal (v_rcp_f32, ~1 ulp) refined by one
// Newton-Raphson step r' = r + r (1 - d r).  Unlike IEEE division it does not
// serialise on VCC, so independent reciprocals overlap.
__device__ __forceinline__ float rcp_nr(float d) {
    const float r = __builtin_amdgcn_rcpf(d);
    const float e = fmaf(-d, r, 1.0f);
    return fmaf(r, e, r);
}

// ---------------------------------------------------------------------------
// Sinkhorn-Knopp on an N x N matrix held one row per lane in a group of
// G = pow2ceil(N) lanes.  Lanes with active == false (padding rows r >= N)
// hold zero rows, stay zero and contribute nothing to column sums.
// Forward (ops_pytorch_backward.py:9-33): T times, A = X/(rowsum+eps),
// Y = A/(colsum+eps); each row / column scale is one Newton-refined
// reciprocal applied by multiplication.
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void sk_row_step(float (&a)[N], float eps, bool active, float& rinv) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < N; ++c) s += a[c];
    rinv = active ? rcp_nr(s + eps) : 0.f;
#pragma unroll
    for (int c = 0; c < N; ++c) a[c] *= rinv;
}

template <int N>
__device__ __forceinline__ void sk_col_step(float (&a)[N], float eps) {
    constexpr int G = pow2ceil(N);
#pragma unroll
    for (int c = 0; c < N; ++c) a[c] *= rcp_nr(group_sum<G>(a[c]) + eps);
}

template <int N>
__device__ __forceinline__ void sk_forward(float (&a)[N], int iters, float eps, bool active) {
    for (int t = 0; t < iters; ++t) {
        float rinv;
        sk_row_step<N>(a, eps, active, rinv);
        sk_col_step<N>(a, eps);
    }
}

// Register budget for the per-iteration history of the backward pass.
template <int N> struct SkHist { static constexpr int TMAX = (N <= 4) ? 32 : (N <= 8 ? 12 : 0); };

// Exact adjoint of sk_forward (lane holds row r of grad_out in `g`, row r of
// the forward input in `x0`; on return `g` holds row r of grad_inp).  With
// A the post-row-step matrix of an iteration, cs its column sums + eps and
// rinv = 1/(rowsum + eps) of the row step:
//   column step: dA[r][c] = (dY[r][c] - sum_r' dY[r'][c] Y[r'][c]) / cs[c]
//   row step:    dX[r][c] = (dA[r][c] - sum_c' dA[r][c'] A[r][c']) * rinv[r]
// For iters <= TMAX the rows A_t and rinv_t of every iteration stay in
// registers; otherwise each iteration's state is recomputed from x0
// (O(iters^2) work, no history).
template <int N>
__device__ __forceinline__ void sk_adjoint_step(float (&g)[N], const float (&A)[N], float rinv, float eps) {
    constexpr int G = pow2ceil(N);
    float dA[N];
#pragma unroll
    for (int c = 0; c < N; ++c) {
        const float cinv = rcp_nr(group_sum<G>(A[c]) + eps);
        const float dot = group_sum<G>(g[c] * (A[c] * cinv));
        dA[c] = (g[c] - dot) * cinv;
    }
    float rdot = 0.f;
#pragma unroll
    for (int c = 0; c < N; ++c) rdot += dA[c] * A[c];
#pragma unroll
    for (int c = 0; c < N; ++c) g[c] = (dA[c] - rdot) * rinv;
}

template <int N>
__device__ __forceinline__ void sk_backward(float (&g)[N], const float (&x0)[N], int iters, float eps, bool active) {
    constexpr int TMAX = SkHist<N>::TMAX;
    if (TMAX > 0 && iters <= TMAX) {
        float hA[TMAX > 0 ? TMAX : 1][N];
        float hr[TMAX > 0 ? TMAX : 1];
        float a[N];
#pragma unroll
        for (int c = 0; c < N; ++c) a[c] = x0[c];
#pragma unroll
        for (int t = 0; t < TMAX; ++t) {
            if (t < iters) {
                sk_row_step<N>(a, eps, active, hr[t]);
#pragma unroll
                for (int c = 0; c < N; ++c) hA[t][c] = a[c];
                sk_col_step<N>(a, eps);
            }
        }
#pragma unroll
        for (int t = TMAX - 1; t >= 0; --t) {
            if (t < iters) sk_adjoint_step<N>(g, hA[t], hr[t], eps);
        }
    } else {
        for (int t = iters - 1; t >= 0; --t) {
            float a[N];
#pragma unroll
            for (int c = 0; c < N; ++c) a[c] = x0[c];
            float rinv = 0.f;
            for (int s = 0; s <= t; ++s) {
                sk_row_step<N>(a, eps, active, rinv);
                if (s < t) sk_col_step<N>(a, eps);
            }
            sk_adjoint_step<N>(g, a, rinv, eps);
        }
    }
}

// The same adjoint with the per-iteration state kept in memory instead of
// registers or recomputed: O(iters) steps for N too large for a register
// history.  Lane r of the matrix's group of G = pow2ceil(N) lanes stores
// column c of iteration t at hist[(t * (N + 1) + c) * G + r] and the row
// scale at c = N (iters * (N + 1) * G floats per matrix).  Each lane reads
// back only what it wrote, so program order is the only ordering needed.
template <int N>
__device__ __forceinline__ void sk_backward_mem(float (&g)[N], const float (&x0)[N], int iters, float eps,
                                                bool active, float* __restrict__ hist, int r) {
    constexpr int G = pow2ceil(N);
    float a[N];
#pragma unroll
    for (int c = 0; c < N; ++c) a[c] = x0[c];
    for (int t = 0; t < iters; ++t) {
        float rinv;
        sk_row_step<N>(a, eps, active, rinv);
        float* h = hist + (int64_t)t * (N + 1) * G + r;
#pragma unroll
        for (int c = 0; c < N; ++c) h[c * G] = a[c];
        h[N * G] = rinv;
        sk_col_step<N>(a, eps);
    }
    // iteration t - 1's state is loaded while iteration t's adjoint runs
    float A[N], ri = 0.f;
    if (iters > 0) {
        const float* h = hist + (int64_t)(iters - 1) * (N + 1) * G + r;
#pragma unroll
        for (int c = 0; c < N; ++c) A[c] = h[c * G];
        ri = h[N * G];
    }
    for (int t = iters - 1; t >= 0; --t) {
        float An[N], rn = 0.f;
#pragma unroll
        for (int c = 0; c < N; ++c) An[c] = 0.f;
        if (t > 0) {
            const float* h = hist + (int64_t)(t - 1) * (N + 1) * G + r;
#pragma unroll
            for (int c = 0; c < N; ++c) An[c] = h[c * G];
            rn = h[N * G];
        }
        sk_adjoint_step<N>(g, A, ri, eps);
#pragma unroll
        for (int c = 0; c < N; ++c) A[c] = An[c];
        ri = rn;
    }
}

// ---------------------------------------------------------------------------
// Sinkhorn-Knopp on an n x n matrix with n <= NM (NM = 16, 32 or 64) held one
// row per lane in a group of NM lanes, for n above the exact instantiations.
// Columns c >= n are padding: they hold zero, take no part in the column
// steps (with eps = 0 their scale would be 1/0) and their adjoint is zero.
// Same formulas as sk_forward / sk_adjoint_step; the backward recomputes each
// iteration's state from x0 (no history: a row is NM registers).
// ---------------------------------------------------------------------------
template <int NM>
__device__ __forceinline__ void skw_col_step(float (&a)[NM], int n, float eps) {
#pragma unroll
    for (int c = 0; c < NM; ++c) {
        if (c < n) a[c] *= rcp_nr(group_sum<NM>(a[c]) + eps);
    }
}

template <int NM>
__device__ __forceinline__ void skw_forward(float (&a)[NM], int n, int iters, float eps, bool active) {
    for (int t = 0; t < iters; ++t) {
        float rinv;
        sk_row_step<NM>(a, eps, active, rinv);
        skw_col_step<NM>(a, n, eps);
    }
}

template <int NM>
__device__ __forceinline__ void skw_adjoint_step(float (&g)[NM], const float (&A)[NM], int n, float rinv,
                                                 float eps) {
    float dA[NM];
#pragma unroll
    for (int c = 0; c < NM; ++c) {
        dA[c] = 0.f;
        if (c < n) {
            const float cinv = rcp_nr(group_sum<NM>(A[c]) + eps);
            const float dot = group_sum<NM>(g[c] * (A[c] * cinv));
            dA[c] = (g[c] - dot) * cinv;
        }
    }
    float rdot = 0.f;
#pragma unroll
    for (int c = 0; c < NM; ++c) rdot += dA[c] * A[c];
#pragma unroll
    for (int c = 0; c < NM; ++c) g[c] = c < n ? (dA[c] - rdot) * rinv : 0.f;
}

template <int NM>
__device__ __forceinline__ void skw_backward(float (&g)[NM], const float (&x0)[NM], int n, int iters, float eps,
                                             bool active) {
    for (int t = iters - 1; t >= 0; --t) {
        float a[NM];
#pragma unroll
        for (int c = 0; c < NM; ++c) a[c] = x0[c];
        float rinv = 0.f;
        for (int s = 0; s <= t; ++s) {
            sk_row_step<NM>(a, eps, active, rinv);
            if (s < t) skw_col_step<NM>(a, n, eps);
        }
        skw_adjoint_step<NM>(g, a, n, rinv, eps);
    }
}

// The same adjoint with each iteration's state kept in memory (O(iters)
// steps instead of O(iters^2)), as sk_backward_mem does: lane r of a group
// of ld lanes (ld >= NM; the lanes of one wave share a history when several
// groups run in it) stores column c < n of iteration t at
// hist[(t * (n + 1) + c) * ld + r] and the row scale at c = n
// (skw_hist_floats(ld, n, iters) floats); each lane reads back only what it
// wrote.  Same arithmetic as skw_backward, so the same results.
template <int NM>
__device__ __forceinline__ void skw_backward_mem(float (&g)[NM], const float (&x0)[NM], int n, int iters,
                                                 float eps, bool active, float* __restrict__ hist, int r, int ld) {
    float a[NM];
#pragma unroll
    for (int c = 0; c < NM; ++c) a[c] = x0[c];
    for (int t = 0; t < iters; ++t) {
        float rinv;
        sk_row_step<NM>(a, eps, active, rinv);
        float* h = hist + (int64_t)t * (n + 1) * ld + r;
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            if (c < n) h[(int64_t)c * ld] = a[c];
        }
        h[(int64_t)n * ld] = rinv;
        skw_col_step<NM>(a, n, eps);
    }
    // iteration t - 1's state is loaded while iteration t's adjoint runs;
    // the padding columns c >= n stay zero, as in the forward
    float A[NM], ri = 0.f;
#pragma unroll
    for (int c = 0; c < NM; ++c) A[c] = 0.f;
    if (iters > 0) {
        const float* h = hist + (int64_t)(iters - 1) * (n + 1) * ld + r;
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            if (c < n) A[c] = h[(int64_t)c * ld];
        }
        ri = h[(int64_t)n * ld];
    }
    for (int t = iters - 1; t >= 0; --t) {
        float An[NM], rn = 0.f;
#pragma unroll
        for (int c = 0; c < NM; ++c) An[c] = 0.f;
        if (t > 0) {
            const float* h = hist + (int64_t)(t - 1) * (n + 1) * ld + r;
#pragma unroll
            for (int c = 0; c < NM; ++c) {
                if (c < n) An[c] = h[(int64_t)c * ld];
            }
            rn = h[(int64_t)n * ld];
        }
        skw_adjoint_step<NM>(g, A, n, ri, eps);
#pragma unroll
        for (int c = 0; c < NM; ++c) A[c] = An[c];
        ri = rn;
    }
}

// floats of skw_backward_mem's history for one group of ld lanes
__host__ __device__ constexpr int64_t skw_hist_floats(int ld, int n, int iters) {
    return (int64_t)(iters > 0 ? iters : 0) * (n + 1) * ld;
}

// ---------------------------------------------------------------------------
// Sinkhorn-Knopp on a 4 x 4 matrix held one element per lane in a 16-lane DPP
// row (lane 4 r + c of the row holds element (r, c)): a row sum is a quad
// reduction, a column sum two rotations within the row, so an iteration is a
// few full-rate instructions (for one shared matrix such as the static H_res,
// where the latency of the chain is the cost).  The adjoint follows the same
// formulas as sk_adjoint_step, with the per-iteration post-row-step element
// and row scale kept in registers for iters <= kSk16Hist.
// ---------------------------------------------------------------------------
constexpr int kSk16Hist = 32;

__device__ __forceinline__ float sk16_row_sum(float v) { return group_sum<4>(v); }
__device__ __forceinline__ float sk16_col_sum(float v) {
    v += dpp::mov<dpp::kRowRor4>(v);
    v += dpp::mov<dpp::kRowRor8>(v);
    return v;
}

__device__ __forceinline__ void sk16_forward(float& a, int iters, float eps) {
    for (int t = 0; t < iters; ++t) {
        a *= rcp_nr(sk16_row_sum(a) + eps);
        a *= rcp_nr(sk16_col_sum(a) + eps);
    }
}

__device__ __forceinline__ void sk16_adjoint_step(float& g, float A, float ri, float eps) {
    const float ci = rcp_nr(sk16_col_sum(A) + eps);
    const float dot = sk16_col_sum(g * (A * ci));
    const float dA = (g - dot) * ci;
    const float rd = sk16_row_sum(dA * A);
    g = (dA - rd) * ri;
}

// g: element of dL/dM in, dL/dX out; x0: element of the forward input X.
__device__ __forceinline__ void sk16_backward(float& g, float x0, int iters, float eps) {
    if (iters <= kSk16Hist) {
        float hA[kSk16Hist], hr[kSk16Hist];
        float a = x0;
#pragma unroll
        for (int t = 0; t < kSk16Hist; ++t) {
            if (t < iters) {
                hr[t] = rcp_nr(sk16_row_sum(a) + eps);
                a *= hr[t];
                hA[t] = a;
                a *= rcp_nr(sk16_col_sum(a) + eps);
            }
        }
#pragma unroll
        for (int t = kSk16Hist - 1; t >= 0; --t) {
            if (t < iters) sk16_adjoint_step(g, hA[t], hr[t], eps);
        }
    } else {
        for (int t = iters - 1; t >= 0; --t) {
            float a = x0, ri = 0.f;
            for (int s = 0; s <= t; ++s) {
                ri = rcp_nr(sk16_row_sum(a) + eps);
                a *= ri;
                if (s < t) a *= rcp_nr(sk16_col_sum(a) + eps);
            }
            sk16_adjoint_step(g, a, ri, eps);
        }
    }
}


// ---------------------------------------------------------------------------
// Sinkhorn-Knopp on one 32 x 32 matrix spread over a 256-lane workgroup, for
// a matrix whose chain of iterations is the latency of a launch (the static
// H_res, or one token's matrix per workgroup).  Lane t holds row t / 8,
// columns 4 (t % 8) .. 4 (t % 8) + 3.  A row is 8 consecutive lanes (DPP
// sum); a column is lanes t, t ^ 8, t ^ 16, ... of each wave (row_ror:8 and
// the lane-swap ops), then the four waves' partials through LDS, added in
// wave order.  Every step is an xor butterfly, so all lanes of a row or
// column hold the same bits of its sum.  One barrier per iteration; the LDS
// partials alternate between two buffers, so a wave's next write never meets
// a slower wave's reads of the previous step.  Same formulas as sk_forward /
// sk_adjoint_step (ops_pytorch_backward.py:9-33, 36-72).
// ---------------------------------------------------------------------------
namespace skb {
constexpr int kThreads = 256;
constexpr int kN = 32;
constexpr int kV = 4;                 // columns per lane
constexpr int kLPR = kN / kV;         // lanes per row (8)
constexpr int kNW = kThreads / kWave; // waves (4)
constexpr int kTMax = 32;             // iterations the adjoint keeps in registers
constexpr int kPartFloats = 2 * kNW * kN;  // LDS column partials, double-buffered
constexpr int kHistFloats = kTMax * kN;    // LDS column scales of the adjoint

__device__ __forceinline__ int row() { return threadIdx.x / kLPR; }
__device__ __forceinline__ int col0() { return (threadIdx.x % kLPR) * kV; }

// In-wave sum over the 8 lanes holding the same columns.
__device__ __forceinline__ float col_wave_sum(float v) {
    v += dpp::mov<dpp::kRowRor8>(v);
    v = xor16_add(v);
    return xor32_add(v);
}

// Column totals of the lane's kV columns; `buf` is kNW * kN floats of LDS.
__device__ __forceinline__ void col_total(float (&v)[kV], float* buf) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    float p[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) p[k] = col_wave_sum(v[k]);
    if (lane < kLPR) *reinterpret_cast<float4*>(buf + wave * kN + lane * kV) = make_float4(p[0], p[1], p[2], p[3]);
    __syncthreads();
    float4 q[kNW];
#pragma unroll
    for (int w = 0; w < kNW; ++w) q[w] = *reinterpret_cast<const float4*>(buf + w * kN + col0());
    float t[kV] = {q[0].x, q[0].y, q[0].z, q[0].w};
#pragma unroll
    for (int w = 1; w < kNW; ++w) {
        t[0] += q[w].x;
        t[1] += q[w].y;
        t[2] += q[w].z;
        t[3] += q[w].w;
    }
#pragma unroll
    for (int k = 0; k < kV; ++k) v[k] = t[k];
}

__device__ __forceinline__ void row_scale(float (&a)[kV], float eps, float& rinv) {
    float s = ((a[0] + a[1]) + a[2]) + a[3];
    s = group_sum<kLPR>(s);
    rinv = rcp_nr(s + eps);
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] *= rinv;
}

__device__ __forceinline__ void col_scale(float (&a)[kV], float eps, float* buf, float (&cinv)[kV]) {
    float s[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) s[k] = a[k];
    col_total(s, buf);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        cinv[k] = rcp_nr(s[k] + eps);
        a[k] *= cinv[k];
    }
}

// a: the lane's four elements of X in, of SK(X) out.  part: kPartFloats of LDS.
__device__ __forceinline__ void forward(float (&a)[kV], int iters, float eps, float* part) {
    for (int t = 0; t < iters; ++t) {
        float ri, ci[kV];
        row_scale(a, eps, ri);
        col_scale(a, eps, part + (t & 1) * kNW * kN, ci);
    }
}

// g: the lane's elements of dL/dM in, dL/dX out; x0: elements of X.
// Requires iters <= kTMax.  part: kPartFloats, hc: kHistFloats of LDS.
__device__ __forceinline__ void backward(float (&g)[kV], const float (&x0)[kV], int iters, float eps, float* part,
                                         float* hc) {
    float hA[kTMax][kV], hr[kTMax];
    float a[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] = x0[k];
    const bool writer = threadIdx.x < kLPR;  // row 0 stores the column scales
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
        if (t < iters) {
            row_scale(a, eps, hr[t]);
#pragma unroll
            for (int k = 0; k < kV; ++k) hA[t][k] = a[k];
            float ci[kV];
            col_scale(a, eps, part + (t & 1) * kNW * kN, ci);
            if (writer) *reinterpret_cast<float4*>(hc + t * kN + col0()) = make_float4(ci[0], ci[1], ci[2], ci[3]);
        }
    }
    __syncthreads();
    // adjoint steps continue the buffer alternation: step t uses (t + 1) & 1
#pragma unroll
    for (int t = kTMax - 1; t >= 0; --t) {
        if (t < iters) {
            const float4 cv = *reinterpret_cast<const float4*>(hc + t * kN + col0());
            const float ci[kV] = {cv.x, cv.y, cv.z, cv.w};
            float d[kV];
#pragma unroll
            for (int k = 0; k < kV; ++k) d[k] = g[k] * (hA[t][k] * ci[k]);
            col_total(d, part + ((t + 1) & 1) * kNW * kN);
            float dA[kV];
#pragma unroll
            for (int k = 0; k < kV; ++k) dA[k] = (g[k] - d[k]) * ci[k];
            float rd = ((dA[0] * hA[t][0] + dA[1] * hA[t][1]) + dA[2] * hA[t][2]) + dA[3] * hA[t][3];
            rd = group_sum<kLPR>(rd);
#pragma unroll
            for (int k = 0; k < kV; ++k) g[k] = (dA[k] - rd) * hr[t];
        }
    }
}

// The same for an n x n matrix with n <= 32 zero-padded to 32 x 32: padded
// rows (r >= n) take a zero row scale and padded columns (c >= n) a zero
// column scale (no 1/0 with eps = 0), so they stay zero and the adjoint
// leaves the real entries as the unpadded one does; g comes back with
// don't-care values in the padded columns.
__device__ __forceinline__ void row_scale_n(float (&a)[kV], float eps, bool active, float& rinv) {
    float s = ((a[0] + a[1]) + a[2]) + a[3];
    s = group_sum<kLPR>(s);
    rinv = active ? rcp_nr(s + eps) : 0.f;
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] *= rinv;
}

__device__ __forceinline__ void col_scale_n(float (&a)[kV], int n, float eps, float* buf, float (&cinv)[kV]) {
    float s[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) s[k] = a[k];
    col_total(s, buf);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        cinv[k] = col0() + k < n ? rcp_nr(s[k] + eps) : 0.f;
        a[k] *= cinv[k];
    }
}

__device__ __forceinline__ void forward_n(float (&a)[kV], int n, int iters, float eps, float* part) {
    const bool active = row() < n;
    for (int t = 0; t < iters; ++t) {
        float ri, ci[kV];
        row_scale_n(a, eps, active, ri);
        col_scale_n(a, n, eps, part + (t & 1) * kNW * kN, ci);
    }
}

__device__ __forceinline__ void backward_n(float (&g)[kV], const float (&x0)[kV], int n, int iters, float eps,
                                           float* part, float* hc) {
    const bool active = row() < n;
    float hA[kTMax][kV], hr[kTMax];
    float a[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] = x0[k];
    const bool writer = threadIdx.x < kLPR;  // row 0 stores the column scales
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
        if (t < iters) {
            row_scale_n(a, eps, active, hr[t]);
#pragma unroll
            for (int k = 0; k < kV; ++k) hA[t][k] = a[k];
            float ci[kV];
            col_scale_n(a, n, eps, part + (t & 1) * kNW * kN, ci);
            if (writer) *reinterpret_cast<float4*>(hc + t * kN + col0()) = make_float4(ci[0], ci[1], ci[2], ci[3]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int t = kTMax - 1; t >= 0; --t) {
        if (t < iters) {
            const float4 cv = *reinterpret_cast<const float4*>(hc + t * kN + col0());
            const float ci[kV] = {cv.x, cv.y, cv.z, cv.w};
            float d[kV];
#pragma unroll
            for (int k = 0; k < kV; ++k) d[k] = g[k] * (hA[t][k] * ci[k]);
            col_total(d, part + ((t + 1) & 1) * kNW * kN);
            float dA[kV];
#pragma unroll
            for (int k = 0; k < kV; ++k) dA[k] = (g[k] - d[k]) * ci[k];
            float rd = ((dA[0] * hA[t][0] + dA[1] * hA[t][1]) + dA[2] * hA[t][2]) + dA[3] * hA[t][3];
            rd = group_sum<kLPR>(rd);
#pragma unroll
            for (int k = 0; k < kV; ++k) g[k] = (dA[k] - rd) * hr[t];
        }
    }
}
}  // namespace skb

// ---------------------------------------------------------------------------
// Sinkhorn-Knopp on one 16 x 16 matrix held by one wave (the static H_res at
// n = 16): lane t holds row t / 4, columns 4 (t % 4) .. 4 (t % 4) + 3.  A row
// is a quad (DPP); a column is lanes t, t +- 4, t +- 8 of each 16-lane row
// (row_ror 4 and 8, as sk16_col_sum) and the four rows (the lane-swap ops),
// so an iteration is a few dozen full-rate instructions with no barrier.
// Same formulas as sk_forward / sk_adjoint_step (ops_pytorch_backward.py:
// 9-33, 36-72); the adjoint keeps each iteration's state in registers
// (iters <= kTMax).  The whole wave must be active.
// ---------------------------------------------------------------------------
namespace skw16 {
constexpr int kN = 16;
constexpr int kV = 4;     // columns per lane
constexpr int kTMax = 32; // iterations the adjoint keeps in registers

__device__ __forceinline__ int row() { return (threadIdx.x & (kWave - 1)) >> 2; }
__device__ __forceinline__ int col0() { return (threadIdx.x & 3) * kV; }

__device__ __forceinline__ float col_sum(float v) {
    v += dpp::mov<dpp::kRowRor4>(v);
    v += dpp::mov<dpp::kRowRor8>(v);
    v = xor16_add(v);
    return xor32_add(v);
}

__device__ __forceinline__ void row_scale(float (&a)[kV], float eps, float& rinv) {
    float s = ((a[0] + a[1]) + a[2]) + a[3];
    s = group_sum<4>(s);
    rinv = rcp_nr(s + eps);
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] *= rinv;
}

__device__ __forceinline__ void col_scale(float (&a)[kV], float eps) {
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] *= rcp_nr(col_sum(a[k]) + eps);
}

// a: the lane's four elements of X in, of SK(X) out.
__device__ __forceinline__ void forward(float (&a)[kV], int iters, float eps) {
    for (int t = 0; t < iters; ++t) {
        float ri;
        row_scale(a, eps, ri);
        col_scale(a, eps);
    }
}

// g: the lane's elements of dL/dM in, dL/dX out; x0: elements of X.
// Requires iters <= kTMax.
__device__ __forceinline__ void backward(float (&g)[kV], const float (&x0)[kV], int iters, float eps) {
    float hA[kTMax][kV], hr[kTMax];
    float a[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] = x0[k];
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
        if (t < iters) {
            row_scale(a, eps, hr[t]);
#pragma unroll
            for (int k = 0; k < kV; ++k) hA[t][k] = a[k];
            col_scale(a, eps);
        }
    }
#pragma unroll
    for (int t = kTMax - 1; t >= 0; --t) {
        if (t < iters) {
            // column step, then the row step of iteration t
            float dA[kV];
#pragma unroll
            for (int k = 0; k < kV; ++k) {
                const float cinv = rcp_nr(col_sum(hA[t][k]) + eps);
                const float dot = col_sum(g[k] * (hA[t][k] * cinv));
                dA[k] = (g[k] - dot) * cinv;
            }
            float rdot = ((dA[0] * hA[t][0] + dA[1] * hA[t][1]) + dA[2] * hA[t][2]) + dA[3] * hA[t][3];
            rdot = group_sum<4>(rdot);
#pragma unroll
            for (int k = 0; k < kV; ++k) g[k] = (dA[k] - rdot) * hr[t];
        }
    }
}

// The same for an n x n matrix with n <= 16 zero-padded to 16 x 16 (rows
// r >= n and columns c >= n hold zeros): padded rows take a zero row scale
// and padded columns no column step (with eps = 0 their scale would be
// 1/0), as the skw_* functions treat their padding.
__device__ __forceinline__ void row_scale_n(float (&a)[kV], float eps, bool active, float& rinv) {
    float s = ((a[0] + a[1]) + a[2]) + a[3];
    s = group_sum<4>(s);
    rinv = active ? rcp_nr(s + eps) : 0.f;
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] *= rinv;
}

__device__ __forceinline__ void col_scale_n(float (&a)[kV], int n, float eps) {
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const float s = col_sum(a[k]);
        if (col0() + k < n) a[k] *= rcp_nr(s + eps);
    }
}

__device__ __forceinline__ void forward_n(float (&a)[kV], int n, int iters, float eps) {
    const bool active = row() < n;
    for (int t = 0; t < iters; ++t) {
        float ri;
        row_scale_n(a, eps, active, ri);
        col_scale_n(a, n, eps);
    }
}

__device__ __forceinline__ void backward_n(float (&g)[kV], const float (&x0)[kV], int n, int iters, float eps) {
    const bool active = row() < n;
    float hA[kTMax][kV], hr[kTMax];
    float a[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) a[k] = x0[k];
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
        if (t < iters) {
            row_scale_n(a, eps, active, hr[t]);
#pragma unroll
            for (int k = 0; k < kV; ++k) hA[t][k] = a[k];
            col_scale_n(a, n, eps);
        }
    }
#pragma unroll
    for (int t = kTMax - 1; t >= 0; --t) {
        if (t < iters) {
            float dA[kV];
#pragma unroll
            for (int k = 0; k < kV; ++k) {
                const bool on = col0() + k < n;
                const float cs = col_sum(hA[t][k]);
                const float cinv = on ? rcp_nr(cs + eps) : 0.f;
                const float dot = col_sum(g[k] * (hA[t][k] * cinv));
                dA[k] = on ? (g[k] - dot) * cinv : 0.f;
            }
            float rdot = ((dA[0] * hA[t][0] + dA[1] * hA[t][1]) + dA[2] * hA[t][2]) + dA[3] * hA[t][3];
            rdot = group_sum<4>(rdot);
#pragma unroll
            for (int k = 0; k < kV; ++k) g[k] = col0() + k < n ? (dA[k] - rdot) * hr[t] : 0.f;
        }
    }
}
}  // namespace skw16

}  // namespace mhc

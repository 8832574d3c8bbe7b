// Dynamic-H mHC layer: per-token H projected from the flattened token row
// (bindings.cpp:880-952 forward, 600-874 backward), and the projection
// operators fused_rmsnorm_matmul / compute_rms (bindings.cpp:480-566).
//
//   x_flat = x[b].reshape(n*C);  r_h = sqrt(mean(x_flat^2) + rms_eps)
//   P = x_flat . Phi^T,  Phi = [phi_pre; phi_post; phi_res]  ([2n+n^2, nC])
//   t_k = alpha_k P_k / r_h + b_k;  h_pre = sigmoid(t_pre),
//   h_post = 2 sigmoid(t_post),  M = SK(exp(t_res as n x n))
//   then the fused aggregate -> RMSNorm -> distribute pass of layer.hip.
//
// Kernels here:
//   phi_split_kernel    Phi (fp32) -> bf16 hi / mid / lo planes [3][32][K]
//                       (hi + mid + lo carries all 24 mantissa bits)
//   proj_mfma_kernel    P partials (split-K) and sum(x^2) partials; bf16
//                       MFMA 16x16x32 on the planes gives fp32 accuracy
//   dyn_coef_fwd_kernel per token: sum partials, t, sigmoid, Sinkhorn
//   dyn_coef_bwd_kernel per token: Sinkhorn adjoint, dP, d r_h, db/dalpha
//   proj_bwd_mfma_kernel dx += dP.Phi + s x_flat, dPhi partials (bf16 MFMA, split operands)
#include "mhc_device.h"
#include "mhc_internal.h"
#include "mhc_rows.h"

namespace mhc {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kNPad = 32;  // projection outputs padded to two 16-wide MFMA tiles

__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
    // A rows = lane % 16, B cols = lane % 16, k = 8 * (lane / 16) + 0..7;
    // D[4 * (lane / 16) + i][lane % 16] in element i.
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) { return pack_bf16x2(lo, hi); }


// ---------------------------------------------------------------------------
// fp32 -> three bf16 terms: v = hi + mid + lo exactly up to the last bit
// for normal values (3 x 8 significant bits = the fp32 mantissa).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void split3(float v, float& h, float& m, float& l) {
    h = bf16_to_f32(f32_to_bf16(v));
    const float r = v - h;
    m = bf16_to_f32(f32_to_bf16(r));
    l = r - m;
}

// Phi -> bf16 planes in MFMA B-fragment order, p = hi / mid / lo:
//   phif[((p * 2 + nt) * (K / 32) + ks) * 64 + lane]  (16 bytes = 8 bf16)
//     = Phi_p[nt * 16 + lane % 16][32 ks + 8 (lane / 16) .. + 7]
// so one wave's B operand of a 32-wide k step is 1 KB contiguous.  More
// than 32 rows are split into output tiles of 32 rows, tile t at
// phif + t * 6 * (K / 32) * 64 holding rows 32 t .. 32 t + 31; rows past np
// are zero.  Grid-stride over tiles * 2 * (K / 32) * 64 fragments.
// With w32 not null the same launch also converts the RMSNorm weight (wdt:
// F32 or BF16, C elements) to fp32 (as weight_f32_kernel).
__global__ __launch_bounds__(256) void phi_split_kernel(const float* __restrict__ pre, const float* __restrict__ post,
                                                        const float* __restrict__ res, int n, int np, int64_t K,
                                                        uint4* __restrict__ phif, const void* __restrict__ wsrc,
                                                        int wdt, int64_t C, float* __restrict__ w32) {
    if (w32) {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < C; i += (int64_t)gridDim.x * blockDim.x)
            w32[i] = wdt == kBF16 ? bf16_to_f32(static_cast<const bf16_t*>(wsrc)[i]) : static_cast<const float*>(wsrc)[i];
    }
    const int64_t ksteps = K / 32;
    const int64_t per_tile = 2 * ksteps * 64;
    const int64_t total = (int64_t)((np + 31) / 32) * per_tile;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = i / per_tile;
        const int64_t it = i - t * per_tile;
        const int lane = (int)(it & 63);
        const int64_t ks = (it >> 6) % ksteps;
        const int nt = (int)((it >> 6) / ksteps);
        const int o = (int)t * 32 + nt * 16 + (lane & 15);
        const int64_t k = ks * 32 + 8 * (lane >> 4);
        float v[8];
        if (o < np) {
            load_run<float, 8>(phi_row(pre, post, res, n, o, K) + k, v);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.f;
        }
        uint32_t w[3][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float h0, m0, l0, h1, m1, l1;
            split3(v[2 * e], h0, m0, l0);
            split3(v[2 * e + 1], h1, m1, l1);
            w[0][e] = pack_bf16(h0, h1);
            w[1][e] = pack_bf16(m0, m1);
            w[2][e] = pack_bf16(l0, l1);
        }
#pragma unroll
        for (int p = 0; p < 3; ++p)
            phif[t * 3 * per_tile + ((int64_t)(p * 2 + nt) * ksteps + ks) * 64 + lane] =
                make_uint4(w[p][0], w[p][1], w[p][2], w[p][3]);
    }
}

// ---------------------------------------------------------------------------
// Split-K projection on MFMA.  Workgroup = TB = 16*MT tokens x one K range,
// walked in stages of 128 k.  A stage of x is loaded with whole-row 16-byte
// pieces (16 lanes per 256-byte row for bf16), so every request is a full
// cache line, and staged in LDS; wave w then takes the 32-wide k step w of
// the stage for all TB tokens (MT A fragments read from LDS) against its B
// fragments of the Phi planes (1 KB contiguous loads).  bf16 x is exact in
// bf16: P = x.(hi + mid + lo) (3 MFMAs per tile); fp32 x is split the same
// way and the six products down to 2^-16 relative weight are kept
// (xh.(hi+mid+lo) + xm.(hi+mid) + xl.hi), leaving terms of order 2^-24.
// Also sum x^2.  blockIdx.z is the 32-row output tile of Phi: partials
// p_part[tile][ks][B][32]; tile 0 also stores ss_part[ks][B].
// Pipeline: x of stage s+2 and Phi of stage s+2 are in flight while stage s
// is on the matrix cores; one barrier per stage.
// ---------------------------------------------------------------------------
template <typename TX> constexpr int proj_mt() { return sizeof(TX) == 2 ? 8 : 4; }
constexpr int kProjKS = 128;  // k per stage

template <typename TX, int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void proj_mfma_kernel(
    const TX* __restrict__ x, const uint4* __restrict__ phif, float* __restrict__ p_part,
    float* __restrict__ ss_part, int64_t B, int64_t K, int64_t kchunk) {
    constexpr int TB = 16 * MT;
    constexpr int KS = kProjKS;
    constexpr int EPV = 16 / (int)sizeof(TX);  // elements per 16-byte piece
    constexpr int VPR = KS / EPV;              // pieces per row of a stage
    constexpr int RPP = 256 / VPR;             // rows per load pass
    constexpr int PASSES = TB / RPP;
    constexpr int PITCH = KS * (int)sizeof(TX) + 16;
    constexpr int XW = sizeof(TX) / 2;         // A pieces per lane per k step
    static_assert(PASSES * RPP == TB, "stage rows");
    static_assert(3 * 9 * MT * 64 * 4 <= 2 * TB * PITCH, "epilogue reuses the stage buffers");
    __shared__ __align__(16) char xs[2][TB * PITCH];

    const int lane = threadIdx.x & 63;
    const int wave = (int)wave_uniform(threadIdx.x >> 6);
    const int row = lane & 15;
    const int kg = lane >> 4;
    // block -> (token block, K split) from the linear id with the K split
    // fastest: workgroups go round-robin over the 8 XCDs by linear id, so
    // with ks a multiple of 8 each XCD serves only its own K splits (and
    // holds only their part of Phi in its L2)
    const int64_t lin = (int64_t)blockIdx.x + (int64_t)blockIdx.y * gridDim.x;
    const int64_t ksplit = lin % gridDim.y;
    const int64_t tblk = lin / gridDim.y;
    const int64_t tok0 = tblk * TB;
    const int64_t kb = ksplit * kchunk;
    const int64_t ke = (kb + kchunk < K) ? kb + kchunk : K;
    const int64_t nst = ke > kb ? (ke - kb + KS - 1) / KS : 0;
    const int64_t ksteps = K / 32;

    f32x4_t acc[MT][2];
    float ss[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        ss[mt] = 0.f;
    }
    // rows of this block past the batch read zeros (resource range)
    const int64_t rows = (B - tok0 < TB) ? B - tok0 : TB;
    const buf_rsrc_t xrs = make_buf_rsrc(x + tok0 * K, (uint32_t)(rows * K * (int64_t)sizeof(TX)));
    const int64_t otile = blockIdx.z;
    const buf_rsrc_t prs = make_buf_rsrc(phif + otile * 6 * ksteps * 64, (uint32_t)(6 * ksteps * 64 * 16));
    const int lrow = threadIdx.x / VPR;
    const int lvec = threadIdx.x % VPR;
    const uint32_t xoff = (uint32_t)(((int64_t)lrow * K + lvec * EPV) * (int64_t)sizeof(TX));
    const uint32_t xpass = (uint32_t)((int64_t)RPP * K * (int64_t)sizeof(TX));

    uint4 F0[PASSES], F1[PASSES], G0[6], G1[6];
    // The whole x offset is per lane: the range check covers the lane offset
    // only, so a column past K in the block's last row reads zeros instead
    // of memory past the tensor.  Columns past ke are zeroed at commit.
    // Blocks start at different stages of their K range, so the workgroups
    // reading one K range at a time spread over its columns (and the memory
    // channels) instead of all reading the same 256 bytes of their rows when
    // the row pitch is a multiple of the channel period.  With ks a multiple
    // of 8 the start goes by token block (an XCD's Phi is its K splits'
    // part); otherwise by XCD, so the blocks of one XCD move through a small
    // window of Phi that stays in its L2.
    const int64_t rot = nst <= 0 ? 0 : (gridDim.y % 8 == 0 ? tblk % nst : ((lin % 8) * nst) / 8);
    auto srot = [&](int64_t st) __attribute__((always_inline)) {
        const int64_t r = st + rot;
        return r < nst ? r : r - nst;
    };
    auto fetch_x = [&](uint4 (&f)[PASSES], int64_t st) __attribute__((always_inline)) {
        const uint32_t col = (uint32_t)((kb + srot(st) * KS) * (int64_t)sizeof(TX));
#pragma unroll
        for (int p = 0; p < PASSES; ++p) f[p] = buf_ld16<true, true>(xrs, xoff + p * xpass + col, 0u);
    };
    auto fetch_phi = [&](uint4 (&g)[6], int64_t st) __attribute__((always_inline)) {
        // this wave's k step of stage st, clamped to the last one (a step
        // past ke meets x = 0, so any finite fragment contributes nothing)
        int64_t kstep = (kb + srot(st) * KS) / 32 + wave;
        kstep = kstep < ksteps ? kstep : ksteps - 1;
        const uint32_t so = (uint32_t)(kstep * 64 * 16);
#pragma unroll
        for (int q = 0; q < 6; ++q) g[q] = buf_ld16<false>(prs, (uint32_t)((q * ksteps * 64 + lane) * 16), so);
    };
    auto commit = [&](const uint4 (&f)[PASSES], int64_t st, int buf) __attribute__((always_inline)) {
        const uint32_t m = (kb + srot(st) * KS + lvec * EPV < ke) ? 0xffffffffu : 0u;
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
            *reinterpret_cast<uint4*>(&xs[buf][(lrow + p * RPP) * PITCH + lvec * 16]) =
                make_uint4(f[p].x & m, f[p].y & m, f[p].z & m, f[p].w & m);
    };
    auto bop = [](const uint4& q) __attribute__((always_inline)) { return u32x4_t{q.x, q.y, q.z, q.w}; };
    auto compute = [&](int buf, const uint4 (&g)[6]) __attribute__((always_inline)) {
        const char* base = &xs[buf][row * PITCH + (wave * 32 + kg * 8) * (int)sizeof(TX)];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if constexpr (sizeof(TX) == 2) {
                const u32x4_t a = bop(*reinterpret_cast<const uint4*>(base + mt * 16 * PITCH));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = __uint_as_float(a[e] << 16), hi = __uint_as_float(a[e] & 0xffff0000u);
                    ss[mt] += lo * lo + hi * hi;
                }
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
                    for (int p = 0; p < 3; ++p) acc[mt][nt] = mfma16x16x32(a, bop(g[p * 2 + nt]), acc[mt][nt]);
                }
            } else {
                float v[8];
#pragma unroll
                for (int q = 0; q < XW; ++q) {
                    const uint4 w = *reinterpret_cast<const uint4*>(base + mt * 16 * PITCH + 16 * q);
                    v[4 * q] = __uint_as_float(w.x);
                    v[4 * q + 1] = __uint_as_float(w.y);
                    v[4 * q + 2] = __uint_as_float(w.z);
                    v[4 * q + 3] = __uint_as_float(w.w);
                }
                u32x4_t ah, am, al;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ss[mt] += v[2 * e] * v[2 * e] + v[2 * e + 1] * v[2 * e + 1];
                    float h0, m0, l0, h1, m1, l1;
                    split3(v[2 * e], h0, m0, l0);
                    split3(v[2 * e + 1], h1, m1, l1);
                    ah[e] = pack_bf16(h0, h1);
                    am[e] = pack_bf16(m0, m1);
                    al[e] = pack_bf16(l0, l1);
                }
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    acc[mt][nt] = mfma16x16x32(ah, bop(g[0 * 2 + nt]), acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(ah, bop(g[1 * 2 + nt]), acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(am, bop(g[0 * 2 + nt]), acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(ah, bop(g[2 * 2 + nt]), acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(am, bop(g[1 * 2 + nt]), acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(al, bop(g[0 * 2 + nt]), acc[mt][nt]);
                }
            }
        }
    };

    // Stages run in pairs with no exit between them (an exit there lets the
    // compiler sink a prefetch to its use); a prefetch past the last stage
    // re-reads stage 0.  buf 0 holds even stages, buf 1 odd ones.
    if (nst > 0) {
        auto clampst = [&](int64_t st) __attribute__((always_inline)) { return st < nst ? st : (int64_t)0; };
        fetch_x(F0, 0);
        fetch_phi(G0, 0);
        commit(F0, 0, 0);
        fetch_x(F1, clampst(1));
        fetch_phi(G1, clampst(1));
        __syncthreads();
        int64_t i = 0;
        for (; i + 2 <= nst; i += 2) {
            fetch_x(F0, clampst(i + 2));
            __builtin_amdgcn_sched_barrier(0);
            compute(0, G0);
            fetch_phi(G0, clampst(i + 2));
            commit(F1, i + 1, 1);
            __syncthreads();
            fetch_x(F1, clampst(i + 3));
            __builtin_amdgcn_sched_barrier(0);
            compute(1, G1);
            fetch_phi(G1, clampst(i + 3));
            commit(F0, i + 2, 0);
            __syncthreads();
        }
        if (i < nst) compute(0, G0);
    }
    __syncthreads();  // the stage buffers become the cross-wave reduction area
    float (*red)[9 * MT][64] = reinterpret_cast<float (*)[9 * MT][64]>(&xs[0][0]);

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
    float* pp = p_part + (otile * gridDim.y + ksplit) * B * kNPad;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t tok = tok0 + mt * 16 + kg * 4 + i;
            if (tok < B) {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) pp[tok * kNPad + nt * 16 + row] = acc[mt][nt][i];
            }
        }
        // lanes row, row+16, row+32, row+48 hold parts of token row's sum
        float s2 = ss[mt];
        s2 = xor32_add(xor16_add(s2));
        const int64_t tok = tok0 + mt * 16 + row;
        if (kg == 0 && tok < B && otile == 0) ss_part[ksplit * B + tok] = s2;
    }
}

// ---------------------------------------------------------------------------
// Projection over more than 128 output rows (2n + n^2 > 128: n >= 16),
// reading Phi once.  Workgroup = 128 output rows (one 32-row output tile
// per wave, two 16-row MFMA tiles that share each x fragment read from LDS)
// x TB = 16 MT tokens x one K range; Phi is the large operand here
// (178 MB at n = 32, C = 1280), so each element of it is loaded by one lane
// of one workgroup per token block and never staged.  x arrives as XPL
// bf16 planes ([XPL][B][K]: fp32 x split hi / mid / lo by
// proj_xsplit_kernel, or bf16 x itself) and goes through LDS, 64 k per
// stage, double-buffered, one barrier per stage.  A wave's Phi fragments
// (its 32 rows x 32 k: 2 x 8 consecutive fp32 per lane) are loaded two
// stages ahead and split into hi / mid / lo in registers (PHI_PLANES: read the
// fragment-order planes of phi_split_kernel instead, as packed for the
// forward-only entry).  Products as proj_mfma_kernel: bf16 x:
// x.(hi + mid + lo); fp32 x: xh.(hi + mid + lo) + xm.(hi + mid) + xl.hi.
// Partials p_part[tile][ks][B][32], the layout proj_mfma_kernel writes;
// with bf16 x the workgroups of output block 0 also store ss_part[ks][B]
// (fp32 x: proj_xsplit_kernel stores it).  Workgroups that stage the same x
// (same token block and K range) get ids on one XCD.
// ---------------------------------------------------------------------------
constexpr int kStreamOB = 128;                    // output rows per workgroup (32 per wave)
constexpr int kStreamKS = 64;                     // k per LDS stage
constexpr int kStreamPitch = kStreamKS * 2 + 16;  // bytes per staged row of one plane

// fp32 x -> xp[3][B][K] bf16 (split3 per element) and ss_part[q][b] = sum
// of x^2 over K range q of the projection: workgroup (b, q), fixed order.
__global__ __launch_bounds__(256) void proj_xsplit_kernel(const float* __restrict__ x, uint4* __restrict__ xp,
                                                          float* __restrict__ ss_part, int64_t B, int64_t K,
                                                          int64_t kchunk, int ks) {
    __shared__ float red[256 / kWave];
    const int64_t b = blockIdx.x / ks;
    const int q = (int)(blockIdx.x % ks);
    const int64_t kb = q * kchunk;
    const int64_t ke = kb + kchunk < K ? kb + kchunk : K;
    const int64_t plane = B * K / 8;  // 16-byte pieces per plane
    float ss[1] = {0.f};
    for (int64_t k = kb + 8 * (int64_t)threadIdx.x; k < ke; k += 8 * (int64_t)blockDim.x) {
        const float4 a = *reinterpret_cast<const float4*>(x + b * K + k);
        const float4 c = *reinterpret_cast<const float4*>(x + b * K + k + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        uint32_t w[3][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float h0, m0, l0, h1, m1, l1;
            split3(v[2 * e], h0, m0, l0);
            split3(v[2 * e + 1], h1, m1, l1);
            w[0][e] = pack_bf16(h0, h1);
            w[1][e] = pack_bf16(m0, m1);
            w[2][e] = pack_bf16(l0, l1);
            ss[0] += v[2 * e] * v[2 * e] + v[2 * e + 1] * v[2 * e + 1];
        }
        const int64_t pc = (b * K + k) / 8;
#pragma unroll
        for (int p2 = 0; p2 < 3; ++p2) xp[p2 * plane + pc] = make_uint4(w[p2][0], w[p2][1], w[p2][2], w[p2][3]);
    }
    block_sum<1>(ss, red);
    if (threadIdx.x == 0) ss_part[(int64_t)q * B + b] = ss[0];
}

// WRAP = 1 or 2 (the MHCResidualWrapper's streams, bf16 storage): x is not
// in memory; xpl is the residual and xb the branch ([B][Cw] each) and the
// stage's 16-byte pieces are read from the stream's source row (stream j =
// k / Cw, each 64-k stage within one stream: Cw % 64 == 0) and, for
// j >= 2, scaled by 0.1^(j-1) and rounded to bf16 at commit (WRAP = 1,
// 'decay') or read as zeros (WRAP = 2, 'zero').
template <int XPL, int MT, bool PHI_PLANES, int WRAP = 0>
__global__ __launch_bounds__(256) void proj_stream_kernel(
    const bf16_t* __restrict__ xpl, const float* __restrict__ phi_pre, const float* __restrict__ phi_post,
    const float* __restrict__ phi_res, int n_pre, const uint4* __restrict__ phif, int np, float* __restrict__ p_part,
    float* __restrict__ ss_part, int64_t B, int64_t K, int64_t kchunk, int ks, int oblocks, int64_t groups,
    const bf16_t* __restrict__ xb = nullptr, int Cw = 0) {
    static_assert(WRAP == 0 || XPL == 1, "the wrapper's streams are bf16 rows");
    constexpr int TB = 16 * MT;
    constexpr int KS = kStreamKS;
    constexpr int PITCH = kStreamPitch;
    constexpr int PIECES = XPL * TB * (KS * 2 / 16);  // 16-byte pieces per stage
    constexpr int PPT = (PIECES + 255) / 256;         // per thread
    __shared__ __align__(16) char xs[2][XPL * TB * PITCH];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row = lane & 15;
    const int kg = lane >> 4;
    // id = 8 (gq * oblocks + oi) + gx for group g = 8 gq + gx (token block
    // x K range): one group's output blocks share an XCD
    const int64_t lin = blockIdx.x;
    const int64_t rest = lin / 8;
    const int oi = (int)(rest % oblocks);
    const int64_t grp = (rest / oblocks) * 8 + lin % 8;
    if (grp >= groups) return;
    const int64_t tblk = grp / ks;
    const int ksplit = (int)(grp % ks);
    const int64_t tok0 = tblk * TB;
    const int ow = oi * kStreamOB + 32 * wave;  // the wave's output tile: rows ow .. ow + 31
    const bool wave_on = ow < np;
    const int64_t kb = ksplit * kchunk;
    const int64_t ke = kb + kchunk < K ? kb + kchunk : K;
    const int nst = ke > kb ? (int)((ke - kb + KS - 1) / KS) : 0;
    const int64_t ksteps = K / 32;
    const int64_t plane = B * K;  // elements per x plane

    f32x4_t acc[MT][2];
    float ss[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        acc[mt][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        acc[mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        ss[mt] = 0.f;
    }
    const bool do_ss = XPL == 1 && oi == 0 && wave == 0;

    // x stage st: piece i = tid + 256 u of this thread = (plane, token row,
    // 16-byte column), the plane fixed per u (TB * 8 is a multiple of 256).
    // Buffer loads: rows past the batch read zero through the per-plane
    // range, columns past the K range are zeroed at commit, no branches.
    static_assert((TB * 8) % 256 == 0, "whole planes per piece round");
    const int64_t rows = B - tok0 < TB ? B - tok0 : TB;
    buf_rsrc_t xr[XPL];
    if constexpr (WRAP != 0) {
        xr[0] = make_buf_rsrc(xpl + tok0 * Cw, (uint32_t)(rows * Cw * 2));
    } else {
#pragma unroll
        for (int p2 = 0; p2 < XPL; ++p2)
            xr[p2] = make_buf_rsrc(xpl + p2 * plane + tok0 * K, (uint32_t)(rows * K * 2));
    }
    const buf_rsrc_t xbr = WRAP != 0 ? make_buf_rsrc(xb + tok0 * Cw, (uint32_t)(rows * Cw * 2)) : xr[0];
    auto fetch_x = [&](uint4 (&f)[PPT], int st) __attribute__((always_inline)) {
        const int64_t k0 = kb + (int64_t)st * KS;
        if constexpr (WRAP != 0) {
            const int j = (int)k0 / Cw;  // wave-uniform
            const int c0 = (int)k0 - j * Cw;
            const bool none = WRAP == 2 && j >= 2;
#pragma unroll
            for (int u = 0; u < PPT; ++u) {
                const int i = threadIdx.x + 256 * u;
                const int r = (i / 8) % TB;
                const int c = i % 8;
                const uint32_t off = none ? kBufOff : (uint32_t)((r * Cw + c0 + 8 * c) * 2);
                f[u] = buf_ld16<false, true>(j == 1 ? xbr : xr[0], off, 0u);
            }
        } else {
#pragma unroll
            for (int u = 0; u < PPT; ++u) {
                const int i = threadIdx.x + 256 * u;
                const int r = (i / 8) % TB;
                const int c = i % 8;
                f[u] = buf_ld16<false, true>(xr[(256 * u) / (TB * 8)], (uint32_t)(((int64_t)r * K + k0 + 8 * c) * 2),
                                             0u);
            }
        }
    };
    auto commit = [&](const uint4 (&f)[PPT], int st, int buf) __attribute__((always_inline)) {
        const int64_t k0 = kb + (int64_t)st * KS;
        // decay streams: the stored stream value bf16(r * 0.1^(j-1))
        float mult = 0.f;
        if constexpr (WRAP == 1) {
            const int j = (int)k0 / Cw;
            double d = 1.0;
            for (int e = 1; e < j; ++e) d *= 0.1;  // Python's 0.1 ** (j - 1), as the wrapper kernels take it
            mult = j >= 2 ? (float)d : 0.f;
        }
#pragma unroll
        for (int u = 0; u < PPT; ++u) {
            const int i = threadIdx.x + 256 * u;
            const int pl = (256 * u) / (TB * 8);
            const int r = (i / 8) % TB;
            const int c = i % 8;
            const uint32_t m = k0 + 8 * c < ke ? 0xffffffffu : 0u;
            uint4 v = f[u];
            if constexpr (WRAP == 1) {
                if (mult != 0.f) {
                    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float lo = __uint_as_float(w[e] << 16) * mult;
                        const float hi = __uint_as_float(w[e] & 0xffff0000u) * mult;
                        w[e] = pack_bf16(lo, hi);
                    }
                    v = make_uint4(w[0], w[1], w[2], w[3]);
                }
            }
            *reinterpret_cast<uint4*>(&xs[buf][(pl * TB + r) * PITCH + 16 * c]) =
                make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
        }
    };
    // Phi fragments of stage st (its two k steps) for the wave's two 16-row
    // MFMA tiles nt: rows ow + 16 nt + row, k = 32 kstep + 8 kg .. + 7;
    // loaded two stages ahead, a step past the last one clamped (x is zero
    // there)
    struct PhiStage {
        float f[2][2][8];
        uint4 q[2][2][3];
    };
    auto fetch_phi = [&](PhiStage& ps, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            int64_t kstep = (kb + (int64_t)st * KS) / 32 + kk;
            kstep = kstep < ksteps ? kstep : ksteps - 1;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                if constexpr (PHI_PLANES) {
                    const int tile = ow / 32;
#pragma unroll
                    for (int p2 = 0; p2 < 3; ++p2)
                        ps.q[kk][nt][p2] =
                            wave_on ? phif[((int64_t)(tile * 6 + p2 * 2 + nt) * ksteps + kstep) * 64 + lane]
                                    : make_uint4(0u, 0u, 0u, 0u);
                } else {
                    // rows past np read the last row (no branch) and are zeroed
                    const int o = ow + 16 * nt + row;
                    const bool ov = o < np;
                    const float* pr =
                        phi_row(phi_pre, phi_post, phi_res, n_pre, ov ? o : np - 1, K) + kstep * 32 + 8 * kg;
                    const float4 a = *reinterpret_cast<const float4*>(pr);
                    const float4 c = *reinterpret_cast<const float4*>(pr + 4);
                    const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) ps.f[kk][nt][e] = ov ? v[e] : 0.f;
                }
            }
        }
    };
    auto phi_planes = [&](const PhiStage& ps, int kk, int nt, u32x4_t& h, u32x4_t& m, u32x4_t& l)
        __attribute__((always_inline)) {
        if constexpr (PHI_PLANES) {
            h = u32x4_t{ps.q[kk][nt][0].x, ps.q[kk][nt][0].y, ps.q[kk][nt][0].z, ps.q[kk][nt][0].w};
            m = u32x4_t{ps.q[kk][nt][1].x, ps.q[kk][nt][1].y, ps.q[kk][nt][1].z, ps.q[kk][nt][1].w};
            l = u32x4_t{ps.q[kk][nt][2].x, ps.q[kk][nt][2].y, ps.q[kk][nt][2].z, ps.q[kk][nt][2].w};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float h0, m0, l0, h1, m1, l1;
                split3(ps.f[kk][nt][2 * e], h0, m0, l0);
                split3(ps.f[kk][nt][2 * e + 1], h1, m1, l1);
                h[e] = pack_bf16(h0, h1);
                m[e] = pack_bf16(m0, m1);
                l[e] = pack_bf16(l0, l1);
            }
        }
    };
    auto compute = [&](int buf, int kk, const u32x4_t (&ph)[2], const u32x4_t (&pm)[2], const u32x4_t (&pl)[2])
        __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const char* base = &xs[buf][(16 * mt + row) * PITCH + (32 * kk + 8 * kg) * 2];
            const uint4 q0 = *reinterpret_cast<const uint4*>(base);
            const u32x4_t a0 = u32x4_t{q0.x, q0.y, q0.z, q0.w};
            if constexpr (XPL == 1) {
                if (do_ss) {
                    const uint32_t wv[4] = {q0.x, q0.y, q0.z, q0.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float lo = __uint_as_float(wv[e] << 16), hi = __uint_as_float(wv[e] & 0xffff0000u);
                        ss[mt] += lo * lo + hi * hi;
                    }
                }
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    acc[mt][nt] = mfma16x16x32(a0, ph[nt], acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(a0, pm[nt], acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(a0, pl[nt], acc[mt][nt]);
                }
            } else {
                const uint4 q1 = *reinterpret_cast<const uint4*>(base + TB * PITCH);
                const uint4 q2 = *reinterpret_cast<const uint4*>(base + 2 * TB * PITCH);
                const u32x4_t a1 = u32x4_t{q1.x, q1.y, q1.z, q1.w};
                const u32x4_t a2 = u32x4_t{q2.x, q2.y, q2.z, q2.w};
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    acc[mt][nt] = mfma16x16x32(a0, ph[nt], acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(a0, pm[nt], acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(a1, ph[nt], acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(a0, pl[nt], acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(a1, pm[nt], acc[mt][nt]);
                    acc[mt][nt] = mfma16x16x32(a2, ph[nt], acc[mt][nt]);
                }
            }
        }
    };

    if (nst > 0) {
        // Phi of stage s lives in ring slot s % 3 (no register copies, so
        // nothing waits for a load before its stage); x is staged one ahead
        uint4 f[PPT];
        PhiStage p0, p1, p2;
        fetch_x(f, 0);
        fetch_phi(p0, 0);
        fetch_phi(p1, 1);
        commit(f, 0, 0);
        __syncthreads();
        // x of the next stage is issued before Phi two ahead: the loads
        // complete in issue order, so the commit's wait leaves Phi in flight
        auto step = [&](int st, const PhiStage& cur, PhiStage& ahead) __attribute__((always_inline)) {
            const int buf = st & 1;
            if (st + 1 < nst) fetch_x(f, st + 1);
            fetch_phi(ahead, st + 2);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                u32x4_t ph[2], pm[2], pl[2];
                phi_planes(cur, kk, 0, ph[0], pm[0], pl[0]);
                phi_planes(cur, kk, 1, ph[1], pm[1], pl[1]);
                if (wave_on || do_ss) compute(buf, kk, ph, pm, pl);
            }
            if (st + 1 < nst) commit(f, st + 1, buf ^ 1);
            __syncthreads();
        };
        int st = 0;
        for (; st + 3 <= nst; st += 3) {
            step(st, p0, p2);
            step(st + 1, p1, p0);
            step(st + 2, p2, p1);
        }
        if (st < nst) step(st, p0, p2);
        if (st + 1 < nst) step(st + 1, p1, p0);
    }
    if (wave_on) {
        // D[token 16 mt + 4 kg + i][output ow + 16 nt + row]
        const int tile = ow / 32;
        float* pp = p_part + ((int64_t)tile * ks + ksplit) * B * kNPad + row;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t t = tok0 + 16 * mt + 4 * kg + i;
                if (t < B) {
                    pp[t * kNPad] = acc[mt][0][i];
                    pp[t * kNPad + 16] = acc[mt][1][i];
                }
            }
        }
    }
    if (do_ss) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            // lanes row, row + 16, row + 32, row + 48 hold parts of token row's sum
            const float s2 = xor32_add(xor16_add(ss[mt]));
            const int64_t t = tok0 + 16 * mt + row;
            if (kg == 0 && t < B) ss_part[(int64_t)ksplit * B + t] = s2;
        }
    }
}

// Split-K partial q of projection output o of token b.  The partials of
// the output tiles are stored tile-major: p_part[o / 32][q][b][o % 32].
__device__ __forceinline__ float p_part_at(const float* __restrict__ p_part, int ks, int64_t B, int q, int64_t b,
                                           int o) {
    return p_part[(((int64_t)(o >> 5) * ks + q) * B + b) * kNPad + (o & 31)];
}

// P[b][o] = sum_ks p_part[.][ks][b][.] for o < np (standalone projection).
__global__ __launch_bounds__(256) void proj_reduce_kernel(const float* __restrict__ p_part, int ks, int64_t B,
                                                          int np, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * np) return;
    const int64_t b = i / np;
    const int o = (int)(i % np);
    float s = 0.f;
    for (int q = 0; q < ks; ++q) s += p_part_at(p_part, ks, B, q, b, o);
    out[i] = s;
}

// ---------------------------------------------------------------------------
// Per-token coefficients (bindings.cpp:909-929).  One token per group of
// G = pow2ceil(n) lanes; lane r owns t_pre[r], t_post[r] and row r of t_res.
// coef[b] = (h_pre, h_post, M row-major); p_out[b] = P (np values); rh[b]
// (p_out and rh may be null: the forward-only entry keeps neither).
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void dyn_coef_fwd_kernel(
    const float* __restrict__ p_part, const float* __restrict__ ss_part, int ks, int64_t B, int64_t K,
    const float* __restrict__ a_pre, const float* __restrict__ a_post, const float* __restrict__ a_res,
    const float* __restrict__ b_pre, const float* __restrict__ b_post, const float* __restrict__ b_res,
    float* __restrict__ coef, float* __restrict__ p_out, float* __restrict__ rh, int iters, float sk_eps,
    float rms_eps) {
    constexpr int G = pow2ceil(N);
    constexpr int NP = 2 * N + N * N;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t tok = gid / G;
    const int r = (int)(gid % G);
    const bool tv = tok < B;
    const bool active = tv && r < N;
    float pp = 0.f, pq = 0.f, pr[N], ss = 0.f;
#pragma unroll
    for (int c = 0; c < N; ++c) pr[c] = 0.f;
    if (tv) {
        for (int q = 0; q < ks; ++q) {
            ss += ss_part[(int64_t)q * B + tok];
            if (r < N) {
                pp += p_part_at(p_part, ks, B, q, tok, r);
                pq += p_part_at(p_part, ks, B, q, tok, N + r);
#pragma unroll
                for (int c = 0; c < N; ++c) pr[c] += p_part_at(p_part, ks, B, q, tok, 2 * N + r * N + c);
            }
        }
    }
    const float r_h = sqrtf(ss / (float)K + rms_eps);
    const float inv = 1.f / r_h;
    const int rr = r < N ? r : 0;
    const float hp = sigmoidf(pp * a_pre[0] * inv + b_pre[rr]);
    const float hq = 2.f * sigmoidf(pq * a_post[0] * inv + b_post[rr]);
    float e[N];
#pragma unroll
    for (int c = 0; c < N; ++c) e[c] = active ? expf(pr[c] * a_res[0] * inv + b_res[rr * N + c]) : 0.f;
    sk_forward<N>(e, iters, sk_eps, active);
    if (active) {
        float* cf = coef + tok * NP;
        cf[r] = hp;
        cf[N + r] = hq;
#pragma unroll
        for (int c = 0; c < N; ++c) cf[2 * N + r * N + c] = e[c];
        if (p_out) {
            float* po = p_out + tok * NP;
            po[r] = pp;
            po[N + r] = pq;
#pragma unroll
            for (int c = 0; c < N; ++c) po[2 * N + r * N + c] = pr[c];
        }
    }
    if (tv && r == 0 && rh) rh[tok] = r_h;
}

// ---------------------------------------------------------------------------
// Per-token coefficient backward (bindings.cpp:777-848):
//   dt_pre = dh_pre_act h_pre (1 - h_pre);  dt_post = dh_post_act h_post (1 - h_post/2)
//   dt_res = SK^T(dM) * exp(t_res)
//   dP_k = alpha_k dt_k / r_h;  d r_h = -sum_k alpha_k dt_k P_k / r_h^2
//   s = d r_h / (K r_h)  (coefficient of x_flat in dx)
// dp_out[b][dp_stride(np)] (np rounded up to 32, zero padded), s_out[b];
// per-workgroup partial sums of db (np values) and dalpha (3) in
// part[blk][np + 3].  RES = false: the Sinkhorn adjoint's output is taken as
// zero (as in dyn_coef16_bwd_kernel<false>), so no adjoint runs and dP_res,
// db_res and dalpha_res are zeros.
// ---------------------------------------------------------------------------
template <int N, bool RES = true>
__global__ __launch_bounds__(256) void dyn_coef_bwd_kernel(
    const float* __restrict__ scal, const float* __restrict__ coef, const float* __restrict__ p,
    const float* __restrict__ rh, int64_t B, int64_t K, const float* __restrict__ a_pre,
    const float* __restrict__ a_post, const float* __restrict__ a_res, const float* __restrict__ b_res,
    float* __restrict__ dp_out, float* __restrict__ s_out, float* __restrict__ part, int iters, float sk_eps) {
    constexpr int G = pow2ceil(N);
    constexpr int NP = 2 * N + N * N;
    constexpr int NS = N * N + 2 * N;
    constexpr int NV = NP + 3;
    __shared__ float red[4 * NV];
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t tok = gid / G;
    const int r = (int)(gid % G);
    const bool tv = tok < B;
    const bool active = tv && r < N;
    const int rr = r < N ? r : 0;
    const int64_t tk = tv ? tok : 0;
    const float* sc = scal + tk * (NS + 2);
    const float* cf = coef + tk * NP;
    const float* pv = p + tk * NP;
    const float ap = a_pre[0], aq = a_post[0], ar = a_res[0];
    const float r_h = rh[tk];
    const float inv = 1.f / r_h;

    float gm[N], e[N], pr[N];
#pragma unroll
    for (int c = 0; c < N; ++c) {
        gm[c] = RES && active ? sc[rr * N + c] : 0.f;
        pr[c] = RES ? pv[2 * N + rr * N + c] : 0.f;
        e[c] = RES && active ? expf(pr[c] * ar * inv + b_res[rr * N + c]) : 0.f;
    }
    if constexpr (RES) sk_backward<N>(gm, e, iters, sk_eps, active);
    const float hp = cf[rr], hq = cf[N + rr];
    const float dt_pre = active ? sc[N * N + N + rr] * hp * (1.f - hp) : 0.f;
    const float dt_post = active ? sc[N * N + rr] * hq * (1.f - 0.5f * hq) : 0.f;
    float dt_res[N];
#pragma unroll
    for (int c = 0; c < N; ++c) dt_res[c] = active ? gm[c] * e[c] : 0.f;
    const float pp = pv[rr], pq = pv[N + rr];
    float lp = 0.f;
#pragma unroll
    for (int c = 0; c < N; ++c) lp += dt_res[c] * pr[c];
    const float l_pre = dt_pre * pp, l_post = dt_post * pq;
    const float tot = group_sum<G>(ap * l_pre + aq * l_post + ar * lp);
    if (active) {
        constexpr int NPT = dp_stride(NP);
        float* dp = dp_out + tok * NPT;
        dp[r] = ap * dt_pre * inv;
        dp[N + r] = aq * dt_post * inv;
#pragma unroll
        for (int c = 0; c < N; ++c) dp[2 * N + r * N + c] = ar * dt_res[c] * inv;
        if (r == 0) {
            for (int o = NP; o < NPT; ++o) dp[o] = 0.f;
            s_out[tok] = -tot * inv * inv * inv / (float)K;
        }
    }
    // per-workgroup partial sums of db and dalpha
    float v[NV];
#pragma unroll
    for (int q = 0; q < N; ++q) {
        v[q] = (r == q) ? dt_pre : 0.f;
        v[N + q] = (r == q) ? dt_post : 0.f;
#pragma unroll
        for (int c = 0; c < N; ++c) v[2 * N + q * N + c] = (r == q) ? dt_res[c] : 0.f;
    }
    v[NP] = l_pre * inv;
    v[NP + 1] = l_post * inv;
    v[NP + 2] = lp * inv;
    block_sum<NV>(v, red);
    if (threadIdx.x < NV) {
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < NV; ++q) t = (q == (int)threadIdx.x) ? v[q] : t;
        part[(int64_t)blockIdx.x * NV + threadIdx.x] = t;
    }
}

// ---------------------------------------------------------------------------
// The same for n >= 16, one token per group of n lanes: the db / dalpha
// terms (np + 3 values, too many to block-sum in registers) are written per
// token to part[b][np + 3] and column-summed over the tokens afterwards.
// The Sinkhorn adjoint keeps its per-iteration state in hist (one slot of
// iters * (n + 1) * n floats per lane group); the groups stride over the
// tokens with a trip count that is the same for every lane of the grid.
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void dyn_coef_bwd_wide_kernel(
    const float* __restrict__ scal, const float* __restrict__ coef, const float* __restrict__ p,
    const float* __restrict__ rh, int64_t B, int64_t K, const float* __restrict__ a_pre,
    const float* __restrict__ a_post, const float* __restrict__ a_res, const float* __restrict__ b_res,
    float* __restrict__ dp_out, float* __restrict__ s_out, float* __restrict__ part, int iters, float sk_eps,
    float* __restrict__ hist) {
    constexpr int NP = 2 * N + N * N;
    constexpr int NS = N * N + 2 * N;
    constexpr int NV = NP + 3;
    constexpr int NPT = dp_stride(NP);
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t slot = gid / N;
    const int64_t slots = (int64_t)gridDim.x * blockDim.x / N;
    const int r = (int)(gid % N);
    float* hs = hist + slot * (int64_t)iters * (N + 1) * N;
    const float ap = a_pre[0], aq = a_post[0], ar = a_res[0];
    for (int64_t base = 0; base < B; base += slots) {
        const int64_t tok = base + slot;
        const bool tv = tok < B;
        const int64_t tk = tv ? tok : 0;
        const float* sc = scal + tk * (NS + 2);
        const float* cf = coef + tk * NP;
        const float* pv = p + tk * NP;
        const float inv = 1.f / rh[tk];

        float gm[N], e[N], pr[N];
#pragma unroll
        for (int c = 0; c < N; ++c) {
            gm[c] = tv ? sc[r * N + c] : 0.f;
            pr[c] = pv[2 * N + r * N + c];
            e[c] = tv ? expf(pr[c] * ar * inv + b_res[r * N + c]) : 0.f;
        }
        sk_backward_mem<N>(gm, e, iters, sk_eps, tv, hs, r);
        const float hp = cf[r], hq = cf[N + r];
        const float dt_pre = tv ? sc[N * N + N + r] * hp * (1.f - hp) : 0.f;
        const float dt_post = tv ? sc[N * N + r] * hq * (1.f - 0.5f * hq) : 0.f;
        float lp = 0.f;
#pragma unroll
        for (int c = 0; c < N; ++c) {
            gm[c] = tv ? gm[c] * e[c] : 0.f;  // dt_res row r
            lp += gm[c] * pr[c];
        }
        const float l_pre = dt_pre * pv[r], l_post = dt_post * pv[N + r];
        const float tot = group_sum<N>(ap * l_pre + aq * l_post + ar * lp);
        const float s_pre = group_sum<N>(l_pre), s_post = group_sum<N>(l_post), s_res = group_sum<N>(lp);
        if (tv) {
            float* dp = dp_out + tok * NPT;
            dp[r] = ap * dt_pre * inv;
            dp[N + r] = aq * dt_post * inv;
#pragma unroll
            for (int c = 0; c < N; ++c) dp[2 * N + r * N + c] = ar * gm[c] * inv;
            float* pt = part + tok * NV;
            pt[r] = dt_pre;
            pt[N + r] = dt_post;
#pragma unroll
            for (int c = 0; c < N; ++c) pt[2 * N + r * N + c] = gm[c];
            if (r == 0) {
                for (int o = NP; o < NPT; ++o) dp[o] = 0.f;
                s_out[tok] = -tot * inv * inv * inv / (float)K;
                pt[NP] = s_pre * inv;
                pt[NP + 1] = s_post * inv;
                pt[NP + 2] = s_res * inv;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Generic n (no compiled instantiation, n <= 64): the formulas of
// dyn_coef_fwd_kernel / dyn_coef_bwd_wide_kernel with n taken at run time,
// one token per group of NM = 16, 32 or 64 lanes (row r of t_res on lane r,
// NM-float rows with the columns c >= n padding, skw_* Sinkhorn).  The
// backward writes its db / dalpha terms per token to part[b][np + 3].
// ---------------------------------------------------------------------------
template <int NM>
__global__ __launch_bounds__(256) void dyn_coef_gen_fwd_kernel(
    const float* __restrict__ p_part, const float* __restrict__ ss_part, int ks, int64_t B, int64_t K,
    const float* __restrict__ a_pre, const float* __restrict__ a_post, const float* __restrict__ a_res,
    const float* __restrict__ b_pre, const float* __restrict__ b_post, const float* __restrict__ b_res,
    float* __restrict__ coef, float* __restrict__ p_out, float* __restrict__ rh, int n, int iters, float sk_eps,
    float rms_eps) {
    const int np = 2 * n + n * n;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t tok = gid / NM;
    const int r = (int)(gid % NM);
    const bool tv = tok < B;
    const bool active = tv && r < n;
    const int rr = r < n ? r : 0;
    float pp = 0.f, pq = 0.f, pr[NM], ss = 0.f;
#pragma unroll
    for (int c = 0; c < NM; ++c) pr[c] = 0.f;
    if (tv) {
        for (int q = 0; q < ks; ++q) {
            ss += ss_part[(int64_t)q * B + tok];
            if (active) {
                pp += p_part_at(p_part, ks, B, q, tok, rr);
                pq += p_part_at(p_part, ks, B, q, tok, n + rr);
#pragma unroll
                for (int c = 0; c < NM; ++c) {
                    if (c < n) pr[c] += p_part_at(p_part, ks, B, q, tok, 2 * n + rr * n + c);
                }
            }
        }
    }
    const float r_h = sqrtf(ss / (float)K + rms_eps);
    const float inv = 1.f / r_h;
    const float hp = sigmoidf(pp * a_pre[0] * inv + b_pre[rr]);
    const float hq = 2.f * sigmoidf(pq * a_post[0] * inv + b_post[rr]);
    float e[NM];
#pragma unroll
    for (int c = 0; c < NM; ++c) e[c] = (active && c < n) ? expf(pr[c] * a_res[0] * inv + b_res[rr * n + c]) : 0.f;
    skw_forward<NM>(e, n, iters, sk_eps, active);
    if (active) {
        float* cf = coef + tok * np;
        cf[r] = hp;
        cf[n + r] = hq;
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            if (c < n) cf[2 * n + r * n + c] = e[c];
        }
        if (p_out) {
            float* po = p_out + tok * np;
            po[r] = pp;
            po[n + r] = pq;
#pragma unroll
            for (int c = 0; c < NM; ++c) {
                if (c < n) po[2 * n + r * n + c] = pr[c];
            }
        }
    }
    if (tv && r == 0 && rh) rh[tok] = r_h;
}

// Backward: groups of NM lanes take tokens slot, slot + slots, ... (a trip
// count the same for every lane of the grid).  With hist, each group keeps
// its Sinkhorn adjoint's per-iteration state in its own
// skw_hist_floats(NM, n, iters) floats of hist (O(iters) steps); without,
// the state is recomputed per iteration.  RES = false: the adjoint's output
// is taken as zero (as in dyn_coef_bwd_kernel<N, false>).
template <int NM, bool RES>
__global__ __launch_bounds__(256) void dyn_coef_gen_bwd_kernel(
    const float* __restrict__ scal, const float* __restrict__ coef, const float* __restrict__ p,
    const float* __restrict__ rh, int64_t B, int64_t K, const float* __restrict__ a_pre,
    const float* __restrict__ a_post, const float* __restrict__ a_res, const float* __restrict__ b_res,
    float* __restrict__ dp_out, float* __restrict__ s_out, float* __restrict__ part, int n, int iters,
    float sk_eps, float* __restrict__ hist) {
    const int np = 2 * n + n * n;
    const int ns = n * n + 2 * n;
    const int nv = np + 3;
    const int npt = dp_stride(np);
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t slot = gid / NM;
    const int64_t slots = (int64_t)gridDim.x * blockDim.x / NM;
    const int r = (int)(gid % NM);
    float* hs = hist ? hist + slot * skw_hist_floats(NM, n, iters) : nullptr;
    const float ap = a_pre[0], aq = a_post[0], ar = a_res[0];
    for (int64_t base = 0; base < B; base += slots) {
        const int64_t tok = base + slot;
        const bool tv = tok < B;
        const bool active = tv && r < n;
        const int rr = r < n ? r : 0;
        const int64_t tk = tv ? tok : 0;
        const float* sc = scal + tk * (ns + 2);
        const float* cf = coef + tk * np;
        const float* pv = p + tk * np;
        const float inv = 1.f / rh[tk];
        float gm[NM], e[NM], pr[NM];
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            const bool on = RES && active && c < n;
            gm[c] = on ? sc[rr * n + c] : 0.f;
            pr[c] = on ? pv[2 * n + rr * n + c] : 0.f;
            e[c] = on ? expf(pr[c] * ar * inv + b_res[rr * n + c]) : 0.f;
        }
        if constexpr (RES) {
            if (hs) {
                skw_backward_mem<NM>(gm, e, n, iters, sk_eps, active, hs, r, NM);
            } else {
                skw_backward<NM>(gm, e, n, iters, sk_eps, active);
            }
        }
        const float hp = cf[rr], hq = cf[n + rr];
        const float dt_pre = active ? sc[n * n + n + rr] * hp * (1.f - hp) : 0.f;
        const float dt_post = active ? sc[n * n + rr] * hq * (1.f - 0.5f * hq) : 0.f;
        float lp = 0.f;
#pragma unroll
        for (int c = 0; c < NM; ++c) {
            gm[c] = (active && c < n) ? gm[c] * e[c] : 0.f;  // dt_res row r
            lp += gm[c] * pr[c];
        }
        const float l_pre = active ? dt_pre * pv[rr] : 0.f, l_post = active ? dt_post * pv[n + rr] : 0.f;
        const float tot = group_sum<NM>(ap * l_pre + aq * l_post + ar * lp);
        const float s_pre = group_sum<NM>(l_pre), s_post = group_sum<NM>(l_post), s_res = group_sum<NM>(lp);
        if constexpr (!RES) {
            // the H_res rows' zeros, written by the whole lane group in
            // consecutive runs
            if (tv) {
                float* dp = dp_out + tok * npt + 2 * n;
                float* pt = part + tok * nv + 2 * n;
                for (int q = r; q < n * n; q += NM) {
                    dp[q] = 0.f;
                    pt[q] = 0.f;
                }
            }
        }
        if (active) {
            float* dp = dp_out + tok * npt;
            dp[r] = ap * dt_pre * inv;
            dp[n + r] = aq * dt_post * inv;
            float* pt = part + tok * nv;
            pt[r] = dt_pre;
            pt[n + r] = dt_post;
            if constexpr (RES) {
#pragma unroll
                for (int c = 0; c < NM; ++c) {
                    if (c < n) {
                        dp[2 * n + r * n + c] = ar * gm[c] * inv;
                        pt[2 * n + r * n + c] = gm[c];
                    }
                }
            }
            if (r == 0) {
                for (int o = np; o < npt; ++o) dp[o] = 0.f;
                s_out[tok] = -tot * inv * inv * inv / (float)K;
                pt[np] = s_pre * inv;
                pt[np + 1] = s_post * inv;
                pt[np + 2] = s_res * inv;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// n = 32: one token per 256-lane workgroup, the token's 32 x 32 matrix spread
// over the workgroup (skb: lane t holds row i = t / 8, columns c0 .. c0 + 3
// with c0 = 4 (t % 8)), so its Sinkhorn chain takes a barrier and a few
// instructions per iteration instead of 32 columns' reductions on one lane.
// Same formulas and outputs as dyn_coef_fwd_kernel / dyn_coef_bwd_wide_kernel;
// the backward keeps the iteration state in registers (iters <= skb::kTMax).
// P row o of token b sits in tile o / 32, so a lane's four t_res columns are
// one 16-byte run of a partial row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(skb::kThreads) void dyn_coef32_fwd_kernel(
    const float* __restrict__ p_part, const float* __restrict__ ss_part, int ks, int64_t B, int64_t K,
    const float* __restrict__ a_pre, const float* __restrict__ a_post, const float* __restrict__ a_res,
    const float* __restrict__ b_pre, const float* __restrict__ b_post, const float* __restrict__ b_res,
    float* __restrict__ coef, float* __restrict__ p_out, float* __restrict__ rh, int iters, float sk_eps,
    float rms_eps) {
    constexpr int N = skb::kN;
    constexpr int NP = 2 * N + N * N;
    constexpr int V = skb::kV;
    __shared__ float part[skb::kPartFloats];
    const int64_t tok = blockIdx.x;
    const int i = skb::row(), c0 = skb::col0();
    float pp = 0.f, pq = 0.f, pr[V] = {0.f, 0.f, 0.f, 0.f}, ss = 0.f;
    // unrolled so that the loads of several splits are in flight together
    // (the sums stay in split order)
#pragma unroll 8
    for (int q = 0; q < ks; ++q) {
        ss += ss_part[(int64_t)q * B + tok];
        pp += p_part_at(p_part, ks, B, q, tok, i);
        pq += p_part_at(p_part, ks, B, q, tok, N + i);
        const float4 v = *reinterpret_cast<const float4*>(
            p_part + (((int64_t)(2 + i) * ks + q) * B + tok) * kNPad + c0);
        pr[0] += v.x;
        pr[1] += v.y;
        pr[2] += v.z;
        pr[3] += v.w;
    }
    const float r_h = sqrtf(ss / (float)K + rms_eps);
    const float inv = 1.f / r_h;
    float e[V];
#pragma unroll
    for (int k = 0; k < V; ++k) e[k] = expf(pr[k] * a_res[0] * inv + b_res[i * N + c0 + k]);
    skb::forward(e, iters, sk_eps, part);
    float* cf = coef + tok * NP;
#pragma unroll
    for (int k = 0; k < V; ++k) cf[2 * N + i * N + c0 + k] = e[k];
    if (c0 == 0) {
        cf[i] = sigmoidf(pp * a_pre[0] * inv + b_pre[i]);
        cf[N + i] = 2.f * sigmoidf(pq * a_post[0] * inv + b_post[i]);
    }
    if (p_out) {
        float* po = p_out + tok * NP;
#pragma unroll
        for (int k = 0; k < V; ++k) po[2 * N + i * N + c0 + k] = pr[k];
        if (c0 == 0) {
            po[i] = pp;
            po[N + i] = pq;
        }
    }
    if (threadIdx.x == 0 && rh) rh[tok] = r_h;
}

__global__ __launch_bounds__(skb::kThreads) void dyn_coef32_bwd_kernel(
    const float* __restrict__ scal, const float* __restrict__ coef, const float* __restrict__ p,
    const float* __restrict__ rh, int64_t B, int64_t K, const float* __restrict__ a_pre,
    const float* __restrict__ a_post, const float* __restrict__ a_res, const float* __restrict__ b_res,
    float* __restrict__ dp_out, float* __restrict__ s_out, float* __restrict__ part, int iters, float sk_eps) {
    (void)B;  // the grid is one workgroup per token
    constexpr int N = skb::kN;
    constexpr int NP = 2 * N + N * N;
    constexpr int NS = N * N + 2 * N;
    constexpr int NV = NP + 3;
    constexpr int NPT = dp_stride(NP);
    constexpr int V = skb::kV;
    __shared__ float pbuf[skb::kPartFloats];
    __shared__ float hc[skb::kHistFloats];
    __shared__ float red[skb::kNW][4];
    const int64_t tok = blockIdx.x;
    const int i = skb::row(), c0 = skb::col0();
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const float ap = a_pre[0], aq = a_post[0], ar = a_res[0];
    const float* sc = scal + tok * (NS + 2);
    const float* cf = coef + tok * NP;
    const float* pv = p + tok * NP;
    const float inv = 1.f / rh[tok];
    float gm[V], e[V], pr[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
        gm[k] = sc[i * N + c0 + k];
        pr[k] = pv[2 * N + i * N + c0 + k];
        e[k] = expf(pr[k] * ar * inv + b_res[i * N + c0 + k]);
    }
    skb::backward(gm, e, iters, sk_eps, pbuf, hc);
    const float hp = cf[i], hq = cf[N + i];
    const float dt_pre = sc[N * N + N + i] * hp * (1.f - hp);
    const float dt_post = sc[N * N + i] * hq * (1.f - 0.5f * hq);
    float lp = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
        gm[k] *= e[k];  // dt_res
        lp += gm[k] * pr[k];
    }
    lp = group_sum<skb::kLPR>(lp);
    const float l_pre = dt_pre * pv[i], l_post = dt_post * pv[N + i];
    // sums over the 32 rows: one lane per row, the wave, then the 4 waves
    const bool lead = c0 == 0;
    float v[4] = {ap * l_pre + aq * l_post + ar * lp, l_pre, l_post, lp};
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = group_sum<kWave>(lead ? v[k] : 0.f);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) red[wave][k] = v[k];
    }
    float* dp = dp_out + tok * NPT;
#pragma unroll
    for (int k = 0; k < V; ++k) dp[2 * N + i * N + c0 + k] = ar * gm[k] * inv;
    float* pt = part + tok * NV;
#pragma unroll
    for (int k = 0; k < V; ++k) pt[2 * N + i * N + c0 + k] = gm[k];
    if (lead) {
        dp[i] = ap * dt_pre * inv;
        dp[N + i] = aq * dt_post * inv;
        pt[i] = dt_pre;
        pt[N + i] = dt_post;
    }
    for (int o = NP + (int)threadIdx.x; o < NPT; o += skb::kThreads) dp[o] = 0.f;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t[4] = {red[0][0], red[0][1], red[0][2], red[0][3]};
#pragma unroll
        for (int w = 1; w < skb::kNW; ++w) {
#pragma unroll
            for (int k = 0; k < 4; ++k) t[k] += red[w][k];
        }
        s_out[tok] = -t[0] * inv * inv * inv / (float)K;
        pt[NP] = t[1] * inv;
        pt[NP + 1] = t[2] * inv;
        pt[NP + 2] = t[3] * inv;
    }
}

// ---------------------------------------------------------------------------
// n = 4: one token per 16-lane DPP row.  Lane l holds element (l/4, l%4) of
// t_res and, for l < 8, t_pre[l] (l < 4) or t_post[l-4] (the coefficient
// order), so the Sinkhorn iterations are a few DPP steps per lane
// (sk16_forward / sk16_backward) and the per-token loads and stores are
// contiguous.  Lanes of tokens past the batch compute on token 0 and store
// nothing.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dyn_coef16_fwd_kernel(
    const float* __restrict__ p_part, const float* __restrict__ ss_part, int ks, int64_t B, int64_t K,
    const float* __restrict__ a_pre, const float* __restrict__ a_post, const float* __restrict__ a_res,
    const float* __restrict__ b_pre, const float* __restrict__ b_post, const float* __restrict__ b_res,
    float* __restrict__ coef, float* __restrict__ p_out, float* __restrict__ rh, int iters, float sk_eps,
    float rms_eps) {
    constexpr int N = 4;
    constexpr int NP = 2 * N + N * N;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t tok = gid >> 4;
    const int l = (int)(gid & 15);
    const bool tv = tok < B;
    const int64_t tk = tv ? tok : 0;
    float pres = 0.f, ppq = 0.f, ss = 0.f;
    for (int q = 0; q < ks; ++q) {
        const float* pb = p_part + ((int64_t)q * B + tk) * kNPad;
        ss += ss_part[(int64_t)q * B + tk];
        pres += pb[2 * N + l];
        ppq += pb[l & 7];
    }
    const float r_h = sqrtf(ss / (float)K + rms_eps);
    const float inv = 1.f / r_h;
    const float h = (l < N) ? sigmoidf(ppq * a_pre[0] * inv + b_pre[l & 3])
                            : 2.f * sigmoidf(ppq * a_post[0] * inv + b_post[(l - N) & 3]);
    float e = expf(pres * a_res[0] * inv + b_res[l]);
    sk16_forward(e, iters, sk_eps);
    if (tv) {
        float* cf = coef + tok * NP;
        cf[2 * N + l] = e;
        if (l < 2 * N) cf[l] = h;
        if (p_out) {
            float* po = p_out + tok * NP;
            po[2 * N + l] = pres;
            if (l < 2 * N) po[l] = ppq;
        }
        if (l == 0 && rh) rh[tok] = r_h;
    }
}

int dyn_coef16_bwd_blocks(int64_t B) {
    int64_t g = (B + 15) / 16;
    if (g > 1024) g = 1024;
    return (int)(g < 1 ? 1 : g);
}

// Backward of dyn_coef16_fwd_kernel (the formulas of dyn_coef_bwd_kernel).
// Workgroups stride over groups of 16 tokens; each lane sums its db / dalpha
// terms over its tokens in order, then the block reduces them into
// part[blk][27] = (db_pre[4], db_post[4], db_res[16], dalpha_pre, dalpha_post,
// dalpha_res).  RES = false: the Sinkhorn adjoint's output is taken as zero
// (a dM constant down each column, which the final column normalisation
// removes), so dP_res, db_res and dalpha_res are zeros.
template <bool RES>
__global__ __launch_bounds__(256) void dyn_coef16_bwd_kernel(
    const float* __restrict__ scal, const float* __restrict__ coef, const float* __restrict__ p,
    const float* __restrict__ rh, int64_t B, int64_t K, const float* __restrict__ a_pre,
    const float* __restrict__ a_post, const float* __restrict__ a_res, const float* __restrict__ b_res,
    float* __restrict__ dp_out, float* __restrict__ s_out, float* __restrict__ part, int iters, float sk_eps) {
    constexpr int N = 4;
    constexpr int NP = 2 * N + N * N;
    constexpr int NS = N * N + 2 * N;
    constexpr int NV = NP + 3;
    __shared__ float red[4][NV];
    const int l = threadIdx.x & 15;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const float ap = a_pre[0], aq = a_post[0], ar = a_res[0];
    const float apq = (l < N) ? ap : aq;
    float acc_pp = 0.f, acc_res = 0.f, acc_a = 0.f, acc_b = 0.f, acc_c = 0.f;
    const int64_t groups = (B + 15) / 16;
    for (int64_t grp = blockIdx.x; grp < groups; grp += gridDim.x) {  // uniform trip count per block
        const int64_t tok = grp * 16 + (threadIdx.x >> 4);
        const bool tv = tok < B;
        const int64_t tk = tv ? tok : 0;
        const float* sc = scal + tk * (NS + 2);
        const float* cf = coef + tk * NP;
        const float* pv = p + tk * NP;
        const float inv = 1.f / rh[tk];
        const float pr = pv[2 * N + l];
        float dt_res = 0.f;
        if constexpr (RES) {
            const float e = expf(pr * ar * inv + b_res[l]);
            float g = sc[l];  // dM element
            sk16_backward(g, e, iters, sk_eps);
            dt_res = g * e;
        }
        const float hv = cf[l & 7];
        // dh_post_act[q] at sc[N*N + q], dh_pre_act[q] at sc[N*N + N + q]
        const float dh = (l < N) ? sc[N * N + N + (l & 3)] : sc[N * N + ((l - N) & 3)];
        const float dt_pp = (l < N) ? dh * hv * (1.f - hv) : dh * hv * (1.f - 0.5f * hv);
        const float lpp = (l < 2 * N) ? dt_pp * pv[l & 7] : 0.f;  // l_pre or l_post
        const float lres = dt_res * pr;
        const float tot = group_sum<16>(apq * lpp + ar * lres);
        if (tv) {
            float* dp = dp_out + tok * kNPad;
            dp[2 * N + l] = ar * dt_res * inv;
            if (l < 2 * N) dp[l] = apq * dt_pp * inv;
            else dp[2 * N + N * N + (l - 2 * N)] = 0.f;  // padding entries 24..31
            if (l == 0) s_out[tok] = -tot * inv * inv * inv / (float)K;
            if (l < 2 * N) acc_pp += dt_pp;
            acc_res += dt_res;
            if (l < N) acc_a += lpp * inv;
            else if (l < 2 * N) acc_b += lpp * inv;
            acc_c += lres * inv;
        }
    }
    // lanes of one slot: l, l+16, l+32, l+48 of every wave, then the waves
    acc_a = group_sum<16>(acc_a);
    acc_b = group_sum<16>(acc_b);
    acc_c = group_sum<16>(acc_c);
    float v[5] = {acc_pp, acc_res, acc_a, acc_b, acc_c};
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        v[k] = xor32_add(xor16_add(v[k]));
    }
    if (lane < 16) {
        if (l < 2 * N) red[wave][l] = v[0];
        red[wave][2 * N + l] = v[1];
        if (l == 0) {
            red[wave][NP] = v[2];
            red[wave][NP + 1] = v[3];
            red[wave][NP + 2] = v[4];
        }
    }
    __syncthreads();
    if (threadIdx.x < NV) {
        const int nw = blockDim.x >> 6;
        float t = 0.f;
        for (int w = 0; w < nw; ++w) t += red[w][threadIdx.x];
        part[(int64_t)blockIdx.x * NV + threadIdx.x] = t;
    }
}

// out[c] = sum_r part[r][c] for a few columns (db, dalpha); one workgroup
// per 32 columns, as 32 columns x 32 row phases, each phase summing every
// 32nd row in order and the phases added in order (deterministic).
__global__ __launch_bounds__(1024) void small_column_sum_kernel(const float* __restrict__ part, int rows, int cols,
                                                                float* __restrict__ out_db, float* __restrict__ out_da,
                                                                int np) {
    __shared__ float red[32][33];
    const int cl = threadIdx.x & 31;
    const int ph = threadIdx.x >> 5;
    for (int c0 = blockIdx.x * 32; c0 < cols; c0 += gridDim.x * 32) {
        const int col = c0 + cl;
        float s = 0.f;
        if (col < cols) {
            // the phase's rows in order, 8 loads in flight
            int q = ph;
            for (; q + 224 < rows; q += 256) {
                float a[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) a[k] = part[(int64_t)(q + 32 * k) * cols + col];
#pragma unroll
                for (int k = 0; k < 8; ++k) s += a[k];
            }
            for (; q < rows; q += 32) s += part[(int64_t)q * cols + col];
        }
        red[ph][cl] = s;
        __syncthreads();
        if (ph == 0 && col < cols) {
            float t = 0.f;
            for (int k = 0; k < 32; ++k) t += red[k][cl];
            if (col < np) out_db[col] = t;
            else out_da[col - np] = t;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Projection backward on the bf16 matrix cores, over the flattened rows
// x[b][k] (k = j*C + c for the layer):
//   dx[b][k] = dx_in[b][k] + s[b] x[b][k] + sum_o dP[b][o] Phi[o][k]
//   dPhi_part[tile][o][k] = sum_{b in tile} dP[b][o] x[b][k]
// In the layer backward dx_in is the stream part already written by the row
// kernel (bindings.cpp:834-848 adds the same two terms to grad_x_flat).
// One launch covers the 32-row output tile o0 .. o0 + np - 1 of Phi (np <=
// 32, dP pointing at its column o0); projections with more rows run one
// launch per tile, the later ones accumulating without the s term.
//
// fp32 operands are split into bf16 hi + lo (v = hi + lo to 2^-16 relative);
// products keep hi.hi + hi.lo + lo.hi, so both products carry ~2^-16
// relative error per term (bf16 x is exact and needs no lo part).
// MFMA 16x16x32 bf16 layout: A row = lane % 16, B column = lane % 16, the
// lane's 8 reduction indices are 8 (lane / 16) .. + 7; D register i of lane l
// is D[4 (l / 16) + i][l % 16].
//   dx_proj^T (16 columns x 16 tokens): A = Phi^T, B = dP^T, reducing over o
//     (padded to 32: one step); lane l then holds token l % 16 at four
//     consecutive columns, so its epilogue is 8-byte LDS accesses;
//   dPhi (16 o x 16 columns): A = dP^T, B = x over the stage's 32 tokens.
// Each stage's dP is split into hi/lo bf16 once, when it is written to LDS,
// in token-major and o-major copies, so both operands are single 16-byte
// reads.  Workgroup = 4 waves x 32 columns; stages of 32 tokens; x and dx_in
// tiles arrive with coalesced 16-byte loads (two stages in flight), results
// return to the dx tile in LDS and leave with coalesced 16-byte stores.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void split_pack8(const float (&v)[8], u32x4_t& hi, u32x4_t& lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float h0 = bf16_to_f32(f32_to_bf16(v[2 * e]));
        const float h1 = bf16_to_f32(f32_to_bf16(v[2 * e + 1]));
        hi[e] = pack_bf16(h0, h1);
        lo[e] = pack_bf16(v[2 * e] - h0, v[2 * e + 1] - h1);
    }
}

// Four consecutive elements at an 8-byte aligned LDS address (8-byte accesses only).
template <typename TX>
__device__ __forceinline__ void lds_get4(const char* p, float (&v)[4]) {
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
__device__ __forceinline__ void lds_put4(char* p, const float (&v)[4]) {
    uint2* q = reinterpret_cast<uint2*>(p);
    if constexpr (sizeof(TX) == 2) {
        q[0] = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
    } else {
        q[0] = make_uint2(__float_as_uint(v[0]), __float_as_uint(v[1]));
        q[1] = make_uint2(__float_as_uint(v[2]), __float_as_uint(v[3]));
    }
}

// LDS row pitch of a 128-column stage tile (8-byte aligned rows; 8 extra
// bytes spread the token rows read by the four lane groups over the banks).
template <typename TX, int CB> constexpr int pb_pitch() { return CB * (int)sizeof(TX) + 8; }
constexpr int kDpPitch = 40;  // bf16 per row of the split dP copies (32 + 8 pad)

// Waves per SIMD the register allocation targets: four for bf16 x (128
// registers, no spills; four 35.6 KB workgroups share a CU's LDS), two for
// fp32 x, whose split operands need more.
template <typename TX> constexpr int kPbWaves() { return sizeof(TX) == 2 ? 4 : 2; }
// Waves per workgroup (32 columns each): eight for bf16 x (256 columns), four
// for fp32 x (128 columns).
template <typename TX> constexpr int kPbNW() { return sizeof(TX) == 2 ? 8 : 4; }

template <typename TX, bool ACC, bool HAS_S>
__global__ __launch_bounds__(64 * kPbNW<TX>()) __attribute__((amdgpu_waves_per_eu(kPbWaves<TX>()))) void proj_bwd_mfma_kernel(
    const TX* __restrict__ x, const float* __restrict__ dP, int dp_stride, const float* __restrict__ s_tok,
    const float* __restrict__ phi_pre, const float* __restrict__ phi_post, const float* __restrict__ phi_res,
    int n_pre, int o0, int np, TX* __restrict__ dx, const int32_t* __restrict__ dx_scale, int groups, int C,
    float* __restrict__ dphi_part, int64_t B, int64_t K, int64_t tile) {
    // With bf16 x the incoming dx (ACC) is the row pass's stream part as fp16
    // against power-of-two scales (part_pack4) with exponents
    // dx_scale[b][groups]: each 128 columns of this block (channels c .. c +
    // 127 of one stream) are group (c / 128) % groups of every token.  The
    // sum is rounded once to bf16 on the way out.
    constexpr bool QIN = ACC && sizeof(TX) == 2;
    constexpr int NT = 64 * kPbNW<TX>();
    constexpr int TB = 32;                      // tokens per stage
    constexpr int CB = 32 * kPbNW<TX>();        // columns per workgroup
    constexpr int NG = CB / kPartGroup;         // stream-part scale groups per workgroup
    constexpr int EPV = 16 / sizeof(TX);        // elements per 16-byte vector
    constexpr int VPR = CB / EPV;               // vectors per tile row
    constexpr int RPP = NT / VPR;               // tile rows per load pass
    constexpr int PASSES = TB / RPP;
    constexpr int PITCH = pb_pitch<TX, CB>();
    static_assert(PASSES * RPP == TB && CB % kPartGroup == 0 && NG * TB <= NT, "stage shape");
    // Only the dx tile is double-buffered: a stage's store reads it while
    // the next stage is committed.  x, the dP copies and s of the next
    // stage are committed after the barrier that ends the compute reading
    // them, so one copy each suffices (35.6 KB of LDS for bf16 x: four
    // workgroups fit a CU).
    __shared__ __align__(16) char x_lds[TB * PITCH];
    __shared__ __align__(16) char dx_lds[2][TB * PITCH];
    __shared__ __align__(16) bf16_t dps_lds[4][32 * kDpPitch];  // hi_row, lo_row, hi_col, lo_col
    __shared__ float s_lds[TB];
    __shared__ int q_lds[QIN ? NG : 1][QIN ? TB : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int64_t kb0 = (int64_t)blockIdx.x * CB;
    const int wc0 = wave * 32;
    const bool wave_on = kb0 + wc0 < K;  // K % 32 == 0: whole waves are in or out

    const int lrow = tid / VPR;
    const int lvec = tid % VPR;
    const int64_t lcol = kb0 + (int64_t)lvec * EPV;
    const bool lcol_ok = lcol < K;
    // dP loaders: lanes 0..255, token tid / 8, outputs 4 (tid % 8) .. + 3
    const bool dp_on = tid < 256;
    const int dtk = (tid & 255) >> 3;
    const int dpo = (tid & 7) * 4;

    // dx_proj A operands (Phi^T): Phi[8 lg + e][column 16 ct + lr]
    u32x4_t phh[2], phl[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int64_t k = kb0 + wc0 + 16 * ct + lr;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int o = 8 * lg + e;
            v[e] = (wave_on && o < np) ? phi_row(phi_pre, phi_post, phi_res, n_pre, o0 + o, K)[k] : 0.f;
        }
        split_pack8(v, phh[ct], phl[ct]);
    }
    f32x4_t accP[2][2];
#pragma unroll
    for (int ot = 0; ot < 2; ++ot) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) accP[ot][ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    const int64_t t_begin = (int64_t)blockIdx.y * tile;
    const int64_t t_end = (t_begin + tile < B) ? t_begin + tile : B;
    const int64_t nrows = t_end > t_begin ? t_end - t_begin : 0;

    // Every global access goes through a buffer resource over this block's
    // rows [t_begin, t_end) (under 2 GiB each: proj_bwd_tiles): rows past
    // t_end and lanes with nothing to load read zeros and such stores are
    // dropped, so no access sits behind a branch and the compiler's wait
    // counts stay exact across the two-stage prefetch.  Offsets are bytes.
    const uint32_t xrow = (uint32_t)(K * (int64_t)sizeof(TX));
    const buf_rsrc_t rs_x = make_buf_rsrc(x + t_begin * K, (uint32_t)(nrows * xrow));
    const buf_rsrc_t rs_dx = make_buf_rsrc(dx + t_begin * K, (uint32_t)(nrows * xrow));
    const buf_rsrc_t rs_p = make_buf_rsrc(dP + t_begin * dp_stride, (uint32_t)(nrows * dp_stride * 4));
    const buf_rsrc_t rs_s = make_buf_rsrc(HAS_S ? s_tok + t_begin : s_tok, HAS_S ? (uint32_t)(nrows * 4) : 0u);
    // step loaders: lane tid < NG TB takes group tid / TB of token tid % TB
    const int qg = tid / TB;
    const int grp = QIN ? (int)(((kb0 + (int64_t)qg * kPartGroup) % C) / kPartGroup) % groups : 0;
    const buf_rsrc_t rs_q =
        make_buf_rsrc(QIN ? dx_scale + t_begin * groups : dx_scale, QIN ? (uint32_t)(nrows * groups * 4) : 0u);
    const uint32_t xo = lcol_ok ? (uint32_t)lrow * xrow + (uint32_t)(lcol * (int64_t)sizeof(TX)) : kBufOff;
    const uint32_t po = dp_on ? (uint32_t)(dtk * dp_stride + dpo) * 4u : kBufOff;
    const uint32_t so = tid < TB ? (uint32_t)tid * 4u : kBufOff;
    const uint32_t qo = tid < NG * TB ? (uint32_t)((tid % TB) * groups + grp) * 4u : kBufOff;

    // Two register sets of fetched row tiles: stage i+2 is fetched while
    // stage i computes and stage i+1 (fetched one stage earlier) moves into
    // LDS.  The stage's small records (dP, s, steps) are fetched one stage
    // ahead, before the row tiles of the stage after, so that waiting for
    // them leaves those in flight.
    struct Fetched {
        uint4 x[PASSES], d[PASSES];
    };
    struct Small {
        uint4 dp;
        uint32_t s, q;
    };
    Fetched f0, f1;
    Small sm;
    // the stage of rows rel .. rel + TB - 1 (relative to t_begin)
    auto fetch = [&](Fetched& f, uint32_t rel) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const uint32_t off = xo + (rel + p * RPP) * xrow;
            f.x[p] = buf_ld16<true>(rs_x, off, 0u);
            if constexpr (ACC) f.d[p] = buf_ld16<true>(rs_dx, off, 0u);
        }
    };
    auto fetch_small = [&](uint32_t rel) __attribute__((always_inline)) {
        sm.dp = buf_ld16<false>(rs_p, po + rel * (uint32_t)dp_stride * 4u, 0u);
        sm.s = HAS_S ? buf_ld4(rs_s, so + rel * 4u, 0u) : 0u;
        sm.q = QIN ? buf_ld4(rs_q, qo + rel * (uint32_t)groups * 4u, 0u) : 0u;
    };
    auto commit = [&](const Fetched& f, int buf) __attribute__((always_inline)) {
        // s and the steps are consumed behind a branch below; an empty use of
        // their registers makes every lane wait for them in straight-line
        // code, so the compiler's wait counts do not carry them as possibly
        // in flight past it.
        asm volatile("" ::"v"(sm.s), "v"(sm.q), "v"(sm.dp.x), "v"(sm.dp.y), "v"(sm.dp.z), "v"(sm.dp.w));
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int row = lrow + p * RPP;
            const uint4 vx = f.x[p];
            uint2* px = reinterpret_cast<uint2*>(&x_lds[row * PITCH + lvec * 16]);
            px[0] = make_uint2(vx.x, vx.y);
            px[1] = make_uint2(vx.z, vx.w);
            if constexpr (ACC) {
                const uint4 vd = f.d[p];
                uint2* pd = reinterpret_cast<uint2*>(&dx_lds[buf][row * PITCH + lvec * 16]);
                pd[0] = make_uint2(vd.x, vd.y);
                pd[1] = make_uint2(vd.z, vd.w);
            }
        }
        // dP of token dtk, o = dpo .. dpo + 3: split once into hi / lo bf16,
        // token-major (one 8-byte write each) and o-major copies
        if (dp_on) {
            const uint32_t dw4[4] = {sm.dp.x, sm.dp.y, sm.dp.z, sm.dp.w};
            float hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float v = dpo + q < np ? __uint_as_float(dw4[q]) : 0.f;
                hi[q] = bf16_to_f32(f32_to_bf16(v));
                lo[q] = v - hi[q];
            }
            *reinterpret_cast<uint2*>(&dps_lds[0][dtk * kDpPitch + dpo]) =
                make_uint2(pack_bf16(hi[0], hi[1]), pack_bf16(hi[2], hi[3]));
            *reinterpret_cast<uint2*>(&dps_lds[1][dtk * kDpPitch + dpo]) =
                make_uint2(pack_bf16(lo[0], lo[1]), pack_bf16(lo[2], lo[3]));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                dps_lds[2][(dpo + q) * kDpPitch + dtk] = f32_to_bf16(hi[q]);
                dps_lds[3][(dpo + q) * kDpPitch + dtk] = f32_to_bf16(lo[q]);
            }
        }
        if constexpr (HAS_S) {
            if (tid < TB) s_lds[tid] = __uint_as_float(sm.s);
        }
        if constexpr (QIN) {
            if (tid < NG * TB) q_lds[qg][tid % TB] = (int)sm.q;
        }
    };
    auto read16 = [&](const bf16_t* p) __attribute__((always_inline)) -> u32x4_t {
        const uint4 q = *reinterpret_cast<const uint4*>(p);
        return u32x4_t{q.x, q.y, q.z, q.w};
    };
    auto compute = [&](int cur) __attribute__((always_inline)) {
        if (!wave_on) return;
        const char* xt = x_lds;
        char* dt = dx_lds[cur];
        // dPhi: A = dP^T (o = 16 ot + lr, tokens 8 lg .. + 7), B = x (same tokens, column 16 ct + lr)
        u32x4_t xh[2], xl[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int c = wc0 + 16 * ct + lr;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = VecIO<TX>::scalar(reinterpret_cast<const TX*>(xt + (8 * lg + e) * PITCH) + c);
            if constexpr (sizeof(TX) == 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) xh[ct][e] = pack_bf16(v[2 * e], v[2 * e + 1]);  // exact
            } else {
                split_pack8(v, xh[ct], xl[ct]);
            }
        }
#pragma unroll
        for (int ot = 0; ot < 2; ++ot) {
            const u32x4_t ah = read16(&dps_lds[2][(16 * ot + lr) * kDpPitch + 8 * lg]);
            const u32x4_t al = read16(&dps_lds[3][(16 * ot + lr) * kDpPitch + 8 * lg]);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                accP[ot][ct] = mfma16x16x32(ah, xh[ct], accP[ot][ct]);
                accP[ot][ct] = mfma16x16x32(al, xh[ct], accP[ot][ct]);
                if constexpr (sizeof(TX) == 4) accP[ot][ct] = mfma16x16x32(ah, xl[ct], accP[ot][ct]);
            }
        }
        // dx_proj^T: D[column 16 ct + 4 lg + i][token 16 tt + lr]
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 16 * tt + lr;
            const u32x4_t bh = read16(&dps_lds[0][t * kDpPitch + 8 * lg]);
            const u32x4_t bl = read16(&dps_lds[1][t * kDpPitch + 8 * lg]);
            const float st = HAS_S ? s_lds[t] : 0.f;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                f32x4_t d = f32x4_t{0.f, 0.f, 0.f, 0.f};
                d = mfma16x16x32(phh[ct], bh, d);
                d = mfma16x16x32(phl[ct], bh, d);
                d = mfma16x16x32(phh[ct], bl, d);
                // epilogue: four consecutive columns of token t, in place in the dx tile
                const int c0 = wc0 + 16 * ct + 4 * lg;
                const int boff = t * PITCH + c0 * (int)sizeof(TX);  // 8-byte aligned
                float xv[4], dv[4];
                lds_get4<TX>(xt + boff, xv);
                if constexpr (QIN) {
                    part_unpack4(*reinterpret_cast<const uint2*>(dt + boff), q_lds[c0 / kPartGroup][t], dv);
                } else if constexpr (ACC) {
                    lds_get4<TX>(dt + boff, dv);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) dv[i] = 0.f;
                }
                float o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = d[i] + dv[i] + st * xv[i];
                lds_put4<TX>(dt + boff, o);
            }
        }
    };
    auto store = [&](uint32_t rel, int cur) __attribute__((always_inline)) {  // dx tile -> HBM, 16-byte pieces
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int row = lrow + p * RPP;
            const uint2* ps = reinterpret_cast<const uint2*>(&dx_lds[cur][row * PITCH + lvec * 16]);
            const uint2 u0 = ps[0], u1 = ps[1];
            buf_st16<true>(rs_dx, xo + (rel + p * RPP) * xrow, 0u, make_uint4(u0.x, u0.y, u1.x, u1.y));
        }
    };

    // Fetches and commits past the last row read zeros.  Whole pairs of
    // stages: with an odd count the last one reads only zeros, adds zeros and
    // stores nothing.  An exit between the two would leave a path (seen by
    // the compiler, never taken) from the first stage back to the loop head
    // with its fetch outstanding, and the wait counts would then hold every
    // loop head until that fetch had landed.
    const uint32_t nr = (uint32_t)nrows;
    fetch_small(0u);
    fetch(f0, 0u);
    commit(f0, 0);
    fetch(f1, TB);
    __syncthreads();
    for (uint32_t r0 = 0; r0 < nr; r0 += 2 * TB) {
        // even stage r0 in LDS buffer 0; f1 holds the rows of stage r0 + TB
        fetch_small(r0 + TB);
        fetch(f0, r0 + 2 * TB);
        compute(0);
        __syncthreads();  // the dx tile is complete
        store(r0, 0);
        commit(f1, 1);
        __syncthreads();
        // odd stage r0 + TB in LDS buffer 1; f0 holds the rows of stage r0 + 2 TB
        fetch_small(r0 + 2 * TB);
        fetch(f1, r0 + 3 * TB);
        compute(1);
        __syncthreads();
        store(r0 + TB, 1);
        commit(f0, 0);
        __syncthreads();
    }
    if (!wave_on) return;
    // dPhi partial: accP[ot][ct] register i holds o = 16 ot + 4 lg + i at column 16 ct + lr
    float* out = dphi_part + (int64_t)blockIdx.y * np * K;
#pragma unroll
    for (int ot = 0; ot < 2; ++ot) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = 16 * ot + 4 * lg + i;
                if (o < np) out[(int64_t)o * K + kb0 + wc0 + 16 * ct + lr] = accP[ot][ct][i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
hipError_t launch_phi_split(const float* pre, const float* post, const float* res, int n, int np, int64_t K,
                            bf16_t* phib, hipStream_t s, const void* weight, int w_dtype, int64_t C, float* w32) {
    const int64_t total = (int64_t)proj_tiles(np) * 2 * (K / 32) * 64;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    MHC_LAUNCH_GGL(phi_split_kernel, dim3((unsigned)blocks), dim3(256), 0, s, pre, post, res, n, np, K,
                       reinterpret_cast<uint4*>(phib), weight, w_dtype, C, w32);
    return hipGetLastError();
}

// Tokens per workgroup of the streaming projection (16 MT): 64 above 32
// tokens (two workgroups per CU fit; 128-token workgroups read Phi once per
// 128 tokens but fit one per CU, and measured slower in the one-tile-per-
// wave form: 165 against 129 us at n = 32, 128 tokens), else 32.
static int proj_stream_mt(int64_t B) { return B > 32 ? 4 : 2; }

template <int XPL, int PHI>
static const void* proj_stream_fn(int mt) {
    if (mt == 2) return reinterpret_cast<const void*>(&proj_stream_kernel<XPL, 2, PHI != 0>);
    return reinterpret_cast<const void*>(&proj_stream_kernel<XPL, 4, PHI != 0>);
}

// The streaming projection pays off where Phi outweighs x (np > 128, n >= 16:
// 288 rows at n = 16, 1088 at n = 32); below that the per-tile kernel, whose
// x re-reads are few, is faster.
bool proj_stream_path(int np) { return np > kStreamOB; }

// K splits of the streaming projection: token blocks x output blocks x
// splits fill two rounds of resident workgroups (occupancy of the fp32-x
// kernel, whose LDS stage is the larger), at least two stages per split.
static int proj_stream_ksplit(int64_t B, int64_t K, int np) {
    const int mt = proj_stream_mt(B);
    const int64_t groups0 = ((B + 16 * mt - 1) / (16 * mt)) * ((np + kStreamOB - 1) / kStreamOB);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, proj_stream_fn<3, 0>(mt), 256, 0) != hipSuccess ||
        per_cu < 1) {
        (void)hipGetLastError();
        per_cu = 1;
    }
    // rounded down: a last partial round would leave most CUs idle while it
    // runs; splits x tokens at most 4096 (the partials the coefficient
    // kernel adds per token: 32 splits at 128 tokens, 128 at 32)
    int64_t ks = 2 * (int64_t)device_cu_count() * per_cu / groups0;
    const int64_t kcap = B > 0 ? (4096 + B - 1) / B : 1;
    if (ks > kcap) ks = kcap;
    const int64_t kmax = (K + 2 * kStreamKS - 1) / (2 * kStreamKS);
    if (ks > kmax) ks = kmax;
    if (ks < 1) ks = 1;
    return (int)ks;
}

// K splits so that token blocks x splits x output tiles fill about two
// workgroups per CU, at least 256 columns per split.
int proj_ksplit(int64_t B, int64_t K, int np) {
    if (proj_stream_path(np)) return proj_stream_ksplit(B, K, np);
    const int64_t blocks = ((B + 127) / 128) * proj_tiles(np);
    int64_t ks = (2 * (int64_t)device_cu_count() + blocks - 1) / blocks;
    const int64_t kmax = (K + 2 * kProjKS - 1) / (2 * kProjKS);
    if (ks > kmax) ks = kmax;
    if (ks < 1) ks = 1;
    return (int)ks;
}

hipError_t launch_proj_mfma(int x_dtype, const void* x, const bf16_t* phib, int np, float* p_part, float* ss_part,
                            int64_t B, int64_t K, int ks, hipStream_t s) {
    if (B == 0) return hipSuccess;
    // 32-bit buffer offsets: a 128-row block of fp32 x and the Phi planes
    if (K % 32 != 0 || K > (int64_t(1) << 22) || np < 1) return hipErrorInvalidValue;
    int64_t kchunk = (K + ks - 1) / ks;
    kchunk = ((kchunk + kProjKS - 1) / kProjKS) * kProjKS;
    // grid z = the 32-row output tiles of Phi (tile 0 also stores sum x^2)
    const unsigned tiles = (unsigned)proj_tiles(np);
    const uint4* phif = reinterpret_cast<const uint4*>(phib);
    const int tok = timing_begin("proj", s);
    if (x_dtype == kBF16) {
        constexpr int MT = proj_mt<bf16_t>();
        const dim3 grid((unsigned)((B + 16 * MT - 1) / (16 * MT)), (unsigned)ks, tiles);
        MHC_LAUNCH_GGL((proj_mfma_kernel<bf16_t, MT>), grid, dim3(256), 0, s, (const bf16_t*)x, phif, p_part,
                           ss_part, B, K, kchunk);
    } else {
        constexpr int MT = proj_mt<float>();
        const dim3 grid((unsigned)((B + 16 * MT - 1) / (16 * MT)), (unsigned)ks, tiles);
        MHC_LAUNCH_GGL((proj_mfma_kernel<float, MT>), grid, dim3(256), 0, s, (const float*)x, phif, p_part,
                           ss_part, B, K, kchunk);
    }
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_proj_stream(int x_dtype, const void* x, bf16_raw_t* xplanes, const float* phi_pre,
                              const float* phi_post, const float* phi_res, int n_pre, const bf16_raw_t* phib, int np,
                              float* p_part, float* ss_part, int64_t B, int64_t K, int ks, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (K % 32 != 0 || np <= kProjTile || ks < 1 || (x_dtype == kF32 && !xplanes)) return hipErrorInvalidValue;
    int64_t kchunk = (K + ks - 1) / ks;
    kchunk = ((kchunk + kStreamKS - 1) / kStreamKS) * kStreamKS;
    const int mt = proj_stream_mt(B);
    const int64_t tb = (B + 16 * mt - 1) / (16 * mt);
    const int ob = (np + kStreamOB - 1) / kStreamOB;
    const int64_t groups = tb * ks;
    const dim3 grid((unsigned)(((groups + 7) / 8) * 8 * ob));
    const int tok = timing_begin("proj", s);
    const bf16_t* xp = reinterpret_cast<const bf16_t*>(x);
    if (x_dtype == kF32) {
        MHC_LAUNCH_GGL(proj_xsplit_kernel, dim3((unsigned)(B * ks)), dim3(256), 0, s, (const float*)x,
                           reinterpret_cast<uint4*>(xplanes), ss_part, B, K, kchunk, ks);
        xp = reinterpret_cast<const bf16_t*>(xplanes);
    }
    const uint4* phif = reinterpret_cast<const uint4*>(phib);
#define MHC_STREAM(XPL_, MT_)                                                                                   \
    if (phib) {                                                                                                 \
        MHC_LAUNCH_GGL((proj_stream_kernel<XPL_, MT_, true>), grid, dim3(256), 0, s, xp, phi_pre, phi_post,   \
                           phi_res, n_pre, phif, np, p_part, ss_part, B, K, kchunk, ks, ob, groups,              \
                           (const bf16_t*)nullptr, 0);                                                          \
    } else {                                                                                                    \
        MHC_LAUNCH_GGL((proj_stream_kernel<XPL_, MT_, false>), grid, dim3(256), 0, s, xp, phi_pre, phi_post,  \
                           phi_res, n_pre, phif, np, p_part, ss_part, B, K, kchunk, ks, ob, groups,              \
                           (const bf16_t*)nullptr, 0);                                                          \
    }
#define MHC_STREAM_MT(XPL_)                               \
    if (mt == 2) {                                        \
        MHC_STREAM(XPL_, 2);                              \
    } else {                                              \
        MHC_STREAM(XPL_, 4);                              \
    }
    if (x_dtype == kF32) {
        MHC_STREAM_MT(3);
    } else {
        MHC_STREAM_MT(1);
    }
#undef MHC_STREAM_MT
#undef MHC_STREAM
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_proj_stream_wrap(bool decay, const void* res, const void* br, int64_t Cw, const bf16_raw_t* phib,
                                   int np, float* p_part, float* ss_part, int64_t B, int64_t K, int ks,
                                   hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (K % 32 != 0 || np <= kProjTile || ks < 1 || !phib || Cw < kStreamKS || Cw % kStreamKS != 0 ||
        K % Cw != 0 || K > (int64_t(1) << 22))
        return hipErrorInvalidValue;
    int64_t kchunk = (K + ks - 1) / ks;
    kchunk = ((kchunk + kStreamKS - 1) / kStreamKS) * kStreamKS;
    const int mt = proj_stream_mt(B);
    const int64_t tb = (B + 16 * mt - 1) / (16 * mt);
    const int ob = (np + kStreamOB - 1) / kStreamOB;
    const int64_t groups = tb * ks;
    const dim3 grid((unsigned)(((groups + 7) / 8) * 8 * ob));
    const int tok = timing_begin("proj", s);
    const bf16_t* rp = reinterpret_cast<const bf16_t*>(res);
    const bf16_t* bp = reinterpret_cast<const bf16_t*>(br);
    const uint4* phif = reinterpret_cast<const uint4*>(phib);
    const int Ci = (int)Cw;
#define MHC_STREAM_W(MT_, W_)                                                                                     \
    MHC_LAUNCH_GGL((proj_stream_kernel<1, MT_, true, W_>), grid, dim3(256), 0, s, rp, nullptr, nullptr, nullptr, 0, \
                   phif, np, p_part, ss_part, B, K, kchunk, ks, ob, groups, bp, Ci)
    if (mt == 2) {
        if (decay) { MHC_STREAM_W(2, 1); } else { MHC_STREAM_W(2, 2); }
    } else {
        if (decay) { MHC_STREAM_W(4, 1); } else { MHC_STREAM_W(4, 2); }
    }
#undef MHC_STREAM_W
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_proj_reduce(const float* p_part, int ks, int64_t B, int np, float* out, hipStream_t s) {
    const int64_t total = B * np;
    if (total == 0) return hipSuccess;
    MHC_LAUNCH_GGL(proj_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, p_part, ks, B, np,
                       out);
    return hipGetLastError();
}

#ifdef MHC_KERNEL_TIMING
// ---------------------------------------------------------------------------
// VALU projection (the benchmark build only, for the A/B against
// proj_mfma_kernel): the same P and sum-x^2 partials from fp32 FMAs.  One
// token per lane; the rows Phi^T[k][0..31] are the same for every lane and
// come through scalar loads; x is staged through LDS in 32-k slices with
// coalesced 16-byte loads.  NP FMAs and one square per element of x.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void phi_t_kernel(const float* __restrict__ phi, int np, int64_t K,
                                                    float* __restrict__ phit) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over K x 32
    if (i >= K * 32) return;
    const int64_t k = i >> 5;
    const int o = (int)(i & 31);
    phit[i] = o < np ? phi[(int64_t)o * K + k] : 0.f;
}

constexpr int kValuTB = 256;  // tokens per workgroup
constexpr int kValuKC = 32;   // k per stage

template <typename TX, int NP>
__global__ __launch_bounds__(256) void proj_valu_kernel(const TX* __restrict__ x, const float* __restrict__ phit,
                                                        float* __restrict__ p_part, float* __restrict__ ss_part,
                                                        int64_t B, int64_t K, int64_t kchunk) {
    constexpr int EPV = 16 / (int)sizeof(TX);
    constexpr int VPR = kValuKC / EPV;
    constexpr int PITCH = kValuKC * (int)sizeof(TX) + 16;
    __shared__ __align__(16) char xs[kValuTB * PITCH];
    const int tid = threadIdx.x;
    const int64_t tok0 = (int64_t)blockIdx.x * kValuTB;
    const int64_t ks = blockIdx.y;
    const int64_t kb = ks * kchunk;
    const int64_t ke = kb + kchunk < K ? kb + kchunk : K;
    float acc[NP];
#pragma unroll
    for (int o = 0; o < NP; ++o) acc[o] = 0.f;
    float ss = 0.f;
    for (int64_t k0 = kb; k0 < ke; k0 += kValuKC) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < VPR; ++i) {
            const int p = tid + 256 * i;
            const int row = p / VPR;
            const int vec = p % VPR;
            const int64_t tok = tok0 + row;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (tok < B) v = *reinterpret_cast<const uint4*>(x + tok * K + k0 + vec * EPV);
            *reinterpret_cast<uint4*>(&xs[row * PITCH + vec * 16]) = v;
        }
        __syncthreads();
        const float* ph = phit + k0 * 32;
#pragma unroll
        for (int v = 0; v < VPR; ++v) {
            const uint4 q = *reinterpret_cast<const uint4*>(&xs[tid * PITCH + v * 16]);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
            float xv[EPV];
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                if constexpr (sizeof(TX) == 2) {
                    xv[e] = __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
                } else {
                    xv[e] = __uint_as_float(w[e]);
                }
            }
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const float* pr = ph + (v * EPV + e) * 32;
                ss = fmaf(xv[e], xv[e], ss);
#pragma unroll
                for (int o = 0; o < NP; ++o) acc[o] = fmaf(xv[e], pr[o], acc[o]);
            }
        }
    }
    const int64_t tok = tok0 + tid;
    if (tok < B) {
        float4* out = reinterpret_cast<float4*>(p_part + (ks * B + tok) * kNPad);
#pragma unroll
        for (int o = 0; o < kNPad; o += 4) {
            out[o / 4] = make_float4(o < NP ? acc[o < NP ? o : 0] : 0.f, o + 1 < NP ? acc[o + 1 < NP ? o + 1 : 0] : 0.f,
                                     o + 2 < NP ? acc[o + 2 < NP ? o + 2 : 0] : 0.f,
                                     o + 3 < NP ? acc[o + 3 < NP ? o + 3 : 0] : 0.f);
        }
        ss_part[ks * B + tok] = ss;
    }
}

int proj_valu_ksplit(int64_t B, int64_t K) {
    const int64_t tb = (B + kValuTB - 1) / kValuTB;
    int64_t ks = (4 * (int64_t)device_cu_count() + tb - 1) / tb;
    const int64_t kmax = K / kValuKC;
    if (ks > kmax) ks = kmax;
    return (int)(ks < 1 ? 1 : ks);
}

hipError_t launch_proj_valu(int x_dtype, const void* x, const float* phi, int np, float* phit, float* p_part,
                            float* ss_part, int64_t B, int64_t K, int ks, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (K % kValuKC != 0 || np < 1 || np > kNPad || ks < 1) return hipErrorInvalidValue;
    MHC_LAUNCH_GGL(phi_t_kernel, dim3((unsigned)((K * 32 + 255) / 256)), dim3(256), 0, s, phi, np, K, phit);
    int64_t kchunk = (K + ks - 1) / ks;
    kchunk = ((kchunk + kValuKC - 1) / kValuKC) * kValuKC;
    const dim3 grid((unsigned)((B + kValuTB - 1) / kValuTB), (unsigned)ks);
    const int tok = timing_begin("proj_valu", s);
#define MHC_VALU(TX_, NP_) \
    MHC_LAUNCH_GGL((proj_valu_kernel<TX_, NP_>), grid, dim3(256), 0, s, (const TX_*)x, phit, p_part, ss_part, B, K, kchunk)
    if (x_dtype == kBF16) {
        if (np <= 8) { MHC_VALU(bf16_t, 8); } else if (np <= 24) { MHC_VALU(bf16_t, 24); } else { MHC_VALU(bf16_t, 32); }
    } else {
        if (np <= 8) { MHC_VALU(float, 8); } else if (np <= 24) { MHC_VALU(float, 24); } else { MHC_VALU(float, 32); }
    }
#undef MHC_VALU
    timing_end(tok, s);
    return hipGetLastError();
}
#endif  // MHC_KERNEL_TIMING

#define MHC_DYN_N(n, ...)                                        \
    switch (n) {                                                 \
        case 2: { constexpr int N_ = 2; __VA_ARGS__; break; }    \
        case 4: { constexpr int N_ = 4; __VA_ARGS__; break; }    \
        case 8: { constexpr int N_ = 8; __VA_ARGS__; break; }    \
        case 16: { constexpr int N_ = 16; __VA_ARGS__; break; }  \
        case 32: { constexpr int N_ = 32; __VA_ARGS__; break; }  \
        default: return hipErrorInvalidValue;                    \
    }

hipError_t launch_dyn_coef_fwd(int n, const float* p_part, const float* ss_part, int ks, int64_t B, int64_t K,
                               const float* a_pre, const float* a_post, const float* a_res, const float* b_pre,
                               const float* b_post, const float* b_res, float* coef, float* p_out, float* rh,
                               int iters, float sk_eps, float rms_eps, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (generic_layer_n(n)) {
#define MHC_DCG_FWD(NM_)                                                                                          \
    MHC_LAUNCH_GGL((dyn_coef_gen_fwd_kernel<NM_>), dim3((unsigned)((B * NM_ + 255) / 256)), dim3(256), 0, s,     \
                       p_part, ss_part, ks, B, K, a_pre, a_post, a_res, b_pre, b_post, b_res, coef, p_out, rh, n,   \
                       iters, sk_eps, rms_eps)
        if (n <= 16) { MHC_DCG_FWD(16); } else if (n <= 32) { MHC_DCG_FWD(32); } else { MHC_DCG_FWD(64); }
#undef MHC_DCG_FWD
        return hipGetLastError();
    }
    if (n == 4) {
        MHC_LAUNCH_GGL(dyn_coef16_fwd_kernel, dim3((unsigned)((B * 16 + 255) / 256)), dim3(256), 0, s, p_part,
                           ss_part, ks, B, K, a_pre, a_post, a_res, b_pre, b_post, b_res, coef, p_out, rh, iters,
                           sk_eps, rms_eps);
        return hipGetLastError();
    }
    if (n == skb::kN) {
        MHC_LAUNCH_GGL(dyn_coef32_fwd_kernel, dim3((unsigned)B), dim3(skb::kThreads), 0, s, p_part, ss_part, ks, B,
                           K, a_pre, a_post, a_res, b_pre, b_post, b_res, coef, p_out, rh, iters, sk_eps, rms_eps);
        return hipGetLastError();
    }
    const int64_t threads = B * pow2ceil(n);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    MHC_DYN_N(n, MHC_LAUNCH_GGL((dyn_coef_fwd_kernel<N_>), dim3(blocks), dim3(256), 0, s, p_part, ss_part, ks, B,
                                    K, a_pre, a_post, a_res, b_pre, b_post, b_res, coef, p_out, rh, iters, sk_eps,
                                    rms_eps));
    return hipGetLastError();
}

// Rows of the db / dalpha partials: one per workgroup, or one per token for
// n >= 16 and for the generic-n kernel.
int dyn_coef_bwd_blocks(int n, int64_t B) {
    if (n == 4) return dyn_coef16_bwd_blocks(B);
    if (n >= 16 || generic_layer_n(n)) return (int)(B < 1 ? 1 : B);
    return (int)((B * pow2ceil(n) + 255) / 256);
}

// Lane groups (token slots) of the n >= 16 coefficient backward: a whole
// number of 256-lane workgroups, at most one slot per token, as many as fit
// kSkHistBytes of history; 0 if not even one workgroup's slots fit.
int dyn_coef_bwd_hist_slots(int n, int64_t B, int iters) {
    if (n < 16 || generic_layer_n(n)) return 0;
    const int per_wg = 256 / n;
    const int64_t slot_bytes = (int64_t)(iters > 0 ? iters : 1) * (n + 1) * n * (int64_t)sizeof(float);
    const int64_t fit_wgs = (int64_t)kSkHistBytes / slot_bytes / per_wg;
    int64_t wgs = (B + per_wg - 1) / per_wg;
    if (wgs > fit_wgs) wgs = fit_wgs;
    if (wgs < 1) return fit_wgs < 1 ? 0 : per_wg;
    return (int)(wgs * per_wg);
}

// Generic n: the coefficient backward's lane-group width, and the workgroups
// of token slots whose Sinkhorn history fits the region the dynamic
// backward's workspace reserves (dyn_coef_gen_hist_bytes; 0: none fit).
static int dyn_coef_gen_nm(int n) { return n <= 16 ? 16 : (n <= 32 ? 32 : 64); }
constexpr int kGenHistIters = 20;  // iterations the reserved region is sized for

size_t dyn_coef_gen_hist_bytes(int n, int64_t B) {
    if (!generic_layer_n(n) || B <= 0) return 0;
    const int nm = dyn_coef_gen_nm(n), per_wg = 256 / nm;
    const int64_t wgs = (B + per_wg - 1) / per_wg;
    const size_t need = (size_t)wgs * per_wg * (size_t)skw_hist_floats(nm, n, kGenHistIters) * sizeof(float);
    return need < kSkHistBytes ? need : kSkHistBytes;
}

static int64_t dyn_coef_gen_hist_wgs(int n, int64_t B, int iters) {
    const int nm = dyn_coef_gen_nm(n), per_wg = 256 / nm;
    const int64_t slot_bytes = skw_hist_floats(nm, n, iters) * (int64_t)sizeof(float);
    if (slot_bytes <= 0) return 0;
    const int64_t fit = (int64_t)dyn_coef_gen_hist_bytes(n, B) / slot_bytes / per_wg;
    const int64_t wgs = (B + per_wg - 1) / per_wg;
    return wgs < fit ? wgs : fit;
}

hipError_t launch_dyn_coef_bwd(int n, const float* scal, const float* coef, const float* p, const float* rh,
                               int64_t B, int64_t K, const float* a_pre, const float* a_post, const float* a_res,
                               const float* b_res, float* dp_out, float* s_out, float* part, int iters, float sk_eps,
                               float* hist, hipStream_t s, bool res_rows) {
    if (B == 0) return hipSuccess;
    if (generic_layer_n(n)) {
        // one token per lane group, or (history in hist) as many token slots
        // as the history region holds, each taking several tokens
        const int nm = dyn_coef_gen_nm(n);
        int64_t blocks = (B * nm + 255) / 256;
        float* h = nullptr;
        if (res_rows && hist && iters > 0) {
            const int64_t wgs = dyn_coef_gen_hist_wgs(n, B, iters);
            if (wgs >= 1) {
                blocks = wgs;
                h = hist;
            }
        }
        if (blocks > 0x7fffffff) return hipErrorInvalidValue;
#define MHC_DCG_BWD(NM_, RES_)                                                                                     \
    MHC_LAUNCH_GGL((dyn_coef_gen_bwd_kernel<NM_, RES_>), dim3((unsigned)blocks), dim3(256), 0, s, scal, coef, p, rh, \
                       B, K, a_pre, a_post, a_res, b_res, dp_out, s_out, part, n, iters, sk_eps, h)
        if (res_rows) {
            if (nm == 16) { MHC_DCG_BWD(16, true); } else if (nm == 32) { MHC_DCG_BWD(32, true); } else { MHC_DCG_BWD(64, true); }
        } else {
            if (nm == 16) { MHC_DCG_BWD(16, false); } else if (nm == 32) { MHC_DCG_BWD(32, false); } else { MHC_DCG_BWD(64, false); }
        }
#undef MHC_DCG_BWD
        return hipGetLastError();
    }
    const unsigned blocks = (unsigned)dyn_coef_bwd_blocks(n, B);
    if (n == 4) {
        if (res_rows) {
            MHC_LAUNCH_GGL(dyn_coef16_bwd_kernel<true>, dim3(blocks), dim3(256), 0, s, scal, coef, p, rh, B, K, a_pre,
                               a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps);
        } else {
            MHC_LAUNCH_GGL(dyn_coef16_bwd_kernel<false>, dim3(blocks), dim3(256), 0, s, scal, coef, p, rh, B, K,
                               a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps);
        }
        return hipGetLastError();
    }
    if (!res_rows && n >= 16) {
        // no adjoint runs: the run-time-n kernel on n-lane groups
        const int64_t gblocks = (B * n + 255) / 256;
        if (gblocks > 0x7fffffff) return hipErrorInvalidValue;
        if (n == 16) {
            MHC_LAUNCH_GGL((dyn_coef_gen_bwd_kernel<16, false>), dim3((unsigned)gblocks), dim3(256), 0, s, scal, coef,
                               p, rh, B, K, a_pre, a_post, a_res, b_res, dp_out, s_out, part, n, iters, sk_eps,
                               (float*)nullptr);
        } else if (n == 32) {
            MHC_LAUNCH_GGL((dyn_coef_gen_bwd_kernel<32, false>), dim3((unsigned)gblocks), dim3(256), 0, s, scal, coef,
                               p, rh, B, K, a_pre, a_post, a_res, b_res, dp_out, s_out, part, n, iters, sk_eps,
                               (float*)nullptr);
        } else {
            return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (!res_rows && (n == 2 || n == 8)) {
        if (n == 2) {
            MHC_LAUNCH_GGL((dyn_coef_bwd_kernel<2, false>), dim3(blocks), dim3(256), 0, s, scal, coef, p, rh, B, K,
                               a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps);
        } else {
            MHC_LAUNCH_GGL((dyn_coef_bwd_kernel<8, false>), dim3(blocks), dim3(256), 0, s, scal, coef, p, rh, B, K,
                               a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps);
        }
        return hipGetLastError();
    }
    if (!res_rows) return hipErrorInvalidValue;
    if (n == skb::kN && iters <= skb::kTMax) {
        MHC_LAUNCH_GGL(dyn_coef32_bwd_kernel, dim3((unsigned)B), dim3(skb::kThreads), 0, s, scal, coef, p, rh, B, K,
                           a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps);
        return hipGetLastError();
    }
    if (n >= 16) {
        const int slots = dyn_coef_bwd_hist_slots(n, B, iters);
        if (!hist || slots < 1) return hipErrorInvalidValue;
        const unsigned wblocks = (unsigned)slots * n / 256;
        if (n == 16) {
            MHC_LAUNCH_GGL((dyn_coef_bwd_wide_kernel<16>), dim3(wblocks), dim3(256), 0, s, scal, coef, p, rh, B, K,
                               a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps, hist);
        } else if (n == 32) {
            MHC_LAUNCH_GGL((dyn_coef_bwd_wide_kernel<32>), dim3(wblocks), dim3(256), 0, s, scal, coef, p, rh, B, K,
                               a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps, hist);
        } else {
            return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (n) {
        case 2: MHC_LAUNCH_GGL((dyn_coef_bwd_kernel<2>), dim3(blocks), dim3(256), 0, s, scal, coef, p, rh, B, K,
                                   a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps); break;
        case 8: MHC_LAUNCH_GGL((dyn_coef_bwd_kernel<8>), dim3(blocks), dim3(256), 0, s, scal, coef, p, rh, B, K,
                                   a_pre, a_post, a_res, b_res, dp_out, s_out, part, iters, sk_eps); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_small_column_sum(const float* part, int rows, int cols, float* out_db, float* out_da, int np,
                                   hipStream_t s) {
    MHC_LAUNCH_GGL(small_column_sum_kernel, dim3((unsigned)((cols + 31) / 32)), dim3(1024), 0, s, part, rows, cols,
                       out_db, out_da, np);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Projection backward over many 32-row output tiles (2n + n^2 > 32 rows:
// n >= 8), fp32 x and dx (bf16 x is upcast before it gets here), for
// batches up to kProjWideMaxB tokens.  The per-tile kernel above would read
// x and dx once per tile (34 times at n = 32); instead, up to 128 rows the
// two small-np kernels below, and above that:
//   dp_split_kernel + proj_bwd_dx2_kernel: dP split into hi / lo planes
//     once; one workgroup per 128 columns x up to 128 tokens loops over the
//     output tiles, dx_proj^T accumulating in MFMA registers (A = Phi^T,
//     split in registers, B = the dP planes through LDS); then one epilogue
//     dx = dx_proj + (ACC ? dx : 0) + s x.
//   dp_tsplit_kernel + x_tsplit_kernel + proj_bwd_dphi_kernel: dP and x
//     split once into transposed hi / lo planes (tokens contiguous); one
//     workgroup per 128 output rows x 128 columns walks all tokens,
//     dPhi = dP^T x in MFMA registers, and stores its rows of dPhi directly
//     (no partials, no column sums).  The row blocks of one column block get
//     ids on one XCD, so they share those x columns through its L2.
// Operands are split hi / lo (hi.hi + lo.hi + hi.lo, as above).
// ---------------------------------------------------------------------------
constexpr int kProjWideMaxB = 1024;

// ---------------------------------------------------------------------------
// Up to 128 output rows (n = 8: 80), where the all-tiles kernels below would
// have few workgroups: dx from one workgroup per 128 columns x 32 tokens
// looping over the output tiles (A = Phi^T, the next tile's values loaded
// while the current one computes, split hi / lo in registers; B = dP^T read
// straight from dP and split), and dPhi from one workgroup per 64 output
// rows x 128 columns walking all tokens in 32-token stages (dP^T and x
// split in registers).  The token blocks (row blocks) of one column block
// run on one XCD and share Phi (those x columns) through its L2.
// ---------------------------------------------------------------------------
// 8 consecutive fp32 (32-byte aligned) as two 16-byte loads
__device__ __forceinline__ void ld8f(const float* p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <bool ACC, bool HAS_S>
__global__ __launch_bounds__(256) void proj_bwd_dx_small_kernel(
    const float* __restrict__ x, const float* __restrict__ dP, int dp_stride, const float* __restrict__ s_tok,
    const float* __restrict__ phi_pre, const float* __restrict__ phi_post, const float* __restrict__ phi_res,
    int n_pre, int np, float* __restrict__ dx, int64_t B, int64_t K) {
    constexpr int CB = 128;
    constexpr int TS = 1;  // 32-token stages per workgroup
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    // Workgroups go round-robin over the 8 XCDs by linear id; the token
    // blocks of one column block are given ids on the same XCD, one after
    // another, so they share that column block's Phi in the XCD's L2.
    const int64_t tblocks = (B + 32 * TS - 1) / (32 * TS);
    const int64_t lin = blockIdx.x;
    const int64_t idx = lin / 8;
    const int64_t cb = (idx / tblocks) * 8 + lin % 8;
    const int64_t kb0 = cb * CB + wave * 32;  // this wave's 32 columns
    if (kb0 >= K) return;  // padding ids, and K % 32 == 0: whole waves are in or out
    const int64_t tb0 = (idx % tblocks) * (32 * TS);
    f32x4_t d[TS][2][2];
#pragma unroll
    for (int st = 0; st < TS; ++st) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) d[st][tt][ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
    }
    // dP columns are read 8 at a time: a stride that is a multiple of 8
    // allows the aligned 16-byte loads (the layer's dP rows are)
    const bool dp_vec = (dp_stride % 8) == 0;
    // A = Phi^T: Phi[o0 + 8 lg + e][column 16 ct + lr]; the next tile's
    // values are loaded while the current tile is on the matrix cores
    float pv[2][8];
    auto load_phi = [&](int o0) __attribute__((always_inline)) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int o = o0 + 8 * lg + e;
                pv[ct][e] = o < np ? phi_row(phi_pre, phi_post, phi_res, n_pre, o, K)[kb0 + 16 * ct + lr] : 0.f;
            }
        }
    };
    load_phi(0);
    for (int o0 = 0; o0 < np; o0 += 32) {
        u32x4_t phh[2], phl[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) split_pack8(pv[ct], phh[ct], phl[ct]);
        if (o0 + 32 < np) load_phi(o0 + 32);
#pragma unroll
        for (int st = 0; st < TS; ++st) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                // B = dP^T: dP[token 16 tt + lr][o0 + 8 lg .. + 7]
                const int64_t t = tb0 + 32 * st + 16 * tt + lr;
                float v[8];
                const int ob = o0 + 8 * lg;
                if (t < B && dp_vec && ob + 8 <= np) {
                    ld8f(dP + t * dp_stride + ob, v);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = (t < B && ob + e < np) ? dP[t * dp_stride + ob + e] : 0.f;
                }
                u32x4_t bh, bl;
                split_pack8(v, bh, bl);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    d[st][tt][ct] = mfma16x16x32(phh[ct], bh, d[st][tt][ct]);
                    d[st][tt][ct] = mfma16x16x32(phl[ct], bh, d[st][tt][ct]);
                    d[st][tt][ct] = mfma16x16x32(phh[ct], bl, d[st][tt][ct]);
                }
            }
        }
    }
    // D[column 16 ct + 4 lg + i][token 16 tt + lr]: four consecutive columns of one token
#pragma unroll
    for (int st = 0; st < TS; ++st) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int64_t t = tb0 + 32 * st + 16 * tt + lr;
            if (t >= B) continue;
            const float sv = HAS_S ? s_tok[t] : 0.f;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const int64_t off = t * K + kb0 + 16 * ct + 4 * lg;
                float4 o = make_float4(d[st][tt][ct][0], d[st][tt][ct][1], d[st][tt][ct][2], d[st][tt][ct][3]);
                if constexpr (ACC) {
                    const float4 a = *reinterpret_cast<const float4*>(dx + off);
                    o.x += a.x; o.y += a.y; o.z += a.z; o.w += a.w;
                }
                if constexpr (HAS_S) {
                    const float4 xv = *reinterpret_cast<const float4*>(x + off);
                    o.x += sv * xv.x; o.y += sv * xv.y; o.z += sv * xv.z; o.w += sv * xv.w;
                }
                *reinterpret_cast<float4*>(dx + off) = o;
            }
        }
    }
}

constexpr int kDphiSmallRows = 64;  // output rows (two 32-row tiles) per workgroup

__global__ __launch_bounds__(256) void proj_bwd_dphi_small_kernel(const float* __restrict__ x, const float* __restrict__ dP,
                                                            int dp_stride, int np, float* __restrict__ dphi,
                                                            int64_t B, int64_t K) {
    constexpr int CB = 128;
    constexpr int OT = kDphiSmallRows / 16;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    // the row blocks of one column block on one XCD (as in proj_bwd_dx_small_kernel)
    const int64_t rblocks = (np + kDphiSmallRows - 1) / kDphiSmallRows;
    const int64_t lin = blockIdx.x;
    const int64_t idx = lin / 8;
    const int o0 = (int)(idx % rblocks) * kDphiSmallRows;
    const int64_t kb0 = ((idx / rblocks) * 8 + lin % 8) * CB + wave * 32;
    if (kb0 >= K) return;
    f32x4_t acc[OT][2];
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) acc[ot][ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    for (int64_t t0 = 0; t0 < B; t0 += 32) {
        // A = dP^T: rows o = o0 + 16 ot + lr, tokens t0 + 8 lg + e
        u32x4_t ah[OT], al[OT];
#pragma unroll
        for (int ot = 0; ot < OT; ++ot) {
            const int o = o0 + 16 * ot + lr;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t t = t0 + 8 * lg + e;
                v[e] = (t < B && o < np) ? dP[t * dp_stride + o] : 0.f;
            }
            split_pack8(v, ah[ot], al[ot]);
        }
        // B = x: tokens t0 + 8 lg + e, column 16 ct + lr
        u32x4_t xh[2], xl[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t t = t0 + 8 * lg + e;
                v[e] = t < B ? x[t * K + kb0 + 16 * ct + lr] : 0.f;
            }
            split_pack8(v, xh[ct], xl[ct]);
        }
#pragma unroll
        for (int ot = 0; ot < OT; ++ot) {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                acc[ot][ct] = mfma16x16x32(ah[ot], xh[ct], acc[ot][ct]);
                acc[ot][ct] = mfma16x16x32(al[ot], xh[ct], acc[ot][ct]);
                acc[ot][ct] = mfma16x16x32(ah[ot], xl[ct], acc[ot][ct]);
            }
        }
    }
    // D[o 16 ot + 4 lg + i][column 16 ct + lr]
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = o0 + 16 * ot + 4 * lg + i;
            if (o >= np) continue;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) dphi[(int64_t)o * K + kb0 + 16 * ct + lr] = acc[ot][ct][i];
        }
    }
}

// dP [B][stride] (np valid columns) -> bf16 planes hi / lo [B][np32]
// (np32 = np rounded up to 32, zero past np): 8 consecutive outputs of a
// token are one 16-byte piece, the B-operand fragment of proj_bwd_dx2_kernel.
__global__ __launch_bounds__(256) void dp_split_kernel(const float* __restrict__ dP, int stride, int np, int np32,
                                                       int64_t B, uint4* __restrict__ dph, uint4* __restrict__ dpl) {
    const int64_t per_row = np32 / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * per_row) return;
    const int64_t t = i / per_row;
    const int o0 = (int)(i % per_row) * 8;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = o0 + e < np ? dP[t * stride + o0 + e] : 0.f;
    u32x4_t h, l;
    split_pack8(v, h, l);
    dph[i] = make_uint4(h[0], h[1], h[2], h[3]);
    dpl[i] = make_uint4(l[0], l[1], l[2], l[3]);
}

// dx over all output tiles, one workgroup per 128 columns x up to 128
// tokens (token blocks of one column block on one XCD, sharing that column
// block's Phi in its L2): wave w owns columns 32 w .. 32 w + 31 (two
// 16-column MFMA tiles ct) for all the workgroup's tokens, so every Phi
// element is loaded and split hi / lo once per token block.  The 32-output
// tile's dP planes (hi, lo: 16 KB for 128 tokens) go through LDS, shared by
// the four waves, double-buffered; the Phi fragments (A = Phi^T: 8 outputs
// of one column per lane, two tiles) are loaded two output tiles ahead.
// Products hi.hi + lo.hi + hi.lo (as proj_bwd_mfma_kernel); then
// dx = dx_proj + (ACC ? dx : 0) + (HAS_S ? s x : 0).
constexpr int kDx2Tok = 128;                 // tokens per workgroup
constexpr int kDx2Pitch = 64 + 16;           // bytes per token row of one dP plane tile in LDS

template <bool ACC, bool HAS_S>
__global__ __launch_bounds__(256) void proj_bwd_dx2_kernel(
    const float* __restrict__ x, const uint4* __restrict__ dph, const uint4* __restrict__ dpl, int np32,
    const float* __restrict__ s_tok, const float* __restrict__ phi_pre, const float* __restrict__ phi_post,
    const float* __restrict__ phi_res, int n_pre, int np, float* __restrict__ dx, int64_t B, int64_t K) {
    constexpr int CB = 128;
    constexpr int TT = kDx2Tok / 16;
    constexpr int PITCH = kDx2Pitch;
    __shared__ __align__(16) char dps[2][2][kDx2Tok * PITCH];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int64_t tblocks = (B + kDx2Tok - 1) / kDx2Tok;
    const int64_t cblocks = (K + CB - 1) / CB;
    const int64_t lin = blockIdx.x;
    const int64_t idx = lin / 8;
    const int64_t cb = (idx / tblocks) * 8 + lin % 8;
    if (cb >= cblocks) return;  // padding ids: the whole workgroup
    const int64_t tok0 = (idx % tblocks) * kDx2Tok;
    const int64_t kb0 = cb * CB + wave * 32;
    const bool wave_on = kb0 < K;  // K % 32 == 0: whole waves are in or out
    const int tiles = np32 / 32;
    const int64_t prow = np32 / 8;  // 16-byte pieces per token row of a plane

    f32x4_t d[TT][2];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        d[tt][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        d[tt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    // dP planes of output tile ot: piece i = tid + 256 u = (plane, token, 16-byte column)
    auto fetch_dp = [&](uint4 (&f)[4], int ot) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = threadIdx.x + 256 * u;
            const int pl = i / (kDx2Tok * 4);
            const int r = (i / 4) % kDx2Tok;
            const int c = i % 4;
            const int64_t t = tok0 + r;
            const uint4* src = pl == 0 ? dph : dpl;
            f[u] = (t < B && ot < tiles) ? src[t * prow + ot * 4 + c] : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto commit = [&](const uint4 (&f)[4], int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = threadIdx.x + 256 * u;
            const int pl = i / (kDx2Tok * 4);
            const int r = (i / 4) % kDx2Tok;
            const int c = i % 4;
            *reinterpret_cast<uint4*>(&dps[buf][pl][r * PITCH + 16 * c]) = f[u];
        }
    };
    // A = Phi^T fragments of output tile ot: Phi[32 ot + 8 lg + e][kb0 + 16 ct + lr]
    struct PhiTile {
        float v[2][8];
    };
    auto fetch_phi = [&](PhiTile& pt, int ot) __attribute__((always_inline)) {
        const int64_t col = wave_on ? kb0 + lr : 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int o = 32 * ot + 8 * lg + e;
            const bool ov = o < np;
            const float* pr = phi_row(phi_pre, phi_post, phi_res, n_pre, ov ? o : np - 1, K) + col;
            const float a = pr[0], b = pr[16];
            pt.v[0][e] = ov ? a : 0.f;
            pt.v[1][e] = ov ? b : 0.f;
        }
    };
    auto tile_step = [&](int ot, const PhiTile& cur, PhiTile& ahead, uint4 (&f)[4]) __attribute__((always_inline)) {
        const int buf = ot & 1;
        if (ot + 1 < tiles) fetch_dp(f, ot + 1);
        fetch_phi(ahead, ot + 2 < tiles ? ot + 2 : tiles - 1);
        if (wave_on) {
            u32x4_t ah[2], al[2];
            split_pack8(cur.v[0], ah[0], al[0]);
            split_pack8(cur.v[1], ah[1], al[1]);
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                const uint4 qh = *reinterpret_cast<const uint4*>(&dps[buf][0][(16 * tt + lr) * PITCH + 16 * lg]);
                const uint4 ql = *reinterpret_cast<const uint4*>(&dps[buf][1][(16 * tt + lr) * PITCH + 16 * lg]);
                const u32x4_t bh = u32x4_t{qh.x, qh.y, qh.z, qh.w};
                const u32x4_t bl = u32x4_t{ql.x, ql.y, ql.z, ql.w};
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    d[tt][ct] = mfma16x16x32(ah[ct], bh, d[tt][ct]);
                    d[tt][ct] = mfma16x16x32(al[ct], bh, d[tt][ct]);
                    d[tt][ct] = mfma16x16x32(ah[ct], bl, d[tt][ct]);
                }
            }
        }
        if (ot + 1 < tiles) commit(f, buf ^ 1);
        __syncthreads();
    };
    {
        uint4 f[4];
        PhiTile p0, p1, p2;
        fetch_dp(f, 0);
        fetch_phi(p0, 0);
        fetch_phi(p1, tiles > 1 ? 1 : 0);
        commit(f, 0);
        __syncthreads();
        int ot = 0;
        for (; ot + 3 <= tiles; ot += 3) {
            tile_step(ot, p0, p2, f);
            tile_step(ot + 1, p1, p0, f);
            tile_step(ot + 2, p2, p1, f);
        }
        if (ot < tiles) tile_step(ot, p0, p2, f);
        if (ot + 1 < tiles) tile_step(ot + 1, p1, p0, f);
    }
    if (!wave_on) return;
    // D[column 16 ct + 4 lg + i][token 16 tt + lr]: four consecutive columns of one token
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        const int64_t t = tok0 + 16 * tt + lr;
        if (t >= B) continue;
        const float sv = HAS_S ? s_tok[t] : 0.f;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int64_t off = t * K + kb0 + 16 * ct + 4 * lg;
            float4 o = make_float4(d[tt][ct][0], d[tt][ct][1], d[tt][ct][2], d[tt][ct][3]);
            if constexpr (ACC) {
                const float4 a = *reinterpret_cast<const float4*>(dx + off);
                o.x += a.x; o.y += a.y; o.z += a.z; o.w += a.w;
            }
            if constexpr (HAS_S) {
                const float4 xv = *reinterpret_cast<const float4*>(x + off);
                o.x += sv * xv.x; o.y += sv * xv.y; o.z += sv * xv.z; o.w += sv * xv.w;
            }
            *reinterpret_cast<float4*>(dx + off) = o;
        }
    }
}

// Transposed hi / lo planes for dPhi = dP^T x, whose reduction runs over
// tokens: an MFMA fragment wants 8 consecutive tokens of one output row /
// one column, which are strided in the token-major dP and x.  Both are
// split once into [row][Bp] bf16 planes (Bp = tokens rounded up to 32,
// zero past the batch), so the fragments are 16-byte loads and the dPhi
// kernel does no splitting.
//   dpT[o][t] from dP[t][o] (rows up to `rows`, zero past np): one lane
//   per (o, 8 tokens).
__global__ __launch_bounds__(256) void dp_tsplit_kernel(const float* __restrict__ dP, int stride, int np, int rows,
                                                        int64_t B, int64_t Bp, uint4* __restrict__ th,
                                                        uint4* __restrict__ tl) {
    const int64_t groups = Bp / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * groups) return;
    const int o = (int)(i / groups);
    const int64_t t0 = (i % groups) * 8;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (o < np && t0 + e < B) ? dP[(t0 + e) * stride + o] : 0.f;
    u32x4_t h, l;
    split_pack8(v, h, l);
    th[i] = make_uint4(h[0], h[1], h[2], h[3]);
    tl[i] = make_uint4(l[0], l[1], l[2], l[3]);
}

//   xT[k][t] from x[t][k]: a 32-token x 64-column tile through LDS (loads
//   along k, stores along t).
constexpr int kXtCols = 64;
__global__ __launch_bounds__(256) void x_tsplit_kernel(const float* __restrict__ x, int64_t B, int64_t K, int64_t Bp,
                                                       uint4* __restrict__ th, uint4* __restrict__ tl) {
    __shared__ float tile[32][kXtCols + 1];
    const int64_t cb = blockIdx.x;   // column block
    const int64_t tb = blockIdx.y;   // 32-token block
    const int64_t k0 = cb * kXtCols, t0 = tb * 32;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int i = threadIdx.x + 256 * u;
        const int r = i / kXtCols, c = i % kXtCols;
        const int64_t t = t0 + r, k = k0 + c;
        tile[r][c] = (t < B && k < K) ? x[t * K + k] : 0.f;
    }
    __syncthreads();
    const int c = threadIdx.x % kXtCols;
    const int g = threadIdx.x / kXtCols;  // 8-token group 0..3
    const int64_t k = k0 + c;
    if (k >= K) return;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = tile[8 * g + e][c];
    u32x4_t h, l;
    split_pack8(v, h, l);
    const int64_t idx = (k * Bp + t0 + 8 * g) / 8;
    th[idx] = make_uint4(h[0], h[1], h[2], h[3]);
    tl[idx] = make_uint4(l[0], l[1], l[2], l[3]);
}

// dPhi rows: one workgroup per 128 output rows x 128 columns walks all
// tokens, dPhi = hi.hi + lo.hi + hi.lo in MFMA registers, its rows stored
// directly (non-temporal).  A = dP^T (the workgroup's 128 rows, shared by
// its four waves)
// goes through LDS 128 tokens at a time; B = x^T fragments of the wave's
// own 32 columns come straight from the transposed planes, the next 32
// tokens' in flight while the current ones are on the matrix cores.  The
// row blocks of one column block get ids on one XCD, sharing those x
// columns through its L2.
constexpr int kDphiRows = 128;                // output rows (four 32-row tiles) per dPhi workgroup
constexpr int kDphiTok = 128;                 // tokens per LDS chunk of dP^T
constexpr int kDphiPitch = kDphiTok * 2 + 16;  // bytes per row of one plane in LDS

__global__ __launch_bounds__(256) void proj_bwd_dphi_kernel(const uint4* __restrict__ dth, const uint4* __restrict__ dtl,
                                                            const uint4* __restrict__ xth, const uint4* __restrict__ xtl,
                                                            int np, float* __restrict__ dphi, int64_t Bp, int64_t K) {
    constexpr int CB = 128;
    constexpr int OT = kDphiRows / 16;
    constexpr int PITCH = kDphiPitch;
    __shared__ __align__(16) char as[2][kDphiRows * PITCH];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int64_t rblocks = (np + kDphiRows - 1) / kDphiRows;
    const int64_t cblocks = (K + CB - 1) / CB;
    const int64_t lin = blockIdx.x;
    const int64_t idx = lin / 8;
    const int o0 = (int)(idx % rblocks) * kDphiRows;
    const int64_t cb = (idx / rblocks) * 8 + lin % 8;
    if (cb >= cblocks) return;  // padding ids: the whole workgroup
    const int64_t kb0 = cb * CB + wave * 32;
    const bool wave_on = kb0 < K;  // K % 32 == 0: whole waves are in or out
    const int64_t rowp = Bp / 8;   // 16-byte pieces per plane row
    f32x4_t acc[OT][2];
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) acc[ot][ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    auto u4 = [](const uint4& q) __attribute__((always_inline)) { return u32x4_t{q.x, q.y, q.z, q.w}; };
    // B = x^T: column kb0 + 16 ct + lr, tokens t0 + 8 lg .. + 7
    struct BFrag {
        uint4 h[2], l[2];
    };
    auto load_b = [&](BFrag& f, int64_t t0) __attribute__((always_inline)) {
        const int64_t tp = (t0 + 8 * lg) / 8;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int64_t r = (wave_on ? kb0 + 16 * ct + lr : 0) * rowp + tp;
            f.h[ct] = xth[r];
            f.l[ct] = xtl[r];
        }
    };
    for (int64_t c0 = 0; c0 < Bp; c0 += kDphiTok) {
        const int tc = Bp - c0 < kDphiTok ? (int)(Bp - c0) : kDphiTok;  // a multiple of 32
        // dP^T rows o0 .. o0 + 63, tokens c0 .. c0 + tc - 1, both planes:
        // piece i = (plane, row, 16-byte column)
        const int pieces = 2 * kDphiRows * (tc / 8);
        for (int i = threadIdx.x; i < pieces; i += 256) {
            const int pl = i / (kDphiRows * (tc / 8));
            const int r = (i / (tc / 8)) % kDphiRows;
            const int c = i % (tc / 8);
            const uint4* src = pl == 0 ? dth : dtl;
            *reinterpret_cast<uint4*>(&as[pl][r * PITCH + 16 * c]) = src[(int64_t)(o0 + r) * rowp + c0 / 8 + c];
        }
        __syncthreads();
        if (wave_on) {
            BFrag fa, fb;
            int t = 0;
            load_b(fa, c0);
            auto mma = [&](const BFrag& f, int tt) __attribute__((always_inline)) {
#pragma unroll
                for (int ot = 0; ot < OT; ++ot) {
                    const int off = (16 * ot + lr) * PITCH + (tt + 8 * lg) * 2;
                    const u32x4_t ah = u4(*reinterpret_cast<const uint4*>(&as[0][off]));
                    const u32x4_t al = u4(*reinterpret_cast<const uint4*>(&as[1][off]));
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) {
                        acc[ot][ct] = mfma16x16x32(ah, u4(f.h[ct]), acc[ot][ct]);
                        acc[ot][ct] = mfma16x16x32(al, u4(f.h[ct]), acc[ot][ct]);
                        acc[ot][ct] = mfma16x16x32(ah, u4(f.l[ct]), acc[ot][ct]);
                    }
                }
            };
            for (; t + 64 <= tc; t += 64) {
                load_b(fb, c0 + t + 32);
                mma(fa, t);
                if (t + 64 < tc) load_b(fa, c0 + t + 64);
                mma(fb, t + 32);
            }
            if (t < tc) mma(fa, t);
        }
        __syncthreads();  // the chunk is restaged
    }
    if (!wave_on) return;
    // D[o 16 ot + 4 lg + i][column 16 ct + lr]
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = o0 + 16 * ot + 4 * lg + i;
            if (o >= np) continue;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) __builtin_nontemporal_store(acc[ot][ct][i], dphi + (int64_t)o * K + kb0 + 16 * ct + lr);
        }
    }
}

bool proj_bwd_wide_path(int x_dtype, int np, int64_t B) {
    return x_dtype == kF32 && np > kProjTile && B >= 1 && B <= kProjWideMaxB;
}

// scratch of the all-tiles path: [dP hi | dP lo] ([B][np32] bf16),
// [dP^T hi | lo] ([np64][Bp], np64 = np rounded up to the dPhi row block),
// [x^T hi | lo] ([K][Bp]); each plane 256-byte aligned.
struct WideScratch {
    size_t dp_plane, dpt_plane, xt_plane, total;
};
static WideScratch wide_scratch(int np, int64_t B, int64_t K) {
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const int64_t np32 = (int64_t)proj_tiles(np) * kProjTile;
    const int64_t np64 = (np + kDphiRows - 1) / kDphiRows * kDphiRows;  // dPhi row blocks
    const int64_t Bp = (B + 31) / 32 * 32;
    WideScratch w{};
    if (np <= kStreamOB) return w;  // the small-np kernels split in registers
    w.dp_plane = al((size_t)B * np32 * 2);
    w.dpt_plane = al((size_t)np64 * Bp * 2);
    w.xt_plane = al((size_t)K * Bp * 2);
    w.total = 2 * (w.dp_plane + w.dpt_plane + w.xt_plane);
    return w;
}

size_t proj_bwd_wide_scratch_bytes(int np, int64_t B, int64_t K) { return wide_scratch(np, B, K).total; }

int proj_bwd_small_max_rows() { return kStreamOB; }

hipError_t launch_proj_bwd_small(const float* x, const float* dP, int dp_stride, const float* s_tok,
                                 const float* phi_pre, const float* phi_post, const float* phi_res, int n_pre, int np,
                                 float* dx, bool accumulate, float* dphi, int64_t B, int64_t K, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (np <= kProjTile || np > kStreamOB || K % 32 != 0) return hipErrorInvalidValue;
    if (s_tok && !accumulate) return hipErrorInvalidValue;
    const unsigned cblocks = (unsigned)((K + 127) / 128);
    {
        // 1-D grid: 8 XCD lanes x ceil(column blocks / 8) x 32-token blocks
        const unsigned tb32 = (unsigned)((B + 31) / 32);
        const dim3 gs(8u * ((cblocks + 7) / 8) * tb32);
        const int tk = timing_begin("proj_bwd", s);
        if (s_tok) {
            MHC_LAUNCH_GGL((proj_bwd_dx_small_kernel<true, true>), gs, dim3(256), 0, s, x, dP, dp_stride, s_tok,
                               phi_pre, phi_post, phi_res, n_pre, np, dx, B, K);
        } else if (accumulate) {
            MHC_LAUNCH_GGL((proj_bwd_dx_small_kernel<true, false>), gs, dim3(256), 0, s, x, dP, dp_stride, s_tok,
                               phi_pre, phi_post, phi_res, n_pre, np, dx, B, K);
        } else {
            MHC_LAUNCH_GGL((proj_bwd_dx_small_kernel<false, false>), gs, dim3(256), 0, s, x, dP, dp_stride, s_tok,
                               phi_pre, phi_post, phi_res, n_pre, np, dx, B, K);
        }
        hipError_t e = hipGetLastError();
        timing_end(tk, s);
        if (e != hipSuccess) return e;
        const int tg = timing_begin("proj_bwd_dphi", s);
        const unsigned rb = (unsigned)((np + kDphiSmallRows - 1) / kDphiSmallRows);
        MHC_LAUNCH_GGL(proj_bwd_dphi_small_kernel, dim3(8u * ((cblocks + 7) / 8) * rb), dim3(256), 0, s, x, dP,
                           dp_stride, np, dphi, B, K);
        timing_end(tg, s);
        return hipGetLastError();
    }
}

hipError_t launch_proj_bwd_wide(const float* x, const float* dP, int dp_stride, const float* s_tok,
                                const float* phi_pre, const float* phi_post, const float* phi_res, int n_pre, int np,
                                float* dx, bool accumulate, float* dphi, void* scratch, int64_t B, int64_t K,
                                hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (np <= kProjTile || B > kProjWideMaxB || K % 32 != 0) return hipErrorInvalidValue;
    if (s_tok && !accumulate) return hipErrorInvalidValue;
    if (np <= kStreamOB)
        return launch_proj_bwd_small(x, dP, dp_stride, s_tok, phi_pre, phi_post, phi_res, n_pre, np, dx, accumulate,
                                     dphi, B, K, s);
    const unsigned cblocks = (unsigned)((K + 127) / 128);
    if (!scratch) return hipErrorInvalidValue;
    const int np32 = proj_tiles(np) * kProjTile;
    const int64_t Bp = (B + 31) / 32 * 32;
    const WideScratch ws = wide_scratch(np, B, K);
    char* sc = reinterpret_cast<char*>(scratch);
    // dP -> hi / lo bf16 planes in scratch
    uint4* dph = reinterpret_cast<uint4*>(sc);
    uint4* dpl = reinterpret_cast<uint4*>(sc + ws.dp_plane);
    uint4* dth = reinterpret_cast<uint4*>(sc + 2 * ws.dp_plane);
    uint4* dtl = reinterpret_cast<uint4*>(sc + 2 * ws.dp_plane + ws.dpt_plane);
    uint4* xth = reinterpret_cast<uint4*>(sc + 2 * (ws.dp_plane + ws.dpt_plane));
    uint4* xtl = reinterpret_cast<uint4*>(sc + 2 * (ws.dp_plane + ws.dpt_plane) + ws.xt_plane);
    const int64_t pieces = B * (np32 / 8);
    MHC_LAUNCH_GGL(dp_split_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, s, dP, dp_stride, np,
                       np32, B, dph, dpl);
    // 1-D grid: 8 XCD lanes x ceil(column blocks / 8) x token blocks
    const unsigned tblocks = (unsigned)((B + kDx2Tok - 1) / kDx2Tok);
    const dim3 gdx(8u * ((cblocks + 7) / 8) * tblocks);
    const int tok = timing_begin("proj_bwd", s);
    if (s_tok) {
        MHC_LAUNCH_GGL((proj_bwd_dx2_kernel<true, true>), gdx, dim3(256), 0, s, x, dph, dpl, np32, s_tok, phi_pre,
                           phi_post, phi_res, n_pre, np, dx, B, K);
    } else if (accumulate) {
        MHC_LAUNCH_GGL((proj_bwd_dx2_kernel<true, false>), gdx, dim3(256), 0, s, x, dph, dpl, np32, s_tok, phi_pre,
                           phi_post, phi_res, n_pre, np, dx, B, K);
    } else {
        MHC_LAUNCH_GGL((proj_bwd_dx2_kernel<false, false>), gdx, dim3(256), 0, s, x, dph, dpl, np32, s_tok,
                           phi_pre, phi_post, phi_res, n_pre, np, dx, B, K);
    }
    hipError_t e = hipGetLastError();
    timing_end(tok, s);
    if (e != hipSuccess) return e;
    const int tg = timing_begin("proj_bwd_dphi", s);
    const int np64 = (np + kDphiRows - 1) / kDphiRows * kDphiRows;
    const int64_t tgroups = (int64_t)np64 * (Bp / 8);
    MHC_LAUNCH_GGL(dp_tsplit_kernel, dim3((unsigned)((tgroups + 255) / 256)), dim3(256), 0, s, dP, dp_stride, np,
                       np64, B, Bp, dth, dtl);
    MHC_LAUNCH_GGL(x_tsplit_kernel, dim3((unsigned)((K + kXtCols - 1) / kXtCols), (unsigned)(Bp / 32)), dim3(256),
                       0, s, x, B, K, Bp, xth, xtl);
    const unsigned rblocks = (unsigned)((np + kDphiRows - 1) / kDphiRows);
    MHC_LAUNCH_GGL(proj_bwd_dphi_kernel, dim3(8u * ((cblocks + 7) / 8) * rblocks), dim3(256), 0, s, dth, dtl, xth,
                       xtl, np, dphi, Bp, K);
    timing_end(tg, s);
    return hipGetLastError();
}

// Token tiles of the projection backward: column blocks x tiles fill two
// rounds of resident workgroups (rounded down, so a last partial round is
// nearly full rather than leaving most CUs idle while it runs), at least one.
// A token tile's rows of x / dx, plus the three stages the pipeline reads
// past its end, under 2 GiB (the kernel's buffer resources and offsets).
// Tiles are whole pairs of 32-token stages; the pipeline reads up to four
// stages past the end, and offsets stay under 2 GiB.
static int64_t proj_bwd_max_tile(int x_dtype, int64_t K) {
    return ((int64_t(1) << 31) - 1) / (K * (x_dtype == kBF16 ? 2 : 4)) - 4 * 32;
}

int proj_bwd_tiles(int x_dtype, int64_t B, int64_t K) {
    const int cb = 32 * (x_dtype == kBF16 ? kPbNW<bf16_t>() : kPbNW<float>());
    const int64_t gx = (K + cb - 1) / cb;
    const void* fn = x_dtype == kBF16 ? reinterpret_cast<const void*>(&proj_bwd_mfma_kernel<bf16_t, true, true>)
                                      : reinterpret_cast<const void*>(&proj_bwd_mfma_kernel<float, true, true>);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 2 * cb, 0) != hipSuccess || per_cu < 1) {
        (void)hipGetLastError();
        per_cu = 1;
    }
    int64_t tiles = 2 * (int64_t)device_cu_count() * per_cu / gx;
    const int64_t blocks = (B + 31) / 32;
    if (tiles > blocks) tiles = blocks;
    if (tiles < 1) tiles = 1;
    const int64_t mt = proj_bwd_max_tile(x_dtype, K) / 64 * 64;
    if (mt >= 64 && (B + tiles - 1) / tiles > mt) tiles = (B + mt - 1) / mt;
    return (int)tiles;
}

hipError_t launch_proj_bwd(int x_dtype, const void* x, const float* dP, int dp_stride, const float* s_tok,
                           const float* phi_pre, const float* phi_post, const float* phi_res, int n_pre, int o0,
                           int np, void* dx, bool accumulate, float* dphi_part, int tiles, int64_t B, int64_t K,
                           hipStream_t s, const int32_t* dx_scale, int groups) {
    if (B == 0) return hipSuccess;
    if (np < 1 || np > kProjTile || o0 < 0 || K % 32 != 0 || tiles < 1) return hipErrorInvalidValue;
    // bf16 x: one output tile, on the fp16 stream part of the row pass
    const int C = np > 0 ? (int)(K / (n_pre > 0 ? n_pre : 1)) : 0;
    if (x_dtype == kBF16 && (o0 != 0 || dx_scale == nullptr || groups < 1 || C % kPartGroup != 0))
        return hipErrorInvalidValue;
    // token tile: a multiple of two 32-token stages
    int64_t tile = (B + tiles - 1) / tiles;
    tile = ((tile + 63) / 64) * 64;
    if (tile > proj_bwd_max_tile(x_dtype, K)) return hipErrorInvalidValue;  // offsets past 2 GiB
    const int cb = 32 * (x_dtype == kBF16 ? kPbNW<bf16_t>() : kPbNW<float>());  // columns per workgroup
    const dim3 grid((unsigned)((K + cb - 1) / cb), (unsigned)tiles);
#define MHC_PROJ_BWD(TX_, ACC_, S_)                                                                              \
    MHC_LAUNCH_GGL((proj_bwd_mfma_kernel<TX_, ACC_, S_>), grid, dim3(2 * cb), 0, s, (const TX_*)x, dP, dp_stride,  \
                       s_tok, phi_pre, phi_post, phi_res, n_pre, o0, np, (TX_*)dx, dx_scale, groups, C, dphi_part, B, K, \
                       tile)
    // The layer backward accumulates (with the r_h term on the first output
    // tile only); the standalone operator starts from zero on its first tile.
    // An s term without accumulation, or a bf16 dx from zero, is not built.
    const bool has_s = s_tok != nullptr;
    if (has_s && !accumulate) return hipErrorInvalidValue;
    if (x_dtype == kBF16 && !accumulate) return hipErrorInvalidValue;
    const int tok = timing_begin("proj_bwd", s);
    if (x_dtype == kBF16) {
        if (has_s) {
            MHC_PROJ_BWD(bf16_t, true, true);
        } else {
            MHC_PROJ_BWD(bf16_t, true, false);
        }
    } else if (has_s) {
        MHC_PROJ_BWD(float, true, true);
    } else if (accumulate) {
        MHC_PROJ_BWD(float, true, false);
    } else {
        MHC_PROJ_BWD(float, false, false);
    }
#undef MHC_PROJ_BWD
    timing_end(tok, s);
    return hipGetLastError();
}

}  // namespace mhc

// MHCResidualWrapper for the shapes the n = 4 kernels of wrapper.hip do not
// take: expansion rates 2..32 and n = 4 rows those kernels refuse; any
// hidden % 4 == 0 (layer.py:269-322).
//
// The streams are rebuilt from r and b wherever a row pass needs them
// (X_0 = r, X_1 = b, X_j = r * 0.1^(j-1) rounded to the storage dtype in
// 'decay' mode, 0 in 'zero' mode: layer.py:299-310), with n taken at run
// time: per-stream arrays have a compile-time capacity NM in {2, 4, 8, 16,
// 32} (the dPhi / fold kernels: up to 16) and their loops run over it with a
// uniform j < n test, so nothing is indexed at run time in registers.  The
// math is that of wrapper.hip:
//   forward   out = hs (xa / r) w + sum_j cm_j X_j,  xa = sum_j h_pre_j X_j,
//             r = sqrt(mean_c xa^2 + eps),  hs = (1/n) sum_i h_post_i,
//             cm_j = (1/n) sum_i M_ij  (the stream mean of layer.py:316)
//   backward  gxa = (hs / r) w G - k2 xa,  k2 = hs sum(w G xa) / (C r^3),
//             dX_j = cm_j G + h_pre_j gxa (+ dP . Phi_j + s X_j with
//             dynamic H),  d r = sum_j w_j dX_j,  d b = dX_1,
//             w_j = 1, 0, 0.1, 0.01, ... (0 past stream 1 in 'zero' mode),
//             dw = sum_tokens hs G xa / r.
// Kernels:
//   wgen_fwd_kernel    forward row pass, one wave per token
//   wgen_red_kernel    backward row sums, one wave per token: the
//                      coefficient backward's scalars per token (dynamic H)
//                      or summed per wave (static H), and the per-token
//                      factors of d r / d b
//   wgen_dx_kernel     d r, d b (rounded once) and the dw partials:
//                      workgroups of 1024 channels x one token tile; with
//                      dynamic H it adds the layer projection backward's dX
//                      folded over the streams (Sinkhorn settings where the
//                      H_res rows of dP do not vanish, and shapes the fold
//                      kernels do not take)
//   wgen_dphi_mfma_kernel  dynamic H, H_res rows of dP vanishing, n <= 8, or
//                      n <= 16 on rows of 2048 channels or more:
//                      dPhi of the 2n pre / post rows from the rebuilt
//                      streams (bf16 MFMA)
//   wgen_dx_fold_kernel  the same case: d r, d b with dP . Phi folded over
//                      the streams, and the dw partials
//   wgen_synth_kernel  the stream rows [tokens, n*C] as the operand of the
//                      layer's projection kernels (dynamic H: the forward's
//                      in the storage dtype; the backward's in fp32 when the
//                      fold kernels do not run)
#include "mhc_device.h"
#include "mhc_internal.h"

namespace mhc {

namespace {

constexpr double wg_pow01(int e) { return e <= 0 ? 1.0 : 0.1 * wg_pow01(e - 1); }

// Decay multiplier of stream j >= 2: Python's 0.1 ** (j - 1) as fp32 (the
// product r * m is formed in fp32 by the reference's mul; the double
// repeated product rounds to the same fp32 value as 0.1 ** e for e <= 63).
#define MHC_WG_M(e) (float)wg_pow01(e)
constexpr float kWgMult[kWgMaxN] = {
    1.f,          0.f,          MHC_WG_M(1),  MHC_WG_M(2),  MHC_WG_M(3),  MHC_WG_M(4),  MHC_WG_M(5),  MHC_WG_M(6),
    MHC_WG_M(7),  MHC_WG_M(8),  MHC_WG_M(9),  MHC_WG_M(10), MHC_WG_M(11), MHC_WG_M(12), MHC_WG_M(13), MHC_WG_M(14),
    MHC_WG_M(15), MHC_WG_M(16), MHC_WG_M(17), MHC_WG_M(18), MHC_WG_M(19), MHC_WG_M(20), MHC_WG_M(21), MHC_WG_M(22),
    MHC_WG_M(23), MHC_WG_M(24), MHC_WG_M(25), MHC_WG_M(26), MHC_WG_M(27), MHC_WG_M(28), MHC_WG_M(29), MHC_WG_M(30)};
#undef MHC_WG_M

template <typename TX>
__device__ __forceinline__ float wg_round(float v) {
    if constexpr (sizeof(TX) == 2) {
        return bf16_to_f32(f32_to_bf16(v));
    } else {
        return v;
    }
}

// Stream j of the synthesised row (j is a constant after unrolling).
template <typename TX, bool DECAY>
__device__ __forceinline__ float wg_stream(int j, float r, float b) {
    if (j == 0) return r;
    if (j == 1) return b;
    return DECAY ? wg_round<TX>(r * kWgMult[j]) : 0.f;
}

// d r weight of stream j.
template <bool DECAY>
__device__ __forceinline__ float wg_rweight(int j) {
    return j == 0 ? 1.f : (j == 1 ? 0.f : (DECAY ? kWgMult[j] : 0.f));
}

// h_pre, cm = (1/n) column sums of M and hs = (1/n) sum h_post of one token
// (every lane of the wave calls it with the same cf).
template <int NM>
__device__ __forceinline__ void wg_coefs(const float* __restrict__ cf, int n, float (&hp)[NM], float (&cm)[NM],
                                         float& hs) {
    const float inv_n = 1.f / (float)n;
    hs = 0.f;
    if constexpr (NM > 8) {
        // lane j sums column j of M (n loads a lane instead of n^2
        // unrolled ones), then the wave reads the n values back
        const int lane = threadIdx.x & (kWave - 1);
        float hl = 0.f, cl = 0.f;
        if (lane < n) {
            hl = cf[lane];
            float sc = 0.f;
            for (int i = 0; i < n; ++i) sc += cf[2 * n + i * n + lane];
            cl = sc * inv_n;
        }
        for (int i = 0; i < n; ++i) hs += cf[n + i];
        hs *= inv_n;
#pragma unroll
        for (int j = 0; j < NM; ++j) {
            hp[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hl), j));
            cm[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cl), j));
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        hp[j] = 0.f;
        cm[j] = 0.f;
        if (j < n) {
            hp[j] = cf[j];
            hs += cf[n + j];
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < NM; ++i) {
                if (i < n) s += cf[2 * n + i * n + j];
            }
            cm[j] = s * inv_n;
        }
    }
    hs *= inv_n;
}

template <typename TX, int NM, bool DECAY>
__device__ __forceinline__ float wg_xa(float r, float b, const float (&hp)[NM], int n) {
    float xa = 0.f;
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        if (j < n) xa += hp[j] * wg_stream<TX, DECAY>(j, r, b);
    }
    return xa;
}

constexpr int kWgU = 4;  // 4-channel chunks per lane in flight

}  // namespace

// ---------------------------------------------------------------------------
// Forward row pass: one wave per token, 4-channel chunks (lane l takes
// chunks l, l + 64, ...).  Pass 1 forms sum xa^2 (r and b read through the
// cache), pass 2 reads them again (last use) with the weight and stores the
// fp32 output.
// ---------------------------------------------------------------------------
template <typename TX, int NM, bool DECAY>
__global__ __launch_bounds__(256) void wgen_fwd_kernel(const TX* __restrict__ res, const TX* __restrict__ br,
                                                       const float* __restrict__ w, const float* __restrict__ coef,
                                                       int64_t coef_stride, float* __restrict__ out, int64_t B, int C,
                                                       int n, float eps) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t b = (int64_t)blockIdx.x * (blockDim.x / kWave) + (int64_t)wave_uniform(threadIdx.x / kWave);
    if (b >= B) return;
    float hp[NM], cm[NM], hs;
    wg_coefs<NM>(coef + b * coef_stride, n, hp, cm, hs);
    const TX* rb = res + b * (int64_t)C;
    const TX* bb = br + b * (int64_t)C;
    const int nq = C / 4;
    float ss = 0.f;
    for (int q0 = 0; q0 < nq; q0 += kWgU * kWave) {
        float rv[kWgU][4], bv[kWgU][4];
#pragma unroll
        for (int u = 0; u < kWgU; ++u) {
            const int q = q0 + u * kWave + lane;
            const int c0 = (q < nq ? q : 0) * 4;
            load_run<TX, 4>(rb + c0, rv[u]);
            load_run<TX, 4>(bb + c0, bv[u]);
        }
#pragma unroll
        for (int u = 0; u < kWgU; ++u) {
            if (q0 + u * kWave + lane >= nq) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float xa = wg_xa<TX, NM, DECAY>(rv[u][e], bv[u][e], hp, n);
                ss += xa * xa;
            }
        }
    }
    float t[1] = {ss};
    wave_sum<1>(t);
    const float inv = 1.f / sqrtf(t[0] / (float)C + eps);
    float* ob = out + b * (int64_t)C;
    for (int q0 = 0; q0 < nq; q0 += kWgU * kWave) {
        float rv[kWgU][4], bv[kWgU][4], wv[kWgU][4];
#pragma unroll
        for (int u = 0; u < kWgU; ++u) {
            const int q = q0 + u * kWave + lane;
            const int c0 = (q < nq ? q : 0) * 4;
            load_run_nt<TX, 4>(rb + c0, rv[u]);
            load_run_nt<TX, 4>(bb + c0, bv[u]);
            load_run<float, 4>(w + c0, wv[u]);
        }
#pragma unroll
        for (int u = 0; u < kWgU; ++u) {
            const int q = q0 + u * kWave + lane;
            if (q >= nq) continue;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float r = rv[u][e], bvv = bv[u][e];
                float s = hs * (wg_xa<TX, NM, DECAY>(r, bvv, hp, n) * inv * wv[u][e]);
#pragma unroll
                for (int j = 0; j < NM; ++j) {
                    if (j < n) s += cm[j] * wg_stream<TX, DECAY>(j, r, bvv);
                }
                o[e] = s;
            }
            store_run_nt<float, 4>(ob + q * 4, o);
        }
    }
}

// ---------------------------------------------------------------------------
// Backward row sums, one wave per token: ss = sum xa^2, gwx = sum w G xa,
// u_j = sum G X_j, v_j = sum w G X_j, z_j = sum xa X_j, and from them the
// coefficient backward's scalars (dM_ij = u_j / n, dh_post_act_i =
// gwx / (n r), dh_pre_act_j = hs v_j / r - k2 z_j, then 1/r and k2): per
// token in scal_out[b][n*n+2n+2] (dynamic H), or (STATIC) summed over the
// tokens each wave takes (grid stride) into scal_out[wave][n*n+2n]; the
// static sums are kept per stream (lane j: sum u_j / n and sum dh_pre_act_j,
// every lane: sum dh_post_act), since dM_ij does not depend on i, and
// spread over the n*n+2n slots once per wave.  Both write the per-token
// factors of d r / d b, ep_out[b][kWgEp]:
//   [A_r, B_r hs/r, A_b, B_b hs/r, hs/r, -B_r k2, -B_b k2, 0, h_pre_0..7]
// with A_r = sum_j w_j cm_j, B_r = sum_j w_j h_pre_j, A_b = cm_1,
// B_b = h_pre_1, so that d r = A_r G + B_r gxa and d b = A_b G + B_b gxa
// (h_pre only up to capacity 8: the wider kernels read it from coef).
// ---------------------------------------------------------------------------
template <typename TX, int NM, bool DECAY, bool STATIC>
__global__ __launch_bounds__(256) void wgen_red_kernel(const float* __restrict__ g, const TX* __restrict__ res,
                                                       const TX* __restrict__ br, const float* __restrict__ w,
                                                       const float* __restrict__ coef, int64_t coef_stride,
                                                       float* __restrict__ scal_out, float* __restrict__ ep_out,
                                                       int64_t B, int C, int n, float eps) {
    constexpr int NR = 2 + 3 * NM;
    constexpr int U = NM > 8 ? 2 : kWgU;  // chunks in flight beside NR sums
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wid = (int64_t)blockIdx.x * (blockDim.x / kWave) + (int64_t)wave_uniform(threadIdx.x / kWave);
    const int64_t nw = STATIC ? (int64_t)gridDim.x * (blockDim.x / kWave) : B;
    const int NS = n * n + 2 * n;
    const float inv_n = 1.f / (float)n;
    const int nq = C / 4;
    float acc_u = 0.f, acc_pre = 0.f, acc_post = 0.f;  // STATIC sums
    // STATIC: one coefficient set for every token (coef_stride unused)
    float hp[NM], cm[NM], hs;
    if constexpr (STATIC) wg_coefs<NM>(coef, n, hp, cm, hs);
    for (int64_t b = wid; b < B; b += nw) {
        if constexpr (!STATIC) wg_coefs<NM>(coef + b * coef_stride, n, hp, cm, hs);
        float rs[NR];
#pragma unroll
        for (int q = 0; q < NR; ++q) rs[q] = 0.f;
        const float* gb = g + b * (int64_t)C;
        const TX* rb = res + b * (int64_t)C;
        const TX* bb = br + b * (int64_t)C;
        for (int q0 = 0; q0 < nq; q0 += U * kWave) {
            float gv[U][4], wv[U][4], rv[U][4], bv[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int q = q0 + u * kWave + lane;
                const int c0 = (q < nq ? q : 0) * 4;
                load_run_nt<float, 4>(gb + c0, gv[u]);
                load_run<float, 4>(w + c0, wv[u]);
                load_run<TX, 4>(rb + c0, rv[u]);
                load_run<TX, 4>(bb + c0, bv[u]);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (q0 + u * kWave + lane >= nq) continue;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float r = rv[u][e], bvv = bv[u][e];
                    const float xa = wg_xa<TX, NM, DECAY>(r, bvv, hp, n);
                    const float gg = gv[u][e];
                    const float wg = wv[u][e] * gg;
                    rs[0] += xa * xa;
                    rs[1] += wg * xa;
#pragma unroll
                    for (int j = 0; j < NM; ++j) {
                        if (j < n) {
                            const float x = wg_stream<TX, DECAY>(j, r, bvv);
                            rs[2 + j] += gg * x;
                            rs[2 + NM + j] += wg * x;
                            rs[2 + 2 * NM + j] += xa * x;
                        }
                    }
                }
            }
        }
        wave_sum<NR>(rs);
        const float inv = 1.f / sqrtf(rs[0] / (float)C + eps);
        const float gwx = rs[1];
        const float k2 = hs * gwx * inv * inv * inv / (float)C;
        if constexpr (STATIC) {
            // lane j's stream sums (u_j, v_j, z_j) into its running sums
            float uu = 0.f, vv = 0.f, zz = 0.f;
#pragma unroll
            for (int jj = 0; jj < NM; ++jj) {
                uu = (jj == lane) ? rs[2 + jj] : uu;
                vv = (jj == lane) ? rs[2 + NM + jj] : vv;
                zz = (jj == lane) ? rs[2 + 2 * NM + jj] : zz;
            }
            acc_u += uu * inv_n;                 // dM_ij = u_j / n
            acc_pre += hs * inv * vv - k2 * zz;  // dh_pre_act_j
            acc_post += gwx * inv * inv_n;       // dh_post_act_i
        } else {
            auto slot = [&](int t) __attribute__((always_inline)) {
                float v = 0.f;
                if (t < n * n) {
                    const int j = t % n;
                    float u = 0.f;
#pragma unroll
                    for (int jj = 0; jj < NM; ++jj) u = (jj == j) ? rs[2 + jj] : u;
                    v = u * inv_n;  // dM_ij = u_j / n
                } else if (t < n * n + n) {
                    v = gwx * inv * inv_n;  // dh_post_act_i
                } else if (t < NS) {
                    const int j = t - n * n - n;
                    float vv = 0.f, zz = 0.f;
#pragma unroll
                    for (int jj = 0; jj < NM; ++jj) {
                        vv = (jj == j) ? rs[2 + NM + jj] : vv;
                        zz = (jj == j) ? rs[2 + 2 * NM + jj] : zz;
                    }
                    v = hs * inv * vv - k2 * zz;  // dh_pre_act_j
                } else if (t == NS) {
                    v = inv;
                } else if (t == NS + 1) {
                    v = k2;
                }
                return v;
            };
            float* so = scal_out + b * (int64_t)(NS + 2);
            for (int t = lane; t < NS + 2; t += kWave) so[t] = slot(t);
        }
        float a_r = cm[0], b_r = hp[0];
#pragma unroll
        for (int j = 2; j < NM; ++j) {
            if (j < n) {
                a_r += wg_rweight<DECAY>(j) * cm[j];
                b_r += wg_rweight<DECAY>(j) * hp[j];
            }
        }
        const float a_b = cm[1], b_b = hp[1];
        const float hsi = hs * inv;
        float rec[kWgEp];
        rec[0] = a_r;
        rec[1] = b_r * hsi;
        rec[2] = a_b;
        rec[3] = b_b * hsi;
        rec[4] = hsi;
        rec[5] = -b_r * k2;
        rec[6] = -b_b * k2;
        rec[7] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) rec[8 + j] = NM <= 8 && j < NM ? hp[j < NM ? j : 0] : 0.f;
        float ev = 0.f;
#pragma unroll
        for (int k = 0; k < kWgEp; ++k) ev = (lane == k) ? rec[k] : ev;
        if (lane < kWgEp) ep_out[b * kWgEp + lane] = ev;
    }
    if constexpr (STATIC) {
        // slots [dM (n x n) | dh_post_act (n) | dh_pre_act (n)]; the
        // trip count is uniform, so every lane takes part in the shuffles
        float* so = scal_out + wid * (int64_t)NS;
        for (int t0 = 0; t0 < NS; t0 += kWave) {
            const int t = t0 + lane;
            const int src = t < n * n ? t % n : (t < n * n + n ? 0 : t - n * n - n);
            const float vu = __shfl(acc_u, src);
            const float vp = __shfl(acc_pre, src);
            if (t < NS) so[t] = t < n * n ? vu : (t < n * n + n ? acc_post : vp);
        }
    }
}

// ---------------------------------------------------------------------------
// d r, d b and dw partials.  Workgroup = 256 lanes x 4 channels (1024
// channels) x one tile of tokens; each lane walks the tile's tokens with
// the per-token factors (uniform loads) and keeps its channels' dw sum.
// DYN: dX [B][n*C] (fp32: the projection backward's dP . Phi per stream)
// and the r_h term s X enter as d r += sum_j w_j (dX_j + s X_j),
// d b += dX_1 + s b, with s = s_tok[b].
// ---------------------------------------------------------------------------
template <typename TX, int NM, bool DECAY, bool DYN>
__global__ __launch_bounds__(256) void wgen_dx_kernel(const float* __restrict__ g, const TX* __restrict__ res,
                                                      const TX* __restrict__ br, const float* __restrict__ w,
                                                      const float* __restrict__ coef, int64_t coef_stride,
                                                      const float* __restrict__ ep, const float* __restrict__ dX,
                                                      const float* __restrict__ s_tok, TX* __restrict__ dres,
                                                      TX* __restrict__ dbr, float* __restrict__ dw_part, int64_t B,
                                                      int C, int n, int64_t tile) {
    const int64_t c0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const bool active = c0 < C;
    const int64_t t0 = (int64_t)blockIdx.y * tile;
    const int64_t t1 = t0 + tile < B ? t0 + tile : B;
    const int64_t K = (int64_t)n * C;
    float wv[4] = {0.f, 0.f, 0.f, 0.f}, dw[4] = {0.f, 0.f, 0.f, 0.f};
    if (active) load_run<float, 4>(w + c0, wv);
    for (int64_t b = t0; b < t1; ++b) {
        const float* e = ep + b * kWgEp;
        const float e0 = e[0], e1 = e[1], e2 = e[2], e3 = e[3], e4 = e[4], e5 = e[5], e6 = e[6];
        // h_pre from the record (one scalar load with the factors) up to
        // capacity 8, else from the coefficients
        const float* cf = coef + b * coef_stride;
        float hp[NM];
#pragma unroll
        for (int j = 0; j < NM; ++j) hp[j] = NM <= 8 ? e[8 + (j < 8 ? j : 0)] : (j < n ? cf[j] : 0.f);
        const float sv = DYN ? s_tok[b] : 0.f;
        if (!active) continue;
        const int64_t o = b * (int64_t)C + c0;
        float gv[4], rv[4], bv[4];
        load_run_nt<float, 4>(g + o, gv);
        load_run_nt<TX, 4>(res + o, rv);
        load_run_nt<TX, 4>(br + o, bv);
        float dx[NM][4];
        if constexpr (DYN) {
#pragma unroll
            for (int j = 0; j < NM; ++j) {
                if (j < n && (j < 2 || DECAY)) load_run_nt<float, 4>(dX + b * K + (int64_t)j * C + c0, dx[j]);
            }
        }
        float dr[4], db[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float xa = wg_xa<TX, NM, DECAY>(rv[q], bv[q], hp, n);
            const float gg = gv[q];
            const float wg = wv[q] * gg;
            float a = e0 * gg + e1 * wg + e5 * xa;
            float c = e2 * gg + e3 * wg + e6 * xa;
            if constexpr (DYN) {
                a += dx[0][q] + sv * rv[q];
#pragma unroll
                for (int j = 2; j < NM; ++j) {
                    if (j < n && DECAY) a += kWgMult[j] * (dx[j][q] + sv * wg_stream<TX, DECAY>(j, rv[q], bv[q]));
                }
                c += dx[1][q] + sv * bv[q];
            }
            dr[q] = a;
            db[q] = c;
            dw[q] += e4 * gg * xa;
        }
        store_run<TX, 4>(dres + o, dr);
        store_run<TX, 4>(dbr + o, db);
    }
    if (active) store_run<float, 4>(dw_part + (int64_t)blockIdx.y * C + c0, dw);
}

// ---------------------------------------------------------------------------
// The projection backward over the pre / post rows of dP (the H_res rows
// vanish: every stream receives G / n through the stream mean), without
// the stream rows in memory:
//   dphi_part[tile][o][j*C + c] = sum over the tile's tokens of
//                                 dP[t][o] X_j[t][c],  o < rows = 2n
// ---------------------------------------------------------------------------

namespace {
// two consecutive elements (4- or 8-byte aligned) as one load
template <typename TX>
__device__ __forceinline__ void wg_load2(const TX* p, float (&v)[2]) {
    if constexpr (sizeof(TX) == 2) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
        v[0] = __uint_as_float(w << 16);
        v[1] = __uint_as_float(w & 0xffff0000u);
    } else {
        const float2 f = *reinterpret_cast<const float2*>(p);
        v[0] = f.x;
        v[1] = f.y;
    }
}
}  // namespace

// ---------------------------------------------------------------------------
// The dPhi partials on bf16 MFMA 16x16x32: M = the rows o of dP (16,
// zero past rows), N = 16 channels, K = 32 tokens.  A = dP^T split into hi
// and lo bf16 parts (fp32 dP to 2^-16), B = X_j rebuilt from r and b (exact
// in one bf16 plane with bf16 storage; split hi / lo with fp32 storage).
// Workgroup = 4 waves x 16 channels (64 channels) x one token tile; each
// 32-token step stages the r and b tile [32][64] and dP^T [16][32] in LDS,
// and each wave runs 2 (bf16) or 3 (fp32) MFMAs per stream.
// ---------------------------------------------------------------------------
namespace {
typedef __bf16 gbf16x8_t __attribute__((ext_vector_type(8)));
typedef float gf32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int gu32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ gf32x4_t gmfma(gu32x4_t a, gu32x4_t b, gf32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gbf16x8_t, a), __builtin_bit_cast(gbf16x8_t, b),
                                                   c, 0, 0, 0);
}

// 8 fp32 -> hi / lo bf16 parts, packed in MFMA operand order (element e in
// half e % 2 of word e / 2)
__device__ __forceinline__ void g_split8(const float (&v)[8], gu32x4_t& hi, gu32x4_t& lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float h0 = bf16_to_f32(f32_to_bf16(v[2 * e]));
        const float h1 = bf16_to_f32(f32_to_bf16(v[2 * e + 1]));
        hi[e] = pack_bf16x2(h0, h1);
        lo[e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
    }
}
}  // namespace

constexpr int kWgDphiCB = 64;  // channels per workgroup of the MFMA dPhi kernel

template <typename TX, int NM, bool DECAY>
__global__ __launch_bounds__(256) void wgen_dphi_mfma_kernel(const TX* __restrict__ res, const TX* __restrict__ br,
                                                             const float* __restrict__ dP, int dp_stride, int rows,
                                                             float* __restrict__ dphi_part, int64_t B, int C, int n,
                                                             int64_t tile) {
    constexpr int CB = kWgDphiCB;
    constexpr int TS = 32;
    constexpr int RP = CB + 4;          // LDS row pitch (elements)
    constexpr int MI = (2 * NM + 15) / 16;  // 16-row MFMA tiles of the 2n rows
    __shared__ __align__(16) float rl[TS][RP];
    __shared__ __align__(16) float bl[TS][RP];
    __shared__ __align__(16) float dpt[16 * MI][TS + 4];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int64_t cb0 = (int64_t)blockIdx.x * CB;
    const int64_t t0 = (int64_t)blockIdx.y * tile;
    const int64_t t1 = t0 + tile < B ? t0 + tile : B;
    gf32x4_t acc[NM][MI];
#pragma unroll
    for (int j = 0; j < NM; ++j) {
#pragma unroll
        for (int m = 0; m < MI; ++m) acc[j][m] = gf32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    for (int64_t s0 = t0; s0 < t1; s0 += TS) {
        // r and b tile: 32 tokens x 64 channels in 4-channel pieces, two per
        // thread (a piece is all in or all out of the row: C % 4 == 0)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = tid + 256 * u;
            const int tt = i / (CB / 4);
            const int c4 = (i % (CB / 4)) * 4;
            const int64_t t = s0 + tt;
            const int64_t c = cb0 + c4;
            float rv[4] = {0.f, 0.f, 0.f, 0.f}, bv[4] = {0.f, 0.f, 0.f, 0.f};
            if (t < t1 && c < C) {
                load_run<TX, 4>(res + t * C + c, rv);
                load_run<TX, 4>(br + t * C + c, bv);
            }
            *reinterpret_cast<float4*>(&rl[tt][c4]) = make_float4(rv[0], rv[1], rv[2], rv[3]);
            *reinterpret_cast<float4*>(&bl[tt][c4]) = make_float4(bv[0], bv[1], bv[2], bv[3]);
        }
        // dP^T tile [16 MI rows][32 tokens]
#pragma unroll
        for (int u = 0; u < 2 * MI; ++u) {
            const int i = tid + 256 * u;
            const int o = i / TS;
            const int tt = i % TS;
            const int64_t t = s0 + tt;
            dpt[o][tt] = (o < rows && t < t1) ? dP[t * dp_stride + o] : 0.f;
        }
        __syncthreads();
        // A = dP^T: row o = 16 m + lr, tokens 8 lg .. + 7
        gu32x4_t ah[MI], al[MI];
#pragma unroll
        for (int m = 0; m < MI; ++m) {
            float av[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) av[e] = dpt[16 * m + lr][8 * lg + e];
            g_split8(av, ah[m], al[m]);
        }
        // B = X_j: tokens 8 lg .. + 7 of channel 16 wave + lr
        float rv[8], bv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            rv[e] = rl[8 * lg + e][16 * wave + lr];
            bv[e] = bl[8 * lg + e][16 * wave + lr];
        }
#pragma unroll
        for (int j = 0; j < NM; ++j) {
            if (j < n) {
                float xv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = wg_stream<TX, DECAY>(j, rv[e], bv[e]);
                if constexpr (sizeof(TX) == 2) {
                    gu32x4_t xb;
#pragma unroll
                    for (int e = 0; e < 4; ++e) xb[e] = pack_bf16x2(xv[2 * e], xv[2 * e + 1]);  // exact
#pragma unroll
                    for (int m = 0; m < MI; ++m) {
                        acc[j][m] = gmfma(ah[m], xb, acc[j][m]);
                        acc[j][m] = gmfma(al[m], xb, acc[j][m]);
                    }
                } else {
                    gu32x4_t xh, xl;
                    g_split8(xv, xh, xl);
#pragma unroll
                    for (int m = 0; m < MI; ++m) {
                        acc[j][m] = gmfma(ah[m], xh, acc[j][m]);
                        acc[j][m] = gmfma(al[m], xh, acc[j][m]);
                        acc[j][m] = gmfma(ah[m], xl, acc[j][m]);
                    }
                }
            }
        }
        __syncthreads();
    }
    // D[o = 16 m + 4 lg + i][channel 16 wave + lr]
    const int64_t c = cb0 + 16 * wave + lr;
    if (c >= C) return;
    const int64_t K = (int64_t)n * C;
    float* part = dphi_part + (int64_t)blockIdx.y * rows * K;
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        if (j < n) {
#pragma unroll
            for (int m = 0; m < MI; ++m) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int o = 16 * m + 4 * lg + i;
                    if (o < rows) part[o * K + (int64_t)j * C + c] = acc[j][m][i];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// d r, d b and dw partials with the projection's term formed here from dP
// (rows o < rows = 2n, the H_res rows vanishing):
//   d r += sum_o dP[t][o] Phi_r[o][c] + s sum_j w_j X_j,  Phi_r = sum_j w_j Phi_j
//   d b += sum_o dP[t][o] Phi_1[o][c] + s b
// on top of the stream parts of wgen_dx_kernel.  Two channels per lane, so
// the folded Phi columns of the lane (2 x rows x 2 floats) stay in registers
// across the token loop; workgroup = 512 channels x one token tile.
// ---------------------------------------------------------------------------
template <typename TX, int NM, bool DECAY>
__global__ __launch_bounds__(256) void wgen_dx_fold_kernel(
    const float* __restrict__ g, const TX* __restrict__ res, const TX* __restrict__ br, const float* __restrict__ w,
    const float* __restrict__ coef, int64_t coef_stride, const float* __restrict__ ep, const float* __restrict__ dP,
    int dp_stride, int rows,
    const float* __restrict__ s_tok, const float* __restrict__ phi_pre, const float* __restrict__ phi_post,
    TX* __restrict__ dres, TX* __restrict__ dbr, float* __restrict__ dw_part, int64_t B, int C, int n,
    int64_t tile) {
    const int64_t c0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 2;
    const bool active = c0 < C;  // C % 4 == 0: both channels
    const int64_t t0 = (int64_t)blockIdx.y * tile;
    const int64_t t1 = t0 + tile < B ? t0 + tile : B;
    const int64_t K = (int64_t)n * C;
    constexpr int RW = 2 * NM;  // pre / post rows of dP at most
    float pr[RW][2], pb[RW][2];
#pragma unroll
    for (int o = 0; o < RW; ++o) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            float vr = 0.f, vb = 0.f;
            if (active && o < rows) {
                const float* row = o < n ? phi_pre + (int64_t)o * K : phi_post + (int64_t)(o - n) * K;
                vr = row[c0 + e];
#pragma unroll
                for (int j = 2; j < NM; ++j) {
                    if (j < n && DECAY) vr += kWgMult[j] * row[(int64_t)j * C + c0 + e];
                }
                vb = row[C + c0 + e];
            }
            pr[o][e] = vr;
            pb[o][e] = vb;
        }
    }
    float wv[2] = {0.f, 0.f}, dw[2] = {0.f, 0.f};
    if (active) {
        wv[0] = w[c0];
        wv[1] = w[c0 + 1];
    }
    for (int64_t b = t0; b < t1; ++b) {
        const float* e = ep + b * kWgEp;
        const float e0 = e[0], e1 = e[1], e2 = e[2], e3 = e[3], e4 = e[4], e5 = e[5], e6 = e[6];
        // h_pre from the record (one scalar load with the factors) up to
        // capacity 8, else from the coefficients
        const float* cf = coef + b * coef_stride;
        float hp[NM];
#pragma unroll
        for (int j = 0; j < NM; ++j) hp[j] = NM <= 8 ? e[8 + (j < 8 ? j : 0)] : (j < n ? cf[j] : 0.f);
        const float sv = s_tok[b];
        const float* d = dP + b * dp_stride;
        float dv[RW];
#pragma unroll
        for (int o = 0; o < RW; ++o) dv[o] = o < rows ? d[o] : 0.f;
        if (!active) continue;
        const int64_t off = b * (int64_t)C + c0;
        const float2 gg2 = *reinterpret_cast<const float2*>(g + off);
        const float gv[2] = {gg2.x, gg2.y};
        float rv[2], bv[2];
        wg_load2<TX>(res + off, rv);
        wg_load2<TX>(br + off, bv);
        float dr[2], db[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float xa = wg_xa<TX, NM, DECAY>(rv[q], bv[q], hp, n);
            const float gq = gv[q];
            const float wg = wv[q] * gq;
            float pa = 0.f, pc = 0.f;
#pragma unroll
            for (int o = 0; o < RW; ++o) {
                pa += dv[o] * pr[o][q];
                pc += dv[o] * pb[o][q];
            }
            float xs = rv[q];
#pragma unroll
            for (int j = 2; j < NM; ++j) {
                if (j < n && DECAY) xs += kWgMult[j] * wg_stream<TX, DECAY>(j, rv[q], bv[q]);
            }
            dr[q] = e0 * gq + e1 * wg + e5 * xa + pa + sv * xs;
            db[q] = e2 * gq + e3 * wg + e6 * xa + pc + sv * bv[q];
            dw[q] += e4 * gq * xa;
        }
        if constexpr (sizeof(TX) == 2) {
            *reinterpret_cast<uint32_t*>(dres + off) = pack_bf16x2(dr[0], dr[1]);
            *reinterpret_cast<uint32_t*>(dbr + off) = pack_bf16x2(db[0], db[1]);
        } else {
            *reinterpret_cast<float2*>(dres + off) = make_float2(dr[0], dr[1]);
            *reinterpret_cast<float2*>(dbr + off) = make_float2(db[0], db[1]);
        }
    }
    if (active) {
        dw_part[(int64_t)blockIdx.y * C + c0] = dw[0];
        dw_part[(int64_t)blockIdx.y * C + c0 + 1] = dw[1];
    }
}

// ---------------------------------------------------------------------------
// The stream rows X[b][j*C + c] (x_flat of the layer, layer.py:138) in TO.
// ---------------------------------------------------------------------------
template <typename TX, typename TO, int NM, bool DECAY>
__global__ __launch_bounds__(256) void wgen_synth_kernel(const TX* __restrict__ res, const TX* __restrict__ br,
                                                         TO* __restrict__ X, int64_t B, int C, int n) {
    const int64_t nq = C / 4;
    const int64_t total = B * nq;
    const int64_t K = (int64_t)n * C;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = i / nq;
        const int64_t c0 = (i - b * nq) * 4;
        float rv[4], bv[4];
        load_run_nt<TX, 4>(res + b * C + c0, rv);
        load_run_nt<TX, 4>(br + b * C + c0, bv);
        TO* xb = X + b * K + c0;
#pragma unroll
        for (int j = 0; j < NM; ++j) {
            if (j < n) {
                float x[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) x[q] = wg_stream<TX, DECAY>(j, rv[q], bv[q]);
                store_run<TO, 4>(xb + (int64_t)j * C, x);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
bool wgen_supported(int n, int64_t C) { return n >= 2 && n <= kWgMaxN && C >= 4 && C % 4 == 0 && C <= (1 << 28); }

// capacities of the dPhi / fold kernels (n <= kWgFoldMaxN)
#define MHC_WG_NM(n, ...)                    \
    if ((n) <= 2) {                          \
        constexpr int NM_ = 2; __VA_ARGS__;  \
    } else if ((n) <= 4) {                   \
        constexpr int NM_ = 4; __VA_ARGS__;  \
    } else if ((n) <= 8) {                   \
        constexpr int NM_ = 8; __VA_ARGS__;  \
    } else {                                 \
        constexpr int NM_ = 16; __VA_ARGS__; \
    }

// capacities of the row kernels (n <= kWgMaxN)
#define MHC_WG_NM_WIDE(n, ...)               \
    if ((n) <= 16) {                         \
        MHC_WG_NM(n, __VA_ARGS__)            \
    } else {                                 \
        constexpr int NM_ = 32; __VA_ARGS__; \
    }

// dt x decay x capacity dispatch of one kernel template K<TX, NM, DECAY, ...>
#define MHC_WG_DISPATCH_BY(NMX, dt, decay, n, ...)                            \
    if ((dt) == kBF16) {                                                       \
        using TX_ = bf16_t;                                                    \
        if (decay) { constexpr bool D_ = true; NMX(n, __VA_ARGS__); }          \
        else { constexpr bool D_ = false; NMX(n, __VA_ARGS__); }               \
    } else {                                                                   \
        using TX_ = float;                                                     \
        if (decay) { constexpr bool D_ = true; NMX(n, __VA_ARGS__); }          \
        else { constexpr bool D_ = false; NMX(n, __VA_ARGS__); }               \
    }
#define MHC_WG_DISPATCH(dt, decay, n, ...) MHC_WG_DISPATCH_BY(MHC_WG_NM, dt, decay, n, __VA_ARGS__)
#define MHC_WG_DISPATCH_WIDE(dt, decay, n, ...) MHC_WG_DISPATCH_BY(MHC_WG_NM_WIDE, dt, decay, n, __VA_ARGS__)

hipError_t launch_wgen_fwd(int dt, int n, bool decay, const void* res, const void* br, const float* w,
                           const float* coef, int64_t coef_stride, float* out, int64_t B, int64_t C, float eps,
                           hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!wgen_supported(n, C)) return hipErrorInvalidValue;
    const int64_t blocks = (B + 3) / 4;  // one token per wave
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const int Ci = (int)C;
    const int tok = timing_begin("wrap_fwd", s);
    MHC_WG_DISPATCH_WIDE(dt, decay, n,
                    MHC_LAUNCH_GGL((wgen_fwd_kernel<TX_, NM_, D_>), dim3((unsigned)blocks), dim3(256), 0, s,
                                   (const TX_*)res, (const TX_*)br, w, coef, coef_stride, out, B, Ci, n, eps));
    timing_end(tok, s);
    return hipGetLastError();
}

int wgen_red_static_grid(int64_t B) {
    int64_t g = (B + 3) / 4;
    const int64_t cap = 4 * (int64_t)device_cu_count();
    if (g > cap) g = cap;
    if (g < 1) g = 1;
    return (int)g;
}

hipError_t launch_wgen_red(int dt, int n, bool decay, bool stat, const float* g, const void* res, const void* br,
                           const float* w, const float* coef, int64_t coef_stride, float* scal_out, float* ep_out,
                           int64_t B, int64_t C, float eps, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!wgen_supported(n, C)) return hipErrorInvalidValue;
    const int64_t blocks = stat ? wgen_red_static_grid(B) : (B + 3) / 4;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const int Ci = (int)C;
    const int tok = timing_begin("wrap_bwd_reduce", s);
    if (stat) {
        MHC_WG_DISPATCH_WIDE(dt, decay, n,
                        MHC_LAUNCH_GGL((wgen_red_kernel<TX_, NM_, D_, true>), dim3((unsigned)blocks), dim3(256), 0, s,
                                       g, (const TX_*)res, (const TX_*)br, w, coef, coef_stride, scal_out, ep_out, B,
                                       Ci, n, eps));
    } else {
        MHC_WG_DISPATCH_WIDE(dt, decay, n,
                             MHC_LAUNCH_GGL((wgen_red_kernel<TX_, NM_, D_, false>), dim3((unsigned)blocks), dim3(256),
                                            0, s, g, (const TX_*)res, (const TX_*)br, w, coef, coef_stride, scal_out,
                                            ep_out, B, Ci, n, eps));
    }
    timing_end(tok, s);
    return hipGetLastError();
}

// Token tiles of wgen_dx_kernel: column blocks x tiles about eight
// workgroups per CU, at most one tile per token.
int wgen_dx_tiles(int64_t B, int64_t C) {
    const int64_t gx = (C + 1023) / 1024;
    int64_t tiles = (8 * (int64_t)device_cu_count() + gx - 1) / gx;
    if (tiles > B) tiles = B;
    if (tiles < 1) tiles = 1;
    return (int)tiles;
}

hipError_t launch_wgen_dx(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                          const float* w, const float* coef, int64_t coef_stride, const float* ep, const float* dX,
                          const float* s_tok, void* dres, void* dbr, float* dw_part, int tiles, int64_t B, int64_t C,
                          hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!wgen_supported(n, C) || tiles < 1) return hipErrorInvalidValue;
    if (dX && !s_tok) return hipErrorInvalidValue;
    const int64_t tile = (B + tiles - 1) / tiles;
    const dim3 grid((unsigned)((C + 1023) / 1024), (unsigned)tiles);
    const int Ci = (int)C;
    const int tok = timing_begin("wrap_proj_bwd", s);
    if (dX) {
        MHC_WG_DISPATCH_WIDE(dt, decay, n,
                             MHC_LAUNCH_GGL((wgen_dx_kernel<TX_, NM_, D_, true>), grid, dim3(256), 0, s, g,
                                            (const TX_*)res, (const TX_*)br, w, coef, coef_stride, ep, dX, s_tok,
                                            (TX_*)dres, (TX_*)dbr, dw_part, B, Ci, n, tile));
    } else {
        MHC_WG_DISPATCH_WIDE(dt, decay, n,
                             MHC_LAUNCH_GGL((wgen_dx_kernel<TX_, NM_, D_, false>), grid, dim3(256), 0, s, g,
                                            (const TX_*)res, (const TX_*)br, w, coef, coef_stride, ep, dX, s_tok,
                                            (TX_*)dres, (TX_*)dbr, dw_part, B, Ci, n, tile));
    }
    timing_end(tok, s);
    return hipGetLastError();
}

// Token tiles of wgen_dphi_mfma_kernel: 64-channel column blocks x tiles about
// eight workgroups per CU, at most one tile per token.
int wgen_dphi_tiles(int64_t B, int64_t C) {
    const int64_t gx = (C + kWgDphiCB - 1) / kWgDphiCB;
    int64_t tiles = (8 * (int64_t)device_cu_count() + gx - 1) / gx;
    if (tiles > B) tiles = B;
    if (tiles < 1) tiles = 1;
    return (int)tiles;
}

hipError_t launch_wgen_dphi(int dt, int n, bool decay, const void* res, const void* br, const float* dP,
                            int dp_stride, int rows, float* dphi_part, int tiles, int64_t B, int64_t C,
                            hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!wgen_supported(n, C) || n > kWgFoldMaxN || tiles < 1 || rows < 1 || rows > 2 * n)
        return hipErrorInvalidValue;
    const int64_t tile = (B + tiles - 1) / tiles;
    const dim3 grid((unsigned)((C + kWgDphiCB - 1) / kWgDphiCB), (unsigned)tiles);
    const int Ci = (int)C;
    const int tok = timing_begin("proj_bwd_dphi", s);
    MHC_WG_DISPATCH(dt, decay, n,
                    MHC_LAUNCH_GGL((wgen_dphi_mfma_kernel<TX_, NM_, D_>), grid, dim3(256), 0, s, (const TX_*)res,
                                   (const TX_*)br, dP, dp_stride, rows, dphi_part, B, Ci, n, tile));
    timing_end(tok, s);
    return hipGetLastError();
}

// Token tiles of wgen_dx_fold_kernel: 512-channel column blocks x tiles
// about eight workgroups per CU, each tile at least 64 tokens (every
// workgroup first folds its channels' Phi columns over the n streams: 4n^2
// loads a lane, which a tile of a few tokens would not amortise).
int wgen_fold_tiles(int64_t B, int64_t C) {
    const int64_t gx = (C + 511) / 512;
    int64_t tiles = (8 * (int64_t)device_cu_count() + gx - 1) / gx;
    const int64_t by_tokens = (B + 63) / 64;
    if (tiles > by_tokens) tiles = by_tokens;
    if (tiles < 1) tiles = 1;
    return (int)tiles;
}

hipError_t launch_wgen_dx_fold(int dt, int n, bool decay, const float* g, const void* res, const void* br,
                               const float* w, const float* coef, int64_t coef_stride, const float* ep,
                               const float* dP, int dp_stride, int rows,
                               const float* s_tok, const float* phi_pre, const float* phi_post, void* dres,
                               void* dbr, float* dw_part, int tiles, int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!wgen_supported(n, C) || n > kWgFoldMaxN || tiles < 1 || rows < 1 || rows > 2 * n)
        return hipErrorInvalidValue;
    const int64_t tile = (B + tiles - 1) / tiles;
    const dim3 grid((unsigned)((C + 511) / 512), (unsigned)tiles);
    const int Ci = (int)C;
    const int tok = timing_begin("wrap_proj_bwd", s);
    MHC_WG_DISPATCH(dt, decay, n,
                    MHC_LAUNCH_GGL((wgen_dx_fold_kernel<TX_, NM_, D_>), grid, dim3(256), 0, s, g, (const TX_*)res,
                                   (const TX_*)br, w, coef, coef_stride, ep, dP, dp_stride, rows, s_tok, phi_pre,
                                   phi_post, (TX_*)dres, (TX_*)dbr, dw_part, B, Ci, n, tile));
    timing_end(tok, s);
    return hipGetLastError();
}

hipError_t launch_wgen_synth(int dt, int out_dt, int n, bool decay, const void* res, const void* br, void* X,
                             int64_t B, int64_t C, hipStream_t s) {
    if (B == 0) return hipSuccess;
    if (!wgen_supported(n, C)) return hipErrorInvalidValue;
    int64_t blocks = (B * (C / 4) + 255) / 256;
    const int64_t cap = 16 * (int64_t)device_cu_count();
    if (blocks > cap) blocks = cap;
    const int Ci = (int)C;
    const int tok = timing_begin("wrap_synth", s);
    if (out_dt == kF32) {
        MHC_WG_DISPATCH_WIDE(dt, decay, n,
                             MHC_LAUNCH_GGL((wgen_synth_kernel<TX_, float, NM_, D_>), dim3((unsigned)blocks), dim3(256),
                                            0, s, (const TX_*)res, (const TX_*)br, (float*)X, B, Ci, n));
    } else {
        MHC_WG_DISPATCH_WIDE(dt, decay, n,
                             MHC_LAUNCH_GGL((wgen_synth_kernel<TX_, TX_, NM_, D_>), dim3((unsigned)blocks), dim3(256),
                                            0, s, (const TX_*)res, (const TX_*)br, (TX_*)X, B, Ci, n));
    }
    timing_end(tok, s);
    return hipGetLastError();
}

#undef MHC_WG_DISPATCH_WIDE
#undef MHC_WG_DISPATCH
#undef MHC_WG_DISPATCH_BY
#undef MHC_WG_NM_WIDE
#undef MHC_WG_NM

}  // namespace mhc

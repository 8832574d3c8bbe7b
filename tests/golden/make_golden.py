"""Writes the golden vectors of the mHC path into tests/golden/*.npz.

    python tests/golden/make_golden.py

The reference repository holds no golden vectors, known-answer tests or
fixtures for this path (its only checks are doc snippets of invariants,
docs/troubleshooting.md:226-266), so the vectors here are computed by an
independent float64 restatement: plain numpy loops over the closed-form
forward AND the hand-derived backward formulas of the reference
(bindings.cpp:654-848 for the dynamic layer; rmsnorm.cpp:394-411 for the
RMSNorm adjoint), with the Sinkhorn forward / adjoint of oracle/sinkhorn.c.
Nothing here calls torch autograd or oracle/reference.py, so the fixtures
pin that oracle from the outside (tests/test_golden.py) and the HIP kernels
are checked against them on the GPU.

Inputs are seeded; values that the GPU reads as bf16 are generated
bf16-representable.  Files are small (< 400 KB total) and load with
numpy.load(allow_pickle=False).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import csk  # noqa: E402

ITERS, SK_EPS, RMS_EPS = 20, 1e-8, 1e-5


def bf16_round(a):
    """Round-to-nearest-even to bfloat16, returned as float64."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def sk(a):
    return csk.sinkhorn_fwd(a, ITERS, SK_EPS)


def sk_vjp(g, a):
    return csk.sinkhorn_bwd(g, a, ITERS, SK_EPS)


# ---------------------------------------------------------------------------
# One token row of the layer with activated coefficients, and its adjoint
# (layer.py:143-168; Appendix-style closed forms).
# ---------------------------------------------------------------------------

def row_fwd(x, w, hp, hq, M):
    """x [n, C] -> out [n, C], plus (xa, r, y)."""
    n, C = x.shape
    xa = sum(hp[i] * x[i] for i in range(n))
    r = np.sqrt(np.mean(xa * xa) + RMS_EPS)
    y = xa / r * w
    out = np.empty_like(x)
    for i in range(n):
        out[i] = hq[i] * y + sum(M[i, j] * x[j] for j in range(n))
    return out, xa, r, y


def row_bwd(G, x, w, hp, hq, M):
    """Adjoint of row_fwd for cotangent G [n, C]: (dx, dw, dhp_act, dhq_act, dM)."""
    n, C = x.shape
    _, xa, r, y = row_fwd(x, w, hp, hq, M)
    dM = np.array([[np.dot(G[i], x[j]) for j in range(n)] for i in range(n)])
    dhq = np.array([np.dot(G[i], y) for i in range(n)])
    gy = sum(hq[i] * G[i] for i in range(n))
    dw = gy * xa / r
    dot = np.dot(gy * w, xa)
    gxa = w * gy / r - xa * dot / (C * r ** 3)  # rmsnorm.cpp:394-411
    dx = np.empty_like(x)
    for j in range(n):
        dx[j] = hp[j] * gxa + sum(M[i, j] * G[i] for i in range(n))
    dhp = np.array([np.dot(gxa, x[j]) for j in range(n)])
    return dx, dw, dhp, dhq, dM


# ---------------------------------------------------------------------------
# Cases
# ---------------------------------------------------------------------------

def case_sinkhorn(rng):
    a = np.exp(rng.standard_normal((6, 4, 4)))
    g = rng.standard_normal((6, 4, 4))
    return {"inp": a, "grad_out": g, "out": sk(a), "grad_inp": sk_vjp(g, a)}


def case_ops(rng):
    B, n, C = 5, 4, 64
    x = rng.standard_normal((B, C))
    w = 1.0 + 0.1 * rng.standard_normal(C)
    g = rng.standard_normal((B, C))
    rms = np.sqrt(np.mean(x * x, axis=1) + RMS_EPS)
    y = x / rms[:, None] * w
    dot = np.sum(g * w * x, axis=1)
    gx = w * g / rms[:, None] - x * (dot / (C * rms ** 3))[:, None]
    gw = np.sum(g * x / rms[:, None], axis=0)
    xs = rng.standard_normal((B, n, C))
    H = rng.standard_normal((B, n))
    ga = rng.standard_normal((B, C))
    h = sigmoid(H)
    agg = np.einsum("bi,bic->bc", h, xs)
    agg_gx = h[:, :, None] * ga[:, None, :]
    agg_gh = np.einsum("bc,bic->bi", ga, xs) * h * (1 - h)
    Hq = rng.standard_normal((B, n))
    Mt = sk(np.exp(rng.standard_normal((B, n, n))))
    gd = rng.standard_normal((B, n, C))
    hq = 2 * sigmoid(Hq)
    dist = hq[:, :, None] * x[:, None, :] + np.einsum("bij,bjc->bic", Mt, xs)
    dist_gx = np.einsum("bij,bic->bjc", Mt, gd)
    dist_gy = np.einsum("bi,bic->bc", hq, gd)
    dist_gM = np.einsum("bic,bjc->bij", gd, xs)
    dist_gH = np.einsum("bic,bc->bi", gd, x) * hq * (1 - hq / 2)
    return {"x": x, "w": w, "g": g, "rms": rms, "y": y, "gx": gx, "gw": gw,
            "xs": xs, "H_pre": H, "ga": ga, "agg": agg, "agg_gx": agg_gx, "agg_gH": agg_gh,
            "H_post": Hq, "M": Mt, "gd": gd, "dist": dist, "dist_gx": dist_gx, "dist_gy": dist_gy,
            "dist_gM": dist_gM, "dist_gH": dist_gH}


def static_layer(x, w, H_pre, H_post, H_res, G):
    B, n, C = x.shape
    hp, hq = sigmoid(H_pre), 2 * sigmoid(H_post)
    E = np.exp(H_res)
    M = sk(E[None])[0]
    out = np.empty_like(x)
    dx = np.empty_like(x)
    dw = np.zeros(C)
    dhp = np.zeros(n)
    dhq = np.zeros(n)
    dM = np.zeros((n, n))
    for b in range(B):
        out[b] = row_fwd(x[b], w, hp, hq, M)[0]
        dxb, dwb, dhpb, dhqb, dMb = row_bwd(G[b], x[b], w, hp, hq, M)
        dx[b] = dxb
        dw += dwb
        dhp += dhpb
        dhq += dhqb
        dM += dMb
    dH_res = sk_vjp(dM[None], E[None])[0] * E
    return out, dx, dw, dhp * hp * (1 - hp), dhq * hq * (1 - hq / 2), dH_res


def case_static(rng, x_bf16):
    B, n, C = 6, 4, 64
    x = rng.standard_normal((B, n, C))
    if x_bf16:
        x = bf16_round(x)
    w = bf16_round(1.0 + 0.1 * rng.standard_normal(C))
    H_pre, H_post = rng.standard_normal(n), rng.standard_normal(n)
    H_res = rng.standard_normal((n, n))
    G = rng.standard_normal((B, n, C))
    out, dx, dw, dHp, dHq, dHr = static_layer(x, w, H_pre, H_post, H_res, G)
    return {"x": x, "weight": w, "H_pre": H_pre, "H_post": H_post, "H_res": H_res, "grad": G, "out": out,
            "d_x": dx, "d_weight": dw, "d_H_pre": dHp, "d_H_post": dHq, "d_H_res": dHr}


def dynamic_layer(x, w, phi, alpha, bias, G):
    """phi [np, nC] rows (pre, post, res); alpha [3]; bias [np].  Forward
    bindings.cpp:899-940, backward bindings.cpp:654-848."""
    B, n, C = x.shape
    K = n * C
    out = np.empty_like(x)
    dx = np.empty_like(x)
    dw = np.zeros(C)
    dphi = np.zeros_like(phi)
    dalpha = np.zeros(3)
    dbias = np.zeros_like(bias)
    sl = [slice(0, n), slice(n, 2 * n), slice(2 * n, 2 * n + n * n)]
    for b in range(B):
        xf = x[b].reshape(K)
        r_h = np.sqrt(np.mean(xf * xf) + RMS_EPS)
        P = phi @ xf
        t = np.concatenate([alpha[k] * P[sl[k]] / r_h for k in range(3)]) + bias
        hp, hq = sigmoid(t[sl[0]]), 2 * sigmoid(t[sl[1]])
        E = np.exp(t[sl[2]].reshape(n, n))
        M = sk(E[None])[0]
        out[b] = row_fwd(x[b], w, hp, hq, M)[0]
        dxb, dwb, dhp, dhq, dM = row_bwd(G[b], x[b], w, hp, hq, M)
        dt = np.concatenate([dhp * hp * (1 - hp), dhq * hq * (1 - hq / 2),
                             (sk_vjp(dM[None], E[None])[0] * E).reshape(n * n)])
        dbias += dt
        for k in range(3):
            dalpha[k] += np.dot(dt[sl[k]], P[sl[k]]) / r_h
        dP = np.concatenate([alpha[k] * dt[sl[k]] / r_h for k in range(3)])
        dphi += np.outer(dP, xf)
        d_r = -sum(alpha[k] * np.dot(dt[sl[k]], P[sl[k]]) for k in range(3)) / r_h ** 2
        dxf = dxb.reshape(K) + dP @ phi + d_r * xf / (K * r_h)
        dx[b] = dxf.reshape(n, C)
        dw += dwb
    return out, dx, dw, dphi, dalpha, dbias


def case_dynamic(rng, x_bf16):
    B, n, C = 5, 4, 32
    K = n * C
    npj = 2 * n + n * n
    x = rng.standard_normal((B, n, C))
    if x_bf16:
        x = bf16_round(x)
    w = bf16_round(1.0 + 0.1 * rng.standard_normal(C))
    phi = 0.3 * rng.standard_normal((npj, K))
    alpha = np.array([0.4, 0.3, 0.5])
    bias = 0.3 * rng.standard_normal(npj)
    G = rng.standard_normal((B, n, C))
    out, dx, dw, dphi, dalpha, dbias = dynamic_layer(x, w, phi, alpha, bias, G)
    return {"x": x, "weight": w, "phi": phi, "alpha": alpha, "bias": bias, "grad": G, "out": out, "d_x": dx,
            "d_weight": dw, "d_phi": dphi, "d_alpha": dalpha, "d_bias": dbias}


def case_wrapper(rng):
    """MHCResidualWrapper 'decay' (layer.py:287-322) on bf16 residual/branch
    [B=2, T=3, C=32]: X = [r, b, bf16(r*0.1), bf16(r*0.01)], dynamic layer,
    mean over streams.  Gradients are the exact chain rule through the
    synthesis (d r = dX0 + 0.1 dX2 + 0.01 dX3, d b = dX1)."""
    Bo, T, n, C = 2, 3, 4, 32
    K = n * C
    npj = 2 * n + n * n
    r = bf16_round(rng.standard_normal((Bo, T, C)))
    br = bf16_round(rng.standard_normal((Bo, T, C)))
    w = bf16_round(1.0 + 0.1 * rng.standard_normal(C))
    phi = 0.3 * rng.standard_normal((npj, K))
    alpha = np.array([0.4, 0.3, 0.5])
    bias = 0.3 * rng.standard_normal(npj)
    Gm = rng.standard_normal((Bo, T, C))
    N = Bo * T
    rf, bf = r.reshape(N, C), br.reshape(N, C)
    mult = [float(np.float32(0.1 ** (i - 1))) for i in range(n)]
    X = np.stack([rf, bf] + [bf16_round(rf * mult[i]) for i in range(2, n)], axis=1)
    G = np.repeat(Gm.reshape(N, 1, C), n, axis=1) / n
    out, dX, dw, dphi, dalpha, dbias = dynamic_layer(X, w, phi, alpha, bias, G)
    d_r = dX[:, 0] + sum(mult[i] * dX[:, i] for i in range(2, n))
    return {"residual": r, "branch": br, "weight": w, "phi": phi, "alpha": alpha, "bias": bias, "grad": Gm,
            "out": out.mean(axis=1).reshape(Bo, T, C), "d_residual": d_r.reshape(Bo, T, C),
            "d_branch": dX[:, 1].reshape(Bo, T, C), "d_weight": dw, "d_phi": dphi, "d_alpha": dalpha,
            "d_bias": dbias}


CASES = {
    "sinkhorn": lambda: case_sinkhorn(np.random.default_rng(101)),
    "ops": lambda: case_ops(np.random.default_rng(102)),
    "static_f32": lambda: case_static(np.random.default_rng(103), False),
    "static_bf16": lambda: case_static(np.random.default_rng(104), True),
    "dynamic_f32": lambda: case_dynamic(np.random.default_rng(105), False),
    "dynamic_bf16": lambda: case_dynamic(np.random.default_rng(106), True),
    "wrapper_bf16": lambda: case_wrapper(np.random.default_rng(107)),
}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()

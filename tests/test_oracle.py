"""Pins of the CPU oracle (oracle/reference.py) against mathematics, library
routines and an independent C restatement - never against a retyped copy of
its own formulas.  CPU only."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import csk
from oracle import reference as R
from tests.conftest import assert_close



@pytest.fixture(autouse=True)
def _float64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _pos(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.exp(torch.randn(*shape, generator=g, dtype=torch.float64))


# ---------------------------------------------------------------------------
# Sinkhorn-Knopp
# ---------------------------------------------------------------------------

def test_sinkhorn_doubly_stochastic():
    a = _pos((64, 4, 4), 0)
    m = R.sinkhorn_knopp(a, 20, 1e-8)
    # last step is a column normalisation: column sums are s/(s+eps)
    assert_close(m.sum(-2), torch.ones(64, 4), 0, 1e-7, "col sums")
    assert_close(m.sum(-1), torch.ones(64, 4), 0, 1e-4, "row sums")
    assert bool((m >= 0).all())


def test_sinkhorn_constant_matrix_is_uniform():
    for n in (1, 2, 3, 4, 8):
        a = torch.full((3, n, n), 2.5)
        m = R.sinkhorn_knopp(a, 20, 0.0)
        assert_close(m, torch.full_like(m, 1.0 / n), 1e-15, 0, f"n={n}")


def test_sinkhorn_n1_eps0_is_one():
    a = _pos((5, 1, 1), 1)
    assert_close(R.sinkhorn_knopp(a, 7, 0.0), torch.ones(5, 1, 1), 0, 1e-15, "n=1")


def test_sinkhorn_permutation_equivariance():
    a = _pos((8, 4, 4), 2)
    p = torch.eye(4)[[2, 0, 3, 1]]
    q = torch.eye(4)[[1, 3, 0, 2]]
    lhs = R.sinkhorn_knopp(p @ a @ q, 20, 1e-8)
    rhs = p @ R.sinkhorn_knopp(a, 20, 1e-8) @ q
    assert_close(lhs, rhs, 1e-13, 1e-15, "P A Q")


def test_sinkhorn_diagonal_scaling_invariance_of_limit():
    a = _pos((4, 4, 4), 3)
    d1 = torch.diag_embed(_pos((4, 4), 4))
    d2 = torch.diag_embed(_pos((4, 4), 5))
    lhs = R.sinkhorn_knopp(d1 @ a @ d2, 300, 0.0)
    rhs = R.sinkhorn_knopp(a, 300, 0.0)
    assert_close(lhs, rhs, 0, 1e-9, "D1 A D2")


def test_sinkhorn_matches_c_restatement():
    for n in (1, 3, 4, 6):
        a = _pos((16, n, n), 10 + n)
        for iters in (0, 1, 20):
            ref = torch.from_numpy(csk.sinkhorn_fwd(a.numpy(), iters, 1e-8))
            assert_close(R.sinkhorn_knopp(a, iters, 1e-8), ref, 1e-14, 0, f"fwd n={n} T={iters}")


def test_sinkhorn_bwd_autograd_matches_explicit_adjoint():
    for n in (2, 4, 5):
        a = _pos((16, n, n), 20 + n)
        g = torch.randn(16, n, n, generator=torch.Generator().manual_seed(n))
        for iters in (1, 20, 40):
            ref = torch.from_numpy(csk.sinkhorn_bwd(g.numpy(), a.numpy(), iters, 1e-8))
            assert_close(R.sinkhorn_knopp_bwd(g, a, iters, 1e-8), ref, 1e-10, 1e-13, f"bwd n={n} T={iters}")


def test_sinkhorn_gradcheck():
    a = _pos((2, 3, 3), 30).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: R.sinkhorn_knopp(t, 5, 1e-8), (a,))


def test_sinkhorn_column_constant_cotangent_vanishes():
    # The last step normalises columns, so any cotangent constant down each
    # column (e.g. from loss = sum(y)) has a zero VJP.
    a = _pos((6, 4, 4), 40)
    g = torch.randn(6, 1, 4).expand(6, 4, 4)
    gi = R.sinkhorn_knopp_bwd(g, a, 20, 1e-8)
    assert float(gi.abs().max()) < 1e-12


# ---------------------------------------------------------------------------
# RMSNorm / aggregate / distribute / projection
# ---------------------------------------------------------------------------

def test_rmsnorm_matches_library_rms_norm():
    x = torch.randn(16, 96)
    w = 1 + 0.1 * torch.randn(96)
    y, rms = R.rmsnorm(x, w, 1e-5)
    assert_close(y, F.rms_norm(x, (96,), w, 1e-5), 1e-13, 1e-15, "rms_norm")
    assert_close(rms, torch.sqrt((x * x).mean(-1) + 1e-5), 1e-15, 0, "rms")


def test_rmsnorm_constant_row_closed_form():
    a = 0.37
    x = torch.full((3, 50), a)
    w = torch.linspace(0.5, 1.5, 50)
    y, _ = R.rmsnorm(x, w, 1e-5)
    assert_close(y, (a / math.sqrt(a * a + 1e-5)) * w.expand(3, 50), 1e-14, 0, "closed form")


def test_aggregate_and_distribute_brute_force():
    B, n, C = 3, 4, 5
    x = torch.randn(B, n, C)
    hp = torch.randn(B, n)
    hq = torch.randn(B, n)
    m = _pos((B, n, n), 50)
    y = torch.randn(B, C)
    agg, hact = R.stream_aggregate(x, hp)
    out, qact = R.stream_distribute_mix_add(y, hq, m, x)
    for b in range(B):
        for c in range(C):
            s = sum(1 / (1 + math.exp(-hp[b, i].item())) * x[b, i, c].item() for i in range(n))
            assert abs(agg[b, c].item() - s) < 1e-12
            for i in range(n):
                t = 2 / (1 + math.exp(-hq[b, i].item())) * y[b, c].item()
                t += sum(m[b, i, j].item() * x[b, j, c].item() for j in range(n))
                assert abs(out[b, i, c].item() - t) < 1e-12
    assert_close(hact, torch.sigmoid(hp), 0, 1e-15, "h_pre act")
    assert_close(qact, 2 * torch.sigmoid(hq), 0, 1e-15, "h_post act")


@pytest.mark.parametrize("which", ["rmsnorm", "aggregate", "distribute", "projection"])
def test_op_gradcheck(which):
    g = torch.Generator().manual_seed(7)
    if which == "rmsnorm":
        x = torch.randn(3, 6, generator=g).requires_grad_(True)
        w = torch.randn(6, generator=g).requires_grad_(True)
        f, args = (lambda a, b: R.rmsnorm(a, b, 1e-5)[0]), (x, w)
    elif which == "aggregate":
        x = torch.randn(2, 3, 4, generator=g).requires_grad_(True)
        h = torch.randn(2, 3, generator=g).requires_grad_(True)
        f, args = (lambda a, b: R.stream_aggregate(a, b)[0]), (x, h)
    elif which == "distribute":
        y = torch.randn(2, 4, generator=g).requires_grad_(True)
        h = torch.randn(2, 3, generator=g).requires_grad_(True)
        m = torch.rand(2, 3, 3, generator=g).requires_grad_(True)
        x = torch.randn(2, 3, 4, generator=g).requires_grad_(True)
        f, args = (lambda a, b, c, d: R.stream_distribute_mix_add(a, b, c, d)[0]), (y, h, m, x)
    else:
        x = torch.randn(3, 8, generator=g).requires_grad_(True)
        p = torch.randn(5, 8, generator=g).requires_grad_(True)
        f, args = R.projection, (x, p)
    assert torch.autograd.gradcheck(f, args)


# ---------------------------------------------------------------------------
# Whole layers
# ---------------------------------------------------------------------------

def _static_params(n, C, seed):
    d = R.static_layer_inputs(2, n, C, seed=seed, x_dtype=torch.float64)
    return d


def test_static_layer_gradcheck():
    d = _static_params(4, 8, 1)
    args = [d["x"].double(), d["weight"].double(), d["H_pre"].double(), d["H_post"].double(), d["H_res"].double()]
    args = [a.clone().requires_grad_(True) for a in args]
    f = lambda x, w, a, b, c: R.mhc_layer_static(x, w, a, b, c, 6, 1e-8, 1e-5, dtype=torch.float64)
    assert torch.autograd.gradcheck(f, args)


def test_static_layer_identity_mixing_closed_form():
    # H_res with a dominant diagonal gives M ~= I; H_post -> -inf gives
    # h_post ~= 0, so the layer is the identity on x.
    x = torch.randn(5, 4, 16)
    H_res = 40.0 * torch.eye(4)
    out = R.mhc_layer_static(x, torch.ones(16), torch.zeros(4), torch.full((4,), -60.0), H_res, 20, 0.0, 1e-5,
                             dtype=torch.float64)
    assert_close(out, x, 0, 1e-12, "identity")


def test_static_layer_single_stream_closed_form():
    # n = 1: M = 1 (eps=0), h_pre = sigmoid(a), h_post = 2 sigmoid(b):
    # out = x + h_post * rmsnorm(h_pre * x) * w = x + h_post * rmsnorm(x) * w
    # (RMSNorm is scale invariant up to eps; use eps -> 0).
    x = torch.randn(6, 1, 32)
    w = 1 + 0.1 * torch.randn(32)
    a, b = torch.tensor([0.3]), torch.tensor([-0.7])
    out = R.mhc_layer_static(x, w, a, b, torch.zeros(1, 1), 20, 0.0, 1e-30, dtype=torch.float64)
    want = x[:, 0] + 2 * torch.sigmoid(b) * F.rms_norm(x[:, 0], (32,), w, 1e-30)
    assert_close(out[:, 0], want, 1e-12, 1e-12, "n=1")


def test_dynamic_layer_with_zero_projection_equals_static_layer():
    # phi = 0 makes every token's H equal to the bias: the dynamic layer must
    # reduce to the static layer with H = b.
    n, C = 4, 16
    d = R.dynamic_layer_inputs(3, n, C, seed=3, x_dtype=torch.float64, b_std=1.0)
    z = torch.zeros_like
    dyn = R.mhc_layer_dynamic(d["x"], d["weight"], z(d["phi_pre"]), z(d["phi_post"]), z(d["phi_res"]),
                              d["alpha_pre"], d["alpha_post"], d["alpha_res"], d["b_pre"], d["b_post"], d["b_res"],
                              20, 1e-8, 1e-5, dtype=torch.float64)
    sta = R.mhc_layer_static(d["x"], d["weight"], d["b_pre"], d["b_post"], d["b_res"], 20, 1e-8, 1e-5,
                             dtype=torch.float64)
    assert_close(dyn, sta, 1e-13, 1e-14, "phi=0")


def test_dynamic_layer_gradcheck():
    n, C = 2, 4
    d = R.dynamic_layer_inputs(2, n, C, seed=4, x_dtype=torch.float64, alpha=0.7, phi_std=0.5, b_std=0.5)
    names = ["x", "weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res",
             "b_pre", "b_post", "b_res"]
    args = [d[k].double().clone().requires_grad_(True) for k in names]
    f = lambda *a: R.mhc_layer_dynamic(*a, 4, 1e-8, 1e-5, dtype=torch.float64)
    assert torch.autograd.gradcheck(f, args)


def test_dynamic_backward_matches_reference_formulas():
    """Autograd of the dynamic layer vs the reference's hand-written parameter
    gradients (bindings.cpp:798-848), built from the forward intermediates
    and the C Sinkhorn adjoint: d_b, d_alpha, d_phi and the r_h term."""
    n, C, B = 4, 8, 5
    d = R.dynamic_layer_inputs(B, n, C, seed=6, x_dtype=torch.float64, alpha=0.3, phi_std=0.3, b_std=0.3)
    names = ["x", "weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res",
             "b_pre", "b_post", "b_res"]
    leaf = {k: d[k].double().clone().requires_grad_(True) for k in names}
    co = R.dynamic_h_coefficients(leaf["x"], leaf["phi_pre"], leaf["phi_post"], leaf["phi_res"],
                                  leaf["alpha_pre"], leaf["alpha_post"], leaf["alpha_res"],
                                  leaf["b_pre"], leaf["b_post"], leaf["b_res"], 20, 1e-8, 1e-5)
    h_pre, h_post, M = co["h_pre"], co["h_post"], co["M"]
    h_pre.retain_grad(); h_post.retain_grad(); M.retain_grad()
    out = R._layer_core(leaf["x"], leaf["weight"], h_pre, h_post, M, 1e-5)
    g = torch.randn(B, n, C, generator=torch.Generator().manual_seed(1))
    out.backward(g)
    # reference formulas from the activated-H gradients
    p, r_h = co["p"].detach(), co["r_h"].detach()
    inv = 1 / r_h
    dt_pre = h_pre.grad * h_pre.detach() * (1 - h_pre.detach())
    dt_post = h_post.grad * h_post.detach() * (1 - h_post.detach() / 2)
    E = torch.exp(co["t_res"].detach())
    dE = torch.from_numpy(csk.sinkhorn_bwd(M.grad.numpy(), E.numpy(), 20, 1e-8))
    dt_res = (dE * E).reshape(B, n * n)
    a = [float(d["alpha_pre"]), float(d["alpha_post"]), float(d["alpha_res"])]
    dts = [dt_pre, dt_post, dt_res]
    ps = [p[:, :n], p[:, n:2 * n], p[:, 2 * n:]]
    assert_close(leaf["b_pre"].grad, dt_pre.sum(0), 1e-10, 1e-12, "d_b_pre")
    assert_close(leaf["b_post"].grad, dt_post.sum(0), 1e-10, 1e-12, "d_b_post")
    assert_close(leaf["b_res"].grad.reshape(-1), dt_res.sum(0), 1e-10, 1e-12, "d_b_res")
    for k, nm in enumerate(["alpha_pre", "alpha_post", "alpha_res"]):
        assert_close(leaf[nm].grad, (dts[k] * ps[k] * inv[:, None]).sum(), 1e-10, 1e-12, nm)
    xf = leaf["x"].detach().reshape(B, n * C)
    for k, nm in enumerate(["phi_pre", "phi_post", "phi_res"]):
        dp = dts[k] * (a[k] * inv[:, None])
        assert_close(leaf[nm].grad.reshape(dp.shape[1], -1), dp.t() @ xf, 1e-10, 1e-12, nm)
    # x gradient: stream part from autograd with H held fixed, plus the
    # projection and r_h terms of bindings.cpp:834-848.
    xs = leaf["x"].detach().clone().requires_grad_(True)
    out2 = R._layer_core(xs, leaf["weight"].detach(), h_pre.detach(), h_post.detach(), M.detach(), 1e-5)
    out2.backward(g)
    phi = torch.cat([d["phi_pre"], d["phi_post"], d["phi_res"]], 0).double()
    dp_all = torch.cat([dts[k] * (a[k] * inv[:, None]) for k in range(3)], 1)
    d_r = -sum((dts[k] * a[k] * ps[k]).sum(1) for k in range(3)) * inv * inv
    dx = xs.grad.reshape(B, -1) + dp_all @ phi + d_r[:, None] * xf * (inv[:, None] / (n * C))
    assert_close(leaf["x"].grad.reshape(B, -1), dx, 1e-10, 1e-12, "d_x")


def test_wrapper_stream_synthesis_closed_form():
    # With M ~= I and h_post ~= 0 the layer is the identity, so the wrapper
    # returns the mean of the synthesised streams.
    B, T, C, n = 2, 3, 8, 4
    res = torch.randn(B, T, C)
    br = torch.randn(B, T, C)
    layer = lambda X: R.mhc_layer_static(X, torch.ones(C), torch.zeros(n), torch.full((n,), -60.0),
                                         40.0 * torch.eye(n), 20, 0.0, 1e-5, dtype=torch.float64)
    out = R.mhc_residual_wrapper(res, br, layer, n, "decay")
    assert out.shape == (B, T, C)
    assert_close(out, (res + br + 0.1 * res + 0.01 * res) / 4, 0, 1e-12, "decay mean")
    out0 = R.mhc_residual_wrapper(res[:, 0], br[:, 0], layer, n, "zero")
    assert out0.shape == (B, C)
    assert_close(out0, (res[:, 0] + br[:, 0]) / 4, 0, 1e-12, "zero mean")
    # T == 1 stays flattened (layer.py:319-320)
    assert R.mhc_residual_wrapper(res[:, :1], br[:, :1], layer, n).shape == (B, C)


def test_wrapper_build_streams_matches_differentiable_synthesis():
    res = torch.randn(4, 8).to(torch.bfloat16)
    br = torch.randn(4, 8).to(torch.bfloat16)
    X = R.build_wrapper_streams(res, br, 4, "decay")
    assert X.dtype == torch.bfloat16
    assert torch.equal(X[:, 2], res * 0.1) and torch.equal(X[:, 3], res * (0.1 ** 2))

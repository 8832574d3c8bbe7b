"""Golden vectors (tests/golden/*.npz, written by tests/golden/make_golden.py
from an independent float64 numpy restatement with the reference's
hand-derived backward formulas).

CPU: the PyTorch oracle (float64 autograd) reproduces every vector.
GPU: the HIP path reproduces them within the fp32 / bf16 tolerances.
"""
import os

import numpy as np
import pytest
import torch

from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, grad_atol

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ITERS, SK_EPS, RMS_EPS = 20, 1e-8, 1e-5


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k].copy()) for k in z.files}


def dyn_params(d, n, dtype, device="cpu", grad=False):
    """Fixture projection / alpha / bias split into the layer's parameters."""
    phi = d["phi"].to(dtype)
    bias = d["bias"].to(dtype)
    out = {
        "phi_pre": phi[:n], "phi_post": phi[n:2 * n], "phi_res": phi[2 * n:].contiguous(),
        "alpha_pre": d["alpha"][0].to(dtype), "alpha_post": d["alpha"][1].to(dtype),
        "alpha_res": d["alpha"][2].to(dtype),
        "b_pre": bias[:n], "b_post": bias[n:2 * n], "b_res": bias[2 * n:].reshape(n, n),
    }
    return {k: v.clone().to(device).requires_grad_(grad) for k, v in out.items()}


DYN_ORDER = ["phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post", "b_res"]


def dyn_grads_match(p, d, n, rtol, frac):
    g_phi = torch.cat([p["phi_pre"].grad, p["phi_post"].grad, p["phi_res"].grad], 0)
    assert_close(g_phi, d["d_phi"], rtol, grad_atol(d["d_phi"], frac), "d_phi")
    g_a = torch.stack([p["alpha_pre"].grad, p["alpha_post"].grad, p["alpha_res"].grad])
    assert_close(g_a, d["d_alpha"], rtol, grad_atol(d["d_alpha"], frac), "d_alpha")
    g_b = torch.cat([p["b_pre"].grad, p["b_post"].grad, p["b_res"].grad.reshape(-1)])
    assert_close(g_b, d["d_bias"], rtol, grad_atol(d["d_bias"], frac), "d_bias")


# ---------------------------------------------------------------------------
# CPU: the oracle against the golden vectors
# ---------------------------------------------------------------------------

def test_oracle_sinkhorn_golden():
    d = load("sinkhorn")
    assert_close(R.sinkhorn_knopp(d["inp"], ITERS, SK_EPS), d["out"], 1e-12, 1e-15, "fwd")
    assert_close(R.sinkhorn_knopp_bwd(d["grad_out"], d["inp"], ITERS, SK_EPS), d["grad_inp"], 1e-9, 1e-13, "bwd")


def test_oracle_ops_golden():
    d = load("ops")
    x = d["x"].clone().requires_grad_(True)
    w = d["w"].clone().requires_grad_(True)
    y, rms = R.rmsnorm(x, w, RMS_EPS)
    assert_close(y, d["y"], 1e-12, 1e-14, "rmsnorm y")
    assert_close(rms, d["rms"], 1e-12, 1e-14, "rmsnorm rms")
    y.backward(d["g"])
    assert_close(x.grad, d["gx"], 1e-10, 1e-13, "rmsnorm dx")
    assert_close(w.grad, d["gw"], 1e-10, 1e-13, "rmsnorm dw")
    xs = d["xs"].clone().requires_grad_(True)
    H = d["H_pre"].clone().requires_grad_(True)
    agg, _ = R.stream_aggregate(xs, H)
    assert_close(agg, d["agg"], 1e-12, 1e-14, "aggregate")
    agg.backward(d["ga"])
    assert_close(xs.grad, d["agg_gx"], 1e-10, 1e-13, "aggregate dx")
    assert_close(H.grad, d["agg_gH"], 1e-10, 1e-13, "aggregate dH")
    y2 = d["x"].clone().requires_grad_(True)
    Hq = d["H_post"].clone().requires_grad_(True)
    M = d["M"].clone().requires_grad_(True)
    xs2 = d["xs"].clone().requires_grad_(True)
    out, _ = R.stream_distribute_mix_add(y2, Hq, M, xs2)
    assert_close(out, d["dist"], 1e-12, 1e-14, "distribute")
    out.backward(d["gd"])
    assert_close(xs2.grad, d["dist_gx"], 1e-10, 1e-13, "distribute dx")
    assert_close(y2.grad, d["dist_gy"], 1e-10, 1e-13, "distribute dy")
    assert_close(M.grad, d["dist_gM"], 1e-10, 1e-13, "distribute dM")
    assert_close(Hq.grad, d["dist_gH"], 1e-10, 1e-13, "distribute dH")


@pytest.mark.parametrize("name", ["static_f32", "static_bf16"])
def test_oracle_static_layer_golden(name):
    d = load(name)
    x = d["x"].clone().requires_grad_(True)
    ps = [d[k].clone().requires_grad_(True) for k in ("weight", "H_pre", "H_post", "H_res")]
    out = R.mhc_layer_static(x, *ps, ITERS, SK_EPS, RMS_EPS, dtype=torch.float64)
    assert_close(out, d["out"], 1e-11, 1e-13, "out")
    out.backward(d["grad"])
    assert_close(x.grad, d["d_x"], 1e-9, 1e-12, "d_x")
    for p, k in zip(ps, ("d_weight", "d_H_pre", "d_H_post", "d_H_res")):
        assert_close(p.grad, d[k], 1e-8, grad_atol(d[k], 1e-10), k)


@pytest.mark.parametrize("name", ["dynamic_f32", "dynamic_bf16"])
def test_oracle_dynamic_layer_golden(name):
    d = load(name)
    n = 4
    x = d["x"].clone().requires_grad_(True)
    w = d["weight"].clone().requires_grad_(True)
    p = dyn_params(d, n, torch.float64, grad=True)
    out = R.mhc_layer_dynamic(x, w, *[p[k] for k in DYN_ORDER], ITERS, SK_EPS, RMS_EPS, dtype=torch.float64)
    assert_close(out, d["out"], 1e-11, 1e-13, "out")
    out.backward(d["grad"])
    assert_close(x.grad, d["d_x"], 1e-9, 1e-12, "d_x")
    assert_close(w.grad, d["d_weight"], 1e-8, grad_atol(d["d_weight"], 1e-10), "d_weight")
    dyn_grads_match(p, d, n, 1e-8, 1e-10)


def test_oracle_wrapper_golden():
    """The bf16 stream synthesis of the oracle equals the fixture's
    (bf16(float(r) * float32(0.1**(i-1))), layer.py:307-308) exactly; the
    layer then runs in float64.  Gradients reach the bf16 leaves rounded to
    bf16 by autograd, hence the bf16 tolerance there."""
    d = load("wrapper_bf16")
    n = 4
    r = d["residual"].to(torch.bfloat16).requires_grad_(True)
    b = d["branch"].to(torch.bfloat16).requires_grad_(True)
    w = d["weight"].clone().requires_grad_(True)
    p = dyn_params(d, n, torch.float64, grad=True)
    layer = lambda X: R.mhc_layer_dynamic(X, w, *[p[k] for k in DYN_ORDER], ITERS, SK_EPS, RMS_EPS,
                                          dtype=torch.float64)
    out = R.mhc_residual_wrapper(r, b, layer, n, "decay")
    assert_close(out, d["out"], 1e-11, 1e-13, "out")
    out.backward(d["grad"].to(out.dtype))
    assert_close(r.grad, d["d_residual"], 1e-2, grad_atol(d["d_residual"], 1e-3), "d_residual")
    assert_close(b.grad, d["d_branch"], 1e-2, grad_atol(d["d_branch"], 1e-3), "d_branch")
    assert_close(w.grad, d["d_weight"], 1e-8, grad_atol(d["d_weight"], 1e-10), "d_weight")
    dyn_grads_match(p, d, n, 1e-8, 1e-10)


def test_oracle_wrapper_golden_exact_leaves():
    """storage_dtype=bf16 on float64 leaves: the decay streams take the same
    bf16 values as with bf16 leaves (so the forward equals the fixture), and
    the gradients reach the leaves unrounded: they equal the fixture's exact
    chain rule d r = dX0 + 0.1 dX2 + 0.01 dX3, d b = dX1."""
    d = load("wrapper_bf16")
    n = 4
    r = d["residual"].double().requires_grad_(True)
    b = d["branch"].double().requires_grad_(True)
    w = d["weight"].clone().requires_grad_(True)
    p = dyn_params(d, n, torch.float64, grad=True)
    layer = lambda X: R.mhc_layer_dynamic(X, w, *[p[k] for k in DYN_ORDER], ITERS, SK_EPS, RMS_EPS,
                                          dtype=torch.float64)
    out = R.mhc_residual_wrapper(r, b, layer, n, "decay", storage_dtype=torch.bfloat16)
    assert_close(out, d["out"], 1e-11, 1e-13, "out")
    out.backward(d["grad"].double())
    assert_close(r.grad, d["d_residual"], 1e-9, grad_atol(d["d_residual"], 1e-12), "d_residual")
    assert_close(b.grad, d["d_branch"], 1e-9, grad_atol(d["d_branch"], 1e-12), "d_branch")
    dyn_grads_match(p, d, n, 1e-8, 1e-10)


# ---------------------------------------------------------------------------
# GPU: the HIP path against the golden vectors
# ---------------------------------------------------------------------------

@pytest.mark.gpu
def test_hip_sinkhorn_golden(device):
    import mhc_ascend_amd as mhc
    d = load("sinkhorn")
    a = d["inp"].float().to(device).requires_grad_(True)
    out = mhc.sinkhorn_knopp(a, ITERS, SK_EPS)
    assert_close(out, d["out"], 1e-4, 1e-6, "fwd")
    out.backward(d["grad_out"].float().to(device))
    assert_close(a.grad, d["grad_inp"], 1e-3, grad_atol(d["grad_inp"]), "bwd")


@pytest.mark.gpu
def test_hip_ops_golden(device):
    import mhc_ascend_amd as mhc
    d = load("ops")
    f = lambda k: d[k].float().to(device).requires_grad_(True)
    x, w = f("x"), f("w")
    y = mhc.rmsnorm(x, w, RMS_EPS)
    assert_close(y, d["y"], 1e-4, 1e-6, "rmsnorm y")
    y.backward(d["g"].float().to(device))
    assert_close(x.grad, d["gx"], 1e-3, grad_atol(d["gx"]), "rmsnorm dx")
    assert_close(w.grad, d["gw"], 1e-3, grad_atol(d["gw"]), "rmsnorm dw")
    xs, H = f("xs"), f("H_pre")
    agg = mhc.stream_aggregate(xs, H)
    assert_close(agg, d["agg"], 1e-4, 1e-6, "aggregate")
    agg.backward(d["ga"].float().to(device))
    assert_close(xs.grad, d["agg_gx"], 1e-3, grad_atol(d["agg_gx"]), "aggregate dx")
    assert_close(H.grad, d["agg_gH"], 1e-3, grad_atol(d["agg_gH"]), "aggregate dH")
    y2, Hq, M, xs2 = f("x"), f("H_post"), f("M"), f("xs")
    out = mhc.stream_distribute_mix_add(y2, Hq, M, xs2)
    assert_close(out, d["dist"], 1e-4, 1e-6, "distribute")
    out.backward(d["gd"].float().to(device))
    assert_close(xs2.grad, d["dist_gx"], 1e-3, grad_atol(d["dist_gx"]), "distribute dx")
    assert_close(y2.grad, d["dist_gy"], 1e-3, grad_atol(d["dist_gy"]), "distribute dy")
    assert_close(M.grad, d["dist_gM"], 1e-3, grad_atol(d["dist_gM"]), "distribute dM")
    assert_close(Hq.grad, d["dist_gH"], 1e-3, grad_atol(d["dist_gH"]), "distribute dH")


@pytest.mark.gpu
@pytest.mark.parametrize("name,xdt", [("static_f32", torch.float32), ("static_bf16", torch.bfloat16)])
def test_hip_static_layer_golden(device, name, xdt):
    import mhc_ascend_amd as mhc
    d = load(name)
    x = d["x"].to(xdt).to(device).requires_grad_(True)
    w = d["weight"].to(torch.bfloat16).to(device).requires_grad_(True)
    ps = [d[k].float().to(device).requires_grad_(True) for k in ("H_pre", "H_post", "H_res")]
    out = mhc.mhc_layer_static(x, w, *ps, ITERS, SK_EPS, RMS_EPS)
    assert out.dtype == torch.float32
    assert_close(out, d["out"], 1e-4, 1e-5, "out")
    out.backward(d["grad"].float().to(device))
    if xdt == torch.float32:
        assert_close(x.grad, d["d_x"], 1e-3, grad_atol(d["d_x"], 1e-3), "d_x")
    else:
        assert_close_bf16(x.grad, d["d_x"], "d_x")
    assert_close_bf16(w.grad, d["d_weight"], "d_weight (bf16 param)")
    for p, k in zip(ps, ("d_H_pre", "d_H_post", "d_H_res")):
        assert_close(p.grad, d[k], 1e-3, grad_atol(d[k]), k)


@pytest.mark.gpu
@pytest.mark.parametrize("name,xdt", [("dynamic_f32", torch.float32), ("dynamic_bf16", torch.bfloat16)])
def test_hip_dynamic_layer_golden(device, name, xdt):
    import mhc_ascend_amd as mhc
    d = load(name)
    n = 4
    x = d["x"].to(xdt).to(device).requires_grad_(True)
    w = d["weight"].to(torch.bfloat16).to(device).requires_grad_(True)
    p = dyn_params(d, n, torch.float32, device=device, grad=True)
    out = mhc.mhc_layer_fused_dynamic_training(x, w, *[p[k] for k in DYN_ORDER], ITERS, SK_EPS, RMS_EPS)
    assert_close(out, d["out"], 1e-4, 1e-5, "out")
    out.backward(d["grad"].float().to(device))
    if xdt == torch.bfloat16:
        assert_close_bf16(x.grad, d["d_x"], "d_x")
    else:
        assert_close(x.grad, d["d_x"], 1e-3, grad_atol(d["d_x"], 1e-3), "d_x")
    assert_close_bf16(w.grad, d["d_weight"], "d_weight (bf16 param)")
    dyn_grads_match(p, d, n, 1e-3, 1e-4)


@pytest.mark.gpu
def test_hip_wrapper_golden(device):
    import mhc_ascend_amd as mhc
    d = load("wrapper_bf16")
    n, C = 4, d["residual"].shape[-1]
    torch.manual_seed(0)
    wrap = mhc.MHCResidualWrapper(C, n).to(device)
    layer = wrap.mhc
    p = dyn_params(d, n, torch.float32)
    with torch.no_grad():
        layer.rmsnorm_weight.copy_(d["weight"].to(torch.bfloat16))
        for k in DYN_ORDER:
            getattr(layer, k).copy_(p[k])
    r = d["residual"].to(torch.bfloat16).to(device).requires_grad_(True)
    b = d["branch"].to(torch.bfloat16).to(device).requires_grad_(True)
    out = wrap(r, b)
    assert out.dtype == torch.float32 and out.shape == d["out"].shape
    assert_close(out, d["out"], 1e-4, 1e-5, "out")
    out.backward(d["grad"].float().to(device))
    assert_close_bf16(r.grad, d["d_residual"], "d_residual")
    assert_close_bf16(b.grad, d["d_branch"], "d_branch")
    gp = {k: getattr(layer, k) for k in DYN_ORDER}
    dyn_grads_match(gp, d, n, 1e-3, 1e-4)
    assert_close_bf16(layer.rmsnorm_weight.grad, d["d_weight"], "d_weight")

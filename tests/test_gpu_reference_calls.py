"""The reference's dynamic-H native pair called with the reference's own call
shapes: the forward returns nine tensors that its autograd Function unpacks
(ops.py:425-448), the backward takes them back with 23 arguments, alphas as
Python floats (ops.py:518-542).  `RefShapedDynamic` below makes exactly those
calls against `mhc_ascend_amd.native`, so it reads as the reference's
MHCLayerDynamicFunction would with this library bound as its native module.

Checked against the float64 oracle at the C4 shape's n and C (n = 4,
C = 4096), for fp32 x (what the reference's ops.py passes, ops.py:622) and
bf16 x; against the fused entries at the full C4 size; and at n = 8 and
n = 32 (several projection tiles, the streaming projection)."""
import pytest
import torch

from mhc_ascend_amd import native
from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, assert_close_dyn_dx_bf16, grad_atol

pytestmark = pytest.mark.gpu

PARAMS = ["weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post",
          "b_res"]


class RefShapedDynamic(torch.autograd.Function):
    """Forward / backward through the nine-tensor forward and the
    23-argument backward of the native module."""

    @staticmethod
    def forward(ctx, x, weight, phi_pre, phi_post, phi_res, a_pre, a_post, a_res, b_pre, b_post, b_res, iters,
                sk_eps, rms_eps):
        n = phi_pre.size(0)
        phi_concat = torch.cat([phi_pre, phi_post, phi_res.reshape(n * n, -1)], dim=0).contiguous()
        outs = native.mhc_layer_fwd_dynamic(x, weight, phi_concat, float(a_pre.item()), float(a_post.item()),
                                            float(a_res.item()), b_pre, b_post, b_res, iters, sk_eps, rms_eps)
        assert len(outs) == 9
        output, rms, x_agg, h_pre, h_post, M, y_norm, x_flat, rms_h = outs
        ctx.save_for_backward(x, weight, rms, x_agg, h_pre, h_post, M, y_norm, x_flat, rms_h, phi_pre, phi_post,
                              phi_res, b_pre, b_post, b_res, a_pre, a_post, a_res)
        ctx.cfg = (iters, sk_eps, rms_eps)
        ctx.fwd = outs
        return output

    @staticmethod
    def backward(ctx, grad_output):
        (x, weight, rms, x_agg, h_pre, h_post, M, y_norm, x_flat, rms_h, phi_pre, phi_post, phi_res, b_pre, b_post,
         b_res, a_pre, a_post, a_res) = ctx.saved_tensors
        iters, sk_eps, rms_eps = ctx.cfg
        grads = native.mhc_layer_bwd_dynamic(
            grad_output.contiguous(), x, weight, rms, x_agg, h_pre, h_post, M, y_norm, x_flat, rms_h, phi_pre,
            phi_post, phi_res, float(a_pre.item()), float(a_post.item()), float(a_res.item()), b_pre, b_post, b_res,
            iters, sk_eps, rms_eps)
        assert len(grads) == 11
        gx, gw, gpp, gpq, gpr, gap, gaq, gar, gbp, gbq, gbr = grads
        return (gx, gw, gpp, gpq, gpr, gap.view_as(a_pre), gaq.view_as(a_post), gar.view_as(a_res), gbp, gbq, gbr,
                None, None, None)


def _run(d, device, x_dtype, iters=20, sk_eps=1e-8, rms_eps=1e-5):
    x = d["x"].to(x_dtype).to(device).requires_grad_(True)
    ps = [d[k].to(device).requires_grad_(True) for k in PARAMS]
    captured = {}

    class Probe(RefShapedDynamic):
        @staticmethod
        def forward(ctx, *args):
            out = RefShapedDynamic.forward(ctx, *args)
            captured["fwd"] = ctx.fwd
            return out

    out = Probe.apply(x, *ps, iters, sk_eps, rms_eps)
    out.backward(d["grad"].to(device))
    return out.detach(), x.grad, [p.grad for p in ps], captured["fwd"]


def _oracle(d, x_dtype, iters=20, sk_eps=1e-8, rms_eps=1e-5):
    x = d["x"].to(x_dtype).double().requires_grad_(True)
    ps = [d[k].double().requires_grad_(True) for k in PARAMS]
    out = R.mhc_layer_dynamic(x, *ps, iters, sk_eps, rms_eps, dtype=torch.float64)
    out.backward(d["grad"].double())
    with torch.no_grad():
        co = R.dynamic_h_coefficients(x.detach(), *[p.detach() for p in ps[1:]], iters, sk_eps, rms_eps)
        x_agg = (co["h_pre"].unsqueeze(-1) * x.detach()).sum(dim=1)
        y, rms = R.rmsnorm(x_agg, ps[0].detach(), rms_eps)
    inter = {"rms": rms, "x_agg": x_agg, "h_pre": co["h_pre"], "h_post": co["h_post"], "M": co["M"], "y_norm": y,
             "rms_h": co["r_h"]}
    return out.detach(), x.grad, [p.grad for p in ps], inter


def _check(got, want, x_dtype, tag):
    out, gx, gp, fwd = got
    rout, rgx, rgp, inter = want
    assert_close(out, rout, 1e-4, 1e-5, f"{tag} output")
    output, rms, x_agg, h_pre, h_post, M, y_norm, x_flat, rms_h = fwd
    B, n, C = out.shape
    assert output.dtype == torch.float32 and tuple(output.shape) == (B, n, C)
    for nm, t, shape in (("rms", rms, (B,)), ("h_pre", h_pre, (B, n)), ("h_post", h_post, (B, n)),
                         ("M", M, (B, n, n)), ("rms_h", rms_h, (B,))):
        assert t.dtype == torch.float32 and tuple(t.shape) == shape, (nm, t.dtype, tuple(t.shape))
        assert_close(t, inter[nm], 1e-4, 1e-6, f"{tag} {nm}")
    for nm, t, shape in (("x_agg", x_agg, (B, C)), ("y_norm", y_norm, (B, C))):
        assert tuple(t.shape) == shape
        assert_close_bf16(t, inter[nm], f"{tag} {nm}")
    assert x_flat.dtype == torch.bfloat16 and tuple(x_flat.shape) == (B, n * C)
    if x_dtype == torch.bfloat16:
        assert gx.dtype == torch.bfloat16
        assert_close_dyn_dx_bf16(gx, rgx, f"{tag} grad_x")
    else:
        assert gx.dtype == torch.float32
        assert_close(gx, rgx, 1e-3, grad_atol(rgx, 1e-5), f"{tag} grad_x")
    for nm, a, e in zip(PARAMS, gp, rgp):
        assert a is not None, f"{tag}: no gradient for {nm}"
        if nm == "weight":
            # the parameter is bf16; autograd casts the fp32 gradient to it
            assert_close_bf16(a, e, f"{tag} d_weight")
        else:
            assert_close(a, e, 1e-3, grad_atol(e, 1e-4), f"{tag} d_{nm}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_reference_call_shapes_c4_width(device, x_dtype):
    """n = 4, C = 4096 (the C4 shape's row), 24 tokens, b != 0 and alpha 0.3
    so that every parameter gradient is well away from zero."""
    d = R.dynamic_layer_inputs(24, 4, 4096, seed=71, alpha=0.3, b_std=0.5)
    got = _run(d, device, x_dtype)
    _check(got, _oracle(d, x_dtype), x_dtype, f"C4 width {x_dtype}")
    assert torch.equal(got[3][7].cpu(), d["x"].to(x_dtype).bfloat16().reshape(24, -1))


@pytest.mark.parametrize("n,B,C", [(2, 9, 320), (8, 20, 1280), (32, 5, 256)])
def test_reference_call_shapes_general_n(device, n, B, C):
    """Several projection tiles (n = 8: 80 rows) and the streaming projection
    (n = 32: 1088 rows) through the same nine-tensor / 23-argument calls."""
    d = R.dynamic_layer_inputs(B, n, C, seed=7 * n + B, alpha=0.3, phi_std=0.05, b_std=0.5)
    got = _run(d, device, torch.float32)
    _check(got, _oracle(d, torch.float32), torch.float32, f"n={n} B={B} C={C}")


def test_reference_call_shapes_full_c4_match_fused_entries(device):
    """Full C4 size (x bf16 [8192, 4, 4096]): the 23-argument backward on the
    nine forward tensors gives the fused entries' gradients (it rebuilds
    their saved state from the nine tensors and a recomputed P)."""
    B, n, C = 8192, 4, 4096
    d = R.dynamic_layer_inputs(B, n, C, seed=45)
    dev = {k: v.to(device) for k, v in d.items()}
    x, g = dev["x"], dev["grad"]
    w = dev["weight"]
    pp, pq, pr = dev["phi_pre"], dev["phi_post"], dev["phi_res"]
    a = [float(dev[k].item()) for k in ("alpha_pre", "alpha_post", "alpha_res")]
    bp, bq, br = dev["b_pre"], dev["b_post"], dev["b_res"]
    phi_concat = torch.cat([pp, pq, pr.reshape(n * n, -1)], dim=0)
    fwd = native.mhc_layer_fwd_dynamic(x, w, phi_concat, *a, bp, bq, br, 20, 1e-8, 1e-5)
    ref_grads = native.mhc_layer_bwd_dynamic(g, x, w, *fwd[1:], pp, pq, pr, *a, bp, bq, br, 20, 1e-8, 1e-5)
    # the fused entries with the fp32 copy of the weight return an fp32
    # weight gradient, as the reference-shaped backward does
    w32 = w.float()
    alphas = [dev[k] for k in ("alpha_pre", "alpha_post", "alpha_res")]
    out, saved = native.mhc_layer_dynamic_fwd(x, w32, pp, pq, pr, *alphas, bp, bq, br)
    fused = native.mhc_layer_dynamic_bwd(g, x, w32, saved, pp, pq, pr, *alphas, bp, bq, br)
    assert torch.equal(fwd[0], out), "nine-tensor forward output differs from the fused forward"
    names = ["grad_x", "d_weight", "d_phi_pre", "d_phi_post", "d_phi_res", "d_alpha_pre", "d_alpha_post",
             "d_alpha_res", "d_b_pre", "d_b_post", "d_b_res"]
    for nm, r, f in zip(names, ref_grads, fused):
        r = r.reshape(f.shape).to(torch.float64)
        f = f.to(torch.float64)
        assert_close(r, f, 1e-5, grad_atol(f, 1e-6), f"full C4 {nm}: reference-shaped vs fused")
    # and the forward tensors against the oracle on a token subsample
    idx = torch.randperm(B, generator=torch.Generator().manual_seed(9))[:16]
    sub = {k: (v[idx] if k in ("x", "grad") else v) for k, v in d.items()}
    _, _, _, inter = _oracle(sub, torch.bfloat16)
    for k, nm in ((3, "h_pre"), (4, "h_post"), (5, "M"), (8, "rms_h"), (1, "rms")):
        assert_close(fwd[k].cpu()[idx], inter[nm], 1e-4, 1e-6, f"full C4 {nm} subsample")
    assert_close_bf16(fwd[6].cpu()[idx], inter["y_norm"], "full C4 y_norm subsample")


def test_reference_call_shapes_argument_errors(device):
    x = torch.randn(3, 4, 64, device=device)
    w = torch.ones(64, device=device, dtype=torch.bfloat16)
    b = torch.zeros(4, device=device)
    with pytest.raises(RuntimeError, match="phi_concat"):
        native.mhc_layer_fwd_dynamic(x, w, torch.zeros(23, 256, device=device), 0.01, 0.01, 0.01, b, b,
                                     torch.zeros(4, 4, device=device))
    with pytest.raises(RuntimeError, match="phi_concat"):
        native.mhc_layer_fwd_dynamic(x, w, torch.zeros(24 * 256, device=device), 0.01, 0.01, 0.01, b, b,
                                     torch.zeros(4, 4, device=device))
    with pytest.raises(RuntimeError, match="3D"):
        native.mhc_layer_bwd_dynamic(torch.zeros(3, 256, device=device), x, w, None, None, None, None, None, None,
                                     None, None, None, None, None, 0.01, 0.01, 0.01, b, b, b)
    empty = native.mhc_layer_fwd_dynamic(torch.zeros(0, 4, 64, device=device), w,
                                         torch.zeros(24, 256, device=device), 0.01, 0.01, 0.01, b, b,
                                         torch.zeros(4, 4, device=device))
    assert [tuple(t.shape) for t in empty] == [(0, 4, 64), (0,), (0, 64), (0, 4), (0, 4), (0, 4, 4), (0, 64),
                                               (0, 256), (0,)]

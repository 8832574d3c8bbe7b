"""Module compatibility on the GPU: layers built by the reference's factories
(create_mhc_layer, layer.py:186-218; replace_residual_with_mhc, layer.py:
332-353) load a state_dict in the reference's layout (names, shapes and
dtypes of layer.py:64-85, bf16 rmsnorm_weight, wrapper keys under 'mhc.')
with strict=True, then run forward + backward on cuda:0 against the float64
oracle evaluated on the same state_dict values."""
import pytest
import torch

from mhc_ascend_amd import create_mhc_layer, replace_residual_with_mhc
from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, grad_atol

pytestmark = pytest.mark.gpu

DYN = ["phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post", "b_res"]
STA = ["H_pre", "H_post", "H_res"]


def reference_state_dict(n, C, dynamic, seed, prefix=""):
    """Values in the reference module's layout (layer.py:64-85: bf16 weight
    first, then the projections, biases and scalar alphas, or H_pre, H_post,
    H_res), drawn so every gradient is well away from zero."""
    g = torch.Generator().manual_seed(seed)
    nC = n * C
    sd = {"rmsnorm_weight": (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16)}
    if dynamic:
        sd["phi_pre"] = 0.05 * torch.randn(n, nC, generator=g)
        sd["phi_post"] = 0.05 * torch.randn(n, nC, generator=g)
        sd["phi_res"] = 0.05 * torch.randn(n * n, nC, generator=g)
        sd["b_pre"] = 0.5 * torch.randn(n, generator=g)
        sd["b_post"] = 0.5 * torch.randn(n, generator=g)
        sd["b_res"] = 0.5 * torch.randn(n, n, generator=g)
        sd["alpha_pre"] = torch.tensor(0.2)
        sd["alpha_post"] = torch.tensor(0.3)
        sd["alpha_res"] = torch.tensor(0.4)
    else:
        sd["H_pre"] = torch.randn(n, generator=g)
        sd["H_post"] = torch.randn(n, generator=g)
        sd["H_res"] = torch.randn(n, n, generator=g)
    return {prefix + k: v for k, v in sd.items()}


def _oracle_layer_fn(sd, dynamic, iters, sk_eps, rms_eps, prefix=""):
    w = sd[prefix + "rmsnorm_weight"].double().requires_grad_(True)
    names = DYN if dynamic else STA
    ps = [sd[prefix + k].double().requires_grad_(True) for k in names]
    if dynamic:
        fn = lambda X: R.mhc_layer_dynamic(X, w, *ps, iters, sk_eps, rms_eps, dtype=torch.float64)
    else:
        fn = lambda X: R.mhc_layer_static(X, w, *ps, iters, sk_eps, rms_eps, dtype=torch.float64)
    return fn, w, ps


@pytest.mark.parametrize("dynamic", [True, False])
@pytest.mark.parametrize("n,C", [(4, 512), (2, 256), (8, 128)])
def test_factory_layer_with_reference_state_dict(device, dynamic, n, C):
    iters, sk_eps, rms_eps = 12, 1e-7, 1e-6
    layer = create_mhc_layer(C, expansion_rate=n, num_sinkhorn_iters=iters, sinkhorn_eps=sk_eps,
                             rmsnorm_eps=rms_eps, use_dynamic_h=dynamic)
    sd = reference_state_dict(n, C, dynamic, seed=10 * n + C + dynamic)
    missing, unexpected = layer.load_state_dict(sd, strict=True)
    assert not missing and not unexpected
    assert layer.rmsnorm_weight.dtype == torch.bfloat16
    layer = layer.to(device)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(19, n, C, generator=g)
    grad = torch.randn(19, n, C, generator=g)
    xd = x.to(device).requires_grad_(True)
    out = layer(xd)
    out.backward(grad.to(device))

    fn, w, ps = _oracle_layer_fn(sd, dynamic, iters, sk_eps, rms_eps)
    xr = x.double().requires_grad_(True)
    ref = fn(xr)
    ref.backward(grad.double())
    tag = f"{'dynamic' if dynamic else 'static'} n={n} C={C}"
    assert out.dtype == torch.float32
    assert_close(out, ref.detach(), 1e-4, 1e-5, f"{tag} out")
    assert_close(xd.grad, xr.grad, 1e-3, grad_atol(xr.grad, 1e-5), f"{tag} dx")
    assert_close_bf16(layer.rmsnorm_weight.grad, w.grad, f"{tag} d_rmsnorm_weight")
    for nm, p in zip(DYN if dynamic else STA, ps):
        assert_close(getattr(layer, nm).grad, p.grad, 1e-3, grad_atol(p.grad, 1e-4), f"{tag} d_{nm}")
    # eval mode: the forward-only path on the same parameters
    layer.eval()
    with torch.no_grad():
        assert_close(layer(x.to(device)), ref.detach(), 1e-4, 1e-5, f"{tag} eval out")


@pytest.mark.parametrize("dynamic", [True, False])
@pytest.mark.parametrize("mode", ["decay", "zero"])
def test_replace_residual_with_mhc_reference_state_dict(device, dynamic, mode):
    """The wrapper factory, a reference-layout checkpoint under 'mhc.', bf16
    residual and branch [B, T, C]; the fused wrapper kernels (n = 4)."""
    n, C = 4, 384
    wrap = replace_residual_with_mhc(C, expansion_rate=n, residual_mode=mode, use_dynamic_h=dynamic)
    sd = reference_state_dict(n, C, dynamic, seed=31 + dynamic, prefix="mhc.")
    missing, unexpected = wrap.load_state_dict(sd, strict=True)
    assert not missing and not unexpected
    wrap = wrap.to(device)
    g = torch.Generator().manual_seed(4)
    res = torch.randn(6, 5, C, generator=g).to(torch.bfloat16)
    br = torch.randn(6, 5, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(6, 5, C, generator=g)
    r = res.to(device).requires_grad_(True)
    b = br.to(device).requires_grad_(True)
    out = wrap(r, b)
    out.backward(grad.to(device))

    fn, w, ps = _oracle_layer_fn(sd, dynamic, 20, 1e-8, 1e-5, prefix="mhc.")
    rr = res.double().requires_grad_(True)
    rb = br.double().requires_grad_(True)
    ref = R.mhc_residual_wrapper(rr, rb, fn, n, mode, storage_dtype=torch.bfloat16)
    ref.backward(grad.double())
    tag = f"wrapper {'dynamic' if dynamic else 'static'} {mode}"
    assert tuple(out.shape) == (6, 5, C) and out.dtype == torch.float32
    assert_close(out, ref.detach(), 1e-4, grad_atol(ref.detach(), 1e-5), f"{tag} out")
    assert_close_bf16(r.grad, rr.grad, f"{tag} d residual")
    assert_close_bf16(b.grad, rb.grad, f"{tag} d branch")
    assert_close_bf16(wrap.mhc.rmsnorm_weight.grad, w.grad, f"{tag} d_rmsnorm_weight")
    for nm, p in zip(DYN if dynamic else STA, ps):
        if nm.endswith("res"):
            # every stream gets G / n through the mean, so the H_res-side
            # gradients vanish up to rounding (see test_gpu_wrapper)
            continue
        assert_close(getattr(wrap.mhc, nm).grad, p.grad, 1e-3, grad_atol(p.grad, 1e-4), f"{tag} d_{nm}")

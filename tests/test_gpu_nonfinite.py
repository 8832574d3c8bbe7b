"""Non-finite inputs on the GPU: a NaN or an infinity in one token of x (or
of the wrapper's residual) must reach the same outputs and gradients as on
the float64 oracle (ops_pytorch_backward.py, layer.py:94-179, 269-322): the
token's outputs and input gradient and every parameter gradient that sums
over it are non-finite, the other tokens stay finite.  Compared element by
element through the masks of torch.isfinite.  The fused wrapper's H_res
gradients, exact zeros for finite inputs (the stream mean makes dM constant
down each column), are non-finite here as the oracle's are."""
import pytest
import torch

import mhc_ascend_amd as mhc
from oracle import reference as R

pytestmark = pytest.mark.gpu

STA = ["H_pre", "H_post", "H_res"]
DYN = ["phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post", "b_res"]


def _masks_match(got, want, what):
    gm = torch.isfinite(got.detach().float().cpu())
    wm = torch.isfinite(want.detach().cpu())
    bad = (gm != wm).sum().item()
    assert bad == 0, f"{what}: finiteness differs at {bad} of {gm.numel()} elements"


def _plant(t, value, idx):
    t = t.clone()
    t[idx] = value
    return t


@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("value", [float("nan"), float("inf")])
def test_layer_nonfinite_token(device, dynamic, value):
    torch.manual_seed(3)
    layer = mhc.MHCLayer(64, 4, use_dynamic_h=dynamic)
    g = torch.Generator().manual_seed(7)
    x = _plant(torch.randn(5, 4, 64, generator=g), value, (2, 1, 9))
    go = torch.randn(5, 4, 64, generator=g)
    names = DYN if dynamic else STA
    # float64 oracle
    w = layer.rmsnorm_weight.detach().double().requires_grad_(True)
    ps = [getattr(layer, k).detach().double().requires_grad_(True) for k in names]
    xr = x.double().requires_grad_(True)
    fn = R.mhc_layer_dynamic if dynamic else R.mhc_layer_static
    ref = fn(xr, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    ref.backward(go.double())
    # GPU
    layer = layer.to(device)
    xd = x.to(device).requires_grad_(True)
    out = layer(xd)
    out.backward(go.to(device))
    _masks_match(out, ref, "out")
    _masks_match(xd.grad, xr.grad, "dx")
    _masks_match(layer.rmsnorm_weight.grad, w.grad, "d weight")
    for k, p in zip(names, ps):
        _masks_match(getattr(layer, k).grad, p.grad, f"d {k}")
    # the other tokens are untouched
    keep = [0, 1, 3, 4]
    assert torch.isfinite(out[keep]).all() and torch.isfinite(xd.grad[keep]).all()


@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("value", [float("nan"), float("inf")])
def test_wrapper_nonfinite_token(device, dynamic, dtype, value):
    torch.manual_seed(4)
    wrap = mhc.MHCResidualWrapper(64, 4, use_dynamic_h=dynamic)
    g = torch.Generator().manual_seed(8)
    res = _plant(torch.randn(6, 64, generator=g), value, (4, 17)).to(dtype)
    br = torch.randn(6, 64, generator=g).to(dtype)
    go = torch.randn(6, 64, generator=g)
    layer = wrap.mhc
    names = DYN if dynamic else STA
    w = layer.rmsnorm_weight.detach().double().requires_grad_(True)
    ps = [getattr(layer, k).detach().double().requires_grad_(True) for k in names]
    r = res.double().requires_grad_(True)
    b = br.double().requires_grad_(True)
    if dynamic:
        fn = lambda X: R.mhc_layer_dynamic(X, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    else:
        fn = lambda X: R.mhc_layer_static(X, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    ref = R.mhc_residual_wrapper(r, b, fn, 4, "decay", storage_dtype=dtype)
    ref.backward(go.double())
    wrap = wrap.to(device)
    rd = res.to(device).requires_grad_(True)
    bd = br.to(device).requires_grad_(True)
    out = wrap(rd, bd)
    out.backward(go.to(device))
    _masks_match(out, ref, "out")
    _masks_match(rd.grad, r.grad, "d residual")
    _masks_match(bd.grad, b.grad, "d branch")
    _masks_match(wrap.mhc.rmsnorm_weight.grad, w.grad, "d weight")
    for k, p in zip(names, ps):
        _masks_match(getattr(wrap.mhc, k).grad, p.grad, f"d {k}")
    keep = [0, 1, 2, 3, 5]
    assert torch.isfinite(out[keep]).all()
    assert torch.isfinite(rd.grad[keep]).all() and torch.isfinite(bd.grad[keep]).all()

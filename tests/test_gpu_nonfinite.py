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


@pytest.mark.parametrize("n", [4, 5, 16])
@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("value", [float("nan"), float("inf")])
def test_wrapper_nonfinite_token(device, n, dynamic, dtype, value):
    torch.manual_seed(4)
    wrap = mhc.MHCResidualWrapper(64, n, use_dynamic_h=dynamic)
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
    ref = R.mhc_residual_wrapper(r, b, fn, n, "decay", storage_dtype=dtype)
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


def _leaves(device, *ts):
    return [t.to(device).requires_grad_(True) for t in ts], [t.double().requires_grad_(True) for t in ts]


@pytest.mark.parametrize("value", [float("nan"), float("inf")])
def test_operators_nonfinite(device, value):
    g = torch.Generator().manual_seed(9)
    # Sinkhorn: one entry of one matrix
    a = _plant(torch.rand(6, 4, 4, generator=g) + 0.1, value, (3, 1, 2))
    ga = torch.randn(6, 4, 4, generator=g)
    (ad,), (ar,) = _leaves(device, a)
    out = mhc.sinkhorn_knopp(ad, 20, 1e-8)
    ref = R.sinkhorn_knopp(ar, 20, 1e-8)
    out.backward(ga.to(device))
    ref.backward(ga.double())
    _masks_match(out, ref, "sinkhorn out")
    _masks_match(ad.grad, ar.grad, "sinkhorn d inp")
    # RMSNorm: one channel of one row
    x = _plant(torch.randn(5, 96, generator=g), value, (2, 40))
    w = 1 + 0.1 * torch.randn(96, generator=g)
    gy = torch.randn(5, 96, generator=g)
    (xd, wd), (xr, wr) = _leaves(device, x, w)
    y = mhc.rmsnorm(xd, wd, 1e-5)
    yr, _ = R.rmsnorm(xr, wr, 1e-5)
    y.backward(gy.to(device))
    yr.backward(gy.double())
    _masks_match(y, yr, "rmsnorm out")
    _masks_match(xd.grad, xr.grad, "rmsnorm dx")
    _masks_match(wd.grad, wr.grad, "rmsnorm dw")
    # stream aggregate: one element of x
    xs = _plant(torch.randn(5, 4, 96, generator=g), value, (1, 2, 7))
    H = torch.randn(5, 4, generator=g)
    go = torch.randn(5, 96, generator=g)
    (xsd, Hd), (xsr, Hr) = _leaves(device, xs, H)
    o = mhc.stream_aggregate(xsd, Hd)
    orf, _ = R.stream_aggregate(xsr, Hr)
    o.backward(go.to(device))
    orf.backward(go.double())
    _masks_match(o, orf, "aggregate out")
    _masks_match(xsd.grad, xsr.grad, "aggregate dx")
    _masks_match(Hd.grad, Hr.grad, "aggregate dH")
    # stream distribute: one element of y
    yv = _plant(torch.randn(5, 96, generator=g), value, (3, 11))
    Hp = torch.randn(5, 4, generator=g)
    M = torch.rand(5, 4, 4, generator=g)
    x2 = torch.randn(5, 4, 96, generator=g)
    g2 = torch.randn(5, 4, 96, generator=g)
    (yd, Hpd, Md, x2d), (yr2, Hpr, Mr, x2r) = _leaves(device, yv, Hp, M, x2)
    d = mhc.stream_distribute_mix_add(yd, Hpd, Md, x2d)
    dr, _ = R.stream_distribute_mix_add(yr2, Hpr, Mr, x2r)
    d.backward(g2.to(device))
    dr.backward(g2.double())
    for got, want, what in ((d, dr, "distribute out"), (yd.grad, yr2.grad, "distribute dy"),
                            (Hpd.grad, Hpr.grad, "distribute dH"), (Md.grad, Mr.grad, "distribute dM"),
                            (x2d.grad, x2r.grad, "distribute dx")):
        _masks_match(got, want, what)


@pytest.mark.parametrize("dynamic", [False, True])
def test_layer_nonfinite_cotangent(device, dynamic):
    torch.manual_seed(5)
    layer = mhc.MHCLayer(64, 4, use_dynamic_h=dynamic)
    g = torch.Generator().manual_seed(10)
    x = torch.randn(5, 4, 64, generator=g)
    go = _plant(torch.randn(5, 4, 64, generator=g), float("nan"), (1, 3, 20))
    names = DYN if dynamic else STA
    w = layer.rmsnorm_weight.detach().double().requires_grad_(True)
    ps = [getattr(layer, k).detach().double().requires_grad_(True) for k in names]
    xr = x.double().requires_grad_(True)
    fn = R.mhc_layer_dynamic if dynamic else R.mhc_layer_static
    fn(xr, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64).backward(go.double())
    layer = layer.to(device)
    xd = x.to(device).requires_grad_(True)
    layer(xd).backward(go.to(device))
    _masks_match(xd.grad, xr.grad, "dx")
    _masks_match(layer.rmsnorm_weight.grad, w.grad, "d weight")
    for k, p in zip(names, ps):
        _masks_match(getattr(layer, k).grad, p.grad, f"d {k}")


@pytest.mark.parametrize("value", [float("nan"), float("inf")])
def test_inference_nonfinite_token(device, value):
    torch.manual_seed(6)
    layer = mhc.MHCLayer(64, 4, use_dynamic_h=True)
    g = torch.Generator().manual_seed(11)
    x = _plant(torch.randn(5, 4, 64, generator=g), value, (0, 2, 33))
    ps = [getattr(layer, k).detach().double() for k in DYN]
    ref = R.mhc_layer_dynamic(x.double(), layer.rmsnorm_weight.detach().double(), *ps, 20, 1e-8, 1e-5,
                              dtype=torch.float64)
    layer = layer.to(device).eval()
    layer.prepare_inference()
    with torch.no_grad():
        out = layer(x.to(device))
    _masks_match(out, ref, "inference out")
    assert torch.isfinite(out[1:]).all()

"""Non-contiguous inputs on the GPU: a strided or transposed view gives the
same bits, in the outputs and in every gradient (whose layout follows the
input's, as torch's own ops do), as the same values stored contiguously."""
import pytest
import torch

import mhc_ascend_amd as mhc

pytestmark = pytest.mark.gpu


def _same(a, b, what):
    for i, (u, v) in enumerate(zip(a, b)):
        assert u.shape == v.shape, f"{what} result {i}: shape {tuple(u.shape)} != {tuple(v.shape)}"
        assert torch.equal(u, v), f"{what} result {i} differs between the view and its contiguous copy"


def _run(module, inputs, go):
    for p in module.parameters():
        p.grad = None
    leaves = [t.detach().requires_grad_(True) for t in inputs]
    out = module(*leaves)
    out.backward(go)
    return [out.detach()] + [t.grad.contiguous() for t in leaves] + [p.grad.clone() for p in module.parameters()]


@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_transposed_input(device, dynamic, dtype):
    torch.manual_seed(1)
    layer = mhc.MHCLayer(256, 4, use_dynamic_h=dynamic).to(device)
    base = torch.randn(37, 256, 4, device=device).to(dtype)
    view = base.transpose(1, 2)  # [37, 4, 256] over [37, 256, 4] storage
    go = torch.randn(37, 4, 256, device=device)
    _same(_run(layer, [view], go), _run(layer, [view.contiguous()], go), "layer")


@pytest.mark.parametrize("n", [4, 3, 16])
@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_wrapper_strided_inputs(device, n, dynamic, dtype):
    torch.manual_seed(2)
    wrap = mhc.MHCResidualWrapper(256, n, use_dynamic_h=dynamic).to(device)
    big = torch.randn(40, 512, device=device).to(dtype)
    r = big[:, ::2]                      # every other channel
    b = torch.randn(256, 40, device=device).to(dtype).t()  # transposed
    go = torch.randn(40, 256, device=device)
    _same(_run(wrap, [r, b], go), _run(wrap, [r.contiguous(), b.contiguous()], go), "wrapper")


def test_operators_strided_inputs(device):
    g = torch.Generator(device=device).manual_seed(3)
    a = torch.rand(8, 4, 4, device=device, generator=g).transpose(1, 2)
    ga = torch.randn(8, 4, 4, device=device, generator=g)

    def sk(t):
        t = t.detach().requires_grad_(True)
        o = mhc.sinkhorn_knopp(t, 20, 1e-8)
        o.backward(ga)
        return [o.detach(), t.grad.contiguous()]

    _same(sk(a), sk(a.contiguous()), "sinkhorn")
    x = torch.randn(64, 384, device=device, generator=g)[:, ::3]
    w = torch.randn(256, device=device, generator=g)[::2]
    gy = torch.randn(64, 128, device=device, generator=g)

    def rms(xv, wv):
        xd, wd = xv.detach().requires_grad_(True), wv.detach().requires_grad_(True)
        y = mhc.rmsnorm(xd, wd, 1e-5)
        y.backward(gy)
        return [y.detach(), xd.grad.contiguous(), wd.grad.contiguous()]

    _same(rms(x, w), rms(x.contiguous(), w.contiguous()), "rmsnorm")
    xs = torch.randn(30, 128, 4, device=device, generator=g).transpose(1, 2)
    H = torch.randn(4, 30, device=device, generator=g).t()
    go = torch.randn(30, 128, device=device, generator=g)

    def agg(xv, Hv):
        xd, Hd = xv.detach().requires_grad_(True), Hv.detach().requires_grad_(True)
        o = mhc.stream_aggregate(xd, Hd)
        o.backward(go)
        return [o.detach(), xd.grad.contiguous(), Hd.grad.contiguous()]

    _same(agg(xs, H), agg(xs.contiguous(), H.contiguous()), "aggregate")
    y = torch.randn(128, 30, device=device, generator=g).t()
    M = torch.rand(30, 4, 4, device=device, generator=g).transpose(1, 2)
    g2 = torch.randn(30, 4, 128, device=device, generator=g)

    def dist(yv, Hv, Mv, xv):
        ts = [t.detach().requires_grad_(True) for t in (yv, Hv, Mv, xv)]
        d = mhc.stream_distribute_mix_add(*ts)
        d.backward(g2)
        return [d.detach()] + [t.grad.contiguous() for t in ts]

    _same(dist(y, H, M, xs), dist(y.contiguous(), H.contiguous(), M.contiguous(), xs.contiguous()), "distribute")

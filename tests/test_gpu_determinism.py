"""Run-to-run determinism on the GPU: the same forward and backward twice
gives the same bits in every output and gradient, at shapes where many
workgroups contribute partial sums to each parameter gradient (fixed-order
reductions, no float atomics)."""
import pytest
import torch

import mhc_ascend_amd as mhc

pytestmark = pytest.mark.gpu


def _twice(fn):
    a = fn()
    b = fn()
    for i, (u, v) in enumerate(zip(a, b)):
        assert torch.equal(u, v), f"result {i} differs between two identical runs"


def _module_run(module, inputs, go):
    for p in module.parameters():
        p.grad = None
    leaves = [t.clone().requires_grad_(True) for t in inputs]
    out = module(*leaves)
    out.backward(go)
    return [out.detach()] + [t.grad for t in leaves] + [p.grad.clone() for p in module.parameters()]


@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_deterministic(device, dynamic, dtype):
    torch.manual_seed(1)
    layer = mhc.MHCLayer(1024, 4, use_dynamic_h=dynamic).to(device)
    x = torch.randn(3000, 4, 1024, device=device).to(dtype)
    go = torch.randn(3000, 4, 1024, device=device)
    _twice(lambda: _module_run(layer, [x], go))


@pytest.mark.parametrize("n", [4, 8, 32])
@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_wrapper_deterministic(device, n, dynamic, dtype):
    torch.manual_seed(2)
    wrap = mhc.MHCResidualWrapper(1024, n, use_dynamic_h=dynamic).to(device)
    r = torch.randn(2500, 1024, device=device).to(dtype)
    b = torch.randn(2500, 1024, device=device).to(dtype)
    go = torch.randn(2500, 1024, device=device)
    _twice(lambda: _module_run(wrap, [r, b], go))


def test_operators_deterministic(device):
    g = torch.Generator(device=device).manual_seed(3)
    x = torch.randn(4000, 1024, device=device, generator=g)
    w = 1 + 0.1 * torch.randn(1024, device=device, generator=g)
    gy = torch.randn(4000, 1024, device=device, generator=g)

    def rms():
        xd, wd = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        y = mhc.rmsnorm(xd, wd, 1e-5)
        y.backward(gy)
        return [y.detach(), xd.grad, wd.grad]

    _twice(rms)
    xs = torch.randn(3000, 4, 512, device=device, generator=g)
    H = torch.randn(4, device=device, generator=g)
    go = torch.randn(3000, 512, device=device, generator=g)

    def agg():
        xd, Hd = xs.clone().requires_grad_(True), H.clone().requires_grad_(True)
        o = mhc.stream_aggregate(xd, Hd.unsqueeze(0).expand(3000, -1))
        o.backward(go)
        return [o.detach(), xd.grad, Hd.grad]

    _twice(agg)
    y = torch.randn(3000, 512, device=device, generator=g)
    M = torch.rand(4, 4, device=device, generator=g)
    g2 = torch.randn(3000, 4, 512, device=device, generator=g)

    def dist():
        yd, Hd, Md, xd = (t.clone().requires_grad_(True) for t in (y, H, M, xs))
        d = mhc.stream_distribute_mix_add(yd, Hd.unsqueeze(0).expand(3000, -1), Md.unsqueeze(0).expand(3000, -1, -1),
                                          xd)
        d.backward(g2)
        return [d.detach(), yd.grad, Hd.grad, Md.grad, xd.grad]

    _twice(dist)

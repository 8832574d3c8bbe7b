"""Zero-token inputs through the public API on the GPU: the standalone
operators (forward and backward), MHCLayer with static and dynamic H and
MHCResidualWrapper (n = 4 and 6, fp32 and bf16, both residual modes) return empty outputs
of the right shape, and every parameter gradient is zero (a sum over no
tokens), as torch's own ops give on the reference's PyTorch path
(ops_pytorch_backward.py, layer.py:94-179, 269-322 applied to empty
tensors)."""
import pytest
import torch

import mhc_ascend_amd as mhc

pytestmark = pytest.mark.gpu


def _zero_grads(module):
    for name, p in module.named_parameters():
        assert p.grad is not None, f"{name}: no gradient"
        assert torch.count_nonzero(p.grad) == 0, f"{name}: gradient over no tokens is not zero"


def test_operators_on_empty_batches(device):
    inp = torch.rand(0, 4, 4, device=device, requires_grad=True)
    out = mhc.sinkhorn_knopp(inp, 20, 1e-8)
    assert out.shape == (0, 4, 4)
    out.backward(torch.ones_like(out))
    assert inp.grad.shape == (0, 4, 4)

    x = torch.randn(0, 64, device=device, requires_grad=True)
    w = torch.ones(64, device=device, requires_grad=True)
    y = mhc.rmsnorm(x, w, 1e-5)
    assert y.shape == (0, 64)
    y.backward(torch.ones_like(y))
    assert x.grad.shape == (0, 64) and torch.count_nonzero(w.grad) == 0

    xs = torch.randn(0, 4, 64, device=device, requires_grad=True)
    H = torch.randn(0, 4, device=device, requires_grad=True)
    a = mhc.stream_aggregate(xs, H)
    assert a.shape == (0, 64)
    a.backward(torch.ones_like(a))
    assert xs.grad.shape == (0, 4, 64) and H.grad.shape == (0, 4)

    yv = torch.randn(0, 64, device=device, requires_grad=True)
    Hp = torch.randn(0, 4, device=device, requires_grad=True)
    M = torch.rand(0, 4, 4, device=device, requires_grad=True)
    xs2 = torch.randn(0, 4, 64, device=device, requires_grad=True)
    d = mhc.stream_distribute_mix_add(yv, Hp, M, xs2)
    assert d.shape == (0, 4, 64)
    d.backward(torch.ones_like(d))
    assert yv.grad.shape == (0, 64) and Hp.grad.shape == (0, 4)
    assert M.grad.shape == (0, 4, 4) and xs2.grad.shape == (0, 4, 64)

    assert mhc.compute_rms(torch.randn(0, 256, device=device)).shape == (0,)


@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_on_empty_batch(device, dynamic, dtype):
    layer = mhc.MHCLayer(64, 4, use_dynamic_h=dynamic).to(device)
    x = torch.randn(0, 4, 64, device=device).to(dtype).requires_grad_(True)
    out = layer(x)
    assert out.shape == (0, 4, 64) and out.dtype == torch.float32
    out.backward(torch.ones_like(out))
    assert x.grad.shape == (0, 4, 64)
    _zero_grads(layer)


@pytest.mark.parametrize("n", [4, 6, 16])
@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["decay", "zero"])
@pytest.mark.parametrize("shape", [(0, 64), (0, 3, 64)])
def test_wrapper_on_empty_batch(device, n, dynamic, dtype, mode, shape):
    wrap = mhc.MHCResidualWrapper(64, n, residual_mode=mode, use_dynamic_h=dynamic).to(device)
    r = torch.randn(*shape, device=device).to(dtype).requires_grad_(True)
    b = torch.randn(*shape, device=device).to(dtype).requires_grad_(True)
    out = wrap(r, b)
    assert tuple(out.shape) == (shape if len(shape) == 2 else (0, 3, 64))
    out.backward(torch.ones_like(out))
    assert r.grad.shape == r.shape and b.grad.shape == b.shape
    _zero_grads(wrap)

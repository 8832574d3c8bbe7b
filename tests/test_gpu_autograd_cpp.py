"""GPU: the C++ autograd nodes of the fused layers and of the fused
MHCResidualWrapper (_mhc_autograd.so, the path mhc_layer_static /
mhc_layer_fused_dynamic_training / MHCLayer / mhc_residual_wrapper take)
against the Python autograd functions over the same C-ABI entry points
(the structure of the reference's ops.py:387-564 autograd function).

Both call the same kernels with the same arguments, so outputs and every
gradient must be equal bit for bit, with the same dtypes and shapes; parity
of that path with the float64 oracle is covered by test_gpu_static.py and
test_gpu_dynamic.py, which run through the C++ nodes.
"""
import pytest
import torch

import mhc_ascend_amd as mhc
from mhc_ascend_amd import _lib, ops
from tests import pyref_autograd as pyref

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _ag():
    ag = _lib.autograd()
    assert ag is not None, "_mhc_autograd.so is not built next to libmhc_hip.so"
    return ag


def _leaves(ts, device):
    return [t.to(device).requires_grad_(True) for t in ts]


def _same(got, want, what):
    assert got.dtype == want.dtype and got.shape == want.shape, (what, got.dtype, want.dtype, got.shape, want.shape)
    assert torch.equal(got, want), f"{what}: C++ and Python autograd paths differ"


def _run(fn, inputs, grad):
    out = fn(*inputs)
    out.backward(grad)
    return out.detach(), [t.grad for t in inputs]


def _x(g, B, n, C, dtype, device, noncontig):
    if noncontig:  # [B, C, n] storage seen as [B, n, C]
        return torch.randn(B, C, n, generator=g).to(device=device, dtype=dtype).transpose(1, 2)
    return torch.randn(B, n, C, generator=g).to(device=device, dtype=dtype)


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,B,C,noncontig", [(4, 37, 1280, False), (4, 5, 64, True), (8, 129, 320, False),
                                             (32, 3, 96, False)])
def test_static_layer_cpp_equals_python(device, x_dtype, n, B, C, noncontig):
    g = _gen(7 * n + B)
    x0 = _x(g, B, n, C, x_dtype, device, noncontig)
    params = [1 + 0.1 * torch.randn(C, generator=g), 0.3 * torch.randn(n, generator=g),
              0.3 * torch.randn(n, generator=g), torch.randn(n, n, generator=g)]
    grad = torch.randn(B, n, C, generator=g).to(device)
    cfg = (20, 1e-8, 1e-5)

    ag = _ag()
    a = [x0.detach().clone().requires_grad_(True)] + _leaves(params, device)
    out_c, gc = _run(lambda *t: ag.static_layer(*t, *cfg), a, grad)
    b = [x0.detach().clone().requires_grad_(True)] + _leaves(params, device)
    out_p, gp = _run(lambda *t: pyref.MHCLayerStaticFunction.apply(*t, *cfg), b, grad)
    _same(out_c, out_p, "out")
    for i, (u, v) in enumerate(zip(gc, gp)):
        _same(u, v, f"grad {i}")
    assert gc[0].dtype == x_dtype


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,B,C", [(4, 37, 1280), (2, 9, 256), (8, 40, 320), (32, 5, 64)])
@pytest.mark.parametrize("float_alpha", [False, True])
def test_dynamic_layer_cpp_equals_python(device, x_dtype, n, B, C, float_alpha):
    g = _gen(11 * n + B)
    x0 = torch.randn(B, n, C, generator=g).to(device=device, dtype=x_dtype)
    nC = n * C
    tens = [1 + 0.1 * torch.randn(C, generator=g), 0.02 * torch.randn(n, nC, generator=g),
            0.02 * torch.randn(n, nC, generator=g), 0.02 * torch.randn(n * n, nC, generator=g)]
    alphas = [torch.tensor(v) for v in (0.5, 0.7, 0.3)]
    bias = [0.1 * torch.randn(n, generator=g), 0.1 * torch.randn(n, generator=g),
            torch.randn(n, n, generator=g)]
    grad = torch.randn(B, n, C, generator=g).to(device)
    cfg = (20, 1e-8, 1e-5)

    def inputs():
        x = x0.detach().clone().requires_grad_(True)
        w, pp, pq, pr = _leaves(tens, device)
        al = [float(a) for a in alphas] if float_alpha else _leaves(alphas, device)
        bp, bq, br = _leaves(bias, device)
        return [x, w, pp, pq, pr, *al, bp, bq, br]

    _ag()
    a = inputs()
    out_c = mhc.mhc_layer_fused_dynamic_training(*a, *cfg)
    out_c.backward(grad)
    b = inputs()
    al = [torch.tensor(v, device=device, dtype=torch.float32) if not torch.is_tensor(v) else v for v in b[5:8]]
    out_p = pyref.MHCLayerDynamicFunction.apply(*b[:5], *al, *b[8:], *cfg)
    out_p.backward(grad)
    _same(out_c.detach(), out_p.detach(), "out")
    for i, (u, v) in enumerate(zip(a, b)):
        if torch.is_tensor(u):
            _same(u.grad, v.grad, f"grad {i}")
    if not float_alpha:
        assert a[5].grad.shape == torch.Size([])


@pytest.mark.parametrize("dynamic", [False, True])
def test_layer_module_runs_cpp_nodes(device, dynamic):
    """MHCLayer's training forward builds the C++ node and its parameters'
    gradients equal the Python function's."""
    torch.manual_seed(3)
    layer = mhc.MHCLayer(256, expansion_rate=4, use_dynamic_h=dynamic).to(device)
    x = torch.randn(17, 4, 256, device=device, requires_grad=True)
    out = layer(x)
    node = out.grad_fn.name()
    assert ("DynamicLayer" if dynamic else "StaticLayer") in node and "Function" not in node, node
    out.sum().backward()
    got = {k: p.grad.clone() for k, p in layer.named_parameters()}
    gx = x.grad.clone()
    layer.zero_grad()
    x.grad = None
    cfg = (layer.num_sinkhorn_iters, layer.sinkhorn_eps, layer.rmsnorm_eps)
    if dynamic:
        ref = pyref.MHCLayerDynamicFunction.apply(x, layer.rmsnorm_weight, layer.phi_pre, layer.phi_post,
                                                layer.phi_res, layer.alpha_pre, layer.alpha_post, layer.alpha_res,
                                                layer.b_pre, layer.b_post, layer.b_res, *cfg)
    else:
        ref = pyref.MHCLayerStaticFunction.apply(x, layer.rmsnorm_weight, layer.H_pre, layer.H_post, layer.H_res,
                                               *cfg)
    _same(out.detach(), ref.detach(), "out")
    ref.sum().backward()
    _same(gx, x.grad, "grad x")
    for k, p in layer.named_parameters():
        _same(got[k], p.grad, f"grad {k}")


def test_cpp_nodes_raise_like_python(device):
    ag = _ag()
    x = torch.randn(3, 4, 64, device=device)
    with pytest.raises(RuntimeError, match="parameter shapes do not match"):
        ag.static_layer(x, torch.ones(63, device=device), torch.zeros(4, device=device),
                        torch.zeros(4, device=device), torch.zeros(4, 4, device=device), 20, 1e-8, 1e-5)
    with pytest.raises(RuntimeError, match="must be on a HIP device"):
        ag.static_layer(x, torch.ones(64), torch.zeros(4, device=device), torch.zeros(4, device=device),
                        torch.zeros(4, 4, device=device), 20, 1e-8, 1e-5)
    with pytest.raises(RuntimeError, match="does not match"):
        ag.dynamic_layer(x, torch.ones(64, device=device), torch.zeros(4, 255, device=device),
                         torch.zeros(4, 256, device=device), torch.zeros(16, 256, device=device),
                         *[torch.tensor(1.0, device=device)] * 3, torch.zeros(4, device=device),
                         torch.zeros(4, device=device), torch.zeros(4, 4, device=device), 20, 1e-8, 1e-5)


@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["decay", "zero"])
def test_wrapper_cpp_equals_python(device, dynamic, dtype, mode):
    """The fused wrapper's C++ node against MHCWrapper*Function: output and
    the gradients of residual, branch and every layer parameter equal."""
    torch.manual_seed(5)
    T, C = 77, 256
    layer = mhc.MHCLayer(C, expansion_rate=4, use_dynamic_h=dynamic).to(device)
    r0 = torch.randn(T, C, device=device).to(dtype)
    b0 = torch.randn(T, C, device=device).to(dtype)
    grad = torch.randn(T, C, device=device)
    cfg = (layer.num_sinkhorn_iters, layer.sinkhorn_eps, layer.rmsnorm_eps)

    def grads_of(fn):
        layer.zero_grad()
        r = r0.clone().requires_grad_(True)
        b = b0.clone().requires_grad_(True)
        out = fn(r, b)
        out.backward(grad)
        return out.detach(), r.grad, b.grad, {k: p.grad.clone() for k, p in layer.named_parameters()}

    _ag()
    got = grads_of(lambda r, b: ops.mhc_residual_wrapper(r, b, layer, mode))
    if dynamic:
        want = grads_of(lambda r, b: pyref.MHCWrapperDynamicFunction.apply(
            r, b, layer.rmsnorm_weight, layer.phi_pre, layer.phi_post, layer.phi_res, layer.alpha_pre,
            layer.alpha_post, layer.alpha_res, layer.b_pre, layer.b_post, layer.b_res, mode, 4, *cfg))
    else:
        want = grads_of(lambda r, b: pyref.MHCWrapperStaticFunction.apply(
            r, b, layer.rmsnorm_weight, layer.H_pre, layer.H_post, layer.H_res, mode, 4, *cfg))
    _same(got[0], want[0], "out")
    _same(got[1], want[1], "grad residual")
    _same(got[2], want[2], "grad branch")
    for k in want[3]:
        _same(got[3][k], want[3][k], f"grad {k}")


def test_wrapper_cpp_raises_like_python(device):
    ag = _ag()
    layer = mhc.MHCLayer(64, expansion_rate=4, use_dynamic_h=False).to(device)
    r = torch.randn(5, 64, device=device)
    args = (layer.rmsnorm_weight, layer.H_pre, layer.H_post, layer.H_res)
    with pytest.raises(ValueError, match="Unknown residual_mode"):
        ag.static_wrapper(r, r, *args, "other", 4, 20, 1e-8, 1e-5)
    with pytest.raises(RuntimeError, match="one shape"):
        ag.static_wrapper(r, r[:4], *args, "decay", 4, 20, 1e-8, 1e-5)

"""GPU parity of the standalone operators (rmsnorm, compute_rms,
stream_aggregate, stream_distribute_mix_add) against the CPU oracle, their
autograd, config C2 shapes, broadcast (stride-0) coefficients, and the
reference's own composition of the static layer from these operators
(layer.py:142-170)."""
import pytest
import torch

import mhc_ascend_amd as mhc
from mhc_ascend_amd import native
from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, grad_atol

pytestmark = pytest.mark.gpu

FWD = dict(rtol=1e-4, atol=1e-5)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _leaf(t, device):
    return t.to(device).requires_grad_(True)


def _ref_leaf(t):
    return t.double().requires_grad_(True)


def _check_out(out, ref, dtype, what):
    if dtype == torch.bfloat16:
        assert_close_bf16(out, ref, what)
    else:
        assert_close(out, ref, what=what, **FWD)


def _check_grad(got, ref, dtype, what, frac=1e-5):
    if dtype == torch.bfloat16:
        assert_close_bf16(got, ref, what)
    else:
        assert_close(got, ref, 1e-3, grad_atol(ref, frac), what)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,C", [(1, 64), (37, 256), (130, 4096), (9, 7168), (5, 1001), (3, 13), (4, 4100)])
def test_rmsnorm(device, dtype, B, C):
    """Includes rows that are not a multiple of the 16-byte vector (1001, 13;
    4100 for bf16), which run the channel-loop kernels."""
    g = _gen(B + C)
    x = torch.randn(B, C, generator=g).to(dtype)
    w = 1 + 0.1 * torch.randn(C, generator=g)
    go = torch.randn(B, C, generator=g).to(dtype)
    xd, wd = _leaf(x, device), _leaf(w, device)
    out = mhc.rmsnorm(xd, wd, 1e-5)
    out.backward(go.to(device))
    xr, wr = _ref_leaf(x), _ref_leaf(w)
    ref, rms = R.rmsnorm(xr, wr, 1e-5)
    ref.backward(go.double())
    _check_out(out, ref.detach(), dtype, f"rmsnorm B={B} C={C}")
    _check_grad(xd.grad, xr.grad, dtype, "rmsnorm dx")
    assert wd.grad.dtype == torch.float32
    assert_close(wd.grad, wr.grad, 1e-3, grad_atol(wr.grad, 1e-4),
                 "rmsnorm dw")
    _, rms_got = native.rmsnorm_fwd(x.to(device), w.to(device), 1e-5)
    assert_close(rms_got, rms.detach(), 1e-5, 0, "rms")


def test_rmsnorm_config_c2(device):
    """Config C2: [16384, 4096] ~ N(0,1), weight ~ N(1, 0.1), eps 1e-5."""
    g = _gen(11)
    x = torch.randn(16384, 4096, generator=g)
    w = 1 + 0.1 * torch.randn(4096, generator=g)
    out, rms = native.rmsnorm_fwd(x.to(device), w.to(device), 1e-5)
    idx = torch.randperm(16384, generator=g)[:256]
    ref, rref = R.rmsnorm(x[idx].double(), w.double(), 1e-5)
    assert_close(out.cpu()[idx], ref, what="C2 rmsnorm", **FWD)
    assert_close(rms.cpu()[idx], rref, 1e-5, 0, "C2 rms")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K", [4 * 1024, 4 * 1001 + 3])
def test_compute_rms(device, dtype, K):
    g = _gen(3)
    x = torch.randn(50, K, generator=g).to(dtype)
    got = mhc.compute_rms(x.to(device), 1e-8)
    assert_close(got, R.compute_rms(x.double(), 1e-8), 1e-5, 0, f"compute_rms K={K}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("B,C", [(3, 64), (65, 1024), (17, 4096)])
def test_stream_aggregate(device, dtype, shared, B, C):
    g = _gen(B * C + shared)
    x = torch.randn(B, 4, C, generator=g).to(dtype)
    H = torch.randn(4, generator=g) if shared else torch.randn(B, 4, generator=g)
    go = torch.randn(B, C, generator=g).to(dtype)
    xd = _leaf(x, device)
    Hd = _leaf(H, device)
    Hin = Hd.unsqueeze(0).expand(B, -1) if shared else Hd
    out = mhc.stream_aggregate(xd, Hin)
    out.backward(go.to(device))
    xr, Hr = _ref_leaf(x), _ref_leaf(H)
    ref, _ = R.stream_aggregate(xr, Hr.unsqueeze(0).expand(B, -1) if shared else Hr)
    ref.backward(go.double())
    _check_out(out, ref.detach(), dtype, "aggregate out")
    _check_grad(xd.grad, xr.grad, dtype, "aggregate dx")
    assert_close(Hd.grad, Hr.grad, 1e-3, grad_atol(Hr.grad, 1e-4),
                 "aggregate dH")


@pytest.mark.parametrize("n,C", [(1, 256), (2, 256), (8, 64), (16, 256), (32, 320), (1, 3), (4, 77), (8, 1001),
                                 (32, 50), (3, 77), (6, 256), (12, 130), (20, 64), (64, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_stream_ops_general_n(device, n, C, dtype):
    """stream_aggregate and stream_distribute_mix_add at n = 1 .. 64 (n = 3,
    6, 12, 20, 64 on the generic kernels, n at run time) and rows that are
    not a multiple of the vector (the distribute backward's
    n*n + n row sums need >= 72 lanes at n = 8; dM comes from the per-token
    Gram kernel at n >= 16)."""
    B = 9
    g = _gen(100 + n)
    x = torch.randn(B, n, C, generator=g).to(dtype)
    H = torch.randn(B, n, generator=g)
    go = torch.randn(B, C, generator=g).to(dtype)
    xd, Hd = _leaf(x, device), _leaf(H, device)
    out = mhc.stream_aggregate(xd, Hd)
    out.backward(go.to(device))
    xr, Hr = _ref_leaf(x), _ref_leaf(H)
    ref, _ = R.stream_aggregate(xr, Hr)
    ref.backward(go.double())
    _check_out(out, ref.detach(), dtype, f"n={n} aggregate out")
    _check_grad(xd.grad, xr.grad, dtype, f"n={n} aggregate dx")
    assert_close(Hd.grad, Hr.grad, 1e-3, grad_atol(Hr.grad, 1e-4),
                 f"n={n} aggregate dH")

    y = torch.randn(B, C, generator=g).to(dtype)
    Hq = torch.randn(B, n, generator=g)
    M = torch.rand(B, n, n, generator=g)
    gd = torch.randn(B, n, C, generator=g)
    xd, yd, Hd, Md = (_leaf(t, device) for t in (x, y, Hq, M))
    out = mhc.stream_distribute(yd, Hd, Md, xd)
    out.backward(gd.to(device))
    xr, yr, Hr, Mr = (_ref_leaf(t) for t in (x, y, Hq, M))
    ref, _ = R.stream_distribute_mix_add(yr, Hr, Mr, xr)
    ref.backward(gd.double())
    assert out.dtype == torch.float32
    assert_close(out, ref.detach(), what=f"n={n} distribute out", **FWD)
    _check_grad(xd.grad, xr.grad, dtype, f"n={n} distribute dx")
    _check_grad(yd.grad, yr.grad, dtype, f"n={n} distribute dy")
    assert_close(Md.grad, Mr.grad, 1e-3, grad_atol(Mr.grad, 1e-4),
                 f"n={n} distribute dM")
    assert_close(Hd.grad, Hr.grad, 1e-3, grad_atol(Hr.grad, 1e-4),
                 f"n={n} distribute dH")


def test_stream_aggregate_config_c2(device):
    """Config C2: x [16384, 4, 4096] ~ N(0,1), H_pre [16384, 4] ~ N(0,1)."""
    g = _gen(12)
    x = torch.randn(16384, 4, 4096, generator=g)
    H = torch.randn(16384, 4, generator=g)
    out, h_act = native.stream_aggregate_fwd(x.to(device), H.to(device))
    idx = torch.randperm(16384, generator=g)[:256]
    ref, href = R.stream_aggregate(x[idx].double(), H[idx].double())
    assert_close(out.cpu()[idx], ref, what="C2 aggregate", **FWD)
    assert_close(h_act.cpu()[idx], href, 1e-6, 1e-7, "C2 h_pre_act")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("B,C", [(3, 64), (65, 1024), (17, 4096)])
def test_stream_distribute_mix_add(device, dtype, shared, B, C):
    g = _gen(B * C + 7 * shared)
    x = torch.randn(B, 4, C, generator=g).to(dtype)
    y = torch.randn(B, C, generator=g).to(dtype)
    if shared:
        H = torch.randn(4, generator=g)
        M = torch.rand(4, 4, generator=g)
    else:
        H = torch.randn(B, 4, generator=g)
        M = torch.rand(B, 4, 4, generator=g)
    go = torch.randn(B, 4, C, generator=g)
    xd, yd, Hd, Md = (_leaf(t, device) for t in (x, y, H, M))
    Hin = Hd.unsqueeze(0).expand(B, -1) if shared else Hd
    Min = Md.unsqueeze(0).expand(B, -1, -1) if shared else Md
    out = mhc.stream_distribute(yd, Hin, Min, xd)
    assert out.dtype == torch.float32
    out.backward(go.to(device))
    xr, yr, Hr, Mr = (_ref_leaf(t) for t in (x, y, H, M))
    ref, _ = R.stream_distribute_mix_add(yr, Hr.unsqueeze(0).expand(B, -1) if shared else Hr,
                                         Mr.unsqueeze(0).expand(B, -1, -1) if shared else Mr, xr)
    ref.backward(go.double())
    assert_close(out, ref.detach(), what="distribute out", **FWD)
    _check_grad(xd.grad, xr.grad, dtype, "distribute dx")
    _check_grad(yd.grad, yr.grad, dtype, "distribute dy")
    assert_close(Hd.grad, Hr.grad, 1e-3, grad_atol(Hr.grad, 1e-4), "distribute dH")
    assert_close(Md.grad, Mr.grad, 1e-3, grad_atol(Mr.grad, 1e-4), "distribute dM")


def test_native_mirror_returns_pre_activation_grads(device):
    """The native mirrors return d/d(activated H) like the reference's
    bindings (the sigmoid derivative is applied by the autograd layer)."""
    g = _gen(5)
    B, C = 6, 256
    x = torch.randn(B, 4, C, generator=g)
    H = torch.randn(B, 4, generator=g)
    go = torch.randn(B, C, generator=g)
    _, h_act = native.stream_aggregate_fwd(x.to(device), H.to(device))
    _, gh = native.stream_aggregate_bwd(go.to(device), x.to(device), h_act)
    want = (go.double()[:, None, :] * x.double()).sum(-1)
    assert_close(gh, want, 1e-4, 1e-5, "grad_H_pre_activated")


@pytest.mark.parametrize("B,C", [(32, 256), (48, 4096)])
def test_reference_static_composition_from_ops(device, B, C):
    """layer.py:142-170 built from the standalone operators: expanded
    (stride-0) H, B per-token Sinkhorns, aggregate -> rmsnorm -> distribute."""
    d = R.static_layer_inputs(B, 4, C, seed=B)
    x = _leaf(d["x"], device)
    w = _leaf(d["weight"].float(), device)
    hp, hq, hr = (_leaf(d[k], device) for k in ("H_pre", "H_post", "H_res"))
    agg = mhc.stream_aggregate(x, hp.unsqueeze(0).expand(B, -1))
    y = mhc.rmsnorm(agg, w, 1e-5)
    m = mhc.sinkhorn_knopp(torch.exp(hr.unsqueeze(0).expand(B, -1, -1)), 20, 1e-8)
    out = mhc.stream_distribute_mix_add(y, hq.unsqueeze(0).expand(B, -1), m, x)
    out.backward(d["grad"].to(device))
    xr = _ref_leaf(d["x"])
    pr = [_ref_leaf(d[k].float()) for k in ("weight", "H_pre", "H_post", "H_res")]
    ref = R.mhc_layer_static(xr, *pr, 20, 1e-8, 1e-5, dtype=torch.float64)
    ref.backward(d["grad"].double())
    assert_close(out, ref.detach(), what="composition out", **FWD)
    assert_close(x.grad, xr.grad, 1e-3, grad_atol(xr.grad, 1e-5), "composition dx")
    for nm, a, e in zip(["dw", "dH_pre", "dH_post", "dH_res"], [w.grad, hp.grad, hq.grad, hr.grad],
                        [p.grad for p in pr]):
        assert_close(a, e, 1e-3, grad_atol(e, 1e-4), f"composition {nm}")


def test_calls_run_on_the_callers_stream(device):
    """The library enqueues on torch's current stream (bindings.cpp:59 uses
    the current NPU stream): under a side stream the raw handle it receives
    is that stream's, and results match the default-stream ones."""
    from mhc_ascend_amd import _lib
    g = _gen(90)
    x = torch.randn(33, 4, 512, generator=g).to(device)
    torch.manual_seed(90)
    layer = mhc.MHCLayer(512, 4, use_dynamic_h=True).to(device)
    with torch.no_grad():
        want = layer(x)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert _lib.stream_of(x) == side.cuda_stream
        with torch.no_grad():
            got = layer(x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert _lib.stream_of(x) == torch.cuda.current_stream().cuda_stream

"""GPU parity: batched Sinkhorn-Knopp and the fused static-H layer against
the CPU oracle (float64) on identical seeded inputs.

Tolerances: fp32 forward rtol 1e-4 / atol 1e-5;
gradients rtol 1e-3 with an absolute floor of 1e-5 (per-token tensors) or
1e-4 (token-summed parameter gradients) times max|ref|; values stored in
bf16: one rounding to nearest (2^-8 relative) plus 1e-3 max|ref|.
"""
import pytest
import torch

import mhc_ascend_amd as mhc
from mhc_ascend_amd import native
from oracle import csk
from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, grad_atol

pytestmark = pytest.mark.gpu

FWD = dict(rtol=1e-4, atol=1e-5)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------
# Sinkhorn-Knopp
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8, 9, 16, 24, 32, 64])
@pytest.mark.parametrize("iters", [0, 1, 20, 40])
def test_sinkhorn_fwd_bwd_matches_oracle(device, n, iters):
    B = 333  # not a multiple of the matrices per wave
    g = _gen(100 * n + iters)
    a = torch.exp(torch.randn(B, n, n, generator=g))
    go = torch.randn(B, n, n, generator=g)
    ad = a.to(device).requires_grad_(True)
    out = mhc.sinkhorn_knopp(ad, iters, 1e-8)
    out.backward(go.to(device))
    ref = torch.from_numpy(csk.sinkhorn_fwd(a.double().numpy(), iters, 1e-8))
    gref = torch.from_numpy(csk.sinkhorn_bwd(go.double().numpy(), a.double().numpy(), iters, 1e-8))
    assert_close(out, ref, what=f"SK fwd n={n} T={iters}", **FWD)
    # n = 1 has an analytically ~0 gradient: absolute floor 1e-6
    assert_close(ad.grad, gref, 1e-3, max(grad_atol(gref, 1e-5), 1e-6), f"SK bwd n={n} T={iters}")


@pytest.mark.parametrize("n", [3, 5, 6, 7, 12, 20, 40])
def test_sinkhorn_padded_groups_with_zero_eps(device, n):
    """n that is not a power of two leaves padding lanes in each lane group
    (and, above 8, padding columns in each row); with eps = 0 they must not
    divide by zero into the real rows' sums."""
    g = _gen(7 + n)
    a = torch.exp(torch.randn(100, n, n, generator=g))
    go = torch.randn(100, n, n, generator=g)
    ad = a.to(device).requires_grad_(True)
    out = mhc.sinkhorn_knopp(ad, 20, 0.0)
    out.backward(go.to(device))
    ref = torch.from_numpy(csk.sinkhorn_fwd(a.double().numpy(), 20, 0.0))
    gref = torch.from_numpy(csk.sinkhorn_bwd(go.double().numpy(), a.double().numpy(), 20, 0.0))
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(ad.grad).all())
    assert_close(out, ref, what=f"SK fwd eps=0 n={n}", **FWD)
    assert_close(ad.grad, gref, 1e-3, max(grad_atol(gref, 1e-5), 1e-6), f"SK bwd eps=0 n={n}")


def test_sinkhorn_config_c2_shape(device):
    """Config C2: [65536, 4, 4] ~ U(0,1), 20 iterations, eps 1e-8."""
    g = _gen(2)
    a = torch.rand(65536, 4, 4, generator=g)
    out = native.sinkhorn_knopp_fwd(a.to(device), 20, 1e-8).cpu()
    idx = torch.randperm(65536, generator=g)[:2048]
    ref = torch.from_numpy(csk.sinkhorn_fwd(a[idx].double().numpy(), 20, 1e-8))
    assert_close(out[idx], ref, what="SK C2 subsample", **FWD)
    assert_close(out.sum(-2), torch.ones(65536, 4), 0, 1e-5, "SK C2 column sums")
    go = torch.randn(65536, 4, 4, generator=g)
    gi = native.sinkhorn_knopp_bwd(go.to(device), a.to(device), out.to(device), 20, 1e-8).cpu()
    gref = torch.from_numpy(csk.sinkhorn_bwd(go[idx].double().numpy(), a[idx].double().numpy(), 20, 1e-8))
    assert_close(gi[idx], gref, 1e-3, grad_atol(gref, 1e-5), "SK C2 bwd subsample")


def test_sinkhorn_rejects_non_square(device):
    with pytest.raises(RuntimeError, match="square"):
        native.sinkhorn_knopp_fwd(torch.rand(4, 3, 4, device=device))


# ---------------------------------------------------------------------------
# Fused static-H layer
# ---------------------------------------------------------------------------

def _run_static(d, device, iters=20, sk_eps=1e-8, rms_eps=1e-5, grad=None):
    x = d["x"].to(device).requires_grad_(True)
    ps = [d[k].to(device).requires_grad_(True) for k in ("weight", "H_pre", "H_post", "H_res")]
    out = mhc.mhc_layer_static(x, *ps, iters, sk_eps, rms_eps)
    out.backward((d["grad"] if grad is None else grad).to(device))
    return out, x.grad, [p.grad for p in ps]


def _oracle_static(d, iters=20, sk_eps=1e-8, rms_eps=1e-5, grad=None):
    """Oracle outputs and gradients; also the gradient w.r.t. the mixing
    matrix M (the cotangent entering the Sinkhorn adjoint), which sets the
    scale of fp32 rounding in d_H_res."""
    x = d["x"].double().requires_grad_(True)
    ps = [d[k].double().requires_grad_(True) for k in ("weight", "H_pre", "H_post", "H_res")]
    m = R.sinkhorn_knopp(torch.exp(ps[3]), iters, sk_eps)
    m.retain_grad()
    out = R._layer_core(x, ps[0], torch.sigmoid(ps[1]), 2 * torch.sigmoid(ps[2]), m, rms_eps)
    out.backward((d["grad"] if grad is None else grad).double())
    _oracle_static.dm_scale = float(m.grad.abs().max())
    return out.detach(), x.grad, [p.grad for p in ps]


def _check_static(d, got, want, x_bf16=False, tag="", family_floor=False):
    """family_floor: H_* gradients also get an absolute floor of 1e-5 x the
    largest of the three (n = 1: the RMSNorm is invariant to the scale h_pre,
    so d_H_pre is a cancellation that only eps keeps from zero, and the 1 x 1
    Sinkhorn output is 1 whatever its input)."""
    out, gx, gp = got
    rout, rgx, rgp = want
    fam = max(float(e.abs().max()) for e in rgp[1:])
    assert out.dtype == torch.float32
    assert_close(out, rout, what=f"{tag} out", **FWD)
    if x_bf16:
        assert_close_bf16(gx, rgx, f"{tag} dx (bf16)")
    else:
        assert_close(gx, rgx, 1e-3, grad_atol(rgx, 1e-5), f"{tag} dx")
    names = ["d_weight", "d_H_pre", "d_H_post", "d_H_res"]
    for nm, a, e in zip(names, gp, rgp):
        if nm == "d_weight":
            # the parameter is bf16 (layer.py:65), so autograd stores a bf16 grad
            assert_close_bf16(a, e, f"{tag} {nm}")
        elif nm == "d_H_res":
            # fp32 rounding of the Sinkhorn adjoint scales with |dL/dM|; with
            # loss = sum(y) the exact d_H_res is 0 (column-constant cotangent)
            floor = max(grad_atol(e, 1e-4), 1e-7 * getattr(_oracle_static, "dm_scale", 0.0))
            if family_floor:
                floor = max(floor, 1e-5 * fam)
            assert_close(a, e, 1e-3, floor, f"{tag} {nm}")
        else:
            floor = max(grad_atol(e, 1e-4), 1e-5 * fam) if family_floor else grad_atol(e, 1e-4)
            assert_close(a, e, 1e-3, floor, f"{tag} {nm}")


def test_static_layer_config_c1(device):
    """Config C1 shape [32, 4, 256] fp32 with the module's default init,
    checked with loss = sum(y) (the reference benchmark's cotangent) and with
    a random cotangent (which, unlike sum(y), reaches H_res)."""
    torch.manual_seed(0)
    layer = mhc.MHCLayer(256, 4, use_dynamic_h=False)
    x = torch.randn(32, 4, 256, generator=_gen(0))
    d = {"x": x, "weight": layer.rmsnorm_weight.data, "H_pre": layer.H_pre.data, "H_post": layer.H_post.data,
         "H_res": layer.H_res.data, "grad": torch.randn(32, 4, 256, generator=_gen(1))}
    for grad in (torch.ones(32, 4, 256), d["grad"]):
        _check_static(d, _run_static(d, device, grad=grad), _oracle_static(d, grad=grad), tag="C1")


@pytest.mark.parametrize("B,C", [(1, 64), (7, 256), (64, 1024), (33, 4096), (16, 7168)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_static_layer_matches_oracle(device, B, C, x_dtype):
    d = R.static_layer_inputs(B, 4, C, seed=B + C, x_dtype=x_dtype)
    _check_static(d, _run_static(d, device), _oracle_static(d), x_bf16=x_dtype == torch.bfloat16,
                  tag=f"B={B} C={C} {x_dtype}")


@pytest.mark.parametrize("n,B,C", [(2, 5, 64), (2, 37, 1280), (8, 3, 64), (8, 128, 1280), (8, 9, 4096)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_static_layer_general_n(device, n, B, C, x_dtype):
    """Expansion rates 2 and 8 (the paper's (128, 1280, 8) among them); C=64
    with n=8 is a 16-chunk row whose block reduction of 90 row sums needs
    more lanes than the row has chunks."""
    d = R.static_layer_inputs(B, n, C, seed=n * 1000 + B + C, x_dtype=x_dtype)
    _check_static(d, _run_static(d, device), _oracle_static(d), x_bf16=x_dtype == torch.bfloat16,
                  tag=f"n={n} B={B} C={C} {x_dtype}")


@pytest.mark.parametrize("n,B,C", [(16, 5, 64), (16, 19, 999), (32, 3, 100), (32, 32, 1280)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_static_layer_wide_n(device, n, B, C, x_dtype):
    """Expansion rates 16 and 32 on the channel-loop kernels, dM from the
    per-token Gram kernel; (B, C, n) = (32, 1280, 32) is a paper
    configuration (benchmark.py:307)."""
    d = R.static_layer_inputs(B, n, C, seed=n * 1000 + B + C, x_dtype=x_dtype)
    _check_static(d, _run_static(d, device), _oracle_static(d), x_bf16=x_dtype == torch.bfloat16,
                  tag=f"n={n} B={B} C={C} {x_dtype}")


@pytest.mark.parametrize("n,B,C", [(1, 7, 100), (3, 9, 77), (3, 1100, 64), (5, 4, 320), (6, 17, 256),
                                   (7, 3, 1001), (12, 5, 130), (20, 3, 64), (40, 2, 96), (64, 3, 96)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_static_layer_runtime_n(device, n, B, C, x_dtype):
    """Expansion rates without a fixed-n kernel (the reference takes any n up
    to 64, mhc_types.h:68): the generic row kernels with n at run time, dM on
    zero-padded fp32 MFMA blocks, the shared Sinkhorn and its adjoint on a
    16 / 32 / 64-lane group.  B = 1100 runs more tokens than the backward has
    workgroups (per-workgroup partial sums over several tokens)."""
    d = R.static_layer_inputs(B, n, C, seed=n * 1000 + B + C, x_dtype=x_dtype)
    _check_static(d, _run_static(d, device), _oracle_static(d), x_bf16=x_dtype == torch.bfloat16,
                  tag=f"n={n} B={B} C={C} {x_dtype}", family_floor=n == 1)


@pytest.mark.parametrize("iters", [0, 1, 7, 32, 33, 45])
def test_static_layer_n32_iteration_counts(device, iters):
    """n = 32: the Sinkhorn forward and adjoint on the whole workgroup keep
    up to 32 iterations of state in registers; 33 and more take the
    one-row-per-lane adjoint with its history in the workspace."""
    d = R.static_layer_inputs(5, 32, 64, seed=3200 + iters)
    _check_static(d, _run_static(d, device, iters=iters), _oracle_static(d, iters=iters), tag=f"n=32 T={iters}")


@pytest.mark.parametrize("n,C", [(2, 1), (2, 7), (4, 250), (4, 1001), (8, 13), (8, 10240)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_static_layer_ragged_hidden(device, n, C, x_dtype):
    """Hidden sizes that are not a multiple of the 4-channel chunk (the
    reference pads such rows, stream_ops.cpp:66-68) run the channel-loop
    kernels; (8, 10240) fits the register forward but not its backward."""
    d = R.static_layer_inputs(6, n, C, seed=7 * n + C, x_dtype=x_dtype)
    _check_static(d, _run_static(d, device), _oracle_static(d), x_bf16=x_dtype == torch.bfloat16,
                  tag=f"n={n} C={C} {x_dtype}")


def test_static_layer_module_n32(device):
    """MHCLayer(expansion_rate=32) through the module, non-trivial H."""
    torch.manual_seed(32)
    layer = mhc.MHCLayer(320, 32, use_dynamic_h=False).to(device)
    with torch.no_grad():
        layer.H_pre.normal_()
        layer.H_post.normal_()
        layer.H_res.normal_()
    x = torch.randn(9, 32, 320, generator=_gen(32))
    g = torch.randn(9, 32, 320, generator=_gen(33))
    xd = x.to(device).requires_grad_(True)
    out = layer(xd)
    out.backward(g.to(device))
    d = {"x": x, "grad": g, "weight": layer.rmsnorm_weight.detach().cpu(), "H_pre": layer.H_pre.detach().cpu(),
         "H_post": layer.H_post.detach().cpu(), "H_res": layer.H_res.detach().cpu()}
    rout, rgx, rgp = _oracle_static(d)
    assert_close(out, rout, what="n=32 module out", **FWD)
    assert_close(xd.grad, rgx, 1e-3, grad_atol(rgx, 1e-5), "n=32 module dx")
    assert_close(layer.H_pre.grad, rgp[1], 1e-3, grad_atol(rgp[1], 1e-4), "n=32 module d_H_pre")
    assert_close(layer.H_res.grad, rgp[3], 1e-3, grad_atol(rgp[3], 1e-4), "n=32 module d_H_res")


def test_static_layer_module_general_n(device):
    """MHCLayer(expansion_rate=8) forward/backward through the module."""
    torch.manual_seed(8)
    layer = mhc.MHCLayer(1280, 8, use_dynamic_h=False).to(device)
    with torch.no_grad():
        layer.H_pre.normal_()
        layer.H_post.normal_()
        layer.H_res.normal_()
    x = torch.randn(6, 8, 1280, generator=_gen(8))
    g = torch.randn(6, 8, 1280, generator=_gen(9))
    xd = x.to(device).requires_grad_(True)
    out = layer(xd)
    out.backward(g.to(device))
    d = {"x": x, "grad": g, "weight": layer.rmsnorm_weight.detach().cpu(), "H_pre": layer.H_pre.detach().cpu(),
         "H_post": layer.H_post.detach().cpu(), "H_res": layer.H_res.detach().cpu()}
    rout, rgx, rgp = _oracle_static(d)
    assert_close(out, rout, what="n=8 module out", **FWD)
    assert_close(xd.grad, rgx, 1e-3, grad_atol(rgx, 1e-5), "n=8 module dx")
    assert_close(layer.H_res.grad, rgp[3], 1e-3, grad_atol(rgp[3], 1e-4), "n=8 module d_H_res")


def test_static_layer_module_matches_functional(device):
    torch.manual_seed(3)
    layer = mhc.MHCLayer(512, 4, use_dynamic_h=False).to(device)
    with torch.no_grad():
        layer.H_pre.normal_()
        layer.H_post.normal_()
        layer.H_res.normal_()
    x = torch.randn(24, 4, 512, generator=_gen(3)).to(device)
    out = layer(x)
    ref = R.mhc_layer_static(x.cpu().double(), layer.rmsnorm_weight.cpu().double(), layer.H_pre.cpu().double(),
                             layer.H_post.cpu().double(), layer.H_res.cpu().double(), 20, 1e-8, 1e-5,
                             dtype=torch.float64)
    assert_close(out, ref, what="module", **FWD)


def test_static_layer_config_c3_full_size(device):
    """Config C3 [8192, 4, 4096] fp32: per-token outputs on a token
    subsample against the oracle; token-summed parameter gradients through
    additivity (full batch == sum of the two halves) and against the oracle
    on a 256-token slice."""
    B, n, C = 8192, 4, 4096
    d = R.static_layer_inputs(B, n, C, seed=33)
    out, gx, gp = _run_static(d, device)
    idx = torch.randperm(B, generator=_gen(5))[:48]
    sub = {k: (v[idx] if k in ("x", "grad") else v) for k, v in d.items()}
    rout, rgx, _ = _oracle_static(sub)
    assert_close(out.detach().cpu()[idx], rout, what="C3 out subsample", **FWD)
    assert_close(gx.cpu()[idx], rgx, 1e-3, grad_atol(rgx, 1e-5), "C3 dx subsample")
    # additivity of the fp32 token-summed gradients (native entry points;
    # the module's bf16 weight grad would add bf16 rounding of each half)
    dev = {k: v.to(device) for k, v in d.items()}

    def native_grads(sl_):
        w32 = dev["weight"].float()
        _, _, saved = native.mhc_layer_static_fwd(dev["x"][sl_], w32, dev["H_pre"], dev["H_post"], dev["H_res"])
        return native.mhc_layer_static_bwd(dev["grad"][sl_], dev["x"][sl_], w32, dev["H_pre"],
                                           dev["H_post"], dev["H_res"], saved)[1:]

    full = native_grads(slice(0, B))
    h1 = native_grads(slice(0, B // 2))
    h2 = native_grads(slice(B // 2, B))
    for nm, f, a, b in zip(["d_weight", "d_H_pre", "d_H_post", "d_H_res"], full, h1, h2):
        # the Sinkhorn adjoint is linear in dM, so d_H_res is additive too
        ssum = a + b
        assert_close(f, ssum, 1e-4, grad_atol(ssum, 1e-4 if nm == "d_H_res" else 1e-5), f"C3 additivity {nm}")
    sl = {k: (v[:256] if k in ("x", "grad") else v) for k, v in d.items()}
    _check_static(sl, _run_static(sl, device), _oracle_static(sl), tag="C3 slice")


def test_static_layer_native_fp32_weight_grad(device):
    """The fp32 weight gradient before autograd casts it to the bf16 parameter."""
    d = R.static_layer_inputs(40, 4, 1024, seed=9)
    dev = {k: v.to(device) for k, v in d.items()}
    w32 = dev["weight"].float()
    out, rms, saved = native.mhc_layer_static_fwd(dev["x"], w32, dev["H_pre"], dev["H_post"], dev["H_res"])
    gx, gw, ghp, ghq, ghr = native.mhc_layer_static_bwd(dev["grad"], dev["x"], w32, dev["H_pre"],
                                                        dev["H_post"], dev["H_res"], saved)
    _, _, rgp = _oracle_static(d)
    assert gw.dtype == torch.float32
    assert_close(gw, rgp[0], 1e-3, grad_atol(rgp[0], 1e-5), "fp32 d_weight")
    # saved rms and coefficients
    xa = (torch.sigmoid(d["H_pre"].double())[None, :, None] * d["x"].double()).sum(1)
    assert_close(rms, torch.sqrt((xa * xa).mean(-1) + 1e-5), 1e-5, 0, "rms")
    m = R.sinkhorn_knopp(torch.exp(d["H_res"].double()), 20, 1e-8)
    assert_close(saved[8:24].view(4, 4), m, 1e-5, 1e-7, "M")
    assert_close(saved[64:64 + 1024], d["weight"].double(), 0, 0, "fp32 weight copy")


def test_static_layer_empty_batch(device):
    d = R.static_layer_inputs(0, 4, 256, seed=1)
    out, gx, gp = _run_static(d, device)
    assert out.shape == (0, 4, 256) and gx.shape == (0, 4, 256)
    for gparam in gp:
        assert float(gparam.float().abs().max()) == 0.0

"""GPU parity of the dynamic-H path: the projection operators
(fused_rmsnorm_matmul fwd/bwd) and the fused dynamic layer (config C4)
against the float64 CPU oracle on identical seeded inputs.

Tolerances: fp32 outputs rtol 1e-4 / atol 1e-5; gradients rtol 1e-3 with an
absolute floor relative to max|ref| (1e-5 per-token, 1e-4 token-summed);
bf16-stored results: one rounding to nearest (2^-8 relative) plus 1e-3 max|ref|."""
import pytest
import torch

import mhc_ascend_amd as mhc
from mhc_ascend_amd import native
from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, assert_close_dyn_dx_bf16, grad_atol

pytestmark = pytest.mark.gpu

FWD = dict(rtol=1e-4, atol=1e-5)
PARAMS = ["weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post",
          "b_res"]


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,K,out_dim", [(1, 32, 1), (3, 96, 8), (70, 1024, 24), (129, 4160, 24), (300, 4096, 32),
                                         (65, 16384, 24), (9, 320, 33), (70, 1024, 80), (40, 2048, 100),
                                         (1500, 96, 40), (37, 1024, 129), (130, 2048, 300), (200, 640, 1088)])
def test_projection(device, dtype, B, K, out_dim):
    """Projection forward / backward against float64; more than 128 output
    rows run the streaming kernel (Phi once, fp32 x as bf16 planes), up to
    1024 tokens the backward's all-tiles path."""
    g = _gen(B + K + out_dim)
    x = torch.randn(B, K, generator=g).to(dtype)
    phi = 0.02 * torch.randn(out_dim, K, generator=g)
    go = torch.randn(B, out_dim, generator=g)
    xd = x.float().to(device).requires_grad_(True) if dtype == torch.float32 else x.to(device)
    pd = phi.to(device).requires_grad_(True)
    out = mhc.fused_rmsnorm_matmul(xd, pd)
    ref = R.projection(x.double(), phi.double())
    # split-bf16 operands: ~2^-16 relative per product
    assert_close(out, ref, 1e-4, grad_atol(ref, 1e-5), f"P B={B} K={K} o={out_dim}")
    gx, gphi = native.fused_rmsnorm_matmul_bwd(go.to(device), x.float().to(device), pd.detach())
    assert_close(gx, go.double() @ phi.double(), 1e-4, grad_atol(go.double() @ phi.double(), 1e-5), "dx")
    gref = go.double().t() @ x.double()
    assert_close(gphi, gref, 1e-4, grad_atol(gref, 1e-5), "dphi")


def _run_dyn(d, device, iters=20, sk_eps=1e-8, rms_eps=1e-5, training=True):
    x = d["x"].to(device).requires_grad_(True)
    ps = [d[k].to(device).requires_grad_(True) for k in PARAMS]
    if training:
        out = mhc.mhc_layer_fused_dynamic_training(x, *ps, iters, sk_eps, rms_eps)
        out.backward(d["grad"].to(device))
        return out, x.grad, [p.grad for p in ps]
    with torch.no_grad():
        return mhc.mhc_layer_fused_dynamic_inference(x, *ps, iters, sk_eps, rms_eps), None, None


def _oracle_dyn(d, iters=20, sk_eps=1e-8, rms_eps=1e-5):
    x = d["x"].double().requires_grad_(True)
    ps = [d[k].double().requires_grad_(True) for k in PARAMS]
    out = R.mhc_layer_dynamic(x, *ps, iters, sk_eps, rms_eps, dtype=torch.float64)
    out.backward(d["grad"].double())
    return out.detach(), x.grad, [p.grad for p in ps]


def _check_dyn(got, want, x_dtype, tag, family_floor=False):
    """family_floor: each parameter gradient also gets an absolute floor of
    1e-5 x the largest gradient of its family (phi_*, alpha_*, b_*).  For n =
    1 the RMSNorm is invariant to the scale h_pre, so the pre-side gradients
    are a cancellation that only eps keeps from zero (fp32 autograd of the
    same math misses them by as much), and the 1 x 1 Sinkhorn output is 1
    whatever its input."""
    out, gx, gp = got
    rout, rgx, rgp = want
    fam = {}
    for nm, e in zip(PARAMS, rgp):
        key = nm.split("_")[0]
        fam[key] = max(fam.get(key, 0.0), float(e.abs().max()))
    assert out.dtype == torch.float32
    assert_close(out, rout, what=f"{tag} out", **FWD)
    if gx is None:
        return
    if x_dtype == torch.bfloat16:
        assert_close_dyn_dx_bf16(gx, rgx, f"{tag} dx (bf16)")
    else:
        assert_close(gx, rgx, 1e-3, grad_atol(rgx, 1e-5), f"{tag} dx")
    for nm, a, e in zip(PARAMS, gp, rgp):
        if nm == "weight":
            assert_close_bf16(a, e, f"{tag} d_weight (bf16 param)")
        else:
            floor = grad_atol(e, 1e-4)
            if family_floor:
                floor = max(floor, 1e-5 * fam[nm.split("_")[0]])
            assert_close(a, e, 1e-3, floor, f"{tag} d_{nm}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,C", [(1, 64), (7, 256), (64, 1024), (33, 4096)])
def test_dynamic_layer_matches_oracle(device, x_dtype, B, C):
    d = R.dynamic_layer_inputs(B, 4, C, seed=B + C, x_dtype=x_dtype, b_std=0.5)
    _check_dyn(_run_dyn(d, device), _oracle_dyn(d), x_dtype, f"B={B} C={C} {x_dtype}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,C", [(5, 64), (40, 1280)])
def test_dynamic_layer_n2_matches_oracle(device, x_dtype, B, C):
    """Expansion rate 2 (8 projection outputs; one row per lane-pair Sinkhorn)."""
    d = R.dynamic_layer_inputs(B, 2, C, seed=2 * B + C, x_dtype=x_dtype, alpha=0.3, phi_std=0.05, b_std=0.5)
    _check_dyn(_run_dyn(d, device), _oracle_dyn(d), x_dtype, f"n=2 B={B} C={C} {x_dtype}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,C", [(3, 64), (37, 320), (128, 1280), (1100, 64)])
def test_dynamic_layer_n8_matches_oracle(device, x_dtype, B, C):
    """Expansion rate 8: 2n + n^2 = 80 projection rows in three 32-row
    output tiles; (128, 1280) is a paper configuration (benchmark.py:306).
    Up to 1024 tokens the projection backward runs over all tiles at once;
    B = 1100 takes the per-tile path."""
    d = R.dynamic_layer_inputs(B, 8, C, seed=8 * B + C, x_dtype=x_dtype, alpha=0.3, phi_std=0.05, b_std=0.5)
    _check_dyn(_run_dyn(d, device), _oracle_dyn(d), x_dtype, f"n=8 B={B} C={C} {x_dtype}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_dynamic_layer_n8_wide_hidden(device, x_dtype):
    """n = 8, C = 10240: the register forward holds the rows, the backward's
    do not fit and run the channel-loop kernel (dM in its row sums)."""
    d = R.dynamic_layer_inputs(4, 8, 10240, seed=81, x_dtype=x_dtype, alpha=0.3, phi_std=0.02, b_std=0.5)
    _check_dyn(_run_dyn(d, device), _oracle_dyn(d), x_dtype, f"n=8 C=10240 {x_dtype}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,B,C", [(16, 5, 64), (32, 3, 96), (32, 32, 1280)])
def test_dynamic_layer_wide_n(device, x_dtype, n, B, C):
    """Expansion rates 16 and 32: 2n + n^2 projection rows (1088 at n = 32)
    in 32-row output tiles, per-token Sinkhorn on n-lane groups, dM from the
    per-token Gram kernel; (32, 1280, 32) is a paper configuration
    (benchmark.py:307)."""
    d = R.dynamic_layer_inputs(B, n, C, seed=n * 100 + B + C, x_dtype=x_dtype, alpha=0.1, phi_std=0.02, b_std=0.5)
    _check_dyn(_run_dyn(d, device), _oracle_dyn(d), x_dtype, f"n={n} B={B} C={C} {x_dtype}")


@pytest.mark.parametrize("iters", [0, 1, 32, 33])
def test_dynamic_layer_n32_iteration_counts(device, iters):
    """n = 32 runs one token per workgroup with the Sinkhorn adjoint's state
    in registers for up to 32 iterations; 33 takes the lane-group adjoint
    with its history in the workspace."""
    d = R.dynamic_layer_inputs(6, 32, 64, seed=3300 + iters, x_dtype=torch.float32, alpha=0.1, phi_std=0.02,
                               b_std=0.5)
    _check_dyn(_run_dyn(d, device, iters=iters), _oracle_dyn(d, iters=iters), torch.float32, f"n=32 T={iters}")


@pytest.mark.parametrize("iters,B", [(25, 40), (30, 5), (1, 5)])
def test_dynamic_layer_runtime_n_iteration_counts(device, iters, B):
    """Generic n (12) with the Sinkhorn history region sized for 20
    iterations: at 25 iterations and 40 tokens fewer token slots fit than
    there are tokens (slots take several tokens each), at 30 iterations and
    5 tokens not even one workgroup's slots fit (each iteration's state is
    recomputed instead), and one iteration."""
    d = R.dynamic_layer_inputs(B, 12, 64, seed=3400 + iters + B, x_dtype=torch.float32, alpha=0.1, phi_std=0.02,
                               b_std=0.5)
    _check_dyn(_run_dyn(d, device, iters=iters), _oracle_dyn(d, iters=iters), torch.float32,
               f"n=12 T={iters} B={B}")


def test_dynamic_layer_unsupported_n_raises(device):
    layer = mhc.MHCLayer(64, 65, use_dynamic_h=True).to(device)
    with pytest.raises(RuntimeError, match="n=65 is not supported"):
        layer(torch.randn(3, 65, 64, device=device))


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,B,C", [(1, 9, 96), (3, 7, 96), (3, 1100, 64), (5, 9, 160), (6, 5, 64), (6, 1100, 64),
                                   (6, 4200, 32), (7, 3, 32), (12, 4, 128), (20, 3, 64), (64, 3, 64), (64, 300, 64)])
def test_dynamic_layer_runtime_n(device, x_dtype, n, B, C):
    """Expansion rates without a fixed-n kernel (the reference takes any n up
    to 64, mhc_types.h:68): the generic row kernels, the per-token Sinkhorn on
    16 / 32 / 64-lane groups with n at run time, dM on zero-padded fp32 MFMA
    blocks; the projection over 2n + n^2 rows (15 .. 4224) in 32-row tiles or
    the streaming kernels.  B = 1100 runs more tokens than the backward has
    workgroups (and, with bf16 x at n = 6, the one-pass projection, also
    over 4200 tokens); at
    n = 64, 300 tokens are more than the Sinkhorn history region's 200 token
    slots, so each slot takes several tokens."""
    d = R.dynamic_layer_inputs(B, n, C, seed=n * 100 + B + C, x_dtype=x_dtype, alpha=0.1, phi_std=0.02, b_std=0.5)
    _check_dyn(_run_dyn(d, device), _oracle_dyn(d), x_dtype, f"n={n} B={B} C={C} {x_dtype}", family_floor=n == 1)


@pytest.mark.parametrize("dynamic", [False, True])
@pytest.mark.parametrize("n", [3, 6, 12])
def test_module_runtime_n(device, dynamic, n):
    """MHCLayer(expansion_rate=n) for n without a fixed-n kernel, through the
    module (parameters, autograd, every gradient), against the oracle."""
    C, B = 256, 6
    torch.manual_seed(n)
    layer = mhc.MHCLayer(C, n, use_dynamic_h=dynamic)
    g = _gen(40 + n)
    names = list(PARAMS[1:]) if dynamic else ["H_pre", "H_post", "H_res"]
    with torch.no_grad():
        layer.rmsnorm_weight.copy_((1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16))
        for k in names:
            t = getattr(layer, k)
            if k.startswith("alpha"):
                t.fill_(0.2)
            elif k.startswith("phi"):
                t.copy_(0.03 * torch.randn(t.shape, generator=g))
            else:
                t.copy_(0.5 * torch.randn(t.shape, generator=g))
    x = torch.randn(B, n, C, generator=g)
    go = torch.randn(B, n, C, generator=g)
    layer = layer.to(device)
    xd = x.to(device).requires_grad_(True)
    out = layer(xd)
    out.backward(go.to(device))
    w = layer.rmsnorm_weight.detach().cpu().double().requires_grad_(True)
    ps = [getattr(layer, k).detach().cpu().double().requires_grad_(True) for k in names]
    xr = x.double().requires_grad_(True)
    if dynamic:
        ref = R.mhc_layer_dynamic(xr, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    else:
        ref = R.mhc_layer_static(xr, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    ref.backward(go.double())
    tag = f"module n={n} dynamic={dynamic}"
    assert_close(out, ref.detach(), what=f"{tag} out", **FWD)
    assert_close(xd.grad, xr.grad, 1e-3, grad_atol(xr.grad, 1e-5), f"{tag} dx")
    assert_close_bf16(layer.rmsnorm_weight.grad, w.grad, f"{tag} d_weight")
    for k, p in zip(names, ps):
        assert_close(getattr(layer, k).grad, p.grad, 1e-3, grad_atol(p.grad, 1e-4), f"{tag} d_{k}")


@pytest.mark.parametrize("alpha,phi_std", [(0.5, 0.05), (2.0, 0.02)])
def test_dynamic_layer_strong_dynamic_h(device, alpha, phi_std):
    """Large alpha makes t (and so h, M) vary strongly per token."""
    d = R.dynamic_layer_inputs(40, 4, 512, seed=int(alpha * 10), x_dtype=torch.float32, alpha=alpha,
                               phi_std=phi_std, b_std=1.0)
    _check_dyn(_run_dyn(d, device), _oracle_dyn(d), torch.float32, f"alpha={alpha}")


def test_dynamic_inference_equals_training_forward(device):
    d = R.dynamic_layer_inputs(16, 4, 256, seed=2, b_std=0.5)
    out_t = _run_dyn(d, device)[0].detach()
    out_i = _run_dyn(d, device, training=False)[0]
    assert torch.equal(out_t, out_i)


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,B,C", [(4, 1, 64), (4, 37, 1280), (2, 9, 256), (4, 300, 4096), (8, 5, 320),
                                   (8, 1100, 64), (32, 4, 1280), (6, 7, 320), (12, 3, 64)])
def test_dynamic_inference_packed_and_bf16_out(device, x_dtype, n, B, C):
    """The forward-only entry on packed parameters: its fp32 output is the
    training forward's bit for bit, its bf16 output is that result rounded to
    nearest even, and the oracle bounds both."""
    d = R.dynamic_layer_inputs(B, n, C, seed=3 * B + C + n, x_dtype=x_dtype, alpha=0.3, phi_std=0.05, b_std=0.5)
    x = d["x"].to(device)
    ps = [d[k].to(device) for k in PARAMS]
    with torch.no_grad():
        fwd_out, _ = native.mhc_layer_dynamic_fwd(x, *ps, 20, 1e-8, 1e-5)
        packed = native.mhc_layer_dynamic_pack(*ps[:4])
        o32 = native.mhc_layer_dynamic_infer(x, packed, *ps[4:], 20, 1e-8, 1e-5)
        o16 = native.mhc_layer_dynamic_infer(x, packed, *ps[4:], 20, 1e-8, 1e-5, out_dtype=torch.bfloat16)
        o16_api = mhc.mhc_layer_fused_dynamic_inference(x, *ps, 20, 1e-8, 1e-5, out_dtype=torch.bfloat16)
    assert o32.dtype == torch.float32 and o16.dtype == torch.bfloat16
    assert torch.equal(o32, fwd_out)
    assert torch.equal(o16, fwd_out.to(torch.bfloat16))
    assert torch.equal(o16_api, o16)
    rout = R.mhc_layer_dynamic(d["x"].double(), *[d[k].double() for k in PARAMS], 20, 1e-8, 1e-5,
                               dtype=torch.float64)
    assert_close(o32, rout, what=f"infer n={n} B={B} C={C}", **FWD)
    assert_close(o16, rout, 2 ** -8, 1e-5, f"infer bf16 out n={n} B={B} C={C}")


def test_dynamic_module_inference_pack_snapshot(device):
    """prepare_inference() packs once; an in-place parameter update drops the
    snapshot, and the eval forward then equals the training forward on the
    new parameters."""
    torch.manual_seed(6)
    layer = mhc.MHCLayer(512, 4).to(device).eval()
    x = torch.randn(20, 4, 512, generator=_gen(6)).to(device)
    with torch.no_grad():
        base = layer(x)
        layer.prepare_inference()
        assert layer._packed() is not None
        assert torch.equal(layer(x), base)
        layer.phi_res.add_(0.05 * torch.randn(layer.phi_res.shape, generator=_gen(7)).to(device))
        assert layer._packed() is None
        after = layer(x)
    assert not torch.equal(after, base)
    layer.train()
    assert torch.equal(after, layer(x).detach())
    layer.eval()
    layer.prepare_inference()
    layer.train()
    assert layer._inference_pack is None


def test_dynamic_module_eval_n32_unpacked_and_packed(device):
    """n = 32 (1088 projection rows): the unpacked eval forward runs the
    streaming training forward, the packed one the forward-only entry on
    the split planes; both equal the training forward bit for bit."""
    torch.manual_seed(32)
    layer = mhc.MHCLayer(128, 32).to(device)
    with torch.no_grad():
        for k in ("phi_pre", "phi_post", "phi_res"):
            getattr(layer, k).normal_(0.0, 0.05)
        layer.alpha_res.fill_(0.2)
    x = torch.randn(40, 32, 128, generator=_gen(33)).to(device)
    train_out = layer(x).detach()
    layer.eval()
    with torch.no_grad():
        unpacked = layer(x)
        layer.prepare_inference()
        packed = layer(x)
    assert torch.equal(unpacked, train_out)
    assert torch.equal(packed, train_out)


def test_dynamic_inference_rejects_bad_arguments(device):
    layer = mhc.MHCLayer(64, 4).to(device)
    scal = [layer.alpha_pre, layer.alpha_post, layer.alpha_res, layer.b_pre, layer.b_post, layer.b_res]
    with torch.no_grad():
        packed = native.mhc_layer_dynamic_pack(layer.rmsnorm_weight, layer.phi_pre, layer.phi_post, layer.phi_res)
        with pytest.raises(RuntimeError, match="packed parameters do not match"):
            native.mhc_layer_dynamic_infer(torch.randn(3, 4, 128, device=device), packed, *scal)
        with pytest.raises(RuntimeError, match="out_dtype"):
            native.mhc_layer_dynamic_infer(torch.randn(3, 4, 64, device=device), packed, *scal,
                                           out_dtype=torch.float16)
        empty = native.mhc_layer_dynamic_infer(torch.randn(0, 4, 64, device=device), packed, *scal)
    assert tuple(empty.shape) == (0, 4, 64)


def test_dynamic_module_train_and_eval(device):
    torch.manual_seed(4)
    layer = mhc.MHCLayer(256, 4, use_dynamic_h=True).to(device)
    with torch.no_grad():
        layer.b_pre.normal_()
        layer.b_res.normal_()
        layer.alpha_res.fill_(0.3)
    x = torch.randn(24, 4, 256, generator=_gen(4)).to(device)
    g = torch.randn(24, 4, 256, generator=_gen(5)).to(device)
    layer.train()
    xt = x.clone().requires_grad_(True)
    out = layer(xt)
    out.backward(g)
    d = {"x": x.cpu(), "grad": g.cpu()}
    for k in PARAMS:
        d[k] = getattr(layer, "rmsnorm_weight" if k == "weight" else k).detach().cpu()
    rout, rgx, rgp = _oracle_dyn(d)
    assert_close(out, rout, what="module out", **FWD)
    assert_close(xt.grad, rgx, 1e-3, grad_atol(rgx, 1e-5), "module dx")
    assert_close(layer.phi_res.grad, rgp[3], 1e-3, grad_atol(rgp[3], 1e-4), "module d_phi_res")
    assert_close(layer.alpha_res.grad, rgp[6], 1e-3, grad_atol(rgp[6], 1e-4), "module d_alpha_res")
    layer.eval()
    with torch.no_grad():
        assert_close(layer(x), rout, what="module eval", **FWD)


def test_dynamic_layer_config_c4_full_size(device):
    """Config C4: x bf16 [8192, 4, 4096], phi ~ N(0, 0.02), alpha 0.01, b 0.
    Per-token outputs on a token subsample vs the oracle; token-summed
    parameter gradients by additivity over two halves (fp32 native grads)
    and against the oracle on a 128-token slice."""
    B, n, C = 8192, 4, 4096
    d = R.dynamic_layer_inputs(B, n, C, seed=44)
    dev = {k: v.to(device) for k, v in d.items()}
    pvals = [dev[k] for k in PARAMS]

    def grads(sl):
        w32 = dev["weight"].float()
        out, saved = native.mhc_layer_dynamic_fwd(dev["x"][sl], w32, *pvals[1:])
        g = native.mhc_layer_dynamic_bwd(dev["grad"][sl], dev["x"][sl], w32, saved, *pvals[1:])
        return out, g

    out, g_full = grads(slice(0, B))
    idx = torch.randperm(B, generator=_gen(6))[:32]
    sub = {k: (v[idx] if k in ("x", "grad") else v) for k, v in d.items()}
    rout, rgx, _ = _oracle_dyn(sub)
    assert_close(out.cpu()[idx], rout, what="C4 out subsample", **FWD)
    assert_close_dyn_dx_bf16(g_full[0].cpu()[idx], rgx, "C4 dx subsample (bf16)")
    _, g1 = grads(slice(0, B // 2))
    _, g2 = grads(slice(B // 2, B))
    names = ["d_weight", "d_phi_pre", "d_phi_post", "d_phi_res", "d_alpha_pre", "d_alpha_post", "d_alpha_res",
             "d_b_pre", "d_b_post", "d_b_res"]
    for k, nm in enumerate(names):
        s = g1[k + 1] + g2[k + 1]
        assert_close(g_full[k + 1], s, 1e-4, grad_atol(s, 1e-5), f"C4 additivity {nm}")
    sl = {k: (v[:128] if k in ("x", "grad") else v) for k, v in d.items()}
    _check_dyn(_run_dyn(sl, device), _oracle_dyn(sl), torch.bfloat16, "C4 slice")


@pytest.mark.parametrize("B,C", [(1000, 1024), (257, 4096), (3001, 2048), (9001, 256)])
def test_dynamic_layer_backward_many_tokens(device, B, C):
    """bf16 x at n = 4 with many tokens per persistent workgroup and a token
    count that fills no launch evenly: every token's dx (B <= 1000) or a
    strided third of them against the oracle, the parameter gradients against
    the oracle (B <= 1000) or by additivity over two parts split inside a
    workgroup's token range.  At B = 9001 the whole batch has more than 512
    rows of db / dalpha partials and takes the separate column-sum launches,
    its two parts the single multi-job launch."""
    n = 4
    d = R.dynamic_layer_inputs(B, n, C, seed=B + C, alpha=0.3, phi_std=0.05, b_std=0.5)
    if B <= 1000:
        _check_dyn(_run_dyn(d, device), _oracle_dyn(d), torch.bfloat16, f"many tokens B={B} C={C}")
        return
    dev = {k: v.to(device) for k, v in d.items()}
    pvals = [dev[k] for k in PARAMS]

    def grads(sl):
        w32 = dev["weight"].float()
        out, saved = native.mhc_layer_dynamic_fwd(dev["x"][sl], w32, *pvals[1:])
        return native.mhc_layer_dynamic_bwd(dev["grad"][sl], dev["x"][sl], w32, saved, *pvals[1:])

    g_full = grads(slice(0, B))
    idx = torch.arange(0, B, 3)
    sub = {k: (v[idx] if k in ("x", "grad") else v) for k, v in d.items()}
    _, rgx, _ = _oracle_dyn(sub)
    assert_close_dyn_dx_bf16(g_full[0].cpu()[idx], rgx, f"many tokens B={B} C={C} dx (every third token)")
    h = 1200  # not a multiple of the block size
    g1, g2 = grads(slice(0, h)), grads(slice(h, B))
    for k in range(1, len(g_full)):
        s = g1[k] + g2[k]
        assert_close(g_full[k], s, 1e-4, grad_atol(s, 1e-5), f"many tokens B={B} additivity {k}")

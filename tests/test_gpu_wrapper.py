"""GPU parity of the fused MHCResidualWrapper (layer.py:225-329) against the
float64 CPU oracle: stream synthesis ('decay' with the storage-dtype rounding
of residual*0.1**(i-1), and 'zero'), the layer (dynamic and static H), the
stream mean and the [B, T, C] reshape; forward and every gradient.

Tolerances: fp32 outputs rtol 1e-4; gradients rtol 1e-3 (fp32 storage) or
one bf16 rounding (2^-8 relative, plus 1e-3 max|ref|) for bf16 storage,
against an oracle whose leaves are exact (float64) so that its gradients are
not rounded; absolute floors relative to max|ref|.  Config C5 runs
at its width C=7168 on a reduced token count (the full-size oracle needs
~200 GB)."""
import pytest
import torch

import mhc_ascend_amd as mhc
from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, grad_atol

pytestmark = pytest.mark.gpu

DYN = ["phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post", "b_res"]
STA = ["H_pre", "H_post", "H_res"]


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _make(C, dynamic, seed, alpha=0.3, phi_std=0.05, n=4):
    torch.manual_seed(seed)
    wrap = mhc.MHCResidualWrapper(C, n, use_dynamic_h=dynamic)
    layer = wrap.mhc
    g = _gen(seed + 1)
    with torch.no_grad():
        layer.rmsnorm_weight.copy_((1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16))
        if dynamic:
            for k in ("phi_pre", "phi_post", "phi_res"):
                getattr(layer, k).copy_(phi_std * torch.randn(getattr(layer, k).shape, generator=g))
            for k in ("alpha_pre", "alpha_post", "alpha_res"):
                getattr(layer, k).fill_(alpha)
            for k in ("b_pre", "b_post", "b_res"):
                getattr(layer, k).copy_(0.3 * torch.randn(getattr(layer, k).shape, generator=g))
        else:
            for k in STA:
                getattr(layer, k).copy_(torch.randn(getattr(layer, k).shape, generator=g))
    return wrap


def _oracle(wrap, res, br, grad, mode):
    """float64 oracle: streams synthesised in the storage dtype, layer in f64."""
    layer = wrap.mhc
    names = DYN if layer.use_dynamic_h else STA
    w = layer.rmsnorm_weight.detach().cpu().double().requires_grad_(True)
    ps = [getattr(layer, k).detach().cpu().double().requires_grad_(True) for k in names]
    # exact leaves holding the storage values; the decay streams rounded to
    # the storage dtype in value only, so the leaf gradients stay unrounded
    r = res.detach().cpu().double().requires_grad_(True)
    b = br.detach().cpu().double().requires_grad_(True)
    it, eps = int(layer.num_sinkhorn_iters), float(layer.sinkhorn_eps)
    if layer.use_dynamic_h:
        fn = lambda X: R.mhc_layer_dynamic(X, w, *ps, it, eps, 1e-5, dtype=torch.float64)
    else:
        fn = lambda X: R.mhc_layer_static(X, w, *ps, it, eps, 1e-5, dtype=torch.float64)
    out = R.mhc_residual_wrapper(r, b, fn, layer.expansion_rate, mode, storage_dtype=res.dtype)
    out.backward(grad.double())
    return out.detach(), r.grad, b.grad, w.grad, [p.grad for p in ps]


def _run(wrap, res, br, grad, device):
    wrap = wrap.to(device)
    r = res.to(device).requires_grad_(True)
    b = br.to(device).requires_grad_(True)
    out = wrap(r, b)
    out.backward(grad.to(device))
    layer = wrap.mhc
    names = DYN if layer.use_dynamic_h else STA
    return out.detach(), r.grad, b.grad, layer.rmsnorm_weight.grad, [getattr(layer, k).grad for k in names]


def _check(got, want, dtype, names, tag, res_vanish=True):
    out, gr, gb, gw, gp = got
    rout, rgr, rgb, rgw, rgp = want
    assert out.dtype == torch.float32 and tuple(out.shape) == tuple(rout.shape), (out.dtype, out.shape, rout.shape)
    assert_close(out, rout, 1e-4, grad_atol(rout, 1e-5), f"{tag} out")
    assert gr.dtype == dtype and gb.dtype == dtype
    if dtype == torch.bfloat16:
        assert_close_bf16(gr, rgr, f"{tag} d residual")
        assert_close_bf16(gb, rgb, f"{tag} d branch")
    else:
        assert_close(gr, rgr, 1e-3, grad_atol(rgr, 1e-5), f"{tag} d residual")
        assert_close(gb, rgb, 1e-3, grad_atol(rgb, 1e-5), f"{tag} d branch")
    assert_close_bf16(gw, rgw, f"{tag} d_weight (bf16 param)")
    # Through the stream mean every stream gets the same cotangent G / n, so
    # dM is constant along i and the Sinkhorn adjoint's last column step
    # cancels it: the H_res-side gradients are 0 up to eps-terms (~1e-20
    # relative) and fp32 rounding.  Their absolute floor therefore comes from
    # the non-vanishing members of the same family.
    fam = {}
    for nm, e in zip(names, rgp):
        key = nm.split("_")[0]
        fam[key] = max(fam.get(key, 0.0), float(e.abs().max()))
    for nm, a, e in zip(names, gp, rgp):
        floor = max(grad_atol(e, 1e-4), 1e-5 * fam[nm.split("_")[0]])
        assert_close(a, e, 1e-3, floor, f"{tag} d_{nm}")
        if nm.endswith("res") and res_vanish:
            assert float(a.abs().max()) <= 1e-5 * fam[nm.split("_")[0]], f"{tag} d_{nm} should vanish"


@pytest.mark.parametrize("dynamic", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["decay", "zero"])
@pytest.mark.parametrize("shape", [(3, 5, 256), (37, 1024), (19, 160), (2, 3, 224)])
def test_wrapper_matches_oracle(device, dynamic, dtype, mode, shape):
    C = shape[-1]
    seed = len(shape) * 100 + C + (7 if dynamic else 0) + (3 if mode == "zero" else 0)
    wrap = _make(C, dynamic, seed)
    wrap.residual_mode = mode
    g = _gen(seed + 2)
    res = torch.randn(*shape, generator=g).to(dtype)
    br = torch.randn(*shape, generator=g).to(dtype)
    grad = torch.randn(*shape, generator=g)
    want = _oracle(wrap, res, br, grad, mode)
    got = _run(wrap, res, br, grad, device)
    _check(got, want, dtype, DYN if dynamic else STA, f"dyn={dynamic} {dtype} {mode} {shape}")


@pytest.mark.parametrize("dynamic", [True, False])
def test_wrapper_config_c5_width(device, dynamic):
    """Config C5 at its width: residual/branch bf16 [B=16, T=4, 7168], phi
    ~ N(0, 0.02), alpha 0.01, b 0 (the layer defaults of layer.py:69-79)."""
    C = 7168
    torch.manual_seed(5)
    wrap = mhc.MHCResidualWrapper(C, 4, use_dynamic_h=dynamic)
    g = _gen(55)
    res = torch.randn(16, 4, C, generator=g).to(torch.bfloat16)
    br = torch.randn(16, 4, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(16, 4, C, generator=g)
    want = _oracle(wrap, res, br, grad, "decay")
    got = _run(wrap, res, br, grad, device)
    _check(got, want, torch.bfloat16, DYN if dynamic else STA, f"C5 width dyn={dynamic}")


@pytest.mark.parametrize("n,dynamic,C", [(2, False, 256), (8, False, 256), (2, True, 256), (8, True, 128),
                                         (32, False, 64), (32, True, 64), (4, False, 250), (6, False, 256),
                                         (6, True, 128), (3, True, 96)])
@pytest.mark.parametrize("mode", ["decay", "zero"])
def test_wrapper_general_n(device, n, dynamic, C, mode):
    """Other expansion rates on fp32 rows: n = 2..8 and 32 run the run-time-n
    wrapper kernels; rows that are not a multiple of 4 build the streams
    with device tensor ops and run them through the layer."""
    torch.manual_seed(n)
    wrap = mhc.MHCResidualWrapper(C, n, use_dynamic_h=dynamic)
    wrap.residual_mode = mode
    layer = wrap.mhc
    g = _gen(70 + n)
    with torch.no_grad():
        layer.rmsnorm_weight.copy_((1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16))
        if dynamic:
            for k in ("phi_pre", "phi_post", "phi_res"):
                getattr(layer, k).copy_(0.05 * torch.randn(getattr(layer, k).shape, generator=g))
            for k in ("alpha_pre", "alpha_post", "alpha_res"):
                getattr(layer, k).fill_(0.3)
        else:
            for k in STA:
                getattr(layer, k).copy_(torch.randn(getattr(layer, k).shape, generator=g))
    res = torch.randn(3, 5, C, generator=g)
    br = torch.randn(3, 5, C, generator=g)
    grad = torch.randn(3, 5, C, generator=g)
    layer_names = DYN if dynamic else STA
    w = layer.rmsnorm_weight.detach().cpu().double().requires_grad_(True)
    ps = [getattr(layer, k).detach().cpu().double().requires_grad_(True) for k in layer_names]
    r = res.clone().requires_grad_(True)
    b = br.clone().requires_grad_(True)
    if dynamic:
        fn = lambda X: R.mhc_layer_dynamic(X, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    else:
        fn = lambda X: R.mhc_layer_static(X, w, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    want_out = R.mhc_residual_wrapper(r, b, fn, n, mode)
    want_out.backward(grad.double())
    got = _run(wrap, res, br, grad, device)
    assert_close(got[0], want_out.detach(), 1e-4, grad_atol(want_out.detach(), 1e-5), f"n={n} out")
    assert_close(got[1], r.grad.double(), 1e-3, grad_atol(r.grad.double(), 1e-5), f"n={n} d residual")
    assert_close(got[2], b.grad.double(), 1e-3, grad_atol(b.grad.double(), 1e-5), f"n={n} d branch")


def test_wrapper_single_token_rows_stay_flat(device):
    """[B, 1, C] comes back as [B, C] (layer.py:319-320)."""
    wrap = _make(128, True, 9).to(device)
    res = torch.randn(6, 1, 128, generator=_gen(10)).to(device)
    br = torch.randn(6, 1, 128, generator=_gen(11)).to(device)
    assert tuple(wrap(res, br).shape) == (6, 128)


def test_wrapper_rejects_unknown_mode(device):
    wrap = _make(64, True, 12).to(device)
    wrap.residual_mode = "bogus"
    x = torch.randn(4, 64, device=device)
    with pytest.raises(ValueError, match="Unknown residual_mode"):
        wrap(x, x)


def test_wrapper_eval_no_grad_matches_training_forward(device):
    wrap = _make(256, True, 13).to(device)
    res = torch.randn(20, 256, generator=_gen(14)).to(device)
    br = torch.randn(20, 256, generator=_gen(15)).to(device)
    out_t = wrap(res, br).detach()
    wrap.eval()
    with torch.no_grad():
        out_e = wrap(res, br)
    assert torch.equal(out_t, out_e)


@pytest.mark.parametrize("n,dynamic", [(4, True), (4, False), (3, True), (3, False), (8, True), (8, False),
                                       (10, True), (16, False)])
@pytest.mark.parametrize("iters,eps", [(0, 1e-8), (1, 1e-8), (1, 0.1), (20, 0.1)])
def test_wrapper_sinkhorn_settings(device, n, dynamic, iters, eps):
    """Both sides of the rule that writes the H_res gradients as zeros.
    num_iters >= 1 with eps <= 1e-6: the last column normalisation removes
    the column-constant dM (zeros written, checked against the oracle's
    near-zero values).  No iterations (M = exp(t), nothing cancels) or a
    large eps (a leftover of order eps): the full Sinkhorn adjoint runs and
    the H_res gradients are checked against the oracle's (with one
    iteration or none they are of the order of the other gradients; after
    20 iterations at eps = 0.1 about 1e-12 of them, measured on the
    oracle).  n = 3 and 8 run the run-time-n kernels (at n = 8 with all 80
    projection rows: the small-np projection backward), n = 10 with dynamic
    H (120 rows: the most the fused wrapper carries when the H_res
    gradients do not vanish) and n = 16 with static H (dynamic H at n = 16
    takes the tensor-op path at the settings that keep the H_res gradients,
    and its bf16 stream gradients are rounded once per stream before
    autograd sums them, more than this test's one-rounding tolerance)."""
    C, B = 256, 37
    seed = 900 + iters + int(eps * 100) + (7 if dynamic else 0) + 10 * n
    wrap = _make(C, dynamic, seed, n=n)
    wrap.mhc.num_sinkhorn_iters = iters
    wrap.mhc.sinkhorn_eps = eps
    g = _gen(seed + 2)
    res = torch.randn(B, C, generator=g).to(torch.bfloat16)
    br = torch.randn(B, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(B, C, generator=g)
    want = _oracle(wrap, res, br, grad, "decay")
    got = _run(wrap, res, br, grad, device)
    vanish = iters >= 1 and eps <= 1e-6
    names = DYN if dynamic else STA
    _check(got, want, torch.bfloat16, names, f"n={n} dyn={dynamic} iters={iters} eps={eps}", res_vanish=vanish)
    if not vanish and iters <= 1:
        # the oracle's H_res gradients are not negligible here
        fam = max(float(e.abs().max()) for nm, e in zip(names, want[4]) if nm.endswith("pre"))
        res_ref = max(float(e.abs().max()) for nm, e in zip(names, want[4]) if nm.endswith("res"))
        assert res_ref > 1e-4 * fam, (res_ref, fam)


@pytest.mark.parametrize("n,dynamic,C", [(2, False, 256), (3, False, 96), (5, False, 160), (8, False, 256),
                                         (2, True, 256), (3, True, 96), (5, True, 96), (6, True, 256),
                                         (7, True, 96), (8, True, 256), (4, True, 264), (4, False, 17000),
                                         (8, True, 4), (2, True, 16), (5, False, 4), (6, True, 1104)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["decay", "zero"])
def test_wrapper_runtime_n_matches_oracle(device, n, dynamic, C, dtype, mode):
    """The run-time-n wrapper kernels (n = 2..8; n = 4 rows the n = 4 kernels
    refuse: 264 channels with dynamic H, 17000 with static H; rows of 4 and
    16 channels, narrower than one wave's chunks; 1104 channels, a partial
    column block of every backward kernel) against the float64 oracle, every
    output and gradient, both storage dtypes and both residual modes."""
    seed = 1000 + 10 * n + (7 if dynamic else 0) + (3 if mode == "zero" else 0)
    wrap = _make(C, dynamic, seed, n=n)
    wrap.residual_mode = mode
    g = _gen(seed + 2)
    shape = (2, 3, C) if C > 1024 else (37, C)
    res = torch.randn(*shape, generator=g).to(dtype)
    br = torch.randn(*shape, generator=g).to(dtype)
    grad = torch.randn(*shape, generator=g)
    want = _oracle(wrap, res, br, grad, mode)
    got = _run(wrap, res, br, grad, device)
    _check(got, want, dtype, DYN if dynamic else STA, f"n={n} C={C} dyn={dynamic} {dtype} {mode}")


@pytest.mark.parametrize("n", [5, 8])
@pytest.mark.parametrize("mode", ["decay", "zero"])
def test_wrapper_runtime_n_many_tokens(device, n, mode):
    """bf16 storage from 1024 tokens up with whole 64-channel stages: the
    forward projection rebuilds the streams from residual and branch inside
    the streaming projection kernel (no stream rows in memory) - against the
    float64 oracle, every output and gradient."""
    C, B = 128, 1100
    seed = 2000 + 10 * n + (3 if mode == "zero" else 0)
    wrap = _make(C, True, seed, n=n)
    wrap.residual_mode = mode
    g = _gen(seed + 2)
    res = torch.randn(B, C, generator=g).to(torch.bfloat16)
    br = torch.randn(B, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(B, C, generator=g)
    want = _oracle(wrap, res, br, grad, mode)
    got = _run(wrap, res, br, grad, device)
    _check(got, want, torch.bfloat16, DYN, f"n={n} B={B} {mode}")


@pytest.mark.parametrize("n,dynamic", [(3, True), (7, True), (5, False), (8, False)])
@pytest.mark.parametrize("tokens", [1, 2, 17])
def test_wrapper_runtime_n_few_tokens(device, n, dynamic, tokens):
    """The run-time-n kernels on 1, 2 and 17 tokens (one wave per token in
    the row passes; token tiles of one or two tokens in the backward) against
    the float64 oracle, every gradient."""
    C = 96
    seed = 3000 + 10 * n + tokens + (7 if dynamic else 0)
    wrap = _make(C, dynamic, seed, n=n)
    g = _gen(seed + 2)
    res = torch.randn(tokens, C, generator=g).to(torch.bfloat16)
    br = torch.randn(tokens, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(tokens, C, generator=g)
    want = _oracle(wrap, res, br, grad, "decay")
    got = _run(wrap, res, br, grad, device)
    _check(got, want, torch.bfloat16, DYN if dynamic else STA, f"n={n} tokens={tokens} dyn={dynamic}")


@pytest.mark.parametrize("n,C", [(9, 96), (12, 256), (16, 160), (20, 64), (32, 256), (32, 4), (16, 1104)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["decay", "zero"])
def test_wrapper_static_wide_n_matches_oracle(device, n, C, dtype, mode):
    """Static H at n = 9..32: the run-time-n kernels with 16- and 32-stream
    capacity (coefficients read back from the lanes, the per-stream sums
    spread over the n*n + 2n scalar slots once per wave) against the float64
    oracle, every output and gradient, both storage dtypes and residual
    modes; in 'decay' mode stream 31 carries residual * 1e-30."""
    seed = 4000 + 10 * n + (3 if mode == "zero" else 0) + (1 if dtype == torch.bfloat16 else 0)
    wrap = _make(C, False, seed, n=n)
    wrap.residual_mode = mode
    g = _gen(seed + 2)
    shape = (2, 3, C) if C > 1024 else (37, C)
    res = torch.randn(*shape, generator=g).to(dtype)
    br = torch.randn(*shape, generator=g).to(dtype)
    grad = torch.randn(*shape, generator=g)
    want = _oracle(wrap, res, br, grad, mode)
    got = _run(wrap, res, br, grad, device)
    _check(got, want, dtype, STA, f"n={n} C={C} {dtype} {mode}")


@pytest.mark.parametrize("n", [16, 32])
def test_wrapper_static_wide_n_many_tokens(device, n):
    """Static H at n = 16 and 32 on 9000 tokens: more tokens than the static
    row-sum grid's waves, so each wave sums several tokens before it spreads
    its per-stream sums - against the float64 oracle, every gradient."""
    C, B = 64, 9000
    seed = 5000 + n
    wrap = _make(C, False, seed, n=n)
    g = _gen(seed + 2)
    res = torch.randn(B, C, generator=g).to(torch.bfloat16)
    br = torch.randn(B, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(B, C, generator=g)
    want = _oracle(wrap, res, br, grad, "decay")
    got = _run(wrap, res, br, grad, device)
    _check(got, want, torch.bfloat16, STA, f"n={n} B={B}")


@pytest.mark.parametrize("n,C", [(9, 96), (12, 256), (16, 160), (20, 64), (32, 128), (16, 1104), (12, 2048),
                                 (16, 2048)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["decay", "zero"])
def test_wrapper_dynamic_wide_n_matches_oracle(device, n, C, dtype, mode):
    """Dynamic H at n = 9..32: the row kernels with 16- and 32-stream
    capacity, the coefficient backward with no Sinkhorn adjoint, and for the
    2n pre / post rows of dP either the dPhi / fold kernels (n <= 16 on rows
    of 2048 channels or more: 32 dP rows in two MFMA tiles) or fp32 stream
    rows for the layer's projection backward (one 32-row tile up to n = 16,
    the small-np kernels above) - against the float64 oracle, every output
    and gradient, both storage dtypes and residual modes."""
    seed = 6000 + 10 * n + (3 if mode == "zero" else 0) + (1 if dtype == torch.bfloat16 else 0)
    wrap = _make(C, True, seed, n=n)
    wrap.residual_mode = mode
    g = _gen(seed + 2)
    shape = (2, 3, C) if C > 1024 else (37, C)
    res = torch.randn(*shape, generator=g).to(dtype)
    br = torch.randn(*shape, generator=g).to(dtype)
    grad = torch.randn(*shape, generator=g)
    want = _oracle(wrap, res, br, grad, mode)
    got = _run(wrap, res, br, grad, device)
    _check(got, want, dtype, DYN, f"n={n} C={C} {dtype} {mode}")


@pytest.mark.parametrize("n,C", [(16, 128), (32, 64)])
def test_wrapper_dynamic_wide_n_many_tokens(device, n, C):
    """Dynamic H at n = 16 and 32 on 1100 bf16 tokens with whole 64-channel
    stages: the forward projection rebuilds the streams inside the streaming
    projection kernel (288 / 1088 rows) - against the float64 oracle, every
    gradient."""
    B = 1100
    seed = 7000 + n
    wrap = _make(C, True, seed, n=n)
    g = _gen(seed + 2)
    res = torch.randn(B, C, generator=g).to(torch.bfloat16)
    br = torch.randn(B, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(B, C, generator=g)
    want = _oracle(wrap, res, br, grad, "decay")
    got = _run(wrap, res, br, grad, device)
    _check(got, want, torch.bfloat16, DYN, f"n={n} B={B}")


@pytest.mark.parametrize("n,C", [(5, 128), (16, 64)])
def test_wrapper_projection_many_token_blocks(device, n, C):
    """4200 bf16 tokens (65 full 64-token blocks of the streaming projection
    and a partial one) with the projection rebuilding the streams from
    residual and branch - against the float64 oracle, every gradient."""
    B = 4200
    seed = 8000 + n
    wrap = _make(C, True, seed, n=n)
    g = _gen(seed + 2)
    res = torch.randn(B, C, generator=g).to(torch.bfloat16)
    br = torch.randn(B, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(B, C, generator=g)
    want = _oracle(wrap, res, br, grad, "decay")
    got = _run(wrap, res, br, grad, device)
    _check(got, want, torch.bfloat16, DYN, f"n={n} B={B}")


def test_wrapper_dynamic_fold_16_streams_many_tokens(device):
    """Dynamic H at n = 16 on 2048-channel rows and 300 tokens: the dPhi /
    fold kernels at their 16-stream capacity over several token tiles -
    against the float64 oracle, every gradient."""
    n, C, B = 16, 2048, 300
    wrap = _make(C, True, 9100, n=n)
    g = _gen(9102)
    res = torch.randn(B, C, generator=g).to(torch.bfloat16)
    br = torch.randn(B, C, generator=g).to(torch.bfloat16)
    grad = torch.randn(B, C, generator=g)
    want = _oracle(wrap, res, br, grad, "decay")
    got = _run(wrap, res, br, grad, device)
    _check(got, want, torch.bfloat16, DYN, f"n={n} C={C} B={B}")

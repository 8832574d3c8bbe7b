"""Config C5 at full size: the fused MHCResidualWrapper (layer.py:269-322) on
residual / branch bf16 [65536, 4, 7168] (262,144 tokens, about 30 GB
resident with the cotangent, outputs and gradients), forward and backward.

The float64 oracle of the whole batch would need ~200 GB of host memory, so
the checks are the size-independent ones:
  * a random token subsample of the output and of d residual / d branch
    against the oracle (per-token quantities: the wrapper is independent
    per token in the forward, and in the backward apart from the parameter
    gradients);
  * additivity of every parameter gradient over two halves of the tokens
    (the gradients are sums over tokens; each half is its own call, with its
    own grid sizing and partial buffers);
  * finiteness of every output.
The full-size persistent grids, the two-round workgroup sizing and the
32-bit buffer offsets only occur at this size."""
import pytest
import torch

from mhc_ascend_amd import native
from oracle import reference as R
from tests.conftest import assert_close, assert_close_bf16, grad_atol

pytestmark = pytest.mark.gpu

BO, T, N, C = 65536, 4, 4, 7168
DYN = ["phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post", "b_res"]
STA = ["H_pre", "H_post", "H_res"]


def _params(dynamic, seed):
    """Layer parameters in the C5 config (phi ~ N(0, 0.02), alpha 0.01, b 0;
    static H ~ N(0, 1) so that the static gradients are not trivial)."""
    g = torch.Generator().manual_seed(seed)
    nC = N * C
    p = {"weight": (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16)}
    if dynamic:
        phi = 0.02 * torch.randn(nC, 2 * N + N * N, generator=g)
        p.update(phi_pre=phi[:, :N].t().contiguous(), phi_post=phi[:, N:2 * N].t().contiguous(),
                 phi_res=phi[:, 2 * N:].t().contiguous(), alpha_pre=torch.tensor(0.01),
                 alpha_post=torch.tensor(0.01), alpha_res=torch.tensor(0.01), b_pre=torch.zeros(N),
                 b_post=torch.zeros(N), b_res=torch.zeros(N, N))
    else:
        p.update(H_pre=torch.randn(N, generator=g), H_post=torch.randn(N, generator=g),
                 H_res=torch.randn(N, N, generator=g))
    return p


def _call(dynamic, r, b, g, w32, pd):
    """Fused wrapper fwd + bwd through the native entries; fp32 parameter
    gradients (so that additivity is checked before any bf16 rounding)."""
    if dynamic:
        args = [pd[k] for k in DYN]
        out, saved = native.wrapper_dynamic_fwd(r, b, "decay", N, w32, *args)
        grads = native.wrapper_dynamic_bwd(g, r, b, "decay", N, w32, saved, *args[:6], args[8])
    else:
        args = [pd[k] for k in STA]
        out, saved = native.wrapper_static_fwd(r, b, "decay", N, w32, *args)
        grads = native.wrapper_static_bwd(g, r, b, "decay", N, w32, *args, saved)
    return out, grads


@pytest.mark.parametrize("dynamic", [True, False])
def test_wrapper_config_c5_full_size(device, dynamic):
    tokens = BO * T
    print(f"[c5 full] dynamic={dynamic} tokens={tokens} C={C}: generating inputs", flush=True)
    gen = torch.Generator(device=device).manual_seed(5 + dynamic)
    r = torch.randn(tokens, C, device=device, generator=gen).to(torch.bfloat16)
    b = torch.randn(tokens, C, device=device, generator=gen).to(torch.bfloat16)
    g = torch.randn(tokens, C, device=device, generator=gen)
    p = _params(dynamic, seed=50 + dynamic)
    pd = {k: v.to(device) for k, v in p.items()}
    w32 = pd["weight"].float()

    out, grads = _call(dynamic, r, b, g, w32, pd)
    torch.cuda.synchronize()
    print("[c5 full] full-size call done", flush=True)
    assert out.dtype == torch.float32 and tuple(out.shape) == (tokens, C)
    assert bool(torch.isfinite(out).all()), "non-finite wrapper output"
    for k, t in enumerate(grads):
        assert bool(torch.isfinite(t.float()).all()), f"non-finite gradient #{k}"
    dr, db = grads[0], grads[1]
    assert dr.dtype == torch.bfloat16 and db.dtype == torch.bfloat16

    # per-token results on a subsample spread over the whole batch (the first
    # and last tokens included: the persistent grids' edges)
    idx = torch.cat([torch.tensor([0, tokens - 1]),
                     torch.randperm(tokens, generator=torch.Generator().manual_seed(8))[:30]])
    idx_d = idx.to(device)
    rs, bs, gs = r[idx_d].cpu(), b[idx_d].cpu(), g[idx_d].cpu()
    names = DYN if dynamic else STA
    wr = p["weight"].double()
    ps = [p[k].double() for k in names]
    if dynamic:
        fn = lambda X: R.mhc_layer_dynamic(X, wr, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    else:
        fn = lambda X: R.mhc_layer_static(X, wr, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)
    rr = rs.double().requires_grad_(True)
    rb = bs.double().requires_grad_(True)
    ref = R.mhc_residual_wrapper(rr, rb, fn, N, "decay", storage_dtype=torch.bfloat16)
    ref.backward(gs.double())
    tag = f"C5 full {'dynamic' if dynamic else 'static'}"
    assert_close(out[idx_d], ref.detach(), 1e-4, grad_atol(ref.detach(), 1e-5), f"{tag} out subsample")
    assert_close_bf16(dr[idx_d], rr.grad, f"{tag} d residual subsample")
    assert_close_bf16(db[idx_d], rb.grad, f"{tag} d branch subsample")
    del rr, rb, ref

    # parameter gradients: additive over two halves of the tokens
    full = [t.clone() for t in grads[2:]]
    del out, grads, dr, db
    half = tokens // 2
    parts = []
    for sl in (slice(0, half), slice(half, tokens)):
        o, gr = _call(dynamic, r[sl], b[sl], g[sl], w32, pd)
        parts.append([t.clone() for t in gr[2:]])
        del o, gr
    torch.cuda.synchronize()
    print("[c5 full] half-size calls done", flush=True)
    pnames = ["d_weight"] + ["d_" + k for k in names]
    sums = [parts[0][k].double() + parts[1][k].double() for k in range(len(pnames))]
    # Through the stream mean every stream gets G / n, so the H_res-side
    # gradients vanish up to rounding; their floor comes from the
    # non-vanishing members of the same family (pre / post / res).
    fam = {}
    for nm, s in zip(pnames, sums):
        key = nm.rsplit("_", 1)[0]
        fam[key] = max(fam.get(key, 0.0), float(s.abs().max()))
    for k, nm in enumerate(pnames):
        s = sums[k]
        f = full[k].double()
        # fp32 sums over 131,072 tokens per half in a fixed order each
        floor = max(grad_atol(s, 1e-5), 1e-6 * fam[nm.rsplit("_", 1)[0]])
        assert_close(f, s, 1e-4, floor, f"{tag} additivity {nm}")

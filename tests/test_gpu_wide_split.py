"""The channel-loop forward's few-token forms (n >= 16) against the float64
oracle.  Below two workgroups per CU (2 x 256 tokens on MI355X) the output
pass runs over token x 256-channel chunks; the row sums then come from
token x chunk partials when the dynamic / forward-only entries' scratch (the
projection's K-split sum-of-squares region, ks x tokens floats) holds
tokens x chunks floats, i.e. when the K split ks is at least the chunk count,
and from one workgroup per token otherwise.  The cases take each form: at
n = 32, C = 1280 (5 chunks) the K split exceeds the chunks; at C = 4096
(16 chunks) and a few hundred tokens it does not; 513 and 520 tokens are
above the few-token threshold, 511 just below.  Per-token outputs are
checked on a token subsample (the forward is independent per token)."""
import pytest
import torch

import mhc_ascend_amd as mhc
from mhc_ascend_amd import native
from oracle import reference as R
from tests.conftest import assert_close, grad_atol

pytestmark = pytest.mark.gpu

PARAMS = ["weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post",
          "b_res"]


def _inputs(B, n, C, seed, x_dtype):
    # projection std scaled with the row length (0.05 at n * C = 40960), so
    # that alpha * P / r_h, the exponent of the Sinkhorn input, keeps the
    # same spread at every width (an unscaled 0.05 at 131072 channels gives
    # exp() a range of e^+-16 and an fp32-conditioned Sinkhorn)
    phi_std = 0.05 * (40960 / (n * C)) ** 0.5
    return R.dynamic_layer_inputs(B, n, C, seed=seed, x_dtype=x_dtype, alpha=0.3, phi_std=phi_std, b_std=0.5)


def _oracle_rows(d, idx):
    x = d["x"][idx].double()
    ps = [d[k].double() for k in PARAMS]
    return R.mhc_layer_dynamic(x, *ps, 20, 1e-8, 1e-5, dtype=torch.float64)


@pytest.mark.parametrize("n,C,B", [(16, 1280, 100), (16, 1280, 511), (16, 4096, 400), (16, 4096, 513),
                                   (32, 1280, 100), (32, 1280, 400), (32, 1280, 520), (32, 4096, 400)])
def test_wide_forward_token_forms(device, n, C, B):
    x_dtype = torch.bfloat16 if B % 2 == 0 else torch.float32
    d = _inputs(B, n, C, seed=n * 7 + C + B, x_dtype=x_dtype)
    dev = {k: v.to(device) for k, v in d.items()}
    ps = [dev[k] for k in PARAMS]
    print(f"[wide split] n={n} C={C} B={B} {x_dtype}", flush=True)
    out_train, _ = native.mhc_layer_dynamic_fwd(dev["x"], *ps)
    with torch.no_grad():
        out_infer = mhc.mhc_layer_fused_dynamic_inference(dev["x"], *ps)
        packed = native.mhc_layer_dynamic_pack(ps[0], ps[1], ps[2], ps[3])
        out_packed = mhc.mhc_layer_fused_dynamic_inference(dev["x"], *ps, packed=packed)
    torch.cuda.synchronize()
    idx = torch.cat([torch.tensor([0, B - 1]), torch.randperm(B, generator=torch.Generator().manual_seed(B))[:6]])
    ref = _oracle_rows(d, idx)
    # fp32 forward tolerance (rtol 1e-4, atol 1e-5); with n * C = 131072 the
    # projection is a 131072-term fp32 dot product whose rounding moves the
    # outputs by about 1e-6 of their largest magnitude, so there the absolute
    # floor is 2e-6 max|ref| (2.3e-5 at max|ref| = 11.6)
    atol = max(1e-5, grad_atol(ref, 2e-6))
    for tag, out in (("training forward", out_train), ("inference", out_infer), ("inference packed", out_packed)):
        assert out.dtype == torch.float32 and tuple(out.shape) == (B, n, C)
        assert_close(out.cpu()[idx], ref, 1e-4, atol, f"n={n} C={C} B={B} {tag}")


def test_wide_backward_few_tokens(device):
    """n = 16, 100 tokens: the chunked channel-loop backward (row sums per
    256-channel chunk into the workspace) and the all-tiles projection
    backward, every gradient against the float64 oracle."""
    B, n, C = 100, 16, 1280
    d = _inputs(B, n, C, seed=77, x_dtype=torch.float32)
    x = d["x"].to(device).requires_grad_(True)
    ps = [d[k].to(device).requires_grad_(True) for k in PARAMS]
    out = mhc.mhc_layer_fused_dynamic_training(x, *ps, 20, 1e-8, 1e-5)
    out.backward(d["grad"].to(device))
    xr = d["x"].double().requires_grad_(True)
    pr = [d[k].double().requires_grad_(True) for k in PARAMS]
    ref = R.mhc_layer_dynamic(xr, *pr, 20, 1e-8, 1e-5, dtype=torch.float64)
    ref.backward(d["grad"].double())
    assert_close(out, ref.detach(), 1e-4, 1e-5, "out")
    assert_close(x.grad, xr.grad, 1e-3, grad_atol(xr.grad, 1e-5), "dx")
    for nm, a, e in zip(PARAMS[1:], ps[1:], pr[1:]):
        assert_close(a.grad, e.grad, 1e-3, grad_atol(e.grad, 1e-4), f"d_{nm}")

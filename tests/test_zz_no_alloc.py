"""The allocation-free static backward (mhc_layer_static_bwd_noalloc, which
has no counterpart in the reference) against the workspace entry
mhc_layer_static_bwd: identical gradients, bit for bit, on two calls in a
row (the second smaller, over the scratch the first one left), and a clear
error for a shape whose workspace exceeds the library's scratch array."""
import pytest
import torch

from mhc_ascend_amd import _lib, native
from oracle import reference as R

pytestmark = pytest.mark.gpu


def _case(device, B, n, C, x_dtype, seed):
    d = R.static_layer_inputs(B, n, C, seed=seed, x_dtype=x_dtype)
    x = d["x"].to(device)
    w = d["weight"].to(device)
    hp, hq, hr = (d[k].to(device) for k in ("H_pre", "H_post", "H_res"))
    _, _, saved = native.mhc_layer_static_fwd(x, w, hp, hq, hr)
    return d["grad"].to(device), x, w, hp, hq, hr, saved


def test_static_bwd_noalloc_matches_workspace_entry(device):
    names = ("grad_x", "grad_weight", "grad_H_pre", "grad_H_post", "grad_H_res")
    # two calls in a row, the second smaller (the scratch keeps the first's contents)
    for B, n, C, xdt, seed in ((4096, 4, 4096, torch.float32, 1), (37, 4, 1024, torch.bfloat16, 2)):
        print(f"[noalloc] B={B} n={n} C={C} {xdt}", flush=True)
        args = _case(device, B, n, C, xdt, seed)
        want = native.mhc_layer_static_bwd(*args)
        got = native.mhc_layer_static_bwd_noalloc(*args)
        torch.cuda.synchronize()
        for nm, a, b in zip(names, got, want):
            assert a.dtype == b.dtype and a.shape == b.shape, nm
            assert torch.equal(a, b), f"B={B} C={C}: {nm} differs from the workspace entry"


def test_static_bwd_noalloc_rejects_shapes_beyond_the_scratch(device):
    lib = _lib.load()
    limit = lib.mhc_noalloc_scratch_bytes()
    assert limit == 16 << 20
    # n = 8, hidden = 10240 (a valid shape, about 21 MiB of workspace on
    # MI355X): rejected on the host before any pointer is used
    with torch.cuda.device(device):
        assert lib.mhc_layer_static_bwd_workspace_size(1 << 20, 8, 10240, 0) > limit
        rc = lib.mhc_layer_static_bwd_noalloc(None, None, 0, 1, None, None, None, None, None, None, None, None, None,
                                              1 << 20, 8, 10240, 20, 1e-8, 1e-5, None)
    assert rc == -2
    assert b"scratch" in lib.mhc_last_error()

"""The C-ABI entries under HIP graph capture.  Every kernel is enqueued on
the caller's stream, zeroing is done by fill kernels (no hipMemsetAsync
nodes) and scratch comes from caller workspaces, so a training or serving
step that calls the library can be captured once and replayed.  Each test
replays the graph several times on new inputs, with eager work and
synchronisations between replays, and checks every replay against the
eager result bit for bit."""
import pytest
import torch

from mhc_ascend_amd import native
from oracle import reference as R

pytestmark = pytest.mark.gpu

DYN = ["weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre", "b_post",
       "b_res"]


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    return graph, outs


def _replays(graph, outs, fn, feeds):
    for feed in feeds:
        feed()
        want = [t.clone() for t in fn()]  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, e in zip(outs, want):
            assert torch.equal(a, e)


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_static_layer_step_replays(device, x_dtype):
    d = R.static_layer_inputs(48, 4, 1024, seed=5, x_dtype=x_dtype)
    x = d["x"].to(device)
    g = d["grad"].to(device)
    w, hp, hq, hr = (d[k].to(device) for k in ("weight", "H_pre", "H_post", "H_res"))

    def step():
        out, rms, saved = native.mhc_layer_static_fwd(x, w, hp, hq, hr, 20, 1e-8, 1e-5)
        grads = native.mhc_layer_static_bwd(g, x, w, hp, hq, hr, saved, 20, 1e-8, 1e-5)
        return [out, rms, *grads]

    graph, outs = _capture(step)
    gen = torch.Generator().manual_seed(6)
    feeds = [lambda: x.copy_(torch.randn(x.shape, generator=gen).to(x_dtype)),
             lambda: g.copy_(torch.randn(g.shape, generator=gen)),
             lambda: hr.copy_(torch.randn(hr.shape, generator=gen))]
    _replays(graph, outs, step, feeds)


@pytest.mark.parametrize("n", [4, 8])
def test_dynamic_layer_step_replays(device, n):
    d = R.dynamic_layer_inputs(40, n, 256, seed=n, x_dtype=torch.bfloat16, alpha=0.3, phi_std=0.05, b_std=0.5)
    x = d["x"].to(device)
    g = d["grad"].to(device)
    ps = [d[k].to(device) for k in DYN]

    def step():
        out, saved = native.mhc_layer_dynamic_fwd(x, *ps, 20, 1e-8, 1e-5)
        grads = native.mhc_layer_dynamic_bwd(g, x, ps[0], saved, *ps[1:], 20, 1e-8, 1e-5)
        return [out, *grads]

    graph, outs = _capture(step)
    gen = torch.Generator().manual_seed(7)
    feeds = [lambda: x.copy_(torch.randn(x.shape, generator=gen).to(torch.bfloat16)),
             lambda: g.copy_(torch.randn(g.shape, generator=gen)),
             lambda: ps[3].copy_(0.05 * torch.randn(ps[3].shape, generator=gen))]
    _replays(graph, outs, step, feeds)


def test_forward_only_entry_replays(device):
    """A serving step: parameters packed outside the graph, the forward-only
    entry (bf16 output) captured."""
    d = R.dynamic_layer_inputs(64, 4, 512, seed=9, x_dtype=torch.bfloat16, alpha=0.3, phi_std=0.05, b_std=0.5)
    x = d["x"].to(device)
    ps = [d[k].to(device) for k in DYN]
    packed = native.mhc_layer_dynamic_pack(*ps[:4])

    def step():
        return [native.mhc_layer_dynamic_infer(x, packed, *ps[4:], 20, 1e-8, 1e-5, out_dtype=torch.bfloat16)]

    graph, outs = _capture(step)
    gen = torch.Generator().manual_seed(10)
    feeds = [lambda: x.copy_(torch.randn(x.shape, generator=gen).to(torch.bfloat16)) for _ in range(3)]
    _replays(graph, outs, step, feeds)

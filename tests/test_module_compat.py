"""Module-level compatibility with the reference's nn.Modules (CPU only).

A model written against src/python/mhc/layer.py must load into this package
unchanged: the same parameter names, shapes and dtypes (layer.py:64-85),
the same random draws under a fixed seed (so seeded runs initialise alike),
the same factories (layer.py:186-218, 332-353) and the wrapper's fixed
settings (layer.py:248-270).  Nothing here launches a kernel.
"""
import pytest
import torch

import mhc_ascend_amd as mhc
from mhc_ascend_amd.layer import MHCLayer, MHCResidualWrapper, create_mhc_layer, replace_residual_with_mhc

# (name, shape, dtype) of every parameter the reference registers, in its
# registration order (layer.py:65, 69-79 dynamic; 65, 82-85 static).
def _reference_params(n, C, dynamic):
    nC = n * C
    rows = [("rmsnorm_weight", (C,), torch.bfloat16)]
    if dynamic:
        rows += [("phi_pre", (n, nC), torch.float32), ("phi_post", (n, nC), torch.float32),
                 ("phi_res", (n * n, nC), torch.float32), ("b_pre", (n,), torch.float32),
                 ("b_post", (n,), torch.float32), ("b_res", (n, n), torch.float32),
                 ("alpha_pre", (), torch.float32), ("alpha_post", (), torch.float32),
                 ("alpha_res", (), torch.float32)]
    else:
        rows += [("H_pre", (n,), torch.float32), ("H_post", (n,), torch.float32),
                 ("H_res", (n, n), torch.float32)]
    return rows


@pytest.mark.parametrize("dynamic", [True, False])
@pytest.mark.parametrize("n,C", [(4, 64), (2, 40), (8, 24)])
def test_state_dict_layout_matches_reference(dynamic, n, C):
    layer = MHCLayer(C, n, use_dynamic_h=dynamic)
    sd = layer.state_dict()
    want = _reference_params(n, C, dynamic)
    assert list(sd.keys()) == [name for name, _, _ in want]
    for name, shape, dtype in want:
        assert tuple(sd[name].shape) == shape, name
        assert sd[name].dtype == dtype, name
    assert [p for p, _ in layer.named_parameters()] == [name for name, _, _ in want]
    assert not list(layer.buffers())


@pytest.mark.parametrize("dynamic", [True, False])
def test_seeded_initialisation_draws_like_the_reference(dynamic):
    """Under one seed the reference draws randn(n, nC), randn(n, nC),
    randn(n*n, nC) for the projections (layer.py:69-71), or randn(n, n) for
    H_res (layer.py:84), and nothing else; ones/zeros/tensor() draw nothing."""
    n, C, a = 4, 48, 0.03
    torch.manual_seed(1234)
    layer = MHCLayer(C, n, use_dynamic_h=dynamic, alpha_init=a)
    after_layer = torch.rand(3)
    torch.manual_seed(1234)
    if dynamic:
        phi_pre = torch.randn(n, n * C) * 0.02
        phi_post = torch.randn(n, n * C) * 0.02
        phi_res = torch.randn(n * n, n * C) * 0.02
        assert torch.equal(layer.phi_pre.data, phi_pre)
        assert torch.equal(layer.phi_post.data, phi_post)
        assert torch.equal(layer.phi_res.data, phi_res)
        assert torch.equal(layer.b_pre.data, torch.zeros(n))
        assert torch.equal(layer.b_post.data, torch.zeros(n))
        assert torch.equal(layer.b_res.data, torch.zeros(n, n))
        for p in (layer.alpha_pre, layer.alpha_post, layer.alpha_res):
            assert p.dim() == 0 and p.item() == pytest.approx(a)
    else:
        h_res = a * torch.randn(n, n)
        assert torch.equal(layer.H_res.data, h_res)
        assert torch.equal(layer.H_pre.data, torch.zeros(n))
        assert torch.equal(layer.H_post.data, torch.zeros(n))
    # the generator advanced exactly as far as the reference's constructor
    assert torch.equal(torch.rand(3), after_layer)
    assert torch.equal(layer.rmsnorm_weight.data, torch.ones(C, dtype=torch.bfloat16))


@pytest.mark.parametrize("dynamic", [True, False])
def test_reference_state_dict_loads_strictly(dynamic):
    """A state_dict written by the reference module (its names, shapes and
    dtypes, arbitrary values) loads with strict=True and round-trips."""
    n, C = 4, 32
    g = torch.Generator().manual_seed(7)
    ref_sd = {name: (torch.randn(shape, generator=g) if shape else torch.randn((), generator=g)).to(dtype)
              for name, shape, dtype in _reference_params(n, C, dynamic)}
    layer = MHCLayer(C, n, use_dynamic_h=dynamic)
    missing, unexpected = layer.load_state_dict(ref_sd, strict=True)
    assert not missing and not unexpected
    for name, t in layer.state_dict().items():
        assert torch.equal(t, ref_sd[name]), name
        assert t.dtype == ref_sd[name].dtype, name


def test_wrapper_state_dict_nests_the_layer_as_mhc():
    """The wrapper keeps its layer under the attribute `mhc` (layer.py:264),
    so checkpoint keys are 'mhc.<param>'."""
    w = MHCResidualWrapper(40, 4, use_dynamic_h=False)
    assert list(w.state_dict().keys()) == ["mhc." + name for name, _, _ in _reference_params(4, 40, False)]
    w = MHCResidualWrapper(40, 4)
    assert list(w.state_dict().keys()) == ["mhc." + name for name, _, _ in _reference_params(4, 40, True)]


def test_create_mhc_layer_forwards_every_setting():
    layer = create_mhc_layer(96, expansion_rate=2, num_sinkhorn_iters=7, sinkhorn_eps=1e-6, rmsnorm_eps=1e-4,
                             use_dynamic_h=False, alpha_init=0.5)
    assert isinstance(layer, MHCLayer)
    assert (layer.hidden_dim, layer.expansion_rate, layer.num_sinkhorn_iters) == (96, 2, 7)
    assert (layer.sinkhorn_eps, layer.rmsnorm_eps, layer.use_dynamic_h) == (1e-6, 1e-4, False)
    assert tuple(layer.H_res.shape) == (2, 2)
    d = create_mhc_layer(32)
    assert d.use_dynamic_h and d.expansion_rate == 4 and d.num_sinkhorn_iters == 20
    assert d.sinkhorn_eps == 1e-8 and d.rmsnorm_eps == 1e-5
    assert d.alpha_pre.item() == pytest.approx(0.01)


def test_replace_residual_with_mhc_forwards_layer_kwargs():
    w = replace_residual_with_mhc(64, expansion_rate=4, residual_mode="zero", num_sinkhorn_iters=5,
                                  use_dynamic_h=False)
    assert isinstance(w, MHCResidualWrapper)
    assert (w.hidden_dim, w.expansion_rate, w.residual_mode) == (64, 4, "zero")
    assert w.mhc.num_sinkhorn_iters == 5 and not w.mhc.use_dynamic_h
    # use_post_norm is accepted and forced off (layer.py:261)
    assert replace_residual_with_mhc(64, use_post_norm=True).use_post_norm is False
    assert "residual_mode=decay" in repr(replace_residual_with_mhc(64))


def test_wrapper_rejects_unknown_mode_before_any_launch():
    """The reference raises ValueError for an unknown residual_mode
    (layer.py:309-310); here it is raised before the inputs are touched, so
    it shows on CPU tensors too."""
    w = MHCResidualWrapper(16, 4, residual_mode="mirror")
    with pytest.raises(ValueError, match="Unknown residual_mode"):
        w(torch.zeros(2, 16), torch.zeros(2, 16))


def test_package_exports_reference_names():
    """The names of mhc/__init__.py:22-39, plus the two layer functions that
    the reference exposes from mhc.ops (ops.py:337, 567)."""
    for name in ("MHCLayer", "MHCResidualWrapper", "create_mhc_layer", "replace_residual_with_mhc",
                 "sinkhorn_knopp", "rmsnorm", "stream_aggregate", "stream_distribute_mix_add",
                 "mhc_layer_fused_dynamic_inference", "mhc_layer_fused_dynamic_training"):
        assert hasattr(mhc, name), name

"""The benchmark build's VALU projection (mhc_timing_proj_valu, the A/B the
benchmark reports against the MFMA projection) computes the same product as
fused_rmsnorm_matmul_fwd (bindings.cpp:480-528): both against a float64
matmul, at the output counts of n = 2 and n = 4 and a full 32-row tile, with
bf16 and fp32 inputs and a batch that is not a multiple of the 256-token
workgroup."""
import pytest
import torch

from mhc_ascend_amd import _lib, native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("out_dim", [8, 24, 32])
def test_valu_projection_matches_mfma_and_fp64(device, dtype, out_dim):
    g = torch.Generator().manual_seed(out_dim)
    B, K = 300, 1024
    x = torch.randn(B, K, generator=g).to(dtype).to(device)
    w = (0.02 * torch.randn(out_dim, K, generator=g)).to(device)
    ref = x.double() @ w.double().t()
    scale = ref.abs().max().item()
    mfma = native.fused_rmsnorm_matmul_fwd(x, w)
    with _lib.timed_build() as lib:
        wsb = lib.mhc_timing_proj_valu_workspace_size(B, K, out_dim)
        ws = torch.empty(wsb, dtype=torch.uint8, device=device)
        valu = torch.empty(B, out_dim, device=device)
        _lib.call("mhc_timing_proj_valu", x.data_ptr(), _lib.dtype_code(dtype), w.data_ptr(), valu.data_ptr(),
                  ws.data_ptr(), wsb, B, K, out_dim, _lib.stream_of(x))
        torch.cuda.synchronize()
    # fp32 accumulation over K = 1024 terms: a few ulp of the largest output
    for name, got in (("valu", valu), ("mfma", mfma)):
        err = (got.double() - ref).abs().max().item() / scale
        assert err < 2e-5, f"{name}: max error {err:.3e} of max |P|"
    assert (valu.double() - mfma.double()).abs().max().item() / scale < 4e-5

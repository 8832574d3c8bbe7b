"""Autograd functions over the HIP kernels (mirror of src/python/mhc/ops.py).

Public functional ops keep the reference's names, arguments and defaults.
Documented differences from the Ascend implementation (all toward the
PyTorch reference math, which is the contract):
  * arithmetic is fp32 end to end; the Ascend path rounds several
    intermediates to bf16 (ops.py:144-147, 257, 282);
  * standalone ops return the dtype of their input instead of bf16;
  * the Sinkhorn backward is the exact gradient (the Ascend kernel's row
    step is approximate, sinkhorn_knopp.cpp:1773-1795);
  * alpha parameters stay on the device (no ``.item()`` host syncs,
    ops.py:459-461, 572-574).
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import native


# =============================================================================
# Sinkhorn-Knopp (ops.py:71-119)
# =============================================================================

class SinkhornKnoppFunction(torch.autograd.Function):
    """Sinkhorn-Knopp doubly stochastic normalisation of [B, n, n]."""

    @staticmethod
    def forward(ctx, inp: torch.Tensor, num_iters: int = 20, eps: float = 1e-8) -> torch.Tensor:
        out = native.sinkhorn_knopp_fwd(inp, num_iters, eps)
        ctx.save_for_backward(inp, out)
        ctx.num_iters = num_iters
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        inp, out = ctx.saved_tensors
        grad_inp = native.sinkhorn_knopp_bwd(grad_out.float().contiguous(), inp, out, ctx.num_iters, ctx.eps)
        return grad_inp, None, None


def sinkhorn_knopp(inp: torch.Tensor, num_iters: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """Apply Sinkhorn-Knopp normalisation to a batch of matrices [B, n, n]."""
    return SinkhornKnoppFunction.apply(inp.float(), num_iters, eps)


# =============================================================================
# Fused static-H layer (layer.py:142-170 as one HBM pass per direction)
# =============================================================================

class MHCLayerStaticFunction(torch.autograd.Function):
    """Static-H mHC layer: aggregate -> RMSNorm -> distribute-mix-add with
    shared H (one Sinkhorn per call instead of one per token)."""

    @staticmethod
    def forward(ctx, x, rmsnorm_weight, H_pre, H_post, H_res, num_iters: int, sinkhorn_eps: float,
                rmsnorm_eps: float):
        out, _rms, saved = native.mhc_layer_static_fwd(x, rmsnorm_weight, H_pre, H_post, H_res, num_iters,
                                                       sinkhorn_eps, rmsnorm_eps)
        ctx.save_for_backward(x, rmsnorm_weight, H_pre, H_post, H_res, saved)
        ctx.cfg = (num_iters, sinkhorn_eps, rmsnorm_eps)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, w, hp, hq, hr, saved = ctx.saved_tensors
        gx, gw, ghp, ghq, ghr = native.mhc_layer_static_bwd(grad_out, x, w, hp, hq, hr, saved, *ctx.cfg)
        return gx.to(x.dtype), gw, ghp.view_as(hp), ghq.view_as(hq), ghr.view_as(hr), None, None, None


def mhc_layer_static(x: torch.Tensor, rmsnorm_weight: torch.Tensor, H_pre: torch.Tensor, H_post: torch.Tensor,
                     H_res: torch.Tensor, sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                     rmsnorm_eps: float = 1e-5) -> torch.Tensor:
    """Static-H mHC layer on x [B, n, C] -> fp32 [B, n, C]."""
    return MHCLayerStaticFunction.apply(x, rmsnorm_weight, H_pre, H_post, H_res, sinkhorn_iters, sinkhorn_eps,
                                        rmsnorm_eps)

"""Autograd functions over the HIP kernels (mirror of src/python/mhc/ops.py).

Public functional ops keep the reference's names, arguments and defaults.
Documented differences from the Ascend implementation (all toward the
PyTorch reference math, which is the contract):
  * arithmetic is fp32 end to end; the Ascend path rounds several
    intermediates to bf16 (ops.py:105-107, 218, 243, 280-281);
  * standalone ops return the dtype of their input instead of bf16;
  * the Sinkhorn backward is the exact gradient (the Ascend kernel's row
    step is approximate, sinkhorn_knopp.cpp:1773-1795);
  * alpha parameters stay on the device (no ``.item()`` host syncs,
    ops.py:362-364, 420-422, 533-535).
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib, native

# Projection rows above which the library's dynamic forward streams the fp32
# projections (2n + n^2 > 128: n >= 16) instead of split planes.
_STREAM_PROJ_ROWS = 128


# =============================================================================
# Sinkhorn-Knopp (ops.py:32-80)
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
# RMSNorm (ops.py:87-136)
# =============================================================================

class RMSNormFunction(torch.autograd.Function):
    """Root Mean Square normalisation of [B, C] rows."""

    @staticmethod
    def forward(ctx, inp: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
        out, rms = native.rmsnorm_fwd(inp, weight, eps)
        ctx.save_for_backward(inp, weight, rms)
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        inp, weight, rms = ctx.saved_tensors
        grad_inp, grad_weight = native.rmsnorm_bwd(grad_out, inp, weight, rms)
        return grad_inp.to(inp.dtype), grad_weight, None


def rmsnorm(inp: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """RMSNorm of inp [B, C]; the output keeps inp's dtype (fp32 or bf16)."""
    return RMSNormFunction.apply(inp, weight, eps)


# =============================================================================
# Stream aggregate (ops.py:143-188)
# =============================================================================

class StreamAggregateFunction(torch.autograd.Function):
    """out = sum_i sigmoid(H_pre_raw[:, i]) * inp[:, i]."""

    @staticmethod
    def forward(ctx, inp: torch.Tensor, H_pre_raw: torch.Tensor) -> torch.Tensor:
        out, h_act = native.stream_aggregate_fwd(inp, H_pre_raw)
        ctx.save_for_backward(inp, h_act)
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        inp, h_act = ctx.saved_tensors
        gx, _, graw = native._aggregate_bwd(grad_out, inp, h_act, True)
        return gx.to(inp.dtype), graw


def stream_aggregate(inp: torch.Tensor, H_pre_raw: torch.Tensor) -> torch.Tensor:
    """Aggregate [B, n, C] streams with sigmoid weights H_pre_raw [B, n]."""
    return StreamAggregateFunction.apply(inp, H_pre_raw)


# =============================================================================
# Stream distribute-mix-add (ops.py:195-265)
# =============================================================================

class StreamDistributeMixAddFunction(torch.autograd.Function):
    """out[:, i] = 2 sigmoid(H_post_raw[:, i]) * y_norm + sum_j M[:, i, j] x[:, j]."""

    @staticmethod
    def forward(ctx, y_norm, H_post_raw, M, x_inp):
        out, h_act = native.stream_distribute_mix_add_fwd(y_norm, H_post_raw, M, x_inp)
        ctx.save_for_backward(x_inp, y_norm, M, h_act)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x_inp, y_norm, M, h_act = ctx.saved_tensors
        gx, gy, gM, _, graw = native._distribute_bwd(grad_out, x_inp, y_norm, M, h_act, True)
        return gy.to(y_norm.dtype), graw, gM, gx.to(x_inp.dtype)


def stream_distribute_mix_add(y_norm: torch.Tensor, H_post_raw: torch.Tensor, M: torch.Tensor,
                              x_inp: torch.Tensor) -> torch.Tensor:
    """Distribute y_norm [B, C] to n streams, mix x_inp [B, n, C] with M and add (fp32 out)."""
    return StreamDistributeMixAddFunction.apply(y_norm, H_post_raw, M, x_inp)


stream_distribute = stream_distribute_mix_add


def compute_rms(x_flat: torch.Tensor, eps: float = 1e-8) -> torch.Tensor:
    """Per-row RMS of x_flat [B, K] (ops.py:318-330); no autograd, as in the reference."""
    return native.compute_rms_fwd(x_flat, eps)


# =============================================================================
# Fused static-H layer (layer.py:142-170 as one HBM pass per direction)
# =============================================================================

def mhc_layer_static(x: torch.Tensor, rmsnorm_weight: torch.Tensor, H_pre: torch.Tensor, H_post: torch.Tensor,
                     H_res: torch.Tensor, sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                     rmsnorm_eps: float = 1e-5) -> torch.Tensor:
    """Static-H mHC layer on x [B, n, C] -> fp32 [B, n, C]: one fused pass per
    direction (layer.py:142-170), autograd node in C++ (_mhc_autograd.so)."""
    return _lib.autograd().static_layer(x, rmsnorm_weight, H_pre, H_post, H_res, int(sinkhorn_iters),
                                        float(sinkhorn_eps), float(rmsnorm_eps))


# =============================================================================
# Dynamic-H projection (ops.py:272-315)
# =============================================================================

class FusedProjectionFunction(torch.autograd.Function):
    """P = x_flat @ phi_concat^T (fp32), with its backward."""

    @staticmethod
    def forward(ctx, x_flat: torch.Tensor, phi_concat: torch.Tensor) -> torch.Tensor:
        out = native.fused_rmsnorm_matmul_fwd(x_flat, phi_concat)
        ctx.save_for_backward(x_flat, phi_concat)
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        x_flat, phi_concat = ctx.saved_tensors
        gx, gphi = native.fused_rmsnorm_matmul_bwd(grad_out, x_flat, phi_concat)
        return gx.to(x_flat.dtype), gphi.to(phi_concat.dtype)


def fused_rmsnorm_matmul(x_flat: torch.Tensor, phi_concat: torch.Tensor) -> torch.Tensor:
    """Project x_flat [B, K] with phi_concat [out_dim, K] -> fp32 [B, out_dim]."""
    return FusedProjectionFunction.apply(x_flat, phi_concat)


# =============================================================================
# Dynamic-H layer (ops.py:337-628)
# =============================================================================

def mhc_layer_fused_dynamic_inference(x_expanded, rmsnorm_weight, phi_pre, phi_post, phi_res, alpha_pre,
                                      alpha_post, alpha_res, b_pre, b_post, b_res, sinkhorn_iters: int = 20,
                                      sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5,
                                      out_dtype: torch.dtype = torch.float32, packed=None) -> torch.Tensor:
    """Dynamic-H forward without autograd state (ops.py:337-380).

    Extensions (keyword-only in practice, defaults give the reference's
    result): ``out_dtype=torch.bfloat16`` writes the output in bf16;
    ``packed`` (from native.mhc_layer_dynamic_pack on the same weight and
    projections) skips the per-call packing of the parameters."""
    if packed is None:
        if out_dtype == torch.float32 and 2 * phi_pre.shape[0] + phi_res.shape[0] > _STREAM_PROJ_ROWS:
            # More than 128 projection rows: the forward reads the fp32
            # projections directly (no packing pass), and its fp32 output is
            # the packed entry's bit for bit.
            return native.mhc_layer_dynamic_fwd(x_expanded, rmsnorm_weight, phi_pre, phi_post, phi_res, alpha_pre,
                                                alpha_post, alpha_res, b_pre, b_post, b_res, sinkhorn_iters,
                                                sinkhorn_eps, rmsnorm_eps)[0]
        packed = native.mhc_layer_dynamic_pack(rmsnorm_weight, phi_pre, phi_post, phi_res)
    return native.mhc_layer_dynamic_infer(x_expanded, packed, alpha_pre, alpha_post, alpha_res, b_pre, b_post, b_res,
                                          sinkhorn_iters, sinkhorn_eps, rmsnorm_eps, out_dtype)


def mhc_layer_fused_dynamic_training(x_expanded, rmsnorm_weight, phi_pre, phi_post, phi_res, alpha_pre, alpha_post,
                                     alpha_res, b_pre, b_post, b_res, sinkhorn_iters: int = 20,
                                     sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5) -> torch.Tensor:
    """Dynamic-H layer with autograd (ops.py:567-628).  Float alphas become
    device tensors; alpha tensors stay on the device (no .item() syncs)."""
    dev = phi_pre.device
    if not torch.is_tensor(alpha_pre):
        alpha_pre = torch.tensor(alpha_pre, device=dev, dtype=torch.float32)
    if not torch.is_tensor(alpha_post):
        alpha_post = torch.tensor(alpha_post, device=dev, dtype=torch.float32)
    if not torch.is_tensor(alpha_res):
        alpha_res = torch.tensor(alpha_res, device=dev, dtype=torch.float32)
    return _lib.autograd().dynamic_layer(x_expanded, rmsnorm_weight, phi_pre, phi_post, phi_res, alpha_pre,
                                         alpha_post, alpha_res, b_pre, b_post, b_res, int(sinkhorn_iters),
                                         float(sinkhorn_eps), float(rmsnorm_eps))


# =============================================================================
# Fused MHCResidualWrapper (layer.py:269-322)
# =============================================================================

def mhc_residual_wrapper(residual: torch.Tensor, branch_output: torch.Tensor, layer, residual_mode: str = "decay"):
    """Fused MHCResidualWrapper on residual / branch_output [tokens, C] for the
    parameters of ``layer`` (an MHCLayer); returns fp32 [tokens, C]."""
    n = layer.expansion_rate
    C = residual.shape[-1]
    # The fused wrapper kernels take 4-channel rows and n = 2..32; with
    # dynamic H also n*C a multiple of the projection's k step of 32, up to
    # 2^22, and past n = 10 (2n + n^2 > 128 projection rows) Sinkhorn
    # settings under which the H_res gradients vanish (at least one
    # iteration, eps <= 1e-6: the defaults).  Other shapes build the n
    # streams with device tensor ops, as layer.py:299-310 does, and run the
    # layer on them (layer.py:313-316).
    fused = 2 <= n <= 32 and C % 4 == 0
    if layer.use_dynamic_h:
        # the library's test, in float32: iters >= 1 and 0 <= eps <= 1e-6f
        eps32 = float(torch.tensor(float(layer.sinkhorn_eps), dtype=torch.float32))
        vanish = int(layer.num_sinkhorn_iters) >= 1 and 0.0 <= eps32 <= float(torch.tensor(1e-6, dtype=torch.float32))
        fused = fused and (n * C) % 32 == 0 and n * C <= 1 << 22 and (n <= 10 or vanish)
    if not fused:
        if n < 2:
            raise RuntimeError("mhc_residual_wrapper: expansion_rate must be >= 2 (stream 1 holds the branch)")
        if residual_mode not in ("zero", "decay"):
            raise ValueError(f"Unknown residual_mode: {residual_mode}")
        X = torch.zeros(residual.shape[0], n, C, device=residual.device, dtype=residual.dtype)
        X[:, 0] = residual
        X[:, 1] = branch_output
        if residual_mode == "decay":
            for i in range(2, n):
                X[:, i] = residual * (0.1 ** (i - 1))
        return layer(X).mean(dim=1)
    iters, sk_eps, rms_eps = int(layer.num_sinkhorn_iters), float(layer.sinkhorn_eps), float(layer.rmsnorm_eps)
    ag = _lib.autograd()
    if layer.use_dynamic_h:
        return ag.dynamic_wrapper(residual, branch_output, layer.rmsnorm_weight, layer.phi_pre, layer.phi_post,
                                  layer.phi_res, layer.alpha_pre, layer.alpha_post, layer.alpha_res, layer.b_pre,
                                  layer.b_post, layer.b_res, residual_mode, n, iters, sk_eps, rms_eps)
    return ag.static_wrapper(residual, branch_output, layer.rmsnorm_weight, layer.H_pre, layer.H_post, layer.H_res,
                             residual_mode, n, iters, sk_eps, rms_eps)

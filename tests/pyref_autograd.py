"""Test-only reference orchestration of the fused layers: torch.autograd
Functions in Python over the same native entry points as the product's C++
autograd nodes (mhc_ascend_amd/csrc/autograd.cpp), in the structure of the
reference's autograd function (ops.py:387-564).  tests/test_gpu_autograd_cpp.py
checks that the two orchestrations give identical results bit for bit; the
package itself runs only the C++ nodes."""
import torch

from mhc_ascend_amd import native


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



class MHCLayerDynamicFunction(torch.autograd.Function):
    """Fused dynamic-H layer: projection -> per-token H -> aggregate ->
    RMSNorm -> distribute-mix-add, and its backward (ops.py:387-564)."""

    @staticmethod
    def forward(ctx, x_expanded, rmsnorm_weight, phi_pre, phi_post, phi_res, alpha_pre, alpha_post, alpha_res, b_pre,
                b_post, b_res, sinkhorn_iters: int, sinkhorn_eps: float, rmsnorm_eps: float):
        out, saved = native.mhc_layer_dynamic_fwd(x_expanded, rmsnorm_weight, phi_pre, phi_post, phi_res, alpha_pre,
                                                  alpha_post, alpha_res, b_pre, b_post, b_res, sinkhorn_iters,
                                                  sinkhorn_eps, rmsnorm_eps)
        ctx.save_for_backward(x_expanded, rmsnorm_weight, saved, phi_pre, phi_post, phi_res, alpha_pre, alpha_post,
                              alpha_res, b_pre, b_post, b_res)
        ctx.cfg = (sinkhorn_iters, sinkhorn_eps, rmsnorm_eps)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        (x, w, saved, phi_pre, phi_post, phi_res, a_pre, a_post, a_res, b_pre, b_post, b_res) = ctx.saved_tensors
        grads = native.mhc_layer_dynamic_bwd(grad_output, x, w, saved, phi_pre, phi_post, phi_res, a_pre, a_post,
                                             a_res, b_pre, b_post, b_res, *ctx.cfg)
        gx, gw, gpp, gpq, gpr, gap, gaq, gar, gbp, gbq, gbr = grads
        return (gx.to(x.dtype), gw, gpp.view_as(phi_pre), gpq.view_as(phi_post), gpr.view_as(phi_res),
                gap.view_as(a_pre), gaq.view_as(a_post), gar.view_as(a_res), gbp.view_as(b_pre),
                gbq.view_as(b_post), gbr.view_as(b_res), None, None, None)



class MHCWrapperDynamicFunction(torch.autograd.Function):
    """Stream synthesis -> dynamic-H layer -> stream mean, fused: the
    [tokens, n, C] stream tensor and the layer output are never materialised."""

    @staticmethod
    def forward(ctx, residual, branch, rmsnorm_weight, phi_pre, phi_post, phi_res, alpha_pre, alpha_post, alpha_res,
                b_pre, b_post, b_res, residual_mode: str, n: int, sinkhorn_iters: int, sinkhorn_eps: float,
                rmsnorm_eps: float):
        out, saved = native.wrapper_dynamic_fwd(residual, branch, residual_mode, n, rmsnorm_weight, phi_pre, phi_post,
                                                phi_res, alpha_pre, alpha_post, alpha_res, b_pre, b_post, b_res,
                                                sinkhorn_iters, sinkhorn_eps, rmsnorm_eps)
        ctx.save_for_backward(residual, branch, rmsnorm_weight, saved, phi_pre, phi_post, phi_res, alpha_pre,
                              alpha_post, alpha_res, b_pre, b_post, b_res)
        ctx.cfg = (residual_mode, n, sinkhorn_iters, sinkhorn_eps, rmsnorm_eps)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        r, b, w, saved, pp, pq, pr, ap, aq, ar, bp, bq, br = ctx.saved_tensors
        mode, n, iters, sk_eps, rms_eps = ctx.cfg
        gr, gb, gw, gpp, gpq, gpr, gap, gaq, gar, gbp, gbq, gbr = native.wrapper_dynamic_bwd(
            grad_out, r, b, mode, n, w, saved, pp, pq, pr, ap, aq, ar, br, iters, sk_eps, rms_eps)
        return (gr.to(r.dtype), gb.to(b.dtype), gw, gpp.view_as(pp), gpq.view_as(pq), gpr.view_as(pr),
                gap.view_as(ap), gaq.view_as(aq), gar.view_as(ar), gbp.view_as(bp), gbq.view_as(bq),
                gbr.view_as(br), None, None, None, None, None)


class MHCWrapperStaticFunction(torch.autograd.Function):
    """Stream synthesis -> static-H layer -> stream mean, fused."""

    @staticmethod
    def forward(ctx, residual, branch, rmsnorm_weight, H_pre, H_post, H_res, residual_mode: str, n: int,
                sinkhorn_iters: int, sinkhorn_eps: float, rmsnorm_eps: float):
        out, saved = native.wrapper_static_fwd(residual, branch, residual_mode, n, rmsnorm_weight, H_pre, H_post,
                                               H_res, sinkhorn_iters, sinkhorn_eps, rmsnorm_eps)
        ctx.save_for_backward(residual, branch, rmsnorm_weight, H_pre, H_post, H_res, saved)
        ctx.cfg = (residual_mode, n, sinkhorn_iters, sinkhorn_eps, rmsnorm_eps)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        r, b, w, hp, hq, hr, saved = ctx.saved_tensors
        mode, n, iters, sk_eps, rms_eps = ctx.cfg
        gr, gb, gw, ghp, ghq, ghr = native.wrapper_static_bwd(grad_out, r, b, mode, n, w, hp, hq, hr, saved, iters,
                                                              sk_eps, rms_eps)
        return (gr.to(r.dtype), gb.to(b.dtype), gw, ghp.view_as(hp), ghq.view_as(hq), ghr.view_as(hr), None, None,
                None, None, None)



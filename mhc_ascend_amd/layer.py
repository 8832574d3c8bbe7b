"""nn.Modules of the mHC layer (mirror of src/python/mhc/layer.py).

Parameter names, shapes, dtypes and initialisation are the reference's, so
state_dicts interchange (layer.py:64-85): ``rmsnorm_weight`` is bf16, the
dynamic-H projections are [out, n*C] fp32 ~ N(0, 0.02), biases zero, alphas
``alpha_init``; static H_pre/H_post are zero and H_res = alpha_init * N(0,1).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops


class MHCLayer(nn.Module):
    """Manifold-Constrained Hyper-Connections layer on x [B, n, C] (layer.py:24-179).

    Args mirror the reference: hidden_dim (C), expansion_rate (n),
    num_sinkhorn_iters, sinkhorn_eps, rmsnorm_eps, use_dynamic_h, alpha_init.
    The output is fp32 [B, n, C] for fp32 or bf16 input (layer.py:101).
    """

    def __init__(
        self,
        hidden_dim: int,
        expansion_rate: int = 4,
        num_sinkhorn_iters: int = 20,
        sinkhorn_eps: float = 1e-8,
        rmsnorm_eps: float = 1e-5,
        use_dynamic_h: bool = True,
        alpha_init: float = 0.01,
    ):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.expansion_rate = expansion_rate
        self.num_sinkhorn_iters = num_sinkhorn_iters
        self.sinkhorn_eps = sinkhorn_eps
        self.rmsnorm_eps = rmsnorm_eps
        self.use_dynamic_h = use_dynamic_h

        n = expansion_rate
        C = hidden_dim
        nC = n * C
        self.rmsnorm_weight = nn.Parameter(torch.ones(hidden_dim, dtype=torch.bfloat16))
        if use_dynamic_h:
            self.phi_pre = nn.Parameter(torch.randn(n, nC) * 0.02)
            self.phi_post = nn.Parameter(torch.randn(n, nC) * 0.02)
            self.phi_res = nn.Parameter(torch.randn(n * n, nC) * 0.02)
            self.b_pre = nn.Parameter(torch.zeros(n))
            self.b_post = nn.Parameter(torch.zeros(n))
            self.b_res = nn.Parameter(torch.zeros(n, n))
            self.alpha_pre = nn.Parameter(torch.tensor(alpha_init))
            self.alpha_post = nn.Parameter(torch.tensor(alpha_init))
            self.alpha_res = nn.Parameter(torch.tensor(alpha_init))
        else:
            self.H_pre = nn.Parameter(torch.zeros(n, dtype=torch.float32))
            self.H_post = nn.Parameter(torch.zeros(n, dtype=torch.float32))
            self.H_res = nn.Parameter((alpha_init * torch.randn(n, n)).float())
        self._inference_pack = None  # (parameter versions, packed tensor)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, n, C = x.shape
        assert n == self.expansion_rate, f"Expected expansion_rate={self.expansion_rate}, got {n}"
        assert C == self.hidden_dim, f"Expected hidden_dim={self.hidden_dim}, got {C}"
        if x.dtype not in (torch.float32, torch.bfloat16):
            x = x.float()
        if self.use_dynamic_h:
            if (not self.training) and (not torch.is_grad_enabled()):
                return ops.mhc_layer_fused_dynamic_inference(
                    x, self.rmsnorm_weight, self.phi_pre, self.phi_post, self.phi_res,
                    self.alpha_pre, self.alpha_post, self.alpha_res, self.b_pre, self.b_post, self.b_res,
                    self.num_sinkhorn_iters, self.sinkhorn_eps, self.rmsnorm_eps, packed=self._packed())
            return ops.mhc_layer_fused_dynamic_training(
                x, self.rmsnorm_weight, self.phi_pre, self.phi_post, self.phi_res,
                self.alpha_pre, self.alpha_post, self.alpha_res, self.b_pre, self.b_post, self.b_res,
                self.num_sinkhorn_iters, self.sinkhorn_eps, self.rmsnorm_eps)
        return ops.mhc_layer_static(x, self.rmsnorm_weight, self.H_pre, self.H_post, self.H_res,
                                    self.num_sinkhorn_iters, self.sinkhorn_eps, self.rmsnorm_eps)

    # ---- forward-only dynamic H ------------------------------------------
    def _pack_key(self):
        return tuple((p.data_ptr(), p._version)
                     for p in (self.rmsnorm_weight, self.phi_pre, self.phi_post, self.phi_res))

    def prepare_inference(self) -> None:
        """Pack the weight and projections once for eval-mode, no-grad
        forwards (dynamic H only), instead of on every call.  The snapshot is
        dropped when a parameter is updated in place (optimizer steps,
        load_state_dict), moved, or the layer is put back into training mode;
        writes through ``.data`` bypass that check, so call this again after
        them."""
        if not self.use_dynamic_h:
            return
        with torch.no_grad():
            packed = ops.native.mhc_layer_dynamic_pack(self.rmsnorm_weight, self.phi_pre, self.phi_post,
                                                       self.phi_res)
        self._inference_pack = (self._pack_key(), packed)

    def _packed(self):
        if self._inference_pack is not None and self._inference_pack[0] == self._pack_key():
            return self._inference_pack[1]
        self._inference_pack = None
        return None

    def train(self, mode: bool = True):
        if mode:
            self._inference_pack = None
        return super().train(mode)

    def extra_repr(self) -> str:
        return (
            f"hidden_dim={self.hidden_dim}, "
            f"expansion_rate={self.expansion_rate}, "
            f"num_sinkhorn_iters={self.num_sinkhorn_iters}, "
            f"use_dynamic_h={self.use_dynamic_h}"
        )


def create_mhc_layer(
    hidden_dim: int,
    expansion_rate: int = 4,
    num_sinkhorn_iters: int = 20,
    sinkhorn_eps: float = 1e-8,
    rmsnorm_eps: float = 1e-5,
    use_dynamic_h: bool = True,
    alpha_init: float = 0.01,
) -> MHCLayer:
    """Factory for :class:`MHCLayer` (layer.py:186-218)."""
    return MHCLayer(hidden_dim=hidden_dim, expansion_rate=expansion_rate, num_sinkhorn_iters=num_sinkhorn_iters,
                    sinkhorn_eps=sinkhorn_eps, rmsnorm_eps=rmsnorm_eps, use_dynamic_h=use_dynamic_h,
                    alpha_init=alpha_init)


class MHCResidualWrapper(nn.Module):
    """Drop-in replacement for ``residual + branch_output`` (layer.py:225-329).

    Streams are synthesised as [residual, branch, residual*0.1**(i-1) ...]
    ('decay') or zeros ('zero'), run through an :class:`MHCLayer` and
    averaged over streams; [B, T, C] inputs come back as [B, T, C] when
    T > 1 and as [B*T, C] otherwise (layer.py:319-320).  ``use_post_norm``
    is accepted and ignored, as in the reference (layer.py:261).

    For hidden % 4 == 0 and n = 2..32 it runs fused
    (ops.mhc_residual_wrapper; with dynamic H past n = 10 at Sinkhorn
    settings under which the H_res gradients vanish, the defaults): the
    layer's [B*T, n, C] output is never materialised, and the stream tensor
    of layer.py:299-310 only where the dynamic projection needs it (n != 4
    with fp32 storage, fewer than 1024 tokens or hidden % 64 != 0, Sinkhorn
    settings that keep the H_res gradients, and the backward past n = 16 or
    past n = 8 on rows narrower than 2048 channels).
    Other shapes build the streams with tensor ops and run the layer.
    """

    def __init__(self, hidden_dim: int, expansion_rate: int = 4, residual_mode: str = 'decay',
                 use_post_norm: bool = True, **mhc_kwargs):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.expansion_rate = expansion_rate
        self.residual_mode = residual_mode
        self.use_post_norm = False
        self.mhc = MHCLayer(hidden_dim=hidden_dim, expansion_rate=expansion_rate, **mhc_kwargs)

    def forward(self, residual: torch.Tensor, branch_output: torch.Tensor) -> torch.Tensor:
        original_shape = residual.shape
        if len(original_shape) == 3:
            B, T, C = original_shape
            residual = residual.reshape(B * T, C)
            branch_output = branch_output.reshape(B * T, C)
        else:
            B, C = original_shape
            T = 1
        if self.residual_mode not in ("zero", "decay"):
            raise ValueError(f"Unknown residual_mode: {self.residual_mode}")
        output = ops.mhc_residual_wrapper(residual, branch_output, self.mhc, self.residual_mode)
        if T > 1:
            output = output.reshape(B, T, C)
        return output

    def extra_repr(self) -> str:
        return (f'hidden_dim={self.hidden_dim}, expansion_rate={self.expansion_rate}, '
                f'residual_mode={self.residual_mode}')


def replace_residual_with_mhc(hidden_dim: int, expansion_rate: int = 4, **kwargs) -> MHCResidualWrapper:
    """Factory for :class:`MHCResidualWrapper` (layer.py:332-353)."""
    return MHCResidualWrapper(hidden_dim=hidden_dim, expansion_rate=expansion_rate, **kwargs)

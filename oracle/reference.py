"""CPU oracle for the mHC hyper-connection layer (test infrastructure only).

This module restates, in plain PyTorch on the CPU, the math of the
reference's mHC path so that the HIP kernels of ``mhc_ascend_amd`` can be
checked against it.  It is *not* part of the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it, and only as the checker or the timed CPU baseline.  The
product path never calls it and raises when its HIP library is missing.

Every function works in any floating dtype; tests run it in float64 on
the same (fp32 / bf16) inputs the GPU sees, so the oracle is the exact
math and the kernel's fp32 rounding is what the tolerance covers.  All
functions are differentiable through autograd; the backward passes of
the reference (hand-written in bindings.cpp:600-874 and the Ascend
kernels) are checked against autograd of these forwards.

Reference files are cited as ``path:line`` relative to the reference
repository root (ParadoxZW/mHC_Ascend).

Parity pins (each is exercised in tests/test_oracle.py):
  * sinkhorn_knopp        - row/col sums -> 1, constant matrix -> 1/n,
                            permutation equivariance, diagonal-scaling
                            invariance, brute-force C restatement
                            (oracle/sinkhorn.c), gradcheck.
  * sinkhorn_knopp_bwd    - float64 autograd of the forward, the explicit
                            adjoint in oracle/sinkhorn.c, gradcheck,
                            column-constant cotangent -> 0.
  * rmsnorm / compute_rms - torch.nn.functional.rms_norm, constant-row
                            closed form, gradcheck.
  * stream_aggregate      - einsum restatement, gradcheck.
  * stream_distribute_mix_add - bmm restatement, gradcheck.
  * projection            - float64 matmul, gradcheck.
  * mhc_layer_static / mhc_layer_dynamic / mhc_residual_wrapper -
                            composition of the above, gradcheck at tiny
                            shapes, closed forms (identity mixing, n=1).
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

__all__ = [
    "sinkhorn_knopp",
    "sinkhorn_knopp_bwd",
    "rmsnorm",
    "compute_rms",
    "stream_aggregate",
    "stream_distribute_mix_add",
    "projection",
    "dynamic_h_coefficients",
    "mhc_layer_static",
    "mhc_layer_dynamic",
    "build_wrapper_streams",
    "mhc_residual_wrapper",
    "static_layer_inputs",
    "dynamic_layer_inputs",
    "wrapper_inputs",
]


# ---------------------------------------------------------------------------
# Standalone operators
# ---------------------------------------------------------------------------

def sinkhorn_knopp(inp: torch.Tensor, num_iters: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """Sinkhorn-Knopp normalisation of a batch of square matrices.

    Follows ops_pytorch_backward.py:9-33: ``num_iters`` times, divide each
    row by (row sum + eps), then each column by (column sum + eps).  The
    ``+eps`` form is the contract (the Ascend kernel's ``sum > eps`` guard,
    sinkhorn_knopp.cpp:183-188, differs by <= eps).

    inp: [..., n, n] non-negative.  Returns the same shape.
    """
    a = inp
    for _ in range(num_iters):
        a = a / (a.sum(dim=-1, keepdim=True) + eps)
        a = a / (a.sum(dim=-2, keepdim=True) + eps)
    return a


def sinkhorn_knopp_bwd(grad_out: torch.Tensor, inp: torch.Tensor, num_iters: int = 20,
                       eps: float = 1e-8) -> torch.Tensor:
    """Exact vector-Jacobian product of :func:`sinkhorn_knopp`.

    The reference's backward entry is bindings.cpp:189-231 (kernel
    sinkhorn_knopp.cpp:1608-1814).  Its row step uses an approximation
    (sRow = dot * rowInv against the post-normalised matrix,
    sinkhorn_knopp.cpp:1773-1795); the contract here is the exact gradient,
    i.e. autograd of the forward above, which this function returns.
    """
    x = inp.detach().clone().requires_grad_(True)
    with torch.enable_grad():
        y = sinkhorn_knopp(x, num_iters, eps)
        (g,) = torch.autograd.grad(y, x, grad_out)
    return g


def compute_rms(x: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """Per-row RMS ``sqrt(mean(x^2) + eps)`` (ops_pytorch_backward.py:65-75;
    kernel compute_rms.cpp:124, bound at bindings.cpp:543-566)."""
    return torch.sqrt((x * x).mean(dim=-1) + eps)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm ``y = x / rms * w`` (ops_pytorch_backward.py:78-91; kernel
    rmsnorm.cpp:170-178).  Returns ``(y, rms)`` as rmsnorm_fwd does
    (bindings.cpp:237-266)."""
    rms = compute_rms(x, eps)
    y = (x / rms.unsqueeze(-1)) * weight.to(x.dtype).unsqueeze(0)
    return y, rms


def stream_aggregate(x: torch.Tensor, h_pre_raw: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``out = sum_i sigmoid(H_pre[:, i]) * x[:, i]`` (ops_pytorch_backward.py:94-111;
    kernel stream_ops.cpp:151-208).  Returns ``(out, H_pre_activated)``."""
    h = torch.sigmoid(h_pre_raw.to(x.dtype))
    out = (h.unsqueeze(-1) * x).sum(dim=1)
    return out, h


def stream_distribute_mix_add(y_norm: torch.Tensor, h_post_raw: torch.Tensor, m: torch.Tensor,
                              x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``out[:, i] = 2*sigmoid(H_post[:, i]) * y + sum_j M[:, i, j] * x[:, j]``
    (ops_pytorch_backward.py:36-62; kernel stream_ops.cpp:403-525).
    Returns ``(out, H_post_activated)``."""
    dt = x.dtype
    h = 2.0 * torch.sigmoid(h_post_raw.to(dt))
    mix = torch.bmm(m.to(dt), x)
    out = h.unsqueeze(-1) * y_norm.to(dt).unsqueeze(1) + mix
    return out, h


def projection(x_flat: torch.Tensor, phi: torch.Tensor) -> torch.Tensor:
    """Dynamic-H projection ``P = x_flat @ phi^T`` (bindings.cpp:480-528,
    ops.py:272-315).  phi is [out_dim, K] (layer.py:69-71 layout)."""
    return x_flat @ phi.to(x_flat.dtype).t()


# ---------------------------------------------------------------------------
# The mHC layer
# ---------------------------------------------------------------------------

def _layer_core(x: torch.Tensor, weight: torch.Tensor, h_pre: torch.Tensor, h_post: torch.Tensor,
                m: torch.Tensor, rms_eps: float) -> torch.Tensor:
    """Aggregate -> RMSNorm -> distribute-mix-add on activated coefficients.

    x [B, n, C]; h_pre, h_post [B, n] or [n]; m [B, n, n] or [n, n].
    Composition of layer.py:148-168 (static) / bindings.cpp:931-940 (dynamic).
    """
    B, n, C = x.shape
    if h_pre.dim() == 1:
        h_pre = h_pre.unsqueeze(0).expand(B, n)
    if h_post.dim() == 1:
        h_post = h_post.unsqueeze(0).expand(B, n)
    if m.dim() == 2:
        m = m.unsqueeze(0).expand(B, n, n)
    x_agg = (h_pre.unsqueeze(-1) * x).sum(dim=1)
    y, _ = rmsnorm(x_agg, weight, rms_eps)
    mix = torch.einsum("bij,bjc->bic", m, x)
    return mix + h_post.unsqueeze(-1) * y.unsqueeze(1)


def mhc_layer_static(x: torch.Tensor, weight: torch.Tensor, H_pre: torch.Tensor, H_post: torch.Tensor,
                     H_res: torch.Tensor, num_iters: int = 20, sinkhorn_eps: float = 1e-8,
                     rmsnorm_eps: float = 1e-5, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Static-H mHC layer (layer.py:142-170; benchmark.py:66-78).

    h_pre = sigmoid(H_pre), h_post = 2*sigmoid(H_post), M = SK(exp(H_res)).
    The reference expands the shared H to [B, ...] and runs B identical
    Sinkhorns (layer.py:144-160); one shared Sinkhorn is the same function
    (benchmark.py:69-71).  The layer casts x to fp32 first (layer.py:101);
    ``dtype`` selects the arithmetic type of this restatement.
    """
    dt = dtype or torch.float32
    x = x.to(dt)
    h_pre = torch.sigmoid(H_pre.to(dt))
    h_post = 2.0 * torch.sigmoid(H_post.to(dt))
    m = sinkhorn_knopp(torch.exp(H_res.to(dt)), num_iters, sinkhorn_eps)
    return _layer_core(x, weight.to(dt), h_pre, h_post, m, rmsnorm_eps)


def dynamic_h_coefficients(x: torch.Tensor, phi_pre: torch.Tensor, phi_post: torch.Tensor,
                           phi_res: torch.Tensor, alpha_pre, alpha_post, alpha_res,
                           b_pre: torch.Tensor, b_post: torch.Tensor, b_res: torch.Tensor,
                           num_iters: int, sinkhorn_eps: float, rmsnorm_eps: float
                           ) -> Dict[str, torch.Tensor]:
    """Per-token H of the dynamic layer (bindings.cpp:899-929).

    x_flat = x.reshape(B, n*C); r_h = sqrt(mean(x_flat^2) + rmsnorm_eps)
    (the main path uses rmsnorm_eps, bindings.cpp:909); P = x_flat @ phi^T
    with phi = [phi_pre; phi_post; phi_res] (ops.py:416-418);
    t_k = alpha_k * P_k / r_h + b_k; t_res reshaped row-major to n x n;
    h_pre = sigmoid, h_post = 2*sigmoid, M = SK(exp(t_res)).
    """
    B, n, C = x.shape
    dt = x.dtype
    x_flat = x.reshape(B, n * C)
    r_h = compute_rms(x_flat, rmsnorm_eps)
    phi = torch.cat([phi_pre.to(dt), phi_post.to(dt), phi_res.to(dt).reshape(n * n, n * C)], dim=0)
    p = projection(x_flat, phi)
    inv = (1.0 / r_h).unsqueeze(-1)
    a_pre = alpha_pre.to(dt) if torch.is_tensor(alpha_pre) else alpha_pre
    a_post = alpha_post.to(dt) if torch.is_tensor(alpha_post) else alpha_post
    a_res = alpha_res.to(dt) if torch.is_tensor(alpha_res) else alpha_res
    t_pre = a_pre * p[:, :n] * inv + b_pre.to(dt)
    t_post = a_post * p[:, n:2 * n] * inv + b_post.to(dt)
    t_res = (a_res * p[:, 2 * n:] * inv + b_res.to(dt).reshape(-1)).reshape(B, n, n)
    h_pre = torch.sigmoid(t_pre)
    h_post = 2.0 * torch.sigmoid(t_post)
    m = sinkhorn_knopp(torch.exp(t_res), num_iters, sinkhorn_eps)
    return {"x_flat": x_flat, "r_h": r_h, "p": p, "t_pre": t_pre, "t_post": t_post,
            "t_res": t_res, "h_pre": h_pre, "h_post": h_post, "M": m}


def mhc_layer_dynamic(x: torch.Tensor, weight: torch.Tensor, phi_pre: torch.Tensor,
                      phi_post: torch.Tensor, phi_res: torch.Tensor, alpha_pre, alpha_post, alpha_res,
                      b_pre: torch.Tensor, b_post: torch.Tensor, b_res: torch.Tensor,
                      num_iters: int = 20, sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5,
                      dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Dynamic-H mHC layer (bindings.cpp:880-952; ops.py:387-628; layer.py:104-141).

    The reference rounds x_flat, phi and P to bf16 around its projection
    (bindings.cpp:906, 913, 526-527); the contract is the exact math, so
    this restatement keeps everything in ``dtype``.
    """
    dt = dtype or torch.float32
    x = x.to(dt)
    co = dynamic_h_coefficients(x, phi_pre, phi_post, phi_res, alpha_pre, alpha_post, alpha_res,
                                b_pre, b_post, b_res, num_iters, sinkhorn_eps, rmsnorm_eps)
    return _layer_core(x, weight.to(dt), co["h_pre"], co["h_post"], co["M"], rmsnorm_eps)


def build_wrapper_streams(residual: torch.Tensor, branch: torch.Tensor, n: int,
                          mode: str = "decay") -> torch.Tensor:
    """Stream synthesis of MHCResidualWrapper (layer.py:287-310).

    Returns X [BT, n, C] in the dtype of ``residual``: X[:,0] = residual,
    X[:,1] = branch, X[:,i>=2] = residual * 0.1**(i-1) ('decay', computed
    in the storage dtype as the reference's slice assignment does) or 0.
    """
    C = residual.shape[-1]
    res = residual.reshape(-1, C)
    br = branch.reshape(-1, C)
    X = torch.zeros(res.shape[0], n, C, dtype=residual.dtype)
    X[:, 0] = res
    if n > 1:
        X[:, 1] = br
    if mode == "decay":
        for i in range(2, n):
            X[:, i] = res * (0.1 ** (i - 1))
    elif mode != "zero":
        raise ValueError(f"Unknown residual_mode: {mode}")
    return X


class _StoredDecay(torch.autograd.Function):
    """res * c stored in ``storage`` (value of the reference's tensor op,
    layer.py:307-308), with the gradient of the product: g * c.  Infinite
    values stay infinite (a straight-through sum s + (value - s) would turn
    them into NaN)."""

    @staticmethod
    def forward(ctx, res, c, storage):
        ctx.c = c
        return (res.detach().float() * torch.tensor(c, dtype=torch.float32)).to(storage).to(res.dtype)

    @staticmethod
    def backward(ctx, g):
        return g * ctx.c, None, None


def mhc_residual_wrapper(residual: torch.Tensor, branch: torch.Tensor, layer_fn, n: int,
                         mode: str = "decay", storage_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """MHCResidualWrapper.forward (layer.py:269-322): synthesise n streams,
    run the layer, average over streams, reshape to [B, T, C] only if T > 1.

    ``layer_fn`` maps X [BT, n, C] -> [BT, n, C]; the synthesis is done with
    differentiable ops so autograd reaches residual and branch.

    ``storage_dtype`` (e.g. bf16) with exact leaves (float64 tensors holding
    storage_dtype values): the 'decay' streams take the value the
    reference's tensor op gives in that dtype, storage_dtype(float32(r) *
    float32(0.1**(i-1))) (layer.py:307-308), while the gradient flows
    through the product with the same float32 constant, as autograd of that
    op does; the leaves' gradients are then not rounded to storage_dtype.
    """
    shape = residual.shape
    C = shape[-1]
    if residual.dim() == 3:
        B, T = shape[0], shape[1]
    else:
        B, T = shape[0], 1
    res = residual.reshape(B * T, C)
    br = branch.reshape(B * T, C)
    streams = [res, br]
    for i in range(2, n):
        if mode != "decay":
            streams.append(torch.zeros_like(res))
        elif storage_dtype is None:
            streams.append(res * (0.1 ** (i - 1)))
        else:
            c = torch.tensor(0.1 ** (i - 1), dtype=torch.float32).item()
            streams.append(_StoredDecay.apply(res, c, storage_dtype))
    X = torch.stack(streams[:n], dim=1)
    out = layer_fn(X).mean(dim=1)
    if T > 1:
        out = out.reshape(B, T, C)
    return out


# ---------------------------------------------------------------------------
# Seeded synthetic inputs of the benchmark configurations
# ---------------------------------------------------------------------------

def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def static_layer_inputs(B: int, n: int, C: int, seed: int = 0, x_dtype=torch.float32,
                        weight_ones: bool = False) -> Dict[str, torch.Tensor]:
    """Config C3 inputs: x ~ N(0,1) [B,n,C]; H_pre, H_post ~ N(0,1) [n];
    H_res ~ N(0,1) [n,n]; w bf16 (layer.py:65) = ones in the config, or
    1 + 0.1 N(0,1) so that tests see the weight; cotangent g ~ N(0,1)
    [B,n,C] materialised."""
    g = _gen(seed)
    d = {
        "x": torch.randn(B, n, C, generator=g).to(x_dtype),
        "H_pre": torch.randn(n, generator=g),
        "H_post": torch.randn(n, generator=g),
        "H_res": torch.randn(n, n, generator=g),
        "weight": (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16),
        "grad": torch.randn(B, n, C, generator=g),
    }
    if weight_ones:
        d["weight"] = torch.ones(C, dtype=torch.bfloat16)
    return d


def dynamic_layer_inputs(B: int, n: int, C: int, seed: int = 0, x_dtype=torch.bfloat16,
                         alpha: float = 0.01, phi_std: float = 0.02,
                         b_std: float = 0.0) -> Dict[str, torch.Tensor]:
    """Config C4 inputs: x ~ N(0,1) stored as ``x_dtype``; phi ~ N(0, phi_std)
    drawn as [nC, 2n+n^2] and split/transposed to the [out, nC] layout of
    layer.py:69-71; alpha = 0.01; b = b_std * N(0,1) (0 in the config)."""
    g = _gen(seed)
    nC = n * C
    x = torch.randn(B, n, C, generator=g).to(x_dtype)
    phi = phi_std * torch.randn(nC, 2 * n + n * n, generator=g)
    d = {
        "x": x,
        "phi_pre": phi[:, :n].t().contiguous(),
        "phi_post": phi[:, n:2 * n].t().contiguous(),
        "phi_res": phi[:, 2 * n:].t().contiguous(),
        "alpha_pre": torch.tensor(alpha),
        "alpha_post": torch.tensor(alpha),
        "alpha_res": torch.tensor(alpha),
        "b_pre": b_std * torch.randn(n, generator=g),
        "b_post": b_std * torch.randn(n, generator=g),
        "b_res": b_std * torch.randn(n, n, generator=g),
        "weight": (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16),
        "grad": torch.randn(B, n, C, generator=g),
    }
    return d


def wrapper_inputs(B: int, T: int, C: int, n: int = 4, seed: int = 0, dtype=torch.bfloat16,
                   alpha: float = 0.01, phi_std: float = 0.02, b_std: float = 0.0) -> Dict[str, torch.Tensor]:
    """Config C5 inputs: residual, branch ~ N(0,1) [B,T,C] in ``dtype``;
    phi as in :func:`dynamic_layer_inputs`; cotangent g ~ N(0,1) fp32 of the
    wrapper output shape."""
    g = _gen(seed)
    nC = n * C
    shape = (B, T, C) if T > 1 else (B, C)
    res = torch.randn(*shape, generator=g).to(dtype)
    br = torch.randn(*shape, generator=g).to(dtype)
    phi = phi_std * torch.randn(nC, 2 * n + n * n, generator=g)
    return {
        "residual": res,
        "branch": br,
        "phi_pre": phi[:, :n].t().contiguous(),
        "phi_post": phi[:, n:2 * n].t().contiguous(),
        "phi_res": phi[:, 2 * n:].t().contiguous(),
        "alpha_pre": torch.tensor(alpha),
        "alpha_post": torch.tensor(alpha),
        "alpha_res": torch.tensor(alpha),
        "b_pre": b_std * torch.randn(n, generator=g),
        "b_post": b_std * torch.randn(n, generator=g),
        "b_res": b_std * torch.randn(n, n, generator=g),
        "weight": (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16),
        "grad": torch.randn(*shape, generator=g),
    }

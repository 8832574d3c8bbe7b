"""Tensor-level host side of the C ABI: the functions of the reference's
native module ``mhc_ascend`` (bindings.cpp:1020-1117) with the same names,
argument order and return tuples, plus the fused-layer entry points.

Each function checks devices, shapes and dtypes the way the reference's
TORCH_CHECKs do (RuntimeError), allocates its outputs with torch's caching
allocator on the input's device, and enqueues the HIP kernels on torch's
current stream.  Nothing synchronises.  There is no CPU path: CPU tensors
raise.
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib
from ._lib import call, dtype_code, ptr, stream_of


def _check_device(fn: str, *tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{fn}: tensors must be on a HIP device (got {t.device}); "
                               "mhc_ascend_amd has no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{fn}: all tensors must be on the same device ({dev} vs {t.device})")
    return dev


def _f32c(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float32).contiguous()


# =============================================================================
# Sinkhorn-Knopp (bindings.cpp:155-231)
# =============================================================================

def sinkhorn_knopp_fwd(inp: torch.Tensor, num_iters: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """out = SK(inp) on [B, n, n] fp32 (bindings.cpp:155-187)."""
    _check_device("sinkhorn_knopp_fwd", inp)
    if inp.dim() != 3:
        raise RuntimeError("Input must be 3D tensor [B, M, N]")
    if inp.size(1) != inp.size(2):
        raise RuntimeError(f"Sinkhorn-Knopp requires square matrices (M == N), got M={inp.size(1)}, N={inp.size(2)}")
    if inp.dtype != torch.float32:
        raise RuntimeError("inp must be float32")
    inp = inp.contiguous()
    out = torch.empty_like(inp)
    with _lib.on_device(inp.device):
        call("mhc_sinkhorn_knopp_fwd", ptr(inp), ptr(out), inp.size(0), inp.size(1), int(num_iters), float(eps),
             stream_of(inp))
    return out


def sinkhorn_knopp_bwd(grad_out: torch.Tensor, inp: torch.Tensor, out: torch.Tensor, num_iters: int = 20,
                       eps: float = 1e-8) -> torch.Tensor:
    """Exact VJP of SK at inp (bindings.cpp:189-231)."""
    _check_device("sinkhorn_knopp_bwd", grad_out, inp, out)
    for name, t in (("grad_out", grad_out), ("inp", inp), ("out", out)):
        if t.dtype != torch.float32:
            raise RuntimeError(f"{name} must be float32")
    if grad_out.shape != inp.shape:
        raise RuntimeError("grad_out shape must match inp")
    if out.shape != inp.shape:
        raise RuntimeError("out shape must match inp")
    if inp.dim() != 3 or inp.size(1) != inp.size(2):
        raise RuntimeError(f"Sinkhorn-Knopp requires square matrices (M == N), got shape {tuple(inp.shape)}")
    grad_out = grad_out.contiguous()
    inp = inp.contiguous()
    grad_inp = torch.empty_like(inp)
    with _lib.on_device(inp.device):
        call("mhc_sinkhorn_knopp_bwd", ptr(grad_out), ptr(inp), 0, ptr(grad_inp), inp.size(0), inp.size(1),
             int(num_iters), float(eps), stream_of(inp))
    return grad_inp


# =============================================================================
# RMSNorm (bindings.cpp:237-301) and compute_rms (bindings.cpp:543-566)
# =============================================================================

def _storage(t: torch.Tensor) -> torch.Tensor:
    """Large-tensor storage: fp32 or bf16, contiguous (others become fp32)."""
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.float()
    return t.contiguous()


def _coef_view(fn: str, t: torch.Tensor, B: int, per: int):
    """A per-token coefficient tensor [B, *] as (fp32 tensor, batch stride):
    a tensor broadcast over the batch (stride 0, e.g. expand()) is passed
    once with stride 0; anything else is made contiguous."""
    if t.dtype != torch.float32:
        t = t.float()
    if t.dim() >= 2 and t.size(0) == B and t.stride(0) == 0:
        one = t[0].contiguous()
        if one.numel() != per:
            raise RuntimeError(f"{fn}: coefficient shape {tuple(t.shape)} does not match n")
        return one, 0
    t = t.contiguous()
    if t.numel() != B * per:
        raise RuntimeError(f"{fn}: coefficient shape {tuple(t.shape)} does not match [B={B}, {per}]")
    return t, per


def rmsnorm_fwd(inp: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """(out, rms) for inp [B, C] (bindings.cpp:237-266).  out keeps inp's dtype."""
    _check_device("rmsnorm_fwd", inp, weight)
    if inp.dim() != 2:
        raise RuntimeError("Input must be 2D tensor [B, C]")
    x = _storage(inp)
    B, C = x.shape
    if weight.numel() != C:
        raise RuntimeError("weight must have C elements")
    w = _f32c(weight)
    out = torch.empty_like(x)
    rms = torch.empty((B,), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        call("mhc_rmsnorm_fwd", ptr(x), dtype_code(x.dtype), ptr(w), ptr(out), ptr(rms), B, C, float(eps),
             stream_of(x))
    return out, rms


def rmsnorm_bwd(grad_out: torch.Tensor, inp: torch.Tensor, weight: torch.Tensor,
                rms: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(grad_inp [inp dtype], grad_weight fp32 [C]) (bindings.cpp:268-301)."""
    _check_device("rmsnorm_bwd", grad_out, inp, weight, rms)
    x = _storage(inp)
    B, C = x.shape
    g = grad_out.to(x.dtype).contiguous()
    if g.shape != x.shape:
        raise RuntimeError("grad_out shape must match inp")
    w, r = _f32c(weight), _f32c(rms)
    gx = torch.empty_like(x)
    gw = torch.empty((C,), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        ws_bytes = _lib.load().mhc_rmsnorm_bwd_workspace_size(B, C, dtype_code(x.dtype))
        ws = torch.empty((max(int(ws_bytes), 1),), dtype=torch.uint8, device=x.device)
        call("mhc_rmsnorm_bwd", ptr(g), ptr(x), dtype_code(x.dtype), ptr(w), ptr(r), ptr(gx), ptr(gw), ptr(ws),
             int(ws_bytes), B, C, stream_of(x))
    return gx, gw


def compute_rms_fwd(inp: torch.Tensor, eps: float = 1e-8) -> torch.Tensor:
    """rms [B] of inp [B, K] (bindings.cpp:543-566)."""
    _check_device("compute_rms_fwd", inp)
    if inp.dim() != 2:
        raise RuntimeError("Input must be 2D tensor [B, K]")
    x = _storage(inp)
    B, K = x.shape
    rms = torch.empty((B,), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        call("mhc_compute_rms_fwd", ptr(x), dtype_code(x.dtype), ptr(rms), B, K, float(eps), stream_of(x))
    return rms


# =============================================================================
# Stream aggregate (bindings.cpp:307-374) and distribute-mix-add (380-460)
# =============================================================================

def stream_aggregate_fwd(inp: torch.Tensor, H_pre_raw: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(out [B, C] in inp's dtype, H_pre_activated [B, n]) (bindings.cpp:307-338)."""
    _check_device("stream_aggregate_fwd", inp, H_pre_raw)
    if inp.dim() != 3:
        raise RuntimeError("Input must be 3D tensor [B, n, C]")
    x = _storage(inp)
    B, n, C = x.shape
    h, hs = _coef_view("stream_aggregate_fwd", H_pre_raw, B, n)
    out = torch.empty((B, C), dtype=x.dtype, device=x.device)
    h_act = torch.empty((B, n), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        call("mhc_stream_aggregate_fwd", ptr(x), dtype_code(x.dtype), ptr(h), hs, ptr(out), ptr(h_act), B, n, C,
             stream_of(x))
    return out, h_act


def _aggregate_bwd(grad_out, inp, H_pre_activated, want_raw: bool):
    _check_device("stream_aggregate_bwd", grad_out, inp, H_pre_activated)
    x = _storage(inp)
    B, n, C = x.shape
    g = grad_out.to(x.dtype).contiguous()
    if g.shape != (B, C):
        raise RuntimeError("grad_out must be [B, C]")
    h, hs = _coef_view("stream_aggregate_bwd", H_pre_activated, B, n)
    gx = torch.empty_like(x)
    gh = torch.empty((B, n), dtype=torch.float32, device=x.device)
    graw = torch.empty((B, n), dtype=torch.float32, device=x.device) if want_raw else None
    with _lib.on_device(x.device):
        call("mhc_stream_aggregate_bwd", ptr(g), ptr(x), dtype_code(x.dtype), ptr(h), hs, ptr(gx), ptr(gh),
             ptr(graw), B, n, C, stream_of(x))
    return gx, gh, graw


def stream_aggregate_bwd(grad_out: torch.Tensor, inp: torch.Tensor,
                         H_pre_activated: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(grad_inp, grad_H_pre_activated) before the sigmoid derivative (bindings.cpp:340-374)."""
    gx, gh, _ = _aggregate_bwd(grad_out, inp, H_pre_activated, False)
    return gx, gh


def stream_distribute_mix_add_fwd(y_norm: torch.Tensor, H_post_raw: torch.Tensor, M: torch.Tensor,
                                  x_inp: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(out fp32 [B, n, C], H_post_activated [B, n]) (bindings.cpp:380-416)."""
    _check_device("stream_distribute_mix_add_fwd", y_norm, H_post_raw, M, x_inp)
    if x_inp.dim() != 3:
        raise RuntimeError("x_inp must be 3D tensor [B, n, C]")
    x = _storage(x_inp)
    B, n, C = x.shape
    y = y_norm.to(x.dtype).contiguous()
    if y.shape != (B, C):
        raise RuntimeError("y_norm must be [B, C]")
    h, hs = _coef_view("stream_distribute_mix_add_fwd", H_post_raw, B, n)
    m, ms = _coef_view("stream_distribute_mix_add_fwd", M, B, n * n)
    out = torch.empty((B, n, C), dtype=torch.float32, device=x.device)
    h_act = torch.empty((B, n), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        call("mhc_stream_distribute_mix_add_fwd", ptr(y), ptr(h), hs, ptr(m), ms, ptr(x), dtype_code(x.dtype),
             ptr(out), ptr(h_act), B, n, C, stream_of(x))
    return out, h_act


def _distribute_bwd(grad_out, x_inp, y_norm, M, H_post_activated, want_raw: bool):
    _check_device("stream_distribute_mix_add_bwd", grad_out, x_inp, y_norm, M, H_post_activated)
    x = _storage(x_inp)
    B, n, C = x.shape
    y = y_norm.to(x.dtype).contiguous()
    g = _f32c(grad_out)
    if g.shape != x.shape:
        raise RuntimeError("grad_out shape must match x_inp")
    m, ms = _coef_view("stream_distribute_mix_add_bwd", M, B, n * n)
    h, hs = _coef_view("stream_distribute_mix_add_bwd", H_post_activated, B, n)
    gx = torch.empty_like(x)
    gy = torch.empty((B, C), dtype=x.dtype, device=x.device)
    gM = torch.empty((B, n, n), dtype=torch.float32, device=x.device)
    gh = torch.empty((B, n), dtype=torch.float32, device=x.device)
    graw = torch.empty((B, n), dtype=torch.float32, device=x.device) if want_raw else None
    with _lib.on_device(x.device):
        call("mhc_stream_distribute_mix_add_bwd", ptr(g), ptr(x), ptr(y), dtype_code(x.dtype), ptr(m), ms, ptr(h),
             hs, ptr(gx), ptr(gy), ptr(gM), ptr(gh), ptr(graw), B, n, C, stream_of(x))
    return gx, gy, gM, gh, graw


def stream_distribute_mix_add_bwd(grad_out: torch.Tensor, x_inp: torch.Tensor, y_norm: torch.Tensor,
                                  M: torch.Tensor, H_post_activated: torch.Tensor):
    """(grad_x, grad_y, grad_M, grad_H_post_activated) (bindings.cpp:418-460)."""
    gx, gy, gM, gh, _ = _distribute_bwd(grad_out, x_inp, y_norm, M, H_post_activated, False)
    return gx, gy, gM, gh


# =============================================================================
# Fused static-H layer (layer.py:142-170)
# =============================================================================

def _layer_x(fn: str, x: torch.Tensor) -> torch.Tensor:
    if x.dim() != 3:
        raise RuntimeError(f"{fn}: x must be 3D [B, n, C]")
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    return x.contiguous()


def _weight(w: torch.Tensor) -> torch.Tensor:
    if w.dtype not in (torch.float32, torch.bfloat16):
        w = w.float()
    return w.contiguous()


def mhc_layer_static_fwd(x: torch.Tensor, rmsnorm_weight: torch.Tensor, H_pre: torch.Tensor,
                         H_post: torch.Tensor, H_res: torch.Tensor, num_iters: int = 20,
                         sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5
                         ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused static-H forward.  Returns (out fp32 [B,n,C], rms [B], saved)
    where ``saved`` holds (h_pre, h_post, M, fp32 weight) for the backward;
    ``saved[:2n+n*n]`` are the activated coefficients."""
    _check_device("mhc_layer_static_fwd", x, rmsnorm_weight, H_pre, H_post, H_res)
    x = _layer_x("mhc_layer_static_fwd", x)
    B, n, C = x.shape
    if rmsnorm_weight.numel() != C or H_pre.numel() != n or H_post.numel() != n or H_res.numel() != n * n:
        raise RuntimeError("mhc_layer_static_fwd: parameter shapes do not match x [B, n, C]")
    w = _weight(rmsnorm_weight)
    hp, hq, hr = _f32c(H_pre), _f32c(H_post), _f32c(H_res)
    out = torch.empty((B, n, C), dtype=torch.float32, device=x.device)
    rms = torch.empty((B,), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    saved = torch.empty((lib.mhc_layer_static_saved_size(n, C) // 4,), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        call("mhc_layer_static_fwd", ptr(x), dtype_code(x.dtype), ptr(w), dtype_code(w.dtype), ptr(hp), ptr(hq),
             ptr(hr), ptr(out), ptr(rms), ptr(saved), B, n, C, int(num_iters), float(sinkhorn_eps),
             float(rmsnorm_eps), stream_of(x))
    return out, rms, saved


def mhc_layer_static_bwd(grad_out: torch.Tensor, x: torch.Tensor, rmsnorm_weight: torch.Tensor,
                         H_pre: torch.Tensor, H_post: torch.Tensor, H_res: torch.Tensor, saved: torch.Tensor,
                         num_iters: int = 20, sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5):
    """Fused static-H backward.  Returns (grad_x [x dtype], grad_weight
    [C, weight dtype], grad_H_pre [n], grad_H_post [n], grad_H_res [n, n])."""
    _check_device("mhc_layer_static_bwd", grad_out, x, rmsnorm_weight, H_pre, H_post, H_res, saved)
    x = _layer_x("mhc_layer_static_bwd", x)
    B, n, C = x.shape
    if grad_out.shape != x.shape:
        raise RuntimeError("mhc_layer_static_bwd: grad_out must match x [B, n, C]")
    g = _f32c(grad_out)
    wdt = rmsnorm_weight.dtype if rmsnorm_weight.dtype in (torch.float32, torch.bfloat16) else torch.float32
    hp, hq, hr = _f32c(H_pre), _f32c(H_post), _f32c(H_res)
    dev = x.device
    grad_x = torch.empty_like(x)
    gw = torch.empty((C,), dtype=wdt, device=dev)
    ghp = torch.empty((n,), dtype=torch.float32, device=dev)
    ghq = torch.empty((n,), dtype=torch.float32, device=dev)
    ghr = torch.empty((n, n), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        ws_bytes = _lib.load().mhc_layer_static_bwd_workspace_size(B, n, C, dtype_code(x.dtype))
        ws = torch.empty((max(int(ws_bytes), 1),), dtype=torch.uint8, device=dev)
        call("mhc_layer_static_bwd", ptr(g), ptr(x), dtype_code(x.dtype), dtype_code(wdt), ptr(hp), ptr(hq),
             ptr(hr), ptr(saved), ptr(grad_x), ptr(gw), ptr(ghp), ptr(ghq), ptr(ghr), ptr(ws), int(ws_bytes), B, n,
             C, int(num_iters), float(sinkhorn_eps), float(rmsnorm_eps), stream_of(x))
    return grad_x, gw, ghp, ghq, ghr


def mhc_layer_static_bwd_noalloc(grad_out: torch.Tensor, x: torch.Tensor, rmsnorm_weight: torch.Tensor,
                                 H_pre: torch.Tensor, H_post: torch.Tensor, H_res: torch.Tensor, saved: torch.Tensor,
                                 num_iters: int = 20, sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5):
    """mhc_layer_static_bwd through the allocation-free entry: the library
    uses its own per-device scratch array instead of a workspace (only the
    outputs are allocated here).  Same results, bit for bit."""
    _check_device("mhc_layer_static_bwd_noalloc", grad_out, x, rmsnorm_weight, H_pre, H_post, H_res, saved)
    x = _layer_x("mhc_layer_static_bwd_noalloc", x)
    B, n, C = x.shape
    if grad_out.shape != x.shape:
        raise RuntimeError("mhc_layer_static_bwd_noalloc: grad_out must match x [B, n, C]")
    g = _f32c(grad_out)
    wdt = rmsnorm_weight.dtype if rmsnorm_weight.dtype in (torch.float32, torch.bfloat16) else torch.float32
    hp, hq, hr = _f32c(H_pre), _f32c(H_post), _f32c(H_res)
    dev = x.device
    grad_x = torch.empty_like(x)
    gw = torch.empty((C,), dtype=wdt, device=dev)
    ghp = torch.empty((n,), dtype=torch.float32, device=dev)
    ghq = torch.empty((n,), dtype=torch.float32, device=dev)
    ghr = torch.empty((n, n), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        call("mhc_layer_static_bwd_noalloc", ptr(g), ptr(x), dtype_code(x.dtype), dtype_code(wdt), ptr(hp), ptr(hq),
             ptr(hr), ptr(saved), ptr(grad_x), ptr(gw), ptr(ghp), ptr(ghq), ptr(ghr), B, n, C, int(num_iters),
             float(sinkhorn_eps), float(rmsnorm_eps), stream_of(x))
    return grad_x, gw, ghp, ghq, ghr


# =============================================================================
# Dynamic-H projection (bindings.cpp:480-541) and fused dynamic layer
# (bindings.cpp:600-952)
# =============================================================================

def _ws(dev, nbytes: int) -> torch.Tensor:
    return torch.empty((max(int(nbytes), 1),), dtype=torch.uint8, device=dev)


def fused_rmsnorm_matmul_fwd(inp: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """P = inp @ weight^T, fp32 [B, out_dim] (bindings.cpp:480-528); inp [B, K]
    fp32 or bf16, weight [out_dim, K].  Split-bf16 MFMA keeps ~fp32 accuracy
    (the reference rounds inputs and P to bf16)."""
    _check_device("fused_rmsnorm_matmul_fwd", inp, weight)
    if inp.dim() != 2 or weight.dim() != 2 or weight.size(1) != inp.size(1):
        raise RuntimeError("fused_rmsnorm_matmul_fwd: expected inp [B, K] and weight [out_dim, K]")
    x = _storage(inp)
    phi = _f32c(weight)
    B, K = x.shape
    out = torch.empty((B, phi.size(0)), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        wsb = _lib.load().mhc_fused_rmsnorm_matmul_fwd_workspace_size(B, K, phi.size(0))
        ws = _ws(x.device, wsb)
        call("mhc_fused_rmsnorm_matmul_fwd", ptr(x), dtype_code(x.dtype), ptr(phi), ptr(out), ptr(ws), int(wsb), B,
             K, phi.size(0), stream_of(x))
    return out


def fused_rmsnorm_matmul_bwd(grad_out: torch.Tensor, x_flat: torch.Tensor,
                             phi_concat: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(grad_x = grad_out @ phi, grad_phi = grad_out^T @ x_flat), fp32 (bindings.cpp:530-541)."""
    _check_device("fused_rmsnorm_matmul_bwd", grad_out, x_flat, phi_concat)
    g, x, phi = _f32c(grad_out), _f32c(x_flat), _f32c(phi_concat)
    B, K = x.shape
    out_dim = phi.size(0)
    gx = torch.empty((B, K), dtype=torch.float32, device=x.device)
    gphi = torch.empty((out_dim, K), dtype=torch.float32, device=x.device)
    with _lib.on_device(x.device):
        wsb = _lib.load().mhc_fused_rmsnorm_matmul_bwd_workspace_size(B, K, out_dim)
        ws = _ws(x.device, wsb)
        call("mhc_fused_rmsnorm_matmul_bwd", ptr(g), ptr(x), ptr(phi), ptr(gx), ptr(gphi), ptr(ws), int(wsb), B, K,
             out_dim, stream_of(x))
    return gx, gphi


def _scalar_param(a, dev) -> torch.Tensor:
    """alpha as a 1-element fp32 device tensor (device pointer, no host sync)."""
    if torch.is_tensor(a):
        return a.detach().to(device=dev, dtype=torch.float32).reshape(1).contiguous()
    return torch.full((1,), float(a), dtype=torch.float32, device=dev)


def _phi_parts(phi_pre, phi_post, phi_res, n, nC):
    parts = [_f32c(phi_pre), _f32c(phi_post), _f32c(phi_res)]
    for t, rows in zip(parts, (n, n, n * n)):
        if t.numel() != rows * nC:
            raise RuntimeError(f"dynamic layer: projection of {tuple(t.shape)} does not match [{rows}, {nC}]")
    return parts


def mhc_layer_dynamic_fwd(x_expanded: torch.Tensor, rmsnorm_weight: torch.Tensor, phi_pre: torch.Tensor,
                          phi_post: torch.Tensor, phi_res: torch.Tensor, alpha_pre, alpha_post, alpha_res,
                          b_pre: torch.Tensor, b_post: torch.Tensor, b_res: torch.Tensor, sinkhorn_iters: int = 20,
                          sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused dynamic-H forward: (out fp32 [B, n, C], saved) where saved holds
    the fp32 weight, per-token (h_pre, h_post, M), P and r_h for the
    backward.  Unlike mhc_layer_fwd_dynamic of the reference (bindings.cpp:
    880-952, 9 tensors) no [B, C] / [B, nC] intermediates are materialised."""
    _check_device("mhc_layer_dynamic_fwd", x_expanded, rmsnorm_weight, phi_pre, phi_post, phi_res, b_pre, b_post,
                  b_res)
    x = _layer_x("mhc_layer_dynamic_fwd", x_expanded)
    B, n, C = x.shape
    dev = x.device
    w = _weight(rmsnorm_weight)
    if w.numel() != C:
        raise RuntimeError("mhc_layer_dynamic_fwd: rmsnorm_weight must have C elements")
    pp, pq, pr = _phi_parts(phi_pre, phi_post, phi_res, n, n * C)
    a = [_scalar_param(v, dev) for v in (alpha_pre, alpha_post, alpha_res)]
    bp, bq, br = _f32c(b_pre), _f32c(b_post), _f32c(b_res)
    out = torch.empty((B, n, C), dtype=torch.float32, device=dev)
    lib = _lib.load()
    saved = torch.empty((lib.mhc_layer_dynamic_saved_size(B, n, C) // 4,), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        wsb = lib.mhc_layer_dynamic_fwd_workspace_size(B, n, C)
        ws = _ws(dev, wsb)
        call("mhc_layer_dynamic_fwd", ptr(x), dtype_code(x.dtype), ptr(w), dtype_code(w.dtype), ptr(pp), ptr(pq),
             ptr(pr), ptr(a[0]), ptr(a[1]), ptr(a[2]), ptr(bp), ptr(bq), ptr(br), ptr(out), ptr(saved), ptr(ws),
             int(wsb), B, n, C, int(sinkhorn_iters), float(sinkhorn_eps), float(rmsnorm_eps), stream_of(x))
    return out, saved


def mhc_layer_dynamic_pack(rmsnorm_weight: torch.Tensor, phi_pre: torch.Tensor, phi_post: torch.Tensor,
                           phi_res: torch.Tensor) -> torch.Tensor:
    """The parameter-only part of the dynamic forward (fp32 weight, projection
    planes) packed for mhc_layer_dynamic_infer: repack after every parameter
    update.  Returns an opaque uint8 device tensor."""
    _check_device("mhc_layer_dynamic_pack", rmsnorm_weight, phi_pre, phi_post, phi_res)
    w = _weight(rmsnorm_weight)
    C = w.numel()
    n = phi_pre.size(0) if phi_pre.dim() > 0 else 0
    pp, pq, pr = _phi_parts(phi_pre, phi_post, phi_res, n, n * C)
    dev = w.device
    lib = _lib.load()
    nbytes = int(lib.mhc_layer_dynamic_packed_size(n, C))
    packed = _ws(dev, nbytes)
    with _lib.on_device(dev):
        call("mhc_layer_dynamic_pack", ptr(w), dtype_code(w.dtype), ptr(pp), ptr(pq), ptr(pr), ptr(packed), nbytes,
             n, C, stream_of(w))
    return packed


def mhc_layer_dynamic_infer(x_expanded: torch.Tensor, packed: torch.Tensor, alpha_pre, alpha_post, alpha_res,
                            b_pre: torch.Tensor, b_post: torch.Tensor, b_res: torch.Tensor, sinkhorn_iters: int = 20,
                            sinkhorn_eps: float = 1e-8, rmsnorm_eps: float = 1e-5,
                            out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Forward-only dynamic-H layer on parameters packed by
    mhc_layer_dynamic_pack: out [B, n, C] in out_dtype (fp32 or bf16).  No
    state for a backward is written (ops.py:337-380)."""
    _check_device("mhc_layer_dynamic_infer", x_expanded, packed, b_pre, b_post, b_res)
    x = _layer_x("mhc_layer_dynamic_infer", x_expanded)
    B, n, C = x.shape
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError("mhc_layer_dynamic_infer: out_dtype must be torch.float32 or torch.bfloat16")
    lib = _lib.load()
    if packed.dtype != torch.uint8 or packed.numel() < lib.mhc_layer_dynamic_packed_size(n, C):
        raise RuntimeError("mhc_layer_dynamic_infer: packed parameters do not match x [B, n, C]")
    dev = x.device
    a = [_scalar_param(v, dev) for v in (alpha_pre, alpha_post, alpha_res)]
    bp, bq, br = _f32c(b_pre), _f32c(b_post), _f32c(b_res)
    if bp.numel() != n or bq.numel() != n or br.numel() != n * n:
        raise RuntimeError("mhc_layer_dynamic_infer: b_pre/b_post must have n and b_res n*n elements")
    out = torch.empty((B, n, C), dtype=out_dtype, device=dev)
    with _lib.on_device(dev):
        wsb = lib.mhc_layer_dynamic_infer_workspace_size(B, n, C)
        ws = _ws(dev, wsb)
        call("mhc_layer_dynamic_infer", ptr(x), dtype_code(x.dtype), ptr(packed), ptr(a[0]), ptr(a[1]), ptr(a[2]),
             ptr(bp), ptr(bq), ptr(br), ptr(out), dtype_code(out_dtype), ptr(ws), int(wsb), B, n, C,
             int(sinkhorn_iters), float(sinkhorn_eps), float(rmsnorm_eps), stream_of(x))
    return out


def mhc_layer_dynamic_bwd(grad_output: torch.Tensor, x_expanded: torch.Tensor, rmsnorm_weight: torch.Tensor,
                          saved: torch.Tensor, phi_pre: torch.Tensor, phi_post: torch.Tensor, phi_res: torch.Tensor,
                          alpha_pre, alpha_post, alpha_res, b_pre: torch.Tensor, b_post: torch.Tensor,
                          b_res: torch.Tensor, sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                          rmsnorm_eps: float = 1e-5):
    """Fused dynamic-H backward.  Returns the reference's 11 gradients
    (bindings.cpp:600-611): grad_x, grad_rmsnorm_weight, d_phi_pre,
    d_phi_post, d_phi_res, d_alpha_pre, d_alpha_post, d_alpha_res, d_b_pre,
    d_b_post, d_b_res."""
    _check_device("mhc_layer_dynamic_bwd", grad_output, x_expanded, rmsnorm_weight, saved, phi_pre, phi_post,
                  phi_res, b_pre, b_post, b_res)
    x = _layer_x("mhc_layer_dynamic_bwd", x_expanded)
    B, n, C = x.shape
    dev = x.device
    if grad_output.shape != x.shape:
        raise RuntimeError("mhc_layer_dynamic_bwd: grad_output must match x [B, n, C]")
    g = _f32c(grad_output)
    wdt = rmsnorm_weight.dtype if rmsnorm_weight.dtype in (torch.float32, torch.bfloat16) else torch.float32
    pp, pq, pr = _phi_parts(phi_pre, phi_post, phi_res, n, n * C)
    a = [_scalar_param(v, dev) for v in (alpha_pre, alpha_post, alpha_res)]
    bp, bq, br = _f32c(b_pre), _f32c(b_post), _f32c(b_res)
    np_ = 2 * n + n * n
    grad_x = torch.empty_like(x)
    gw = torch.empty((C,), dtype=wdt, device=dev)
    gphi = torch.empty((np_, n * C), dtype=torch.float32, device=dev)
    galpha = torch.empty((3,), dtype=torch.float32, device=dev)
    gb = torch.empty((np_,), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        wsb = _lib.load().mhc_layer_dynamic_bwd_workspace_size(B, n, C, dtype_code(x.dtype))
        ws = _ws(dev, wsb)
        call("mhc_layer_dynamic_bwd", ptr(g), ptr(x), dtype_code(x.dtype), dtype_code(wdt), ptr(pp), ptr(pq),
             ptr(pr), ptr(a[0]), ptr(a[1]), ptr(a[2]), ptr(bp), ptr(bq), ptr(br), ptr(saved), ptr(grad_x), ptr(gw),
             ptr(gphi), ptr(galpha), ptr(gb), ptr(ws), int(wsb), B, n, C, int(sinkhorn_iters),
             float(sinkhorn_eps), float(rmsnorm_eps), stream_of(x))
    return (grad_x, gw, gphi[:n], gphi[n:2 * n], gphi[2 * n:], galpha[0], galpha[1], galpha[2], gb[:n],
            gb[n:2 * n], gb[2 * n:].view(n, n))


def _host_float(v) -> float:
    """A scalar argument the reference's binding takes as a C float."""
    return float(v.item()) if torch.is_tensor(v) else float(v)


def mhc_layer_fwd_dynamic(x_expanded: torch.Tensor, rmsnorm_weight: torch.Tensor, phi_concat: torch.Tensor,
                          alpha_pre, alpha_post, alpha_res, b_pre: torch.Tensor, b_post: torch.Tensor,
                          b_res: torch.Tensor, sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                          rmsnorm_eps: float = 1e-5):
    """The reference's dynamic-H forward with its own call shape
    (bindings.cpp:880-952, unpacked at ops.py:425-448): phi_concat =
    [phi_pre; phi_post; phi_res] [2n+n^2, nC], alphas as Python floats (or
    one-element tensors).  Returns its nine tensors in order: output fp32
    [B, n, C], rms [B] (RMS of x_agg), x_agg_bf16 [B, C], H_pre_activated
    [B, n], H_post_activated [B, n], M [B, n, n], y_norm_bf16 [B, C],
    x_flat_bf16 [B, nC], rms_h [B].  Arithmetic is fp32 throughout; the
    three bf16 tensors are rounded on output only."""
    _check_device("mhc_layer_fwd_dynamic", x_expanded, rmsnorm_weight, phi_concat, b_pre, b_post, b_res)
    x = _layer_x("mhc_layer_fwd_dynamic", x_expanded)
    if phi_concat.dim() != 2:
        raise RuntimeError("phi_concat must be [out_dim, n*C]")
    B, n, C = x.shape
    np_ = 2 * n + n * n
    if tuple(phi_concat.shape) != (np_, n * C):
        raise RuntimeError(f"mhc_layer_fwd_dynamic: phi_concat must be [{np_}, {n * C}], got "
                           f"{tuple(phi_concat.shape)}")
    w = _weight(rmsnorm_weight)
    if w.numel() != C:
        raise RuntimeError("mhc_layer_fwd_dynamic: rmsnorm_weight must have C elements")
    phi = _f32c(phi_concat)
    bp, bq, br = _f32c(b_pre), _f32c(b_post), _f32c(b_res)
    if bp.numel() != n or bq.numel() != n or br.numel() != n * n:
        raise RuntimeError("mhc_layer_fwd_dynamic: b_pre/b_post must have n and b_res n*n elements")
    dev = x.device
    f32 = dict(dtype=torch.float32, device=dev)
    b16 = dict(dtype=torch.bfloat16, device=dev)
    output = torch.empty((B, n, C), **f32)
    rms = torch.empty((B,), **f32)
    x_agg = torch.empty((B, C), **b16)
    h_pre = torch.empty((B, n), **f32)
    h_post = torch.empty((B, n), **f32)
    M = torch.empty((B, n, n), **f32)
    y_norm = torch.empty((B, C), **b16)
    x_flat = torch.empty((B, n * C), **b16)
    rms_h = torch.empty((B,), **f32)
    with _lib.on_device(dev):
        wsb = _lib.load().mhc_layer_fwd_dynamic_workspace_size(B, n, C)
        ws = _ws(dev, wsb)
        call("mhc_layer_fwd_dynamic", ptr(x), dtype_code(x.dtype), ptr(w), dtype_code(w.dtype), ptr(phi),
             _host_float(alpha_pre), _host_float(alpha_post), _host_float(alpha_res), ptr(bp), ptr(bq), ptr(br),
             ptr(output), ptr(rms), ptr(x_agg), ptr(h_pre), ptr(h_post), ptr(M), ptr(y_norm), ptr(x_flat),
             ptr(rms_h), ptr(ws), int(wsb), B, n, C, int(sinkhorn_iters), float(sinkhorn_eps), float(rmsnorm_eps),
             stream_of(x))
    return output, rms, x_agg, h_pre, h_post, M, y_norm, x_flat, rms_h


def mhc_layer_bwd_dynamic(grad_output, x_expanded, rmsnorm_weight, rms, x_agg_bf16, H_pre_activated,
                          H_post_activated, M, y_norm_bf16, x_flat_bf16, rms_h, phi_pre, phi_post, phi_res, alpha_pre,
                          alpha_post, alpha_res, b_pre, b_post, b_res, sinkhorn_iters=20, sinkhorn_eps=1e-8,
                          rmsnorm_eps=1e-5):
    """The reference's dynamic-H backward with its 23-argument call shape
    (bindings.cpp:600-874, called at ops.py:518-542; alphas as floats).
    H_pre_activated, H_post_activated, M and rms_h are used as given and P
    is recomputed from x (as the reference does); rms, x_agg_bf16,
    y_norm_bf16 and x_flat_bf16 are recomputed in fp32 from x inside the
    fused row pass and not read.  Returns the 11 gradients in the
    reference's order and dtypes: grad_x, grad_rmsnorm_weight (fp32),
    d_phi_pre, d_phi_post, d_phi_res (shaped like the phi arguments),
    d_alpha_pre, d_alpha_post, d_alpha_res ([1] each), d_b_pre, d_b_post,
    d_b_res."""
    _check_device("mhc_layer_bwd_dynamic", grad_output, x_expanded, rmsnorm_weight, H_pre_activated,
                  H_post_activated, M, rms_h, phi_pre, phi_post, phi_res, b_pre, b_post, b_res)
    if grad_output.dim() != 3:
        raise RuntimeError("grad_output must be 3D tensor [B, n, C]")
    x = _layer_x("mhc_layer_bwd_dynamic", x_expanded)
    B, n, C = x.shape
    if grad_output.shape != x.shape:
        raise RuntimeError("mhc_layer_bwd_dynamic: grad_output must match x [B, n, C]")
    dev = x.device
    g = _f32c(grad_output)
    w = _weight(rmsnorm_weight)
    if w.numel() != C:
        raise RuntimeError("mhc_layer_bwd_dynamic: rmsnorm_weight must have C elements")
    hp, hq, m, rh = _f32c(H_pre_activated), _f32c(H_post_activated), _f32c(M), _f32c(rms_h)
    if hp.numel() != B * n or hq.numel() != B * n or m.numel() != B * n * n or rh.numel() != B:
        raise RuntimeError("mhc_layer_bwd_dynamic: saved H_pre/H_post [B, n], M [B, n, n], rms_h [B] do not match x")
    pp, pq, pr = _phi_parts(phi_pre, phi_post, phi_res, n, n * C)
    bp, bq, br = _f32c(b_pre), _f32c(b_post), _f32c(b_res)
    np_ = 2 * n + n * n
    f32 = dict(dtype=torch.float32, device=dev)
    grad_x = torch.empty_like(x)
    gw = torch.empty((C,), **f32)
    gphi = torch.empty((np_, n * C), **f32)
    small = torch.empty((3 + np_,), **f32)
    ga = small[:3]
    gb = small[3:]
    with _lib.on_device(dev):
        wsb = _lib.load().mhc_layer_bwd_dynamic_workspace_size(B, n, C, dtype_code(x.dtype))
        ws = _ws(dev, wsb)
        call("mhc_layer_bwd_dynamic", ptr(g), ptr(x), dtype_code(x.dtype), ptr(w), dtype_code(w.dtype), None, None,
             ptr(hp), ptr(hq), ptr(m), None, None, ptr(rh), ptr(pp), ptr(pq), ptr(pr), _host_float(alpha_pre),
             _host_float(alpha_post), _host_float(alpha_res), ptr(bp), ptr(bq), ptr(br), ptr(grad_x), ptr(gw),
             ptr(gphi), ptr(gphi[n:]), ptr(gphi[2 * n:]), ptr(ga), ptr(ga[1:]), ptr(ga[2:]), ptr(gb), ptr(gb[n:]),
             ptr(gb[2 * n:]), ptr(ws), int(wsb), B, n, C, int(sinkhorn_iters), float(sinkhorn_eps),
             float(rmsnorm_eps), stream_of(x))
    return (grad_x, gw, gphi[:n].view_as(phi_pre), gphi[n:2 * n].view_as(phi_post),
            gphi[2 * n:].view(phi_res.shape), ga[0:1], ga[1:2], ga[2:3], gb[:n].view_as(b_pre),
            gb[n:2 * n].view_as(b_post), gb[2 * n:].view(b_res.shape))


# =============================================================================
# Fused MHCResidualWrapper (layer.py:269-322): the n streams are synthesised
# from (residual, branch) inside the kernels; outputs are the stream mean.
# =============================================================================

def _wrapper_inputs(fn: str, residual: torch.Tensor, branch: torch.Tensor, residual_mode: str, n: int):
    _check_device(fn, residual, branch)
    if residual.shape != branch.shape or residual.dim() != 2:
        raise RuntimeError(f"{fn}: residual and branch must both be [tokens, hidden] of one shape")
    if residual_mode not in ("decay", "zero"):
        raise ValueError(f"Unknown residual_mode: {residual_mode}")
    if n < 2:
        # the reference writes stream 1 (layer.py:301), which needs n >= 2
        raise RuntimeError(f"{fn}: expansion_rate must be >= 2 (stream 1 holds the branch)")
    r = _storage(residual)
    b = branch.to(r.dtype).contiguous()
    mode = _lib.WRAPPER_DECAY if residual_mode == "decay" else _lib.WRAPPER_ZERO
    return r, b, mode


def wrapper_dynamic_fwd(residual: torch.Tensor, branch: torch.Tensor, residual_mode: str, n: int,
                        rmsnorm_weight: torch.Tensor, phi_pre, phi_post, phi_res, alpha_pre, alpha_post, alpha_res,
                        b_pre, b_post, b_res, sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                        rmsnorm_eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """(mean of the dynamic-H layer's n output streams, fp32 [tokens, C]; saved)."""
    r, b, mode = _wrapper_inputs("wrapper_dynamic_fwd", residual, branch, residual_mode, n)
    _check_device("wrapper_dynamic_fwd", r, rmsnorm_weight, phi_pre, phi_post, phi_res, b_pre, b_post, b_res)
    T, C = r.shape
    dev = r.device
    w = _weight(rmsnorm_weight)
    if w.numel() != C:
        raise RuntimeError("wrapper_dynamic_fwd: rmsnorm_weight must have C elements")
    pp, pq, pr = _phi_parts(phi_pre, phi_post, phi_res, n, n * C)
    a = [_scalar_param(v, dev) for v in (alpha_pre, alpha_post, alpha_res)]
    bp, bq, br = _f32c(b_pre), _f32c(b_post), _f32c(b_res)
    out = torch.empty((T, C), dtype=torch.float32, device=dev)
    lib = _lib.load()
    saved = torch.empty((lib.mhc_wrapper_dynamic_saved_size(T, n, C) // 4,), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        wsb = lib.mhc_wrapper_dynamic_fwd_workspace_size_for(T, n, C, dtype_code(r.dtype))
        ws = _ws(dev, wsb)
        call("mhc_wrapper_dynamic_fwd", ptr(r), ptr(b), dtype_code(r.dtype), mode, ptr(w), dtype_code(w.dtype),
             ptr(pp), ptr(pq), ptr(pr), ptr(a[0]), ptr(a[1]), ptr(a[2]), ptr(bp), ptr(bq), ptr(br), ptr(out),
             ptr(saved), ptr(ws), int(wsb), T, n, C, int(sinkhorn_iters), float(sinkhorn_eps), float(rmsnorm_eps),
             stream_of(r))
    return out, saved


def wrapper_dynamic_bwd(grad_out: torch.Tensor, residual: torch.Tensor, branch: torch.Tensor, residual_mode: str,
                        n: int, rmsnorm_weight: torch.Tensor, saved: torch.Tensor, phi_pre, phi_post, phi_res,
                        alpha_pre, alpha_post, alpha_res, b_res, sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                        rmsnorm_eps: float = 1e-5):
    """(grad_residual, grad_branch, grad_rmsnorm_weight, d_phi_pre, d_phi_post,
    d_phi_res, d_alpha_pre, d_alpha_post, d_alpha_res, d_b_pre, d_b_post, d_b_res)."""
    r, b, mode = _wrapper_inputs("wrapper_dynamic_bwd", residual, branch, residual_mode, n)
    _check_device("wrapper_dynamic_bwd", grad_out, r, rmsnorm_weight, saved, phi_pre, phi_post, phi_res, b_res)
    T, C = r.shape
    dev = r.device
    if grad_out.shape != r.shape:
        raise RuntimeError("wrapper_dynamic_bwd: grad_out must be [tokens, hidden]")
    g = _f32c(grad_out)
    wdt = rmsnorm_weight.dtype if rmsnorm_weight.dtype in (torch.float32, torch.bfloat16) else torch.float32
    pp, pq, pr = _phi_parts(phi_pre, phi_post, phi_res, n, n * C)
    a = [_scalar_param(v, dev) for v in (alpha_pre, alpha_post, alpha_res)]
    br = _f32c(b_res)
    np_ = 2 * n + n * n
    gr = torch.empty_like(r)
    gb = torch.empty_like(b)
    gw = torch.empty((C,), dtype=wdt, device=dev)
    gphi = torch.empty((np_, n * C), dtype=torch.float32, device=dev)
    galpha = torch.empty((3,), dtype=torch.float32, device=dev)
    gbias = torch.empty((np_,), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        wsb = _lib.load().mhc_wrapper_dynamic_bwd_workspace_size_for(T, n, C, dtype_code(r.dtype), mode,
                                                                     int(sinkhorn_iters), float(sinkhorn_eps))
        ws = _ws(dev, wsb)
        call("mhc_wrapper_dynamic_bwd", ptr(g), ptr(r), ptr(b), dtype_code(r.dtype), mode, dtype_code(wdt), ptr(pp),
             ptr(pq), ptr(pr), ptr(a[0]), ptr(a[1]), ptr(a[2]), ptr(br), ptr(saved), ptr(gr), ptr(gb), ptr(gw),
             ptr(gphi), ptr(galpha), ptr(gbias), ptr(ws), int(wsb), T, n, C, int(sinkhorn_iters),
             float(sinkhorn_eps), float(rmsnorm_eps), stream_of(r))
    return (gr, gb, gw, gphi[:n], gphi[n:2 * n], gphi[2 * n:], galpha[0], galpha[1], galpha[2], gbias[:n],
            gbias[n:2 * n], gbias[2 * n:].view(n, n))


def wrapper_static_fwd(residual: torch.Tensor, branch: torch.Tensor, residual_mode: str, n: int,
                       rmsnorm_weight: torch.Tensor, H_pre: torch.Tensor, H_post: torch.Tensor, H_res: torch.Tensor,
                       sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                       rmsnorm_eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """(mean of the static-H layer's n output streams, fp32 [tokens, C]; saved)."""
    r, b, mode = _wrapper_inputs("wrapper_static_fwd", residual, branch, residual_mode, n)
    _check_device("wrapper_static_fwd", r, rmsnorm_weight, H_pre, H_post, H_res)
    T, C = r.shape
    dev = r.device
    w = _weight(rmsnorm_weight)
    if w.numel() != C or H_pre.numel() != n or H_post.numel() != n or H_res.numel() != n * n:
        raise RuntimeError("wrapper_static_fwd: parameter shapes do not match n and C")
    hp, hq, hr = _f32c(H_pre), _f32c(H_post), _f32c(H_res)
    out = torch.empty((T, C), dtype=torch.float32, device=dev)
    lib = _lib.load()
    saved = torch.empty((lib.mhc_layer_static_saved_size(n, C) // 4,), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        call("mhc_wrapper_static_fwd", ptr(r), ptr(b), dtype_code(r.dtype), mode, ptr(w), dtype_code(w.dtype), ptr(hp),
             ptr(hq), ptr(hr), ptr(out), ptr(saved), T, n, C, int(sinkhorn_iters), float(sinkhorn_eps),
             float(rmsnorm_eps), stream_of(r))
    return out, saved


def wrapper_static_bwd(grad_out: torch.Tensor, residual: torch.Tensor, branch: torch.Tensor, residual_mode: str,
                       n: int, rmsnorm_weight: torch.Tensor, H_pre: torch.Tensor, H_post: torch.Tensor,
                       H_res: torch.Tensor, saved: torch.Tensor, sinkhorn_iters: int = 20, sinkhorn_eps: float = 1e-8,
                       rmsnorm_eps: float = 1e-5):
    """(grad_residual, grad_branch, grad_rmsnorm_weight, grad_H_pre, grad_H_post, grad_H_res)."""
    r, b, mode = _wrapper_inputs("wrapper_static_bwd", residual, branch, residual_mode, n)
    _check_device("wrapper_static_bwd", grad_out, r, rmsnorm_weight, H_pre, H_post, H_res, saved)
    T, C = r.shape
    dev = r.device
    if grad_out.shape != r.shape:
        raise RuntimeError("wrapper_static_bwd: grad_out must be [tokens, hidden]")
    g = _f32c(grad_out)
    wdt = rmsnorm_weight.dtype if rmsnorm_weight.dtype in (torch.float32, torch.bfloat16) else torch.float32
    hp, hq, hr = _f32c(H_pre), _f32c(H_post), _f32c(H_res)
    gr = torch.empty_like(r)
    gb = torch.empty_like(b)
    gw = torch.empty((C,), dtype=wdt, device=dev)
    ghp = torch.empty((n,), dtype=torch.float32, device=dev)
    ghq = torch.empty((n,), dtype=torch.float32, device=dev)
    ghr = torch.empty((n, n), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        wsb = _lib.load().mhc_wrapper_static_bwd_workspace_size(T, n, C, dtype_code(r.dtype), mode)
        ws = _ws(dev, wsb)
        call("mhc_wrapper_static_bwd", ptr(g), ptr(r), ptr(b), dtype_code(r.dtype), mode, dtype_code(wdt), ptr(hp),
             ptr(hq), ptr(hr), ptr(saved), ptr(gr), ptr(gb), ptr(gw), ptr(ghp), ptr(ghq), ptr(ghr), ptr(ws), int(wsb),
             T, n, C, int(sinkhorn_iters), float(sinkhorn_eps), float(rmsnorm_eps), stream_of(r))
    return gr, gb, gw, ghp, ghq, ghr

"""ctypes binding of libmhc_hip.so (the C ABI declared in include/mhc_hip.h).

The library is loaded lazily on first use.  ``import torch`` happens first so
that the library's ``libamdhip64.so.7`` dependency resolves to the HIP
runtime torch already loaded (same SONAME) - one runtime per process, and
torch's HIP streams are valid handles for the library.

There is no fallback: if the library or the C++ autograd extension is
missing or fails to load, every op raises ``RuntimeError``.

``timed_build()`` is a benchmark facility: inside it every call goes to
``libmhc_hip_timed.so``, the same sources built with per-kernel HIP-event
timing (include/mhc_hip_timing.h); the product library has no timing state.
"""
from __future__ import annotations

import contextlib
import ctypes
import importlib.util
import os
import threading
from typing import Dict, List, Tuple

import torch  # noqa: F401  (must precede loading the HIP library)

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libmhc_hip.so"
LIB_PATH = os.path.join(_PKG, LIB_NAME)
TIMED_LIB_PATH = os.path.join(_PKG, "libmhc_hip_timed.so")

F32 = 0
BF16 = 1
WRAPPER_DECAY = 0
WRAPPER_ZERO = 1

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes).  Must match include/mhc_hip.h (checked by
# tests/test_abi.py against the header text).
SIGNATURES: Dict[str, Tuple[object, List[object]]] = {
    "mhc_abi_version": (ctypes.c_int, []),
    "mhc_last_error": (ctypes.c_char_p, []),
    "mhc_sinkhorn_knopp_fwd": (ctypes.c_int, [_vp, _vp, _i64, _i32, _i32, _f32, _vp]),
    "mhc_sinkhorn_knopp_bwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _f32, _vp]),
    "mhc_rmsnorm_fwd": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _i64, _i32, _f32, _vp]),
    "mhc_rmsnorm_bwd_workspace_size": (_sz, [_i64, _i32, _i32]),
    "mhc_rmsnorm_bwd": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i32, _vp]),
    "mhc_compute_rms_fwd": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i64, _f32, _vp]),
    "mhc_stream_aggregate_fwd": (ctypes.c_int, [_vp, _i32, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _vp]),
    "mhc_stream_aggregate_bwd": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _i32, _vp]),
    "mhc_stream_distribute_mix_add_fwd": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64, _vp, _i32, _vp, _vp,
                                                         _i64, _i32, _i32, _vp]),
    "mhc_stream_distribute_mix_add_bwd": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _i64, _vp, _i64, _vp, _vp,
                                                         _vp, _vp, _vp, _i64, _i32, _i32, _vp]),
    "mhc_noalloc_scratch_bytes": (_sz, []),
    "mhc_layer_static_bwd_noalloc": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                                    _i64, _i32, _i32, _i32, _f32, _f32, _vp]),
    "mhc_fused_rmsnorm_matmul_fwd_workspace_size": (_sz, [_i64, _i64, _i32]),
    "mhc_fused_rmsnorm_matmul_fwd": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _sz, _i64, _i64, _i32, _vp]),
    "mhc_fused_rmsnorm_matmul_bwd_workspace_size": (_sz, [_i64, _i64, _i32]),
    "mhc_fused_rmsnorm_matmul_bwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i64, _i32, _vp]),
    "mhc_layer_dynamic_saved_size": (_sz, [_i64, _i32, _i32]),
    "mhc_layer_dynamic_fwd_workspace_size": (_sz, [_i64, _i32, _i32]),
    "mhc_layer_dynamic_fwd": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32, _f32, _f32, _vp]),
    "mhc_layer_dynamic_packed_size": (_sz, [_i32, _i32]),
    "mhc_layer_dynamic_pack": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _vp, _sz, _i32, _i32, _vp]),
    "mhc_layer_dynamic_infer_workspace_size": (_sz, [_i64, _i32, _i32]),
    "mhc_layer_dynamic_infer": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _sz,
                                               _i64, _i32, _i32, _i32, _f32, _f32, _vp]),
    "mhc_layer_dynamic_bwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "mhc_layer_dynamic_bwd": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32, _f32,
                                             _f32, _vp]),
    "mhc_layer_fwd_dynamic_workspace_size": (_sz, [_i64, _i32, _i32]),
    "mhc_layer_fwd_dynamic": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _f32, _f32, _f32, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32,
                                             _f32, _f32, _vp]),
    "mhc_layer_bwd_dynamic_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "mhc_layer_bwd_dynamic": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _f32, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32, _f32,
                                             _f32, _vp]),
    "mhc_wrapper_dynamic_saved_size": (_sz, [_i64, _i32, _i32]),
    "mhc_wrapper_dynamic_fwd_workspace_size": (_sz, [_i64, _i32, _i32]),
    "mhc_wrapper_dynamic_fwd_workspace_size_for": (_sz, [_i64, _i32, _i32, _i32]),
    "mhc_wrapper_dynamic_fwd": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                               _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32, _f32, _f32,
                                               _vp]),
    "mhc_wrapper_dynamic_bwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "mhc_wrapper_dynamic_bwd_workspace_size_for": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32, _f32]),
    "mhc_wrapper_dynamic_bwd": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                               _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32,
                                               _f32, _f32, _vp]),
    "mhc_wrapper_static_fwd": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i32,
                                              _i32, _i32, _f32, _f32, _vp]),
    "mhc_wrapper_static_bwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "mhc_wrapper_static_bwd": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                              _vp, _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32, _f32, _f32, _vp]),
    "mhc_layer_static_saved_size": (_sz, [_i32, _i32]),
    "mhc_layer_static_fwd": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                            _i64, _i32, _i32, _i32, _f32, _f32, _vp]),
    "mhc_layer_static_bwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "mhc_layer_static_bwd": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                            _i64, _i32, _i32, _i32, _f32, _f32, _vp]),
}

# The benchmark build's extra entries (include/mhc_hip_timing.h).
TIMING_SIGNATURES: Dict[str, Tuple[object, List[object]]] = {
    "mhc_timing_enable": (ctypes.c_int, [ctypes.c_int]),
    "mhc_timing_reset": (ctypes.c_int, []),
    "mhc_timing_query": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64)]),
    "mhc_timing_proj_valu_workspace_size": (_sz, [_i64, _i64, _i32]),
    "mhc_timing_proj_valu": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _sz, _i64, _i64, _i32, _vp]),
}

_lib = None
_product = None
_lock = threading.Lock()


def _open(path: str, signatures) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise RuntimeError(
            f"mhc_ascend_amd: HIP library {path} is not built; run "
            "`python -m mhc_ascend_amd.csrc.build` (or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in signatures.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load() -> ctypes.CDLL:
    """The library every call goes to (idempotent)."""
    global _lib, _product
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            _product = _open(LIB_PATH, SIGNATURES)
            _lib = _product
    return _lib


AUTOGRAD_PATH = os.path.join(_PKG, "_mhc_autograd.so")
_autograd = None
_autograd_lock = threading.Lock()


def _bind(mod, lib) -> None:
    mod.bind({name: ctypes.cast(getattr(lib, name), ctypes.c_void_p).value for name in mod.entry_names()})


def autograd():
    """The C++ autograd nodes of the fused layers and the fused wrapper
    (``_mhc_autograd.so``, a torch extension built beside the library),
    bound to the loaded library's entry points.  Raises when it is not
    built: the fused layers have no other orchestration."""
    global _autograd
    if _autograd is not None:
        return _autograd
    lib = load()
    with _autograd_lock:
        if _autograd is None:
            if not os.path.exists(AUTOGRAD_PATH):
                raise RuntimeError(
                    f"mhc_ascend_amd: the C++ autograd extension {AUTOGRAD_PATH} is not built; run "
                    "`python -m mhc_ascend_amd.csrc.build` (or __graft_entry__.build())")
            spec = importlib.util.spec_from_file_location("mhc_ascend_amd._mhc_autograd", AUTOGRAD_PATH)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            _bind(mod, lib)
            _autograd = mod
    return _autograd


@contextlib.contextmanager
def timed_build():
    """Benchmark facility: route every call (ctypes and the C++ autograd
    nodes) to libmhc_hip_timed.so for the duration of the block, and yield
    it; its mhc_timing_* entries then time each kernel on its stream.  The
    two builds run the same kernels on the same buffers (identical
    sources), so state such as `saved` buffers carries across."""
    global _lib
    product = load()
    ag = autograd()
    timed = _open(TIMED_LIB_PATH, {**SIGNATURES, **TIMING_SIGNATURES})
    with _lock:
        _lib = timed
        _bind(ag, timed)
    try:
        yield timed
    finally:
        with _lock:
            _lib = product
            _bind(ag, product)


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point; raise RuntimeError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mhc_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_same_device = contextlib.nullcontext()


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of the current torch stream on ``t``'s device."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index if t.device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def on_device(dev: torch.device):
    """Make ``dev`` the current device for a library call (the library sizes
    grids for the current device); a no-op context when it already is."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _same_device
    return torch.cuda.device(dev)


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise RuntimeError(f"mhc_ascend_amd: unsupported storage dtype {dt} (float32 or bfloat16)")


# ---- kernel timing (inside timed_build() only) -----------------------------

def timing_enable(on: bool = True) -> None:
    call("mhc_timing_enable", 1 if on else 0)


def timing_reset() -> None:
    call("mhc_timing_reset")


def timing_query(kernel: str) -> Tuple[float, int]:
    ms = ctypes.c_double(0.0)
    n = _i64(0)
    call("mhc_timing_query", kernel.encode(), ctypes.byref(ms), ctypes.byref(n))
    return ms.value, n.value

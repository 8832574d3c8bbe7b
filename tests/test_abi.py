"""C-ABI surface checks that need no GPU: the library loads, exports every
function include/mhc_hip.h declares with the ctypes signatures the Python
binding uses, and rejects bad arguments before touching the device."""
import ctypes
import os
import re

import pytest
import torch

from mhc_ascend_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mhc_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:int|size_t|const char\s*\*)\s*(mhc_\w+)\s*\(", text, flags=re.M))


def test_header_and_binding_declare_the_same_functions():
    decl = header_functions()
    assert decl, "no functions parsed from the header"
    assert decl == set(_lib.SIGNATURES), (decl ^ set(_lib.SIGNATURES))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_pure_host_entry_points():
    lib = _lib.load()
    assert lib.mhc_abi_version() >= 100
    assert isinstance(lib.mhc_last_error(), bytes)


def test_product_build_has_no_timing_state_and_the_bench_build_does():
    """Per-kernel timing exists only in the benchmark's build of the same
    sources (include/mhc_hip_timing.h); the product library exports none of
    it.  The timed build exports every product entry as well."""
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "mhc_hip_timing.h")).read(), flags=re.S)
    timing = set(re.findall(r"^\s*(?:int|size_t)\s+(mhc_timing_\w+)\s*\(", text, flags=re.M))
    assert timing == set(_lib.TIMING_SIGNATURES)
    product = ctypes.CDLL(_lib.LIB_PATH)
    assert not [n for n in timing if hasattr(product, n)]
    timed = ctypes.CDLL(_lib.TIMED_LIB_PATH)
    missing = [n for n in header_functions() | timing if not hasattr(timed, n)]
    assert not missing, missing


@pytest.mark.parametrize("n,iters,batch", [(0, 20, 4), (4, -1, 4), (4, 20, -1)])
def test_sinkhorn_rejects_bad_arguments_on_host(n, iters, batch):
    lib = _lib.load()
    rc = lib.mhc_sinkhorn_knopp_fwd(1, 1, batch, n, iters, 1e-8, None)
    assert rc == -1
    assert lib.mhc_last_error()


def test_sinkhorn_rejects_n_above_a_wave_on_host():
    """Rows of one matrix live in the lanes of one wave: n <= 64."""
    lib = _lib.load()
    assert lib.mhc_sinkhorn_knopp_fwd(1, 1, 4, 65, 20, 1e-8, None) == -2
    assert b"n > 64" in lib.mhc_last_error()
    assert lib.mhc_sinkhorn_knopp_bwd(1, 1, 1, 1, 4, 65, 20, 1e-8, None) == -2


def test_layer_rejects_unsupported_and_invalid_on_host():
    lib = _lib.load()
    # n above 64 -> UNSUPPORTED; bad dtype -> INVALID; hidden past the
    # channel-loop kernels' LDS row (12288 channels at n = 32) -> UNSUPPORTED
    assert lib.mhc_layer_static_fwd(1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 8, 65, 64, 20, 1e-8, 1e-5, None) == -2
    assert lib.mhc_layer_static_fwd(1, 7, 1, 1, 1, 1, 1, 1, 1, 1, 8, 4, 64, 20, 1e-8, 1e-5, None) == -1
    assert lib.mhc_layer_static_fwd(1, 0, 1, 5, 1, 1, 1, 1, 1, 1, 8, 4, 64, 20, 1e-8, 1e-5, None) == -1
    assert lib.mhc_layer_static_fwd(1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 8, 32, 12289, 20, 1e-8, 1e-5, None) == -2
    assert b"too large for the row kernels" in lib.mhc_last_error()
    # a ragged hidden size passes the host checks (channel-loop kernels)
    assert lib.mhc_layer_static_fwd(None, 0, 1, 1, 1, 1, 1, 1, 1, 1, 8, 4, 66, 20, 1e-8, 1e-5, None) == -1
    # workspace too small
    assert lib.mhc_layer_static_bwd(1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 8, 4, 64, 20, 1e-8, 1e-5,
                                    None) == -3
    assert lib.mhc_layer_static_saved_size(4, 256) == (64 + 256) * 4


def test_expansion_rate_support_on_host():
    """Layers take every n in 1..64 as the reference does (mhc_types.h:68):
    fixed-n kernels for {2, 4, 8, 16, 32}, the generic kernels for the rest,
    dynamic H included (its 2n + n^2 projection rows run as 32-row output
    tiles or, above 128 rows, the streaming kernels); n > 64 is rejected.
    The fused wrapper takes n = 2..32 (other n go through the layer); with
    dynamic H past n = 10 its backward needs Sinkhorn settings under which
    the H_res gradients vanish.  All checked before any device work."""
    lib = _lib.load()
    # static layer: these n pass the host checks; with a null x they fail on that
    for n in (1, 2, 3, 6, 8, 12, 16, 32, 64):
        assert lib.mhc_layer_static_fwd(None, 0, 1, 1, 1, 1, 1, 1, 1, 1, 8, n, 64, 20, 1e-8, 1e-5, None) == -1
        assert b"null x" in lib.mhc_last_error()
    assert lib.mhc_layer_static_fwd(1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 8, 65, 64, 20, 1e-8, 1e-5, None) == -2
    rc = lib.mhc_layer_dynamic_fwd(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1 << 30, 8, 65, 64, 20, 1e-8,
                                   1e-5, None)
    assert rc == -2 and b"n=65 is not supported" in lib.mhc_last_error()
    # dynamic n = 6 passes the shape checks; a null out then fails before any launch
    rc = lib.mhc_layer_dynamic_fwd(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, None, 1, 1, 1 << 30, 8, 6, 64, 20, 1e-8,
                                   1e-5, None)
    assert rc == -1 and b"null x/out" in lib.mhc_last_error()
    # dynamic n = 8 passes the shape checks; a null out then fails before any launch
    rc = lib.mhc_layer_dynamic_fwd(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, None, 1, 1, 1 << 30, 8, 8, 64, 20, 1e-8,
                                   1e-5, None)
    assert rc == -1 and b"null x/out" in lib.mhc_last_error()
    rc = lib.mhc_wrapper_static_fwd(1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 8, 33, 256, 20, 1e-8, 1e-5, None)
    assert rc == -2 and b"the fused wrapper takes n <= 32" in lib.mhc_last_error()
    rc = lib.mhc_wrapper_dynamic_fwd(1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1 << 30, 8, 33, 256, 20,
                                     1e-8, 1e-5, None)
    assert rc == -2 and b"the fused wrapper takes n <= 32" in lib.mhc_last_error()
    # n = 16 and 32 pass the shape checks; a null out then fails before any launch
    for n in (16, 32):
        rc = lib.mhc_wrapper_static_fwd(1, 1, 1, 0, 1, 1, 1, 1, 1, None, 1, 8, n, 256, 20, 1e-8, 1e-5, None)
        assert rc == -1 and b"null residual/branch/out" in lib.mhc_last_error()
        rc = lib.mhc_wrapper_dynamic_fwd(1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, None, 1, 1, 1 << 30, 8, n, 256,
                                         20, 1e-8, 1e-5, None)
        assert rc == -1 and b"null residual/branch/out" in lib.mhc_last_error()
    # dynamic n = 16 backward with no Sinkhorn iteration (H_res gradients kept:
    # 288 projection rows) is refused before the workspace is looked at
    rc = lib.mhc_wrapper_dynamic_bwd(1, 1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, None, 0, 8, 16, 256, 0,
                                     1e-8, 1e-5, None)
    assert rc == -2 and b"needs num_iters >= 1 and sinkhorn_eps <= 1e-6" in lib.mhc_last_error()
    rc = lib.mhc_wrapper_static_fwd(1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 8, 1, 256, 20, 1e-8, 1e-5, None)
    assert rc == -1 and b"n must be >= 2" in lib.mhc_last_error()
    # n = 2 passes the shape checks; a null out then fails before any launch
    rc = lib.mhc_wrapper_static_fwd(1, 1, 1, 0, 1, 1, 1, 1, 1, None, 1, 8, 2, 256, 20, 1e-8, 1e-5, None)
    assert rc == -1 and b"null residual/branch/out" in lib.mhc_last_error()


def test_wrapper_backward_workspace_for_settings_on_host():
    """The settings-aware size query of the wrapper backward: with the H_res
    rows of dP vanishing (num_iters >= 1, eps <= 1e-6) the run-time-n path
    keeps no stream rows, so its size drops below the all-settings query;
    otherwise (and for the n = 4 kernels' shapes) the two agree."""
    lib = _lib.load()
    for n, C in ((8, 7168), (2, 256), (4, 264), (5, 96)):
        full = lib.mhc_wrapper_dynamic_bwd_workspace_size(4096, n, C, 1, 0)
        assert lib.mhc_wrapper_dynamic_bwd_workspace_size_for(4096, n, C, 1, 0, 0, 1e-8) == full
        assert lib.mhc_wrapper_dynamic_bwd_workspace_size_for(4096, n, C, 1, 0, 1, 0.1) == full
        small = lib.mhc_wrapper_dynamic_bwd_workspace_size_for(4096, n, C, 1, 0, 20, 1e-8)
        # X and dX: 8 n C bytes per token
        assert full - small >= 8 * n * C * 4096, (n, C, full, small)
    full = lib.mhc_wrapper_dynamic_bwd_workspace_size(4096, 4, 4096, 1, 0)
    assert lib.mhc_wrapper_dynamic_bwd_workspace_size_for(4096, 4, 4096, 1, 0, 20, 1e-8) == full


def test_wrapper_forward_workspace_for_dtype_on_host():
    """The dtype-aware size query of the wrapper forward: bf16 rows the
    projection rebuilds itself (n >= 5, >= 1024 tokens, hidden % 64 == 0)
    keep no stream rows; other run-time-n shapes keep them in their own
    dtype; the all-dtypes query covers every case."""
    lib = _lib.load()
    for n, C, T in ((8, 7168, 4096), (5, 128, 1100), (3, 96, 4096), (8, 96, 4096), (8, 7168, 512)):
        full = lib.mhc_wrapper_dynamic_fwd_workspace_size(T, n, C)
        f32 = lib.mhc_wrapper_dynamic_fwd_workspace_size_for(T, n, C, 0)
        b16 = lib.mhc_wrapper_dynamic_fwd_workspace_size_for(T, n, C, 1)
        assert b16 <= f32 <= full, (n, C, T, b16, f32, full)
        direct = n >= 5 and T >= 1024 and C % 64 == 0
        if direct:
            assert f32 - b16 >= 4 * n * C * T, (n, C, T)
        else:
            assert f32 - b16 >= 2 * n * C * T - 256, (n, C, T)
    full = lib.mhc_wrapper_dynamic_fwd_workspace_size(4096, 4, 4096)
    assert lib.mhc_wrapper_dynamic_fwd_workspace_size_for(4096, 4, 4096, 1) == full


def test_cpu_tensors_raise_no_fallback():
    import mhc_ascend_amd as mhc
    x = torch.rand(2, 4, 4)
    with pytest.raises(RuntimeError, match="HIP device"):
        mhc.sinkhorn_knopp(x)
    layer = mhc.MHCLayer(16, 4, use_dynamic_h=False)
    with pytest.raises(RuntimeError, match="HIP device"):
        layer(torch.randn(3, 4, 16))


def test_autograd_extension_binds_every_entry():
    """_mhc_autograd.so (built with the library) imports on the CPU and binds
    only entry points the header declares and the ctypes table types."""
    from mhc_ascend_amd import _lib

    ag = _lib.autograd()
    assert ag is not None, f"{_lib.AUTOGRAD_PATH} is not built"
    names = ag.entry_names()
    assert names and all(n in _lib.SIGNATURES for n in names)
    assert callable(ag.static_layer) and callable(ag.dynamic_layer)


def test_autograd_extension_is_required(monkeypatch):
    """The C++ autograd nodes are the only orchestration of the fused layers:
    bound to the loaded library by default, and a clear error (no silent
    fallback) when the extension is missing."""
    from mhc_ascend_amd import _lib

    saved = _lib._autograd
    try:
        _lib._autograd = None
        ag = _lib.autograd()
        assert ag is not None and hasattr(ag, "static_layer")
        _lib._autograd = None
        monkeypatch.setattr(_lib, "AUTOGRAD_PATH", _lib.AUTOGRAD_PATH + ".missing")
        with pytest.raises(RuntimeError, match="autograd extension"):
            _lib.autograd()
    finally:
        _lib._autograd = saved

"""ctypes loader for the C Sinkhorn-Knopp oracle (oracle/sinkhorn.c).

Test infrastructure only.  Builds the library with ``make`` when it is
missing and a compiler is available.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmhc_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        lib.oracle_sinkhorn_fwd.argtypes = [dp, dp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_double]
        lib.oracle_sinkhorn_bwd.argtypes = [dp, dp, dp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_double]
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def sinkhorn_fwd(inp, num_iters=20, eps=1e-8):
    """inp: array-like [B, n, n] -> float64 ndarray [B, n, n]."""
    a = np.ascontiguousarray(np.asarray(inp, dtype=np.float64))
    out = np.empty_like(a)
    rc = _load().oracle_sinkhorn_fwd(_ptr(a), _ptr(out), a.shape[0], a.shape[1], num_iters, eps)
    assert rc == 0
    return out


def sinkhorn_bwd(grad_out, inp, num_iters=20, eps=1e-8):
    """Exact adjoint: grad wrt inp of <grad_out, SK(inp)>."""
    g = np.ascontiguousarray(np.asarray(grad_out, dtype=np.float64))
    a = np.ascontiguousarray(np.asarray(inp, dtype=np.float64))
    gi = np.empty_like(a)
    rc = _load().oracle_sinkhorn_bwd(_ptr(g), _ptr(a), _ptr(gi), a.shape[0], a.shape[1], num_iters, eps)
    assert rc == 0
    return gi

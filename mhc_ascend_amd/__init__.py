"""mhc_ascend_amd - the mHC hyper-connection layer on AMD Instinct MI355X.

Drop-in for the Python API of the reference package ``mhc``
(src/python/mhc/__init__.py:22-39); ``import mhc_ascend_amd as mhc`` keeps
user code unchanged.  All compute runs in hand-written HIP kernels for
gfx950 (``libmhc_hip.so``, C ABI in include/mhc_hip.h); there is no CPU
path.
"""

__version__ = "0.1.0"

from .layer import MHCLayer, create_mhc_layer, MHCResidualWrapper, replace_residual_with_mhc  # noqa: E402
from .ops import (  # noqa: E402
    sinkhorn_knopp,
    rmsnorm,
    stream_aggregate,
    stream_distribute_mix_add,
    stream_distribute,
    compute_rms,
    fused_rmsnorm_matmul,
    mhc_layer_static,
    mhc_layer_fused_dynamic_training,
    mhc_layer_fused_dynamic_inference,
)

__all__ = [
    "MHCLayer",
    "MHCResidualWrapper",
    "create_mhc_layer",
    "replace_residual_with_mhc",
    "sinkhorn_knopp",
    "rmsnorm",
    "stream_aggregate",
    "stream_distribute_mix_add",
    "stream_distribute",
    "compute_rms",
    "fused_rmsnorm_matmul",
    "mhc_layer_static",
    "mhc_layer_fused_dynamic_training",
    "mhc_layer_fused_dynamic_inference",
]

"""mhc_mlx_amd — the fused mHC layer of svdrecbd/mhc-mlx on MI355X (gfx950).

``MHCLayer`` / ``MHCRewire`` keep the reference's module API; the hot path
runs in libmhc_hip.so (hand-written HIP kernels, C ABI in include/mhc_hip.h).
"""

from .layer import MHCLayer, MHCRewire
from .patching import AutoPatcher
from . import ops, reference
from .ops import (
    mhc_forward_fused_hip,
    mhc_forward_fused_hip_autograd,
    mhc_layer_forward,
    mhc_layer_forward_dynamic,
    post_combine,
    residual_add_agg_hip,
    sinkhorn_knopp_hip,
    sinkhorn_knopp_hip_autograd,
    stream_mix_add_hip,
    stream_mix_add_hip_autograd,
    stream_scale,
)
from .profiling import kernel_timer
from .utils import residual_add_agg

__version__ = "0.1.0"

__all__ = [
    "AutoPatcher",
    "MHCLayer",
    "MHCRewire",
    "ops",
    "reference",
    "kernel_timer",
    "mhc_forward_fused_hip",
    "mhc_forward_fused_hip_autograd",
    "mhc_layer_forward",
    "mhc_layer_forward_dynamic",
    "post_combine",
    "residual_add_agg",
    "residual_add_agg_hip",
    "sinkhorn_knopp_hip",
    "sinkhorn_knopp_hip_autograd",
    "stream_mix_add_hip",
    "stream_mix_add_hip_autograd",
    "stream_scale",
    "__version__",
]

"""mhc_mlx_amd — the fused mHC layer of svdrecbd/mhc-mlx on MI355X (gfx950).

``MHCLayer`` / ``MHCRewire`` keep the reference's module API; the hot path
runs in libmhc_hip.so (hand-written HIP kernels, C ABI in include/mhc_hip.h).
"""

from . import tuning

tuning.load()  # the tuning files of the working directory and ~/.cache/mhc-mlx (metal.py:21-33)

from .layer import MHCLayer, MHCRewire  # noqa: E402
from .patching import AutoPatcher  # noqa: E402
from . import ops, reference  # noqa: E402
from .ops import (  # noqa: E402
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
from .profiling import kernel_timer  # noqa: E402
from .utils import residual_add_agg  # noqa: E402

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

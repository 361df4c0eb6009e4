"""The reference's op names (mhc_mlx/metal.py) bound to the HIP ops.

Code written against ``mhc_mlx.metal`` can import the same names from here;
each one is the corresponding ``mhc_mlx_amd.ops`` function.
"""

from .ops import (  # noqa: F401
    mhc_forward_fused_hip as mhc_forward_fused_metal,
    mhc_forward_fused_hip_autograd as mhc_forward_fused_metal_autograd,
    residual_add_agg_hip as residual_add_agg_metal,
    sinkhorn_knopp_hip as sinkhorn_knopp_metal,
    sinkhorn_knopp_hip_autograd as sinkhorn_knopp_metal_autograd,
    stream_mix_add_hip as stream_mix_add_metal,
    stream_mix_add_hip_autograd as stream_mix_add_metal_autograd,
    suggest_threads_per_group,
)
from .tuning import _get_tuned_tpg  # noqa: F401

__all__ = [
    "mhc_forward_fused_metal",
    "mhc_forward_fused_metal_autograd",
    "residual_add_agg_metal",
    "sinkhorn_knopp_metal",
    "sinkhorn_knopp_metal_autograd",
    "stream_mix_add_metal",
    "stream_mix_add_metal_autograd",
    "suggest_threads_per_group",
    "_get_tuned_tpg",
]

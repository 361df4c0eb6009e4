"""Block-level helpers around the mHC layer (mhc_mlx/utils.py)."""

from __future__ import annotations

import torch

from .ops import residual_add_agg_hip

__all__ = ["residual_add_agg"]


def residual_add_agg(x: torch.Tensor, res: torch.Tensor, H_pre: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused residual add + mHC aggregate (utils.py:4-24).

    out = x + res; y_agg = sum_i H_pre[i] * out[:, i]  (one pass over x and res).

    Args:
        x: input [B, n, C]
        res: residual [B, n, C]
        H_pre: pre-scaling factors [n] (used as given, not activated)

    Returns:
        (out [B, n, C] fp32, y_agg [B, C] fp32); differentiable w.r.t. all three inputs.
    """
    return residual_add_agg_hip(x, res, H_pre)

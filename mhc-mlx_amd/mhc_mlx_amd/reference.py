"""Pure-torch restatement of mhc_mlx/reference.py (the reference path).

This is what ``MHCLayer(use_metal=False)`` / ``MHC_MLX_DISABLE_METAL=1`` run,
as the reference's own layer does (layer.py:122-126, 423-431).  It is plain
autograd-capable torch code on whatever device the inputs live on.  MHCLayer
and MHCRewire also run it where the reference runs its MLX path: for n > 64,
and, with one warning per process, for a call the HIP path cannot take (CPU
tensors, a RuntimeError from the library).  The functions in ops.py never
fall back to it.  Function names and semantics follow reference.py:20-184 one
for one.
"""

from __future__ import annotations

import torch

__all__ = [
    "sinkhorn_knopp",
    "activate_pre_post",
    "mixing_matrix_from_logits",
    "stream_aggregate",
    "rms_norm",
    "stream_distribute",
    "stream_mix_ref",
    "mhc_forward_fused_reference",
    "mhc_forward_reference",
]


def sinkhorn_knopp(H: torch.Tensor, iters: int = 20, eps: float = 1e-5) -> torch.Tensor:
    """reference.py:20-48 (also batched over leading axes)."""
    P = H.to(torch.float32) if H.dtype not in (torch.float32, torch.float64) else H
    for _ in range(int(iters)):
        row_sum = P.sum(dim=-1)
        row_scale = torch.where(row_sum > eps, 1.0 / row_sum, torch.ones_like(row_sum))
        P = P * row_scale.unsqueeze(-1)
        col_sum = P.sum(dim=-2)
        col_scale = torch.where(col_sum > eps, 1.0 / col_sum, torch.zeros_like(col_sum))
        P = P * col_scale.unsqueeze(-2)
    return P


def activate_pre_post(H_pre_raw: torch.Tensor, H_post_raw: torch.Tensor):
    """reference.py:51-55."""
    f = lambda t: t.to(torch.float32) if t.dtype not in (torch.float32, torch.float64) else t
    return torch.sigmoid(f(H_pre_raw)), 2.0 * torch.sigmoid(f(H_post_raw))


def mixing_matrix_from_logits(H_res_raw: torch.Tensor, iters: int = 20, eps: float = 1e-5) -> torch.Tensor:
    """reference.py:58-69 (a leading per-token batch axis is this build's extension)."""
    if H_res_raw.ndim < 2 or H_res_raw.shape[-1] != H_res_raw.shape[-2]:
        raise ValueError(f"H_res_raw must be square [n, n], got shape {tuple(H_res_raw.shape)}")
    H = H_res_raw if H_res_raw.dtype in (torch.float32, torch.float64) else H_res_raw.to(torch.float32)
    H_shifted = H - torch.amax(H, dim=-1, keepdim=True)
    return sinkhorn_knopp(torch.exp(H_shifted), iters=iters, eps=eps)


def _up(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype in (torch.float32, torch.float64) else t.to(torch.float32)


def stream_aggregate(x_expanded: torch.Tensor, H_pre: torch.Tensor) -> torch.Tensor:
    """reference.py:72-86: y[b, c] = sum_i H_pre[i] x[b, i, c]."""
    x = _up(x_expanded)
    w = _up(H_pre)
    w3 = w[None, :, None] if w.ndim == 1 else w[:, :, None]
    return (x * w3).sum(dim=1)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """reference.py:89-105."""
    x_f = _up(x)
    w_f = _up(weight)
    mean_sq = (x_f * x_f).mean(dim=-1, keepdim=True)
    inv_rms = 1.0 / torch.sqrt(mean_sq + eps)
    return (x_f * inv_rms) * w_f[None, :]


def stream_distribute(y_norm: torch.Tensor, H_post: torch.Tensor) -> torch.Tensor:
    """reference.py:108-122."""
    y = _up(y_norm)
    w = _up(H_post)
    w3 = w[None, :, None] if w.ndim == 1 else w[:, :, None]
    return y[:, None, :] * w3


def stream_mix_ref(x_expanded: torch.Tensor, M: torch.Tensor) -> torch.Tensor:
    """reference.py:125-145: x_mixed[b, i, c] = sum_j M[i, j] x[b, j, c]."""
    x = _up(x_expanded)
    M_f = _up(M)
    if M_f.ndim == 2:
        return (M_f[None, :, :, None] * x[:, None, :, :]).sum(dim=2)
    return (M_f[:, :, :, None] * x[:, None, :, :]).sum(dim=2)


def mhc_forward_fused_reference(x_expanded, M, H_pre_act, H_post_act, rms_weight, eps: float = 1e-5):
    """reference.py:148-161."""
    y_agg = stream_aggregate(x_expanded, H_pre_act)
    y_norm = rms_norm(y_agg, rms_weight, eps=eps)
    y_dist = stream_distribute(y_norm, H_post_act)
    x_mixed = stream_mix_ref(x_expanded, M)
    return x_mixed + y_dist


def mhc_forward_reference(x_expanded, H_pre_raw, H_post_raw, H_res_raw, rms_weight, sinkhorn_iters: int = 20,
                          eps: float = 1e-5):
    """reference.py:164-184."""
    H_pre_act, H_post_act = activate_pre_post(H_pre_raw, H_post_raw)
    M = mixing_matrix_from_logits(H_res_raw, iters=sinkhorn_iters, eps=eps)
    y_agg = stream_aggregate(x_expanded, H_pre_act)
    y_norm = rms_norm(y_agg, rms_weight, eps=eps)
    y_dist = stream_distribute(y_norm, H_post_act)
    x_mixed = stream_mix_ref(x_expanded, M)
    return x_mixed + y_dist

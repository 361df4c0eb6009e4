"""CPU oracle for the mHC hot path (test infrastructure only).

THIS MODULE IS A CHECKER, NOT PRODUCT CODE.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The HIP library never calls into it and the package
``mhc_mlx_amd`` never imports it.

It restates, in numpy, the pure-MLX reference of svdrecbd/mhc-mlx
(``mhc_mlx/reference.py``) op for op, plus the backward that MLX autograd
derives from it (the reference has no hand-written backward for this path
other than its Metal VJPs, whose contract is ``mhc_mlx/metal.py:2787-2857``).

Precision: every function takes ``dtype``.  ``np.float64`` (default) is the
parity oracle; ``np.float32`` mimics the reference's own fp32 arithmetic
(bf16/fp16 inputs are upcast to fp32 exactly as ``reference.py:84,101`` do)
and is what the CPU baseline times.

Pinning (each function's independent checks live in ``tests/test_oracle_*.py``):

* ``sinkhorn_knopp`` / ``mixing_matrix_from_logits``: pure-Python scalar
  loop restatement (brute force on tiny n), closed forms (rank-1 logits give
  1/n after one iteration, constant logits give 1/n, the 2x2 limit
  sqrt(ad)/(sqrt(ad)+sqrt(bc)), row-shift invariance, unit column sums,
  doubly-stochastic fixed point, identity init -> I).
* ``sinkhorn_knopp_vjp``: torch.autograd (float64) of an independent torch
  restatement, central finite differences, zero row sums of dH (row-shift
  invariance) and dM = 1 c^T -> dH = 0.
* forward composition: pure-Python loops on tiny shapes, identity init
  gives out ~= x, linearity of the mix term, M = I / H_post -> 0 gives x.
* ``mhc_fused_backward`` / ``mhc_backward_reference``: torch.autograd
  (float64) and central finite differences.
* ``post_combine`` (+ backward): explicit (non-folded) formulation, the
  weight-folding equivalence of ``tests/test_folding.py:6-39`` and
  torch.autograd.
* ``residual_add_agg`` (+ backward): pure-Python loops on tiny shapes,
  res = 0 reduces y_agg to ``stream_aggregate``, symmetry in (x, res), a
  one-hot H_pre selects one stream; torch.autograd (float64) and central
  finite differences for the backward.

No function here is "parity unpinned".  The reference itself cannot be
imported in this container (it needs MLX, which is absent), so bitwise MLX
behaviour (reduction order, exp/sigmoid ulps) is out of reach; the contract
is the tolerance of the reference tests (fp32 1e-5, bf16 2e-2).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_round",
    "f16_round",
    "sigmoid",
    "activate_pre_post",
    "sinkhorn_knopp",
    "mixing_matrix_from_logits",
    "sinkhorn_knopp_vjp",
    "stream_aggregate",
    "rms_norm",
    "stream_distribute",
    "stream_mix_ref",
    "mhc_forward_fused_reference",
    "mhc_forward_reference",
    "mhc_fused_backward",
    "mhc_backward_reference",
    "post_combine",
    "post_combine_backward",
    "ds_residual",
    "rewire_linear_forward",
    "rewire_linear_backward",
    "residual_add_agg",
    "residual_add_agg_backward",
]


# --------------------------------------------------------------------------
# dtype helpers
# --------------------------------------------------------------------------

def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), returned as float32.

    Mirrors ``x.astype(mx.bfloat16)`` in the reference (MLX rounds RNE).
    NaN stays NaN; infinities stay infinite.
    """
    f = np.ascontiguousarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    out = np.where(nan, np.float32(np.nan), out)
    return out.reshape(np.shape(a))


def f16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to float16 (RNE), returned as float32."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def sigmoid(z: np.ndarray, dtype=np.float64) -> np.ndarray:
    z = np.asarray(z, dtype=dtype)
    return (1.0 / (1.0 + np.exp(-z))).astype(dtype)


# --------------------------------------------------------------------------
# forward (reference.py restated)
# --------------------------------------------------------------------------

def activate_pre_post(H_pre_raw, H_post_raw, dtype=np.float64):
    """reference.py:51-55: H_pre = sigmoid(raw), H_post = 2*sigmoid(raw)."""
    H_pre_act = sigmoid(H_pre_raw, dtype)
    H_post_act = (2.0 * sigmoid(H_post_raw, dtype)).astype(dtype)
    return H_pre_act, H_post_act


def sinkhorn_knopp(H, iters: int = 20, eps: float = 1e-5, dtype=np.float64):
    """reference.py:20-48, batched over leading axes ([..., n, n]).

    Row step: s = sum_j P_ij; P_ij *= (s > eps ? 1/s : 1).
    Col step: s = sum_i P_ij; P_ij *= (s > eps ? 1/s : 0).
    The scale is formed as a reciprocal and then multiplied, as the reference
    does (reference.py:39-46).
    """
    P = np.array(H, dtype=dtype, copy=True)
    one = dtype(1.0)
    for _ in range(int(iters)):
        row_sum = P.sum(axis=-1)
        with np.errstate(divide="ignore"):
            row_scale = np.where(row_sum > eps, one / row_sum, one).astype(dtype)
        P = P * row_scale[..., :, None]
        col_sum = P.sum(axis=-2)
        with np.errstate(divide="ignore"):
            col_scale = np.where(col_sum > eps, one / col_sum, dtype(0.0)).astype(dtype)
        P = P * col_scale[..., None, :]
    return P


def mixing_matrix_from_logits(H_res_raw, iters: int = 20, eps: float = 1e-5, dtype=np.float64):
    """reference.py:58-69: M = sinkhorn_knopp(exp(H - rowmax(H))).

    The reference accepts only a square 2-D matrix and raises ValueError
    otherwise (reference.py:64-65); a leading batch axis ([B, n, n], one
    matrix per token) is this build's extension and is accepted here.
    """
    H = np.asarray(H_res_raw)
    if H.ndim < 2 or H.shape[-1] != H.shape[-2]:
        raise ValueError(f"H_res_raw must be square [n, n], got shape {H.shape}")
    Hd = H.astype(dtype)
    shifted = Hd - Hd.max(axis=-1, keepdims=True)
    K = np.exp(shifted).astype(dtype)
    return sinkhorn_knopp(K, iters=iters, eps=eps, dtype=dtype)


def stream_aggregate(x, H_pre, dtype=np.float64):
    """reference.py:72-86: y[b, c] = sum_i H_pre[i] x[b, i, c] (H_pre may be [B, n])."""
    xf = np.asarray(x, dtype=dtype)
    w = np.asarray(H_pre, dtype=dtype)
    if w.ndim == 1:
        return (xf * w[None, :, None]).sum(axis=1)
    return (xf * w[:, :, None]).sum(axis=1)


def rms_norm(y, weight, eps: float = 1e-5, dtype=np.float64, return_inv: bool = False):
    """reference.py:89-105: y * (1/sqrt(mean(y^2) + eps)) * w."""
    yf = np.asarray(y, dtype=dtype)
    wf = np.asarray(weight, dtype=dtype)
    mean_sq = (yf * yf).mean(axis=-1, keepdims=True)
    inv = (dtype(1.0) / np.sqrt(mean_sq + dtype(eps))).astype(dtype)
    out = (yf * inv) * wf[None, :]
    if return_inv:
        return out, inv[..., 0]
    return out


def stream_distribute(y_norm, H_post, dtype=np.float64):
    """reference.py:108-122: y_dist[b, i, c] = H_post[i] y_norm[b, c]."""
    y = np.asarray(y_norm, dtype=dtype)
    w = np.asarray(H_post, dtype=dtype)
    if w.ndim == 1:
        return y[:, None, :] * w[None, :, None]
    return y[:, None, :] * w[:, :, None]


def stream_mix_ref(x, M, dtype=np.float64):
    """reference.py:125-145: x_mixed[b, i, c] = sum_j M[i, j] x[b, j, c]."""
    xf = np.asarray(x, dtype=dtype)
    Mf = np.asarray(M, dtype=dtype)
    if Mf.ndim == 2:
        return np.einsum("ij,bjc->bic", Mf, xf)
    return np.einsum("bij,bjc->bic", Mf, xf)


def mhc_forward_fused_reference(x, M, H_pre_act, H_post_act, rms_weight, eps=1e-5, dtype=np.float64):
    """reference.py:148-161."""
    y_agg = stream_aggregate(x, H_pre_act, dtype)
    y_norm = rms_norm(y_agg, rms_weight, eps=eps, dtype=dtype)
    y_dist = stream_distribute(y_norm, H_post_act, dtype)
    x_mixed = stream_mix_ref(x, M, dtype)
    return x_mixed + y_dist


def mhc_forward_reference(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight,
                          sinkhorn_iters: int = 20, eps: float = 1e-5, dtype=np.float64):
    """reference.py:164-184 (static [n] / [n, n] params, or per-token [B, n] / [B, n, n])."""
    H_pre_act, H_post_act = activate_pre_post(H_pre_raw, H_post_raw, dtype)
    M = mixing_matrix_from_logits(H_res_raw, iters=sinkhorn_iters, eps=eps, dtype=dtype)
    return mhc_forward_fused_reference(x, M, H_pre_act, H_post_act, rms_weight, eps, dtype)


def ds_residual(M) -> float:
    """max(|rowsum - 1|, |colsum - 1|) over all matrices in M ([..., n, n])."""
    M = np.asarray(M, dtype=np.float64)
    r = np.abs(M.sum(axis=-1) - 1.0).max()
    c = np.abs(M.sum(axis=-2) - 1.0).max()
    return float(max(r, c))


# --------------------------------------------------------------------------
# backward
# --------------------------------------------------------------------------

def sinkhorn_knopp_vjp(H_res_raw, dM, iters: int = 20, eps: float = 1e-5, dtype=np.float64):
    """Reverse-mode derivative of mixing_matrix_from_logits (reference.py:20-48, 58-69).

    This is what MLX autograd computes for the reference graph (and what the
    Metal VJP ``sinkhorn_knopp_backward.metal`` approximates):

    * row step with scale r = 1/s (unmasked):  dP_in = r*g - r^2 * sum_j(g*P_in)
      masked row (scale 1, constant):          dP_in = g
    * col step with scale c = 1/s (unmasked):  dP_in = c*g - c^2 * sum_i(g*P_in)
      masked col (scale 0, constant):          dP_in = 0
    * exp:  dH_shift = dK * K
    * rowmax shift: the max gradient -sum_j dH_shift[r, j] is shared evenly
      among the maximal entries of row r (torch.amax semantics).  This term is
      zero in exact arithmetic (the first row step cancels any row scaling).
    """
    H = np.asarray(H_res_raw, dtype=dtype)
    G = np.array(dM, dtype=dtype, copy=True)
    mx_ = H.max(axis=-1, keepdims=True)
    K = np.exp(H - mx_).astype(dtype)
    one = dtype(1.0)
    # forward, storing every intermediate
    states = []
    P = K.copy()
    for _ in range(int(iters)):
        rs = P.sum(axis=-1)
        rmask = rs > eps
        with np.errstate(divide="ignore"):
            rscale = np.where(rmask, one / rs, one).astype(dtype)
        P_row_in = P
        P = P * rscale[..., :, None]
        cs = P.sum(axis=-2)
        cmask = cs > eps
        with np.errstate(divide="ignore"):
            cscale = np.where(cmask, one / cs, dtype(0.0)).astype(dtype)
        P_col_in = P
        P = P * cscale[..., None, :]
        states.append((P_row_in, rscale, rmask, P_col_in, cscale, cmask))
    for P_row_in, rscale, rmask, P_col_in, cscale, cmask in reversed(states):
        # col step
        dot = (G * P_col_in).sum(axis=-2)  # [..., n] per column
        Gc = cscale[..., None, :] * G - (cscale * cscale * dot)[..., None, :]
        G = np.where(cmask[..., None, :], Gc, dtype(0.0))
        # row step
        dot = (G * P_row_in).sum(axis=-1)  # [..., n] per row
        Gr = rscale[..., :, None] * G - (rscale * rscale * dot)[..., :, None]
        G = np.where(rmask[..., :, None], Gr, G)
    dshift = G * K
    is_max = (H == mx_)
    cnt = is_max.sum(axis=-1, keepdims=True)
    dH = dshift - is_max * (dshift.sum(axis=-1, keepdims=True) / cnt)
    return dH.astype(dtype)


def mhc_fused_backward(x, M, H_pre_act, H_post_act, rms_weight, dout, eps=1e-5, dtype=np.float64):
    """VJP of mhc_forward_fused_reference, in the contract of metal.py:2787-2857.

    Returns (dx, dM, dH_pre_act, dH_post_act, d_rms_weight): gradients with
    respect to the *activated* H_pre/H_post (metal.py:2857).  For per-token
    params ([B, n] / [B, n, n]) dM/dH_pre/dH_post are per token; d_rms_weight
    is always summed over tokens.

    With g = dout, y = sum_i a_i x_i, inv = 1/sqrt(mean(y^2)+eps):
      dyn  = sum_i p_i g_i            d_r = sum_c dyn * y * w
      dy   = dyn*inv*w - (inv^3/C) * d_r * y
      dx_j = sum_i M_ij g_i + a_j dy
      dM_ij = sum g_i x_j   dA_j = sum dy x_j   dP_i = sum g_i y inv w
      dw    = sum_t dyn * y * inv
    """
    xf = np.asarray(x, dtype=dtype)
    g = np.asarray(dout, dtype=dtype)
    Mf = np.asarray(M, dtype=dtype)
    a = np.asarray(H_pre_act, dtype=dtype)
    p = np.asarray(H_post_act, dtype=dtype)
    w = np.asarray(rms_weight, dtype=dtype)
    B, n, C = xf.shape
    per_token = a.ndim == 2
    a3 = a[:, :, None] if per_token else a[None, :, None]
    p3 = p[:, :, None] if per_token else p[None, :, None]
    y = (xf * a3).sum(axis=1)                                   # [B, C]
    inv = dtype(1.0) / np.sqrt((y * y).mean(axis=-1) + dtype(eps))  # [B]
    dyn = (g * p3).sum(axis=1)                                  # [B, C]
    d_r = (dyn * y * w[None, :]).sum(axis=-1)                   # [B]
    dy = dyn * inv[:, None] * w[None, :] - ((inv ** 3) / C * d_r)[:, None] * y
    if Mf.ndim == 2:
        dx = np.einsum("ij,bic->bjc", Mf, g)
        dM = np.einsum("bic,bjc->ij", g, xf)
    else:
        dx = np.einsum("bij,bic->bjc", Mf, g)
        dM = np.einsum("bic,bjc->bij", g, xf)
    dx = dx + a3 * dy[:, None, :]
    y_norm = y * inv[:, None] * w[None, :]
    if per_token:
        dA = np.einsum("bc,bjc->bj", dy, xf)
        dP = np.einsum("bic,bc->bi", g, y_norm)
    else:
        dA = np.einsum("bc,bjc->j", dy, xf)
        dP = np.einsum("bic,bc->i", g, y_norm)
    dw = (dyn * y * inv[:, None]).sum(axis=0)
    return dx, dM, dA, dP, dw


def mhc_backward_reference(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, dout,
                           sinkhorn_iters: int = 20, eps: float = 1e-5, dtype=np.float64):
    """Full VJP of mhc_forward_reference w.r.t. (x, H_pre_raw, H_post_raw, H_res_raw, rms_weight).

    Chains mhc_fused_backward through the activations of reference.py:53-54
    (d sigmoid = s(1-s); d 2*sigmoid = 2 s(1-s)) and the Sinkhorn VJP.
    """
    H_pre_act, H_post_act = activate_pre_post(H_pre_raw, H_post_raw, dtype)
    M = mixing_matrix_from_logits(H_res_raw, iters=sinkhorn_iters, eps=eps, dtype=dtype)
    dx, dM, dA, dP, dw = mhc_fused_backward(x, M, H_pre_act, H_post_act, rms_weight, dout, eps, dtype)
    s_pre = sigmoid(H_pre_raw, dtype)
    s_post = sigmoid(H_post_raw, dtype)
    dH_pre_raw = dA * s_pre * (1.0 - s_pre)
    dH_post_raw = dP * 2.0 * s_post * (1.0 - s_post)
    dH_res_raw = sinkhorn_knopp_vjp(H_res_raw, dM, iters=sinkhorn_iters, eps=eps, dtype=dtype)
    return dx, dH_pre_raw, dH_post_raw, dH_res_raw, dw


# --------------------------------------------------------------------------
# MHCRewire post-combine (layer.py:302-337, 469-492)
# --------------------------------------------------------------------------

def post_combine(x, y_inner, H_pre_raw, H_post_raw, H_res_raw, sinkhorn_iters=20, eps=1e-5,
                 dtype=np.float64):
    """layer.py:332-337: out = (y_inner + (M diag(H_pre)) x) * H_post, per stream.

    x, y_inner: [B, n, C].
    """
    a, p = activate_pre_post(H_pre_raw, H_post_raw, dtype)
    M = mixing_matrix_from_logits(H_res_raw, iters=sinkhorn_iters, eps=eps, dtype=dtype)
    Mf = M * a[None, :]
    xf = np.asarray(x, dtype=dtype)
    yf = np.asarray(y_inner, dtype=dtype)
    x_mixed = np.einsum("ij,bjc->bic", Mf, xf)
    return (yf + x_mixed) * p[None, :, None]


def post_combine_backward(x, y_inner, H_pre_raw, H_post_raw, H_res_raw, dout,
                          sinkhorn_iters=20, eps=1e-5, dtype=np.float64):
    """VJP of post_combine w.r.t. (x, y_inner, H_pre_raw, H_post_raw, H_res_raw).

    With S_ij = sum g_i x_j, Mf = M diag(a):
      dy_inner_i = p_i g_i
      dx_j = sum_i p_i Mf_ij g_i
      dM_ij = p_i S_ij a_j
      da_j  = sum_i p_i M_ij S_ij
      dp_i  = sum_j Mf_ij S_ij + sum g_i y_i
    """
    a, p = activate_pre_post(H_pre_raw, H_post_raw, dtype)
    M = mixing_matrix_from_logits(H_res_raw, iters=sinkhorn_iters, eps=eps, dtype=dtype)
    xf = np.asarray(x, dtype=dtype)
    yf = np.asarray(y_inner, dtype=dtype)
    g = np.asarray(dout, dtype=dtype)
    Mf = M * a[None, :]
    S = np.einsum("bic,bjc->ij", g, xf)
    Y = np.einsum("bic,bic->i", g, yf)
    dy_inner = g * p[None, :, None]
    dx = np.einsum("ij,bic->bjc", Mf * p[:, None], g)
    dM = p[:, None] * S * a[None, :]
    da = (p[:, None] * M * S).sum(axis=0)
    dp = (Mf * S).sum(axis=1) + Y
    s_pre = sigmoid(H_pre_raw, dtype)
    s_post = sigmoid(H_post_raw, dtype)
    dH_pre_raw = da * s_pre * (1.0 - s_pre)
    dH_post_raw = dp * 2.0 * s_post * (1.0 - s_post)
    dH_res_raw = sinkhorn_knopp_vjp(H_res_raw, dM, iters=sinkhorn_iters, eps=eps, dtype=dtype)
    return dx, dy_inner, dH_pre_raw, dH_post_raw, dH_res_raw


def rewire_linear_forward(x, W, H_pre_raw, H_post_raw, H_res_raw, sinkhorn_iters=20, eps=1e-5,
                          dtype=np.float64):
    """MHCRewire(Linear(dims, dims, bias=False)) forward, layer.py:469-492.

    x: [T, dims] with dims = n*C (stream i is channels [i*C, (i+1)*C)).
    W: [dims, dims] (torch/MLX Linear convention: y = x W^T).
    Returns (out [T, dims], y_inner [T, dims]).
    """
    n = np.asarray(H_pre_raw).shape[0]
    xf = np.asarray(x, dtype=dtype)
    T, dims = xf.shape
    C = dims // n
    a, _ = activate_pre_post(H_pre_raw, H_post_raw, dtype)
    x3 = xf.reshape(T, n, C)
    x_pre = (x3 * a[None, :, None]).reshape(T, dims)
    y_inner = x_pre @ np.asarray(W, dtype=dtype).T
    out = post_combine(x3, y_inner.reshape(T, n, C), H_pre_raw, H_post_raw, H_res_raw,
                       sinkhorn_iters, eps, dtype)
    return out.reshape(T, dims), y_inner


def rewire_linear_backward(x, W, H_pre_raw, H_post_raw, H_res_raw, dout, sinkhorn_iters=20,
                           eps=1e-5, dtype=np.float64):
    """VJP of rewire_linear_forward w.r.t. (x, W, H_pre_raw, H_post_raw, H_res_raw)."""
    n = np.asarray(H_pre_raw).shape[0]
    xf = np.asarray(x, dtype=dtype)
    Wf = np.asarray(W, dtype=dtype)
    T, dims = xf.shape
    C = dims // n
    a, _ = activate_pre_post(H_pre_raw, H_post_raw, dtype)
    x3 = xf.reshape(T, n, C)
    x_pre = (x3 * a[None, :, None]).reshape(T, dims)
    y_inner = x_pre @ Wf.T
    g3 = np.asarray(dout, dtype=dtype).reshape(T, n, C)
    dx3, dy3, dpre, dpost, dres = post_combine_backward(
        x3, y_inner.reshape(T, n, C), H_pre_raw, H_post_raw, H_res_raw, g3,
        sinkhorn_iters, eps, dtype)
    dy = dy3.reshape(T, dims)
    dW = dy.T @ x_pre
    dx_pre3 = (dy @ Wf).reshape(T, n, C)
    dx3 = dx3 + dx_pre3 * a[None, :, None]
    s_pre = sigmoid(H_pre_raw, dtype)
    dpre = dpre + np.einsum("bjc,bjc->j", dx_pre3, x3) * s_pre * (1.0 - s_pre)
    return dx3.reshape(T, dims), dW, dpre, dpost, dres


# --------------------------------------------------------------------------
# residual add + aggregate
# --------------------------------------------------------------------------

def residual_add_agg(x, res, H_pre, dtype=np.float64):
    """utils.py:4-24 / residual_add_agg.metal:39-66: (out, y_agg).

    out[b, i, c] = x + res; y_agg[b, c] = sum_i H_pre[i] * out[b, i, c], with
    y_agg taken from the sum before out is rounded to its output dtype
    (the kernel aggregates the fp32 ``val``, residual_add_agg.metal:55-62).
    H_pre is used as given (no activation).
    """
    val = np.asarray(x, dtype=dtype) + np.asarray(res, dtype=dtype)
    w = np.asarray(H_pre, dtype=dtype)
    y_agg = (val * w[None, :, None]).sum(axis=1)
    return val, y_agg


def residual_add_agg_backward(x, res, H_pre, dout=None, dy_agg=None, dtype=np.float64):
    """VJP of residual_add_agg: (dx, dres, dH_pre); dout / dy_agg of None count as zero."""
    val = np.asarray(x, dtype=dtype) + np.asarray(res, dtype=dtype)
    w = np.asarray(H_pre, dtype=dtype)
    d = np.zeros_like(val) if dout is None else np.asarray(dout, dtype=dtype).copy()
    if dy_agg is None:
        dH = np.zeros(val.shape[1], dtype=dtype)
    else:
        dy = np.asarray(dy_agg, dtype=dtype)
        d = d + w[None, :, None] * dy[:, None, :]
        dH = np.einsum("bc,bic->i", dy, val)
    return d, d.copy(), dH

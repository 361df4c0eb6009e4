"""Accelerated mHC ops: torch.autograd.Functions over libmhc_hip.

Op-level API (the reference's mhc_mlx/metal.py surface, same argument
meaning, same ValueError texts where the reference has them):

* ``sinkhorn_knopp_hip`` / ``sinkhorn_knopp_hip_autograd``
  (metal.py:1525-1577, 2712-2758)
* ``mhc_forward_fused_hip`` / ``mhc_forward_fused_hip_autograd``
  (metal.py:1823-1975, 2761-2900); the VJP returns gradients w.r.t. the
  *activated* H_pre / H_post (metal.py:2857)
* ``stream_mix_add_hip`` / ``stream_mix_add_hip_autograd`` (metal.py:954-1014,
  2661-2709)

Layer-level fused functions (raw logits in, every activation, the Sinkhorn
projection and its VJP inside the library): ``mhc_layer_forward``,
``mhc_layer_forward_dynamic`` (per-token parameters), ``post_combine`` and
``stream_scale`` (MHCRewire, layer.py:302-337, 469-492).

Block helper: ``residual_add_agg_hip`` (metal.py:1673-1731, utils.py:4-24),
differentiable here although the reference's kernel is not.

All work is enqueued on torch's current stream of the input's device.  Every
op requires GPU tensors and the built library; there is no silent fallback.
"""

from __future__ import annotations

import ctypes

import torch

from . import _ext, _lib, profiling
from .profiling import timed

__all__ = [
    "sinkhorn_knopp_hip",
    "sinkhorn_knopp_hip_autograd",
    "mhc_forward_fused_hip",
    "mhc_forward_fused_hip_autograd",
    "stream_mix_add_hip",
    "stream_mix_add_hip_autograd",
    "mhc_layer_forward",
    "mhc_layer_forward_dynamic",
    "post_combine",
    "stream_scale",
    "stream_scale_and_pass",
    "residual_add_agg_hip",
    "suggest_threads_per_group",
]

_MAX_N_ALLOWED = _lib.MAX_N
_MAX_TPG_ALLOWED = 1024

_DTYPE_CODE = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}


# --------------------------------------------------------------------------
# helpers
# --------------------------------------------------------------------------

def _code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}; expected float32, bfloat16 or float16") from None


def _p(t):
    """Device pointer of t as an int (ctypes converts it for the c_void_p argtypes), or None."""
    return t.data_ptr() if t is not None else None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor):
    """hipStream_t of torch's current stream on t's device (as an int)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError(
                "the HIP path needs GPU tensors (got a tensor on %s); move the inputs and the "
                "module to the GPU or construct the layer with use_metal=False" % t.device
            )


def _f32(t: torch.Tensor) -> torch.Tensor:
    """t as contiguous fp32 (t itself when it already is: only its pointer is passed on)."""
    if t.dtype is torch.float32 and t.is_contiguous():
        return t
    return t.detach().to(torch.float32).contiguous()


def _needs_grad(*ts) -> bool:
    if not torch.is_grad_enabled():
        return False
    return any(t is not None and t.requires_grad for t in ts)


_BINDING = None


def _binding():
    """The torch binding (_mhc_torch.so): MHCLayer's forward / backward in C++ over the same C ABI."""
    global _BINDING
    if _BINDING is None:
        _BINDING = _ext.load()
    return _BINDING


def _ws(nbytes: int, dev) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=dev)


def _validate_n(n: int) -> int:
    """metal.py:827-834."""
    if n <= 0:
        raise ValueError("n must be positive")
    if n > _MAX_N_ALLOWED:
        raise ValueError(f"n={n} exceeds MAX_N_ALLOWED={_MAX_N_ALLOWED}. Increase _MAX_N_ALLOWED if needed.")
    return int(n)


def _validate_tpg(tpg) -> None:
    if tpg is None:
        return
    if tpg <= 0:
        raise ValueError("threads_per_group must be positive")
    if tpg > _MAX_TPG_ALLOWED:
        raise ValueError(f"threads_per_group must be <= {_MAX_TPG_ALLOWED}")


def suggest_threads_per_group(C: int, max_tpg: int = _MAX_TPG_ALLOWED) -> int:
    """metal.py:942-951 (kept for API parity; launch shapes are chosen by the library)."""
    if C <= 0:
        raise ValueError("C must be positive")
    if max_tpg <= 0:
        raise ValueError("max_tpg must be positive")
    tpg = 1 << (int(C) - 1).bit_length()
    return int(min(tpg, max_tpg))


def _normalize_output_dtype(output_dtype, x_dtype):
    """metal.py:862-867, 1170-1200: None/float32 -> fp32; half types must match x."""
    if output_dtype is None or output_dtype == torch.float32:
        return torch.float32
    if output_dtype in (torch.float16, torch.bfloat16):
        if x_dtype != output_dtype:
            name = "float16" if output_dtype == torch.float16 else "bfloat16"
            raise ValueError(f"x must be {name} when output_dtype is {name}")
        return output_dtype
    raise ValueError(f"unsupported output_dtype: {output_dtype}")


def _normalize_mix_kernel(mix_kernel: str) -> str:
    key = (mix_kernel or "auto").strip().lower()
    if key in {"auto", "1d", "2d", "col"}:
        return key
    raise ValueError(f"unsupported mix_kernel: {mix_kernel}")


# --------------------------------------------------------------------------
# Sinkhorn-Knopp
# --------------------------------------------------------------------------

def _sk_shape(H: torch.Tensor) -> tuple[int, int]:
    if H.ndim == 2:
        if H.shape[0] != H.shape[1]:
            raise ValueError(f"H_res_raw must be square [n, n], got shape {tuple(H.shape)}")
        return 1, int(H.shape[0])
    if H.ndim == 3 and H.shape[1] == H.shape[2]:
        return int(H.shape[0]), int(H.shape[1])
    raise ValueError(f"H_res_raw must be square [n, n], got shape {tuple(H.shape)}")


def _sinkhorn_fwd(H: torch.Tensor, iters: int, eps: float, state: torch.Tensor | None = None) -> torch.Tensor:
    """M = SK(exp(H)); with `state`, the forward also records its VJP state there."""
    batch, n = _sk_shape(H)
    _validate_n(n)
    Hf = _f32(H)
    M = torch.empty_like(Hf)
    with timed("sinkhorn_fwd"):
        if state is None:
            _lib.call("mhc_sinkhorn_fwd", _p(Hf), _p(M), batch, n, int(iters), float(eps), _stream(Hf))
        else:
            _lib.call("mhc_sinkhorn_fwd_record", _p(Hf), _p(M), _p(state), state.numel(), batch, n, int(iters),
                      float(eps), _stream(Hf))
    return M


def _sinkhorn_bwd(H: torch.Tensor, dM: torch.Tensor, iters: int, eps: float,
                  state: torch.Tensor | None = None) -> torch.Tensor:
    """dH of <dM, SK(exp(H))>, from a recorded state when one is given."""
    batch, n = _sk_shape(H)
    Hf = _f32(H)
    dMf = _f32(dM)
    dH = torch.empty_like(Hf)
    if state is not None:
        with timed("sinkhorn_bwd"):
            _lib.call("mhc_sinkhorn_bwd_recorded", _p(Hf), _p(dMf), _p(dH), _p(state), state.numel(), batch, n,
                      int(iters), float(eps), _stream(Hf))
        return dH
    nb = _lib.query("mhc_sinkhorn_bwd_workspace_bytes", batch, n, int(iters))
    ws = _ws(nb, Hf.device)
    with timed("sinkhorn_bwd"):
        _lib.call("mhc_sinkhorn_bwd", _p(Hf), _p(dMf), _p(dH), batch, n, int(iters), float(eps),
                  _p(ws), nb, _stream(Hf))
    return dH


def _sk_record_buffer(H: torch.Tensor, batch: int, n: int, iters: int) -> torch.Tensor | None:
    """A buffer for the Sinkhorn forward to record its VJP state in, or None.

    The library records for n = 16 (16-byte aligned logits) and 16 < n <= 64,
    unless the knob MHC_SK16_RECORD / MHC_SK_BLK_RECORD is 0; the backward
    then reads the state instead of recomputing the forward iterations.
    """
    if batch <= 0 or (n == 16 and _f32(H).data_ptr() % 16 != 0):
        return None
    nb = _sk_state_bytes(batch, n, iters)
    return torch.empty(nb, dtype=torch.uint8, device=H.device) if nb > 0 else None


class SinkhornFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, H_res_raw, iters, eps):
        state = None
        if ctx.needs_input_grad[0]:
            batch, n = _sk_shape(H_res_raw)
            state = _sk_record_buffer(H_res_raw, batch, n, iters)
        ctx.save_for_backward(H_res_raw, state)
        ctx.iters, ctx.eps = iters, eps
        return _sinkhorn_fwd(H_res_raw, iters, eps, state)

    @staticmethod
    def backward(ctx, dM):
        H, state = ctx.saved_tensors
        return _sinkhorn_bwd(H, dM, ctx.iters, ctx.eps, state).to(H.dtype), None, None


def sinkhorn_knopp_hip(H_res_raw, iters: int = 20, eps: float = 1e-5, threads_per_group=None,
                       verbose: bool = False) -> torch.Tensor:
    """M = sinkhorn_knopp(exp(H_res_raw)) ([n, n], or [B, n, n] per token). No autograd."""
    _validate_tpg(threads_per_group)
    _require_gpu(H_res_raw)
    _sk_shape(H_res_raw)
    with torch.no_grad():
        return _sinkhorn_fwd(H_res_raw, iters, eps)


def sinkhorn_knopp_hip_autograd(H_res_raw, iters: int = 20, eps: float = 1e-5, threads_per_group=None,
                                verbose: bool = False) -> torch.Tensor:
    """Sinkhorn with the HIP VJP through all `iters` iterations (metal.py:2744)."""
    _validate_tpg(threads_per_group)
    _require_gpu(H_res_raw)
    _sk_shape(H_res_raw)
    return SinkhornFn.apply(H_res_raw, int(iters), float(eps))


# --------------------------------------------------------------------------
# fused forward / backward
# --------------------------------------------------------------------------

def _fused_shapes(x, M, H_pre, H_post, rms_weight):
    """metal.py:1848-1873 checks (plus the per-token extension)."""
    if x.ndim != 3:
        raise ValueError(f"x must be [B, n, C], got shape {tuple(x.shape)}")
    B, n, C = (int(s) for s in x.shape)
    per_token = M.ndim == 3
    if M.ndim not in (2, 3):
        raise ValueError(f"M must be [n, n], got shape {tuple(M.shape)}")
    if H_pre.ndim != (2 if per_token else 1):
        raise ValueError(f"H_pre must be [n], got shape {tuple(H_pre.shape)}")
    if H_post.ndim != (2 if per_token else 1):
        raise ValueError(f"H_post must be [n], got shape {tuple(H_post.shape)}")
    if rms_weight.ndim != 1:
        raise ValueError(f"rms_weight must be [C], got shape {tuple(rms_weight.shape)}")
    want_M = (B, n, n) if per_token else (n, n)
    if tuple(M.shape) != want_M:
        raise ValueError(f"M must be shape (n,n)=( {n},{n} ), got {tuple(M.shape)}")
    want_h = (B, n) if per_token else (n,)
    if tuple(H_pre.shape) != want_h:
        raise ValueError(f"H_pre must be shape (n,)=( {n}, ), got {tuple(H_pre.shape)}")
    if tuple(H_post.shape) != want_h:
        raise ValueError(f"H_post must be shape (n,)=( {n}, ), got {tuple(H_post.shape)}")
    if tuple(rms_weight.shape) != (C,):
        raise ValueError(f"rms_weight must be shape (C,)=( {C}, ), got {tuple(rms_weight.shape)}")
    _validate_n(n)
    return B, n, C, per_token


def _fused_fwd(x, M, hpre, hpost, w, eps, out_dtype, h_mode, per_token):
    B, n, C = (int(s) for s in x.shape)
    xc = x.detach().contiguous()
    Mc, hp, hq, wc = _f32(M), _f32(hpre), _f32(hpost), _f32(w)
    out = torch.empty((B, n, C), dtype=out_dtype, device=x.device)
    with timed("fused_fwd"):
        _lib.call("mhc_fused_fwd", _p(xc), _code(xc.dtype), _p(Mc), n * n if per_token else 0, _p(hp),
                  _p(hq), n if per_token else 0, h_mode, _p(wc), _p(out), _code(out_dtype), None, B, n, C,
                  float(eps), _stream(xc))
    return out


def _fused_bwd(x, g, M, hpre, hpost, w, eps, h_mode, per_token):
    """Returns (dx, dM, dh_pre, dh_post, dw); per-token gradients when per_token."""
    B, n, C = (int(s) for s in x.shape)
    dev = x.device
    xc = x.detach().contiguous()
    gdt = g.dtype if g.dtype in (torch.float32, xc.dtype) else torch.float32
    gc = g.detach().to(gdt).contiguous()
    Mc, hp, hq, wc = _f32(M), _f32(hpre), _f32(hpost), _f32(w)
    dx = torch.empty_like(xc)
    if per_token:
        dM = torch.empty((B, n, n), dtype=torch.float32, device=dev)
        dpre = torch.empty((B, n), dtype=torch.float32, device=dev)
        dpost = torch.empty((B, n), dtype=torch.float32, device=dev)
    else:
        dM = torch.empty((n, n), dtype=torch.float32, device=dev)
        dpre = torch.empty((n,), dtype=torch.float32, device=dev)
        dpost = torch.empty((n,), dtype=torch.float32, device=dev)
    dw = torch.empty((C,), dtype=torch.float32, device=dev)
    nb = _lib.query("mhc_fused_bwd_workspace_bytes", B, n, C, int(per_token))
    ws = _ws(nb, dev)
    np_ = ctypes.c_int64(0)
    s = _stream(xc)
    with timed("fused_bwd"):
        _lib.call("mhc_fused_bwd_partials", _p(xc), _code(xc.dtype), _p(gc), _code(gc.dtype), _p(Mc),
                  n * n if per_token else 0, _p(hp), _p(hq), n if per_token else 0, h_mode, _p(wc),
                  _p(dx), _code(xc.dtype), _p(dM) if per_token else None,
                  _p(dpre) if per_token else None, _p(dpost) if per_token else None, _p(ws), nb, B, n,
                  C, float(eps), ctypes.byref(np_), s)
    with timed("reduce_param_grads"):
        _lib.call("mhc_reduce_param_grads", _p(ws), nb, np_.value, n, C, int(per_token), _p(hp), _p(hq),
                  h_mode, None if per_token else _p(dM), None if per_token else _p(dpre),
                  None if per_token else _p(dpost), _p(dw), s)
    return dx, dM, dpre, dpost, dw


class MHCFusedFn(torch.autograd.Function):
    """Fused forward on activated parameters; VJP as metal.py:2787-2857."""

    @staticmethod
    def forward(ctx, x, M, H_pre, H_post, rms_weight, eps, out_dtype):
        per_token = M.ndim == 3
        ctx.save_for_backward(x, M, H_pre, H_post, rms_weight)
        ctx.eps, ctx.per_token = eps, per_token
        return _fused_fwd(x, M, H_pre, H_post, rms_weight, eps, out_dtype, _lib.H_ACTIVATED, per_token)

    @staticmethod
    def backward(ctx, dout):
        x, M, H_pre, H_post, w = ctx.saved_tensors
        dx, dM, dpre, dpost, dw = _fused_bwd(x, dout, M, H_pre, H_post, w, ctx.eps, _lib.H_ACTIVATED,
                                             ctx.per_token)
        return dx, dM, dpre, dpost, dw, None, None


def mhc_forward_fused_hip(x, M, H_pre, H_post, rms_weight, eps: float = 1e-5, threads_per_group=None,
                          output_dtype=None, mix_kernel: str = "auto", verbose: bool = False):
    """Aggregate + RMSNorm + mix + H_post add (metal.py:1823). No autograd.

    Output is float32 unless output_dtype (float16/bfloat16, equal to x's dtype)
    requests the half type directly.
    """
    _fused_shapes(x, M, H_pre, H_post, rms_weight)
    _validate_tpg(threads_per_group)
    _normalize_mix_kernel(mix_kernel)
    out_dtype = _normalize_output_dtype(output_dtype, x.dtype)
    _require_gpu(x, M, H_pre, H_post, rms_weight)
    with torch.no_grad():
        return _fused_fwd(x, M, H_pre, H_post, rms_weight, eps, out_dtype, _lib.H_ACTIVATED, M.ndim == 3)


def mhc_forward_fused_hip_autograd(x, M, H_pre, H_post, rms_weight, eps: float = 1e-5,
                                   threads_per_group=None, fused_backward: bool = True,
                                   output_dtype=None, mix_kernel: str = "auto", verbose: bool = False):
    """Fused forward with the HIP backward (metal.py:2862). Grads w.r.t. activated H."""
    _fused_shapes(x, M, H_pre, H_post, rms_weight)
    _validate_tpg(threads_per_group)
    _normalize_mix_kernel(mix_kernel)
    out_dtype = _normalize_output_dtype(output_dtype, x.dtype)
    _require_gpu(x, M, H_pre, H_post, rms_weight)
    return MHCFusedFn.apply(x, M, H_pre, H_post, rms_weight, float(eps), out_dtype)


# --------------------------------------------------------------------------
# layer-level fused functions (raw logits)
# --------------------------------------------------------------------------

def _layer_fwd(x, hpre, hpost, hres, w, iters, eps, out_dtype, per_token):
    """mhc_layer_fwd: Sinkhorn projection + fused forward from raw parameters. Returns (out, M)."""
    B, n, C = x.shape
    xc = x if x.is_contiguous() else x.contiguous()
    hp, hq, hr, wc = _f32(hpre), _f32(hpost), _f32(hres), _f32(w)
    M = torch.empty_like(hr)
    out = torch.empty((B, n, C), dtype=out_dtype, device=x.device)
    s = _stream(xc)
    if profiling._active is None:
        _lib.call("mhc_layer_fwd", _p(xc), _code(xc.dtype), _p(hp), _p(hq), _p(hr), _p(wc), _p(out),
                  _code(out_dtype), _p(M), B, n, C, int(per_token), int(iters), float(eps), s)
        return out, M
    # under a kernel timer: the same two kernels, launched by separate calls
    with timed("sinkhorn_fwd"):
        _lib.call("mhc_sinkhorn_fwd", _p(hr), _p(M), B if per_token else 1, n, int(iters), float(eps), s)
    with timed("fused_fwd"):
        _lib.call("mhc_fused_fwd", _p(xc), _code(xc.dtype), _p(M), n * n if per_token else 0, _p(hp), _p(hq),
                  n if per_token else 0, _lib.H_RAW, _p(wc), _p(out), _code(out_dtype), None, B, n, C,
                  float(eps), s)
    return out, M


def layer_apply(x, hpre, hpost, hres, w, iters: int, eps: float, out_dtype):
    """MHCLayer's forward with autograd through the torch binding, with the fewest host steps.

    Layer-wide parameters with the layer's shapes; x on a GPU in fp32/bf16/fp16.  Returns None when the
    dtype is not one the library takes or a kernel timer is active (the caller takes the general path);
    raises ValueError for tensors on another device and RuntimeError on a library error.  n > 16 records
    the Sinkhorn VJP state, as mhc_layer_forward does.
    """
    if x.dtype not in _DTYPE_CODE or not x.is_cuda or profiling._active is not None:
        return None
    return _binding().layer_apply(x, hpre, hpost, hres, w, iters, eps, _DTYPE_CODE[out_dtype], False,
                                  x.shape[1] > 16)


def layer_forward_nograd(x, hpre, hpost, hres, w, iters: int, eps: float, out_dtype):
    """mhc_layer_fwd for a call that needs no gradient, with the fewest host steps (small-batch latency).

    One call into the torch binding, which allocates the output and launches on the current stream.
    Takes x on a GPU in fp32/bf16/fp16 and the four layer-wide parameters with the layer's shapes on
    x's device ([n], [n], [n, n], [C]); returns None when that does not hold or a kernel timer is
    active, and the caller takes the general path (mhc_layer_forward).  Raises ValueError for tensors
    on another device and RuntimeError on a library error.  out_dtype: torch.float32, or x's dtype
    when that is 16-bit.
    """
    if x.dtype not in _DTYPE_CODE or not x.is_cuda or profiling._active is not None:
        return None
    return _binding().layer_forward_nograd(x, hpre, hpost, hres, w, iters, eps, _DTYPE_CODE[out_dtype], False)


def _layer_bwd(x, g, hpre, hpost, hres, M, w, iters, eps, per_token):
    """mhc_layer_bwd: (dx, dH_pre_raw, dH_post_raw, dH_res_raw, d_rms_weight)."""
    B, n, C = (int(s) for s in x.shape)
    dev = x.device
    xc = x.detach().contiguous()
    gdt = g.dtype if g.dtype in (torch.float32, xc.dtype) else torch.float32
    gc = g.detach().to(gdt).contiguous()
    hp, hq, hr, Mc, wc = _f32(hpre), _f32(hpost), _f32(hres), _f32(M), _f32(w)
    dx = torch.empty_like(xc)
    dpre = torch.empty_like(hp)
    dpost = torch.empty_like(hq)
    dres = torch.empty_like(hr)
    dw = torch.empty((C,), dtype=torch.float32, device=dev)
    nb = _lib.query("mhc_layer_bwd_workspace_bytes", B, n, C, int(per_token), int(iters))
    ws = _ws(nb, dev)
    s = _stream(xc)
    if profiling._active is None:
        _lib.call("mhc_layer_bwd", _p(xc), _code(xc.dtype), _p(gc), _code(gc.dtype), _p(hp), _p(hq), _p(hr),
                  _p(Mc), _p(wc), _p(dx), _p(dpre), _p(dpost), _p(dres), _p(dw), _p(ws), nb, B, n, C,
                  int(per_token), int(iters), float(eps), s)
        return dx, dpre, dpost, dres, dw
    # under a kernel timer: partial sums and the reduction as separate calls
    np_ = ctypes.c_int64(0)
    if B > 0:
        nbp = _lib.query("mhc_fused_bwd_workspace_bytes", B, n, C, int(per_token))
        with timed("fused_bwd"):
            _lib.call("mhc_fused_bwd_partials", _p(xc), _code(xc.dtype), _p(gc), _code(gc.dtype), _p(Mc),
                      n * n if per_token else 0, _p(hp), _p(hq), n if per_token else 0, _lib.H_RAW, _p(wc),
                      _p(dx), _code(xc.dtype), _p(dres) if per_token else None,
                      _p(dpre) if per_token else None, _p(dpost) if per_token else None, _p(ws), nbp, B, n, C,
                      float(eps), ctypes.byref(np_), s)
    with timed("layer_bwd_reduce"):
        _lib.call("mhc_layer_bwd_reduce", _p(ws), nb, np_.value, _p(hp), _p(hq), _p(hr), _p(dpre), _p(dpost),
                  _p(dres), _p(dw), B, n, C, int(per_token), int(iters), float(eps), s)
    return dx, dpre, dpost, dres, dw


def _sk_state_bytes(B: int, n: int, iters: int) -> int:
    """Bytes of the Sinkhorn state a forward records for its backward (B matrices).

    0 when the library has no recorded path for n, or when the knob
    MHC_SK16_RECORD (n = 16) or MHC_SK_BLK_RECORD (16 < n <= 64) is 0: then
    the VJP recomputes the forward iterations and needs no saved state.
    """
    return int(_lib.query("mhc_sinkhorn_state_bytes", B, n, iters))


def _layer_fwd_recorded(x, hpre, hpost, hres, w, iters, eps, out_dtype, state, per_token):
    """Layer forward that records the Sinkhorn VJP state in `state`. Returns (out, M)."""
    B, n, C = x.shape
    xc = x if x.is_contiguous() else x.contiguous()
    hp, hq, hr, wc = _f32(hpre), _f32(hpost), _f32(hres), _f32(w)
    M = torch.empty_like(hr)
    out = torch.empty((B, n, C), dtype=out_dtype, device=x.device)
    s = _stream(xc)
    with timed("sinkhorn_fwd"):
        _lib.call("mhc_sinkhorn_fwd_record", _p(hr), _p(M), _p(state), state.numel(), B if per_token else 1, n,
                  int(iters), float(eps), s)
    with timed("fused_fwd"):
        _lib.call("mhc_fused_fwd", _p(xc), _code(xc.dtype), _p(M), n * n if per_token else 0, _p(hp), _p(hq),
                  n if per_token else 0, _lib.H_RAW, _p(wc), _p(out), _code(out_dtype), None, B, n, C, float(eps), s)
    return out, M


def _layer_bwd_recorded(x, g, hpre, hpost, hres, M, w, iters, eps, state, per_token):
    """Backward from a recorded Sinkhorn state: (dx, dH_pre_raw, dH_post_raw, dH_res_raw, d_w)."""
    B, n, C = (int(s) for s in x.shape)
    dev = x.device
    xc = x.detach().contiguous()
    gdt = g.dtype if g.dtype in (torch.float32, xc.dtype) else torch.float32
    gc = g.detach().to(gdt).contiguous()
    hp, hq, hr, Mc, wc = _f32(hpre), _f32(hpost), _f32(hres), _f32(M), _f32(w)
    dx = torch.empty_like(xc)
    dpre = torch.empty_like(hp)
    dpost = torch.empty_like(hq)
    dres = torch.empty_like(hr)
    dw = torch.empty((C,), dtype=torch.float32, device=dev)
    # layer-wide: the reduced dM, input of the Sinkhorn VJP; per token the
    # partials pass writes each token's dM to dres and the VJP runs in place
    dM = dres if per_token else torch.empty((n, n), dtype=torch.float32, device=dev)
    nb = _lib.query("mhc_fused_bwd_workspace_bytes", B, n, C, int(per_token))
    ws = _ws(nb, dev)
    s = _stream(xc)
    np_ = ctypes.c_int64(0)
    pt = per_token
    with timed("fused_bwd"):
        # the activated-H chain is applied in the kernel (per token) or the reduction (layer-wide)
        _lib.call("mhc_fused_bwd_partials", _p(xc), _code(xc.dtype), _p(gc), _code(gc.dtype), _p(Mc),
                  n * n if pt else 0, _p(hp), _p(hq), n if pt else 0, _lib.H_RAW, _p(wc), _p(dx), _code(xc.dtype),
                  _p(dres) if pt else None, _p(dpre) if pt else None, _p(dpost) if pt else None,
                  _p(ws), nb, B, n, C, float(eps), ctypes.byref(np_), s)
    with timed("layer_bwd_reduce"):
        _lib.call("mhc_reduce_param_grads", _p(ws), nb, np_.value, n, C, int(pt), None if pt else _p(hp),
                  None if pt else _p(hq), _lib.H_RAW, None if pt else _p(dM), None if pt else _p(dpre),
                  None if pt else _p(dpost), _p(dw), s)
        _lib.call("mhc_sinkhorn_bwd_recorded", _p(hr), _p(dM), _p(dres), _p(state), state.numel(),
                  B if pt else 1, n, int(iters), float(eps), s)
    return dx, dpre, dpost, dres, dw


class MHCLayerFn(torch.autograd.Function):
    """Whole MHCLayer forward/backward from raw parameters (layer.py:383-407).

    Forward: one library call (Sinkhorn projection, then the fused kernel
    with the sigmoid activations applied inside).  Backward: one library call
    (fused dx + partial sums, then a single launch that reduces the partial
    rows in a fixed order, applies the activation chain and runs the Sinkhorn
    VJP).  Parameters are layer-wide ([n], [n], [n, n]) or per token
    ([B, n], [B, n], [B, n, n]).  Per token at n = 16, when a gradient is
    needed, the Sinkhorn forward also records the VJP's state (saved for
    backward like an activation, 256 bytes per token and iteration), and so
    does the layer-wide or per-token forward for 16 < n <= 64 (6 * 32 * 4
    bytes per matrix and iteration at n = 32): the backward then skips
    recomputing the forward iterations.
    """

    @staticmethod
    def forward(ctx, x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, iters, eps, out_dtype):
        per_token = H_res_raw.ndim == 3
        n = int(x.shape[1])
        # with gradients (per token at n = 16, or n > 16): the Sinkhorn forward records the VJP state
        state = None
        if (per_token or n > 16) and any(ctx.needs_input_grad[:5]) and x.shape[0] > 0:
            state = _sk_record_buffer(H_res_raw, int(x.shape[0]) if per_token else 1, n, iters)
        if state is not None:
            out, M = _layer_fwd_recorded(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, iters, eps, out_dtype,
                                         state, per_token)
        else:
            out, M = _layer_fwd(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, iters, eps, out_dtype, per_token)
        ctx.save_for_backward(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, M, state)
        ctx.iters, ctx.eps, ctx.per_token = iters, eps, per_token
        return out

    @staticmethod
    def backward(ctx, dout):
        x, hpre, hpost, hres, w, M, state = ctx.saved_tensors
        if state is not None:
            dx, dpre, dpost, dres, dw = _layer_bwd_recorded(x, dout, hpre, hpost, hres, M, w, ctx.iters, ctx.eps,
                                                            state, ctx.per_token)
        else:
            dx, dpre, dpost, dres, dw = _layer_bwd(x, dout, hpre, hpost, hres, M, w, ctx.iters, ctx.eps,
                                                   ctx.per_token)
        return (dx, dpre.to(hpre.dtype), dpost.to(hpost.dtype), dres.to(hres.dtype), dw.to(w.dtype),
                None, None, None)


def mhc_layer_forward(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, sinkhorn_iters: int = 20,
                      eps: float = 1e-5, output_dtype=None):
    """mhc_forward_reference (reference.py:164-184) on the HIP path, with autograd.

    When no input needs a gradient (inference, torch.no_grad) the kernels are
    called directly, without an autograd node.
    """
    if H_res_raw.ndim != 2 or H_res_raw.shape[0] != H_res_raw.shape[1]:
        raise ValueError(f"H_res_raw must be square [n, n], got shape {tuple(H_res_raw.shape)}")
    _fused_shapes(x, H_res_raw, H_pre_raw, H_post_raw, rms_weight)
    out_dtype = _normalize_output_dtype(output_dtype, x.dtype)
    _require_gpu(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight)
    if not _needs_grad(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight):
        return _layer_fwd(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, int(sinkhorn_iters), float(eps),
                          out_dtype, False)[0]
    if profiling._active is None:
        # the same Function in C++ (backward without Python); n > 16 records the Sinkhorn state
        return _binding().layer_apply(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, int(sinkhorn_iters),
                                      float(eps), _DTYPE_CODE[out_dtype], False, int(x.shape[1]) > 16)
    return MHCLayerFn.apply(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, int(sinkhorn_iters),
                            float(eps), out_dtype)


def mhc_layer_forward_dynamic(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, sinkhorn_iters: int = 20,
                              eps: float = 1e-5, output_dtype=None):
    """Per-token extension: H_pre_raw/H_post_raw [B, n], H_res_raw [B, n, n] logits."""
    if H_res_raw.ndim != 3 or H_res_raw.shape[1] != H_res_raw.shape[2]:
        raise ValueError(f"H_res_raw must be [B, n, n], got shape {tuple(H_res_raw.shape)}")
    _fused_shapes(x, H_res_raw, H_pre_raw, H_post_raw, rms_weight)
    out_dtype = _normalize_output_dtype(output_dtype, x.dtype)
    _require_gpu(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight)
    if profiling._active is None and _needs_grad(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight):
        return _binding().layer_apply(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, int(sinkhorn_iters),
                                      float(eps), _DTYPE_CODE[out_dtype], True, True)
    return MHCLayerFn.apply(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight, int(sinkhorn_iters),
                            float(eps), out_dtype)


# --------------------------------------------------------------------------
# stream mix + add (MHCRewire post-combine) and pre-scale
# --------------------------------------------------------------------------

def _mix_shapes(x, M, y):
    if x.ndim != 3:
        raise ValueError(f"x must be [B, n, C], got shape {tuple(x.shape)}")
    if M.ndim != 2:
        raise ValueError(f"M must be [n, n], got shape {tuple(M.shape)}")
    if y is not None and tuple(y.shape) != tuple(x.shape):
        raise ValueError(f"y_dist must match x shape, got {tuple(y.shape)} vs {tuple(x.shape)}")
    B, n, C = (int(s) for s in x.shape)
    if tuple(M.shape) != (n, n):
        raise ValueError(f"M must be shape (n,n)=( {n},{n} ), got {tuple(M.shape)}")
    _validate_n(n)
    return B, n, C


def _y_dtype_ok(x, y):
    return y is None or y.dtype == x.dtype or y.dtype == torch.float32


def _mix_fwd(x, y, M, hpre, hpost, h_mode, out_dtype):
    B, n, C = (int(s) for s in x.shape)
    xc = x.detach().contiguous()
    yc = None
    if y is not None:
        yc = y.detach()
        if not _y_dtype_ok(xc, yc):
            yc = yc.to(torch.float32)
        yc = yc.contiguous()
    Mc = _f32(M)
    hp = _f32(hpre) if hpre is not None else None
    hq = _f32(hpost) if hpost is not None else None
    out = torch.empty((B, n, C), dtype=out_dtype, device=x.device)
    with timed("stream_mix_add_fwd"):
        _lib.call("mhc_stream_mix_add_fwd", _p(xc), _code(xc.dtype), _p(yc),
                  _code(yc.dtype) if yc is not None else _code(xc.dtype), _p(Mc), _p(hp), _p(hq), h_mode,
                  _p(out), _code(out_dtype), B, n, C, _stream(xc))
    return out


def _mix_bwd(x, y, g, M, hpre, hpost, h_mode, want_dy):
    B, n, C = (int(s) for s in x.shape)
    dev = x.device
    xc = x.detach().contiguous()
    yc = None
    ydt = xc.dtype
    if y is not None:
        yc = y.detach()
        if not _y_dtype_ok(xc, yc):
            yc = yc.to(torch.float32)
        yc = yc.contiguous()
        ydt = yc.dtype
    gdt = g.dtype if g.dtype in (torch.float32, xc.dtype) else torch.float32
    gc = g.detach().to(gdt).contiguous()
    Mc = _f32(M)
    hp = _f32(hpre) if hpre is not None else None
    hq = _f32(hpost) if hpost is not None else None
    dx = torch.empty_like(xc)
    dy = torch.empty((B, n, C), dtype=ydt, device=dev) if want_dy else None
    dM = torch.empty((n, n), dtype=torch.float32, device=dev)
    dpre = torch.empty((n,), dtype=torch.float32, device=dev) if h_mode != _lib.H_NONE else None
    dpost = torch.empty((n,), dtype=torch.float32, device=dev) if h_mode != _lib.H_NONE else None
    nb = _lib.query("mhc_stream_mix_add_bwd_workspace_bytes", B, n, C)
    ws = _ws(nb, dev)
    with timed("stream_mix_add_bwd"):
        _lib.call("mhc_stream_mix_add_bwd", _p(xc), _code(xc.dtype), _p(yc), _code(ydt), _p(gc),
                  _code(gc.dtype), _p(Mc), _p(hp), _p(hq), h_mode, _p(dx), _code(xc.dtype), _p(dy),
                  _code(ydt), _p(dM), _p(dpre), _p(dpost), _p(ws), nb, B, n, C, _stream(xc))
    return dx, dy, dM, dpre, dpost


class StreamMixAddFn(torch.autograd.Function):
    """out = M x + y_dist (fp32 out); VJP dx = M^T g, dM = sum g x^T, dy = g."""

    @staticmethod
    def forward(ctx, x, M, y_dist):
        ctx.save_for_backward(x, M)
        return _mix_fwd(x, y_dist, M, None, None, _lib.H_NONE, torch.float32)

    @staticmethod
    def backward(ctx, dout):
        x, M = ctx.saved_tensors
        dx, _, dM, _, _ = _mix_bwd(x, None, dout, M, None, None, _lib.H_NONE, want_dy=False)
        return dx, dM, dout


def stream_mix_add_hip(x, M, y_dist, threads_per_group=None, verbose: bool = False):
    """out = stream_mix(x, M) + y_dist, fp32 (metal.py:954-1014). No autograd."""
    _mix_shapes(x, M, y_dist)
    _validate_tpg(threads_per_group)
    _require_gpu(x, M, y_dist)
    with torch.no_grad():
        return _mix_fwd(x, y_dist, M, None, None, _lib.H_NONE, torch.float32)


def stream_mix_add_hip_autograd(x, M, y_dist, threads_per_group=None, verbose: bool = False):
    """Stream mix + add with the HIP backward (metal.py:2695)."""
    _mix_shapes(x, M, y_dist)
    _validate_tpg(threads_per_group)
    _require_gpu(x, M, y_dist)
    return StreamMixAddFn.apply(x, M, y_dist)


class PostCombineFn(torch.autograd.Function):
    """out = H_post * (y_inner + (M diag(H_pre)) x) from raw logits (layer.py:302-337)."""

    @staticmethod
    def forward(ctx, x, y_inner, H_pre_raw, H_post_raw, H_res_raw, iters, eps, out_dtype):
        # with a gradient for H_res_raw the Sinkhorn forward records its VJP state (n >= 16)
        state = None
        if ctx.needs_input_grad[4]:
            state = _sk_record_buffer(H_res_raw, 1, int(H_res_raw.shape[-1]), iters)
        M = _sinkhorn_fwd(H_res_raw, iters, eps, state)
        ctx.save_for_backward(x, y_inner, H_pre_raw, H_post_raw, H_res_raw, M, state)
        ctx.iters, ctx.eps = iters, eps
        return _mix_fwd(x, y_inner, M, H_pre_raw, H_post_raw, _lib.H_RAW, out_dtype)

    @staticmethod
    def backward(ctx, dout):
        x, y, hpre, hpost, hres, M, state = ctx.saved_tensors
        dx, dy, dM, dpre, dpost = _mix_bwd(x, y, dout, M, hpre, hpost, _lib.H_RAW, want_dy=True)
        dres = _sinkhorn_bwd(hres, dM, ctx.iters, ctx.eps, state)
        return (dx, dy.to(y.dtype), dpre.to(hpre.dtype), dpost.to(hpost.dtype), dres.to(hres.dtype), None,
                None, None)


def post_combine(x, y_inner, H_pre_raw, H_post_raw, H_res_raw, sinkhorn_iters: int = 20, eps: float = 1e-5,
                 output_dtype=None):
    """MHCRewire post-combine on [B, n, C] views; output fp32 unless output_dtype."""
    B, n, C = _mix_shapes(x, H_res_raw, y_inner)
    out_dtype = torch.float32 if output_dtype is None else output_dtype
    if out_dtype not in (torch.float32, x.dtype):
        raise ValueError(f"unsupported output_dtype: {output_dtype}")
    _require_gpu(x, y_inner, H_pre_raw, H_post_raw, H_res_raw)
    return PostCombineFn.apply(x, y_inner, H_pre_raw, H_post_raw, H_res_raw, int(sinkhorn_iters),
                               float(eps), out_dtype)


class StreamScaleFn(torch.autograd.Function):
    """x_pre = sigmoid(H_pre_raw)_i * x_i (layer.py:476-480).

    With ``passthrough`` the Function also returns x itself (sharing its storage) for the caller's other
    use of x, MHCRewire's post-combine.  Both x-gradient contributions then arrive at this node, and the
    VJP writes dx = a_i g_i + g_pass in the same pass that reads g and x (the library's dx accumulator)
    instead of leaving their sum to a separate elementwise add.
    """

    @staticmethod
    def forward(ctx, x, H_pre_raw, passthrough):
        B, n, C = (int(s) for s in x.shape)
        xc = x.detach().contiguous()
        hp = _f32(H_pre_raw)
        out = torch.empty_like(xc)
        with timed("stream_scale_fwd"):
            _lib.call("mhc_stream_scale_fwd", _p(xc), _code(xc.dtype), _p(hp), _lib.H_RAW, _p(out),
                      _code(xc.dtype), B, n, C, _stream(xc))
        ctx.save_for_backward(x, H_pre_raw)
        ctx.set_materialize_grads(False)
        return (out, x) if passthrough else out

    @staticmethod
    def backward(ctx, dout, dpass=None):
        x, hpre = ctx.saved_tensors
        if dout is None:
            return dpass, None, None
        B, n, C = (int(s) for s in x.shape)
        xc = x.detach().contiguous()
        gdt = dout.dtype if dout.dtype in (torch.float32, xc.dtype) else torch.float32
        gc = dout.detach().to(gdt).contiguous()
        acc = None if dpass is None else dpass.detach().to(xc.dtype).contiguous()
        hp = _f32(hpre)
        dx = torch.empty_like(xc)
        dpre = torch.empty((n,), dtype=torch.float32, device=xc.device)
        nb = _lib.query("mhc_stream_scale_bwd_workspace_bytes", B, n, C)
        ws = _ws(nb, xc.device)
        with timed("stream_scale_bwd"):
            _lib.call("mhc_stream_scale_bwd", _p(xc), _code(xc.dtype), _p(gc), _code(gc.dtype), _p(hp),
                      _lib.H_RAW, _p(acc), _p(dx), _code(xc.dtype), _p(dpre), _p(ws), nb, B, n, C, _stream(xc))
        return dx, dpre.to(hpre.dtype), None


def _stream_scale_check(x, H_pre_raw):
    if x.ndim != 3 or H_pre_raw.ndim != 1 or H_pre_raw.shape[0] != x.shape[1]:
        raise ValueError(f"x must be [B, n, C] and H_pre_raw [n], got {tuple(x.shape)}, {tuple(H_pre_raw.shape)}")
    _validate_n(int(x.shape[1]))
    _require_gpu(x, H_pre_raw)


def stream_scale(x, H_pre_raw):
    """Pre-scale of MHCRewire: [B, n, C] * sigmoid(H_pre_raw)[n]."""
    _stream_scale_check(x, H_pre_raw)
    return StreamScaleFn.apply(x, H_pre_raw, False)


def stream_scale_and_pass(x, H_pre_raw):
    """(stream_scale(x, H_pre_raw), x): the second output is x for a second use (MHCRewire's
    post-combine) whose gradient the pre-scale's VJP adds into dx in its own pass."""
    _stream_scale_check(x, H_pre_raw)
    return StreamScaleFn.apply(x, H_pre_raw, True)


# --------------------------------------------------------------------------
# residual add + aggregate (utils.py:4-24, metal.py:1673-1731)
# --------------------------------------------------------------------------

def _res_inputs(x, res):
    """Both inputs in one dtype: a mixed pair is promoted to fp32 (exact for bf16 / fp16), as the
    reference upcasts bf16 operands to fp32 before its kernel (metal.py:856-859, 1718-1719)."""
    xc, rc = x.detach(), res.detach()
    if xc.dtype != rc.dtype:
        xc, rc = xc.to(torch.float32), rc.to(torch.float32)
    _code(xc.dtype)
    return xc.contiguous(), rc.contiguous()


class ResidualAddAggFn(torch.autograd.Function):
    """(out, y_agg) = (x + res, sum_i H_pre[i] (x + res)[:, i]); H_pre is used as given.

    Backward (an extension; the reference kernel is not differentiable):
    dx = dres = dout + H_pre[i] dy_agg, dH_pre[i] = sum dy_agg (x + res)[:, i].
    """

    @staticmethod
    def forward(ctx, x, res, H_pre, out_dtype):
        B, n, C = (int(s) for s in x.shape)
        xc, rc = _res_inputs(x, res)
        hp = _f32(H_pre)
        out = torch.empty((B, n, C), dtype=out_dtype, device=x.device)
        y_agg = torch.empty((B, C), dtype=torch.float32, device=x.device)
        with timed("residual_add_agg"):
            _lib.call("mhc_residual_add_agg_fwd", _p(xc), _p(rc), _code(xc.dtype), _p(hp), _lib.H_ACTIVATED,
                      _p(out), _code(out_dtype), _p(y_agg), B, n, C, _stream(xc))
        ctx.save_for_backward(x, res, H_pre)
        ctx.set_materialize_grads(False)
        return out, y_agg

    @staticmethod
    def backward(ctx, dout, dy):
        x, res, hpre = ctx.saved_tensors
        B, n, C = (int(s) for s in x.shape)
        xc, rc = _res_inputs(x, res)
        hp = _f32(hpre)
        want_h = ctx.needs_input_grad[2]
        gc = None
        if dout is not None:
            gdt = dout.dtype if dout.dtype in (torch.float32, xc.dtype) else torch.float32
            gc = dout.detach().to(gdt).contiguous()
        dyc = None if dy is None else dy.detach().to(torch.float32).contiguous()
        dx = torch.empty_like(xc) if ctx.needs_input_grad[0] else None
        dres = torch.empty_like(xc) if ctx.needs_input_grad[1] else None
        dpre = torch.empty((n,), dtype=torch.float32, device=xc.device) if want_h else None
        nb = _lib.query("mhc_residual_add_agg_bwd_workspace_bytes", B, n, C) if want_h else 0
        ws = _ws(nb, xc.device)
        with timed("residual_add_agg_bwd"):
            _lib.call("mhc_residual_add_agg_bwd", _p(xc), _p(rc), _code(xc.dtype), _p(gc),
                      _code(gc.dtype) if gc is not None else _code(xc.dtype), _p(dyc), _p(hp), _lib.H_ACTIVATED,
                      _p(dx), _p(dres), _p(dpre), _p(ws), nb, B, n, C, _stream(xc))
        if dx is not None and dx.dtype != x.dtype:
            dx = dx.to(x.dtype)
        if dres is not None and dres.dtype != res.dtype:
            dres = dres.to(res.dtype)
        return dx, dres, (dpre.to(hpre.dtype) if dpre is not None else None), None


def residual_add_agg_hip(x, res, H_pre, threads_per_group=None, output_dtype=None, verbose: bool = False):
    """Fused residual add + aggregate (metal.py:1673-1731), differentiable.

    Returns (out [B, n, C], y_agg [B, C] fp32) with out = x + res and
    y_agg = sum_i H_pre[i] * out[:, i].  ``out`` is fp32 unless
    ``output_dtype`` names float16 / bfloat16 (any input dtype, as the
    reference allows).  ``threads_per_group`` is validated as the reference
    does; launch shapes are chosen by the library.
    """
    if x.ndim != 3:
        raise ValueError(f"x must be [B, n, C], got shape {tuple(x.shape)}")
    if tuple(res.shape) != tuple(x.shape):
        raise ValueError(f"res must match x shape, got {tuple(res.shape)} vs {tuple(x.shape)}")
    B, n, C = (int(s) for s in x.shape)
    _validate_n(n)
    if threads_per_group is not None and threads_per_group <= 0:
        raise ValueError("threads_per_group must be positive")
    if H_pre.ndim != 1 or int(H_pre.shape[0]) != n:
        raise ValueError(f"H_pre must be [n]=[{n}], got shape {tuple(H_pre.shape)}")
    if output_dtype is None:
        out_dtype = torch.float32
    elif output_dtype in (torch.float32, torch.float16, torch.bfloat16):
        out_dtype = output_dtype
    else:
        raise ValueError(f"unsupported output_dtype: {output_dtype}")
    _require_gpu(x, res, H_pre)
    return ResidualAddAggFn.apply(x, res, H_pre, out_dtype)

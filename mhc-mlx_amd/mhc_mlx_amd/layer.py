"""MHCLayer / MHCRewire: torch modules with the reference's constructor and
call contract (mhc_mlx/layer.py:58-492), backed by libmhc_hip on MI355X.

Forward semantics (layer.py:1-12):
  H_pre_act = sigmoid(H_pre_raw), H_post_act = 2 sigmoid(H_post_raw)
  M = sinkhorn_knopp(exp(H_res_raw))
  out = stream_mix(x, M) + H_post_act * rms_norm(sum_i H_pre_act[i] x[:, i], w)

Paths:
* accelerated (default, ``use_metal=True`` on a host with a GPU): one
  autograd Function per call (Sinkhorn + fused kernel forward; fused
  backward + reduction + Sinkhorn VJP), all in libmhc_hip.
* reference: the torch restatement in reference.py.  It runs when
  ``use_metal=False``, when ``MHC_MLX_DISABLE_METAL=1`` / ``MHC_HIP_DISABLE=1``,
  or when no GPU is visible (``metal_available`` is False), as the reference
  layer does when Metal is absent (layer.py:122-126), and for n > 64.  With
  ``compile_reference`` (on by default where the HIP path is selected, as in
  the reference) CPU tensors run it through ``torch.compile``.

Failures of the accelerated path follow the reference (layer.py:28-29,
158-173, 306-330, 408-422): a RuntimeError raised by the library (a HIP
error, an allocation failure) or inputs that the HIP path cannot take (CPU
tensors) are reported once through ``warnings.warn`` and the module flag
``_METAL_FAILED``, and that call runs the reference path.  A GPU host whose
libmhc_hip.so is missing or unloadable is an installation error: the
constructor raises RuntimeError naming the build command instead of
degrading silently.  Argument errors (ValueError) always propagate.

The reference's dispatch-policy knobs are accepted with the same validation
and the same predicates (``_should_avoid_fused`` etc.).  The policy routes
the reference to its MLX path for shapes its Metal kernels handled badly;
libmhc_hip serves every n <= 64 shape with its own kernels, so here the
predicates are informational and every such call stays on the HIP path.
"""

from __future__ import annotations

import os
import warnings

import torch
import torch.nn as nn

from . import _lib, ops, profiling
from . import reference as ref

__all__ = ["MHCLayer", "MHCRewire", "hip_available"]

# Set once the accelerated path has handed a call to the reference path
# (layer.py:28-29); the warning is issued only the first time.
_METAL_FAILED = False

_HIP_AVAILABLE: bool | None = None



_ENV = os.environ


def _disabled_by_env() -> bool:
    return _ENV.get("MHC_MLX_DISABLE_METAL") == "1" or _ENV.get("MHC_HIP_DISABLE") == "1"


def hip_available() -> bool:
    """Whether the HIP path can run here: a GPU is visible and libmhc_hip.so loads.

    The analogue of the reference's ``hasattr(mx.fast, "metal_kernel")``
    (layer.py:122).  False when torch sees no GPU.  With a GPU visible the
    library must load: a missing or broken build raises RuntimeError (naming
    the build command) rather than reporting False.
    """
    global _HIP_AVAILABLE
    if _HIP_AVAILABLE is None:
        if not torch.cuda.is_available():
            _HIP_AVAILABLE = False
        else:
            _lib.load()
            _HIP_AVAILABLE = True
    return _HIP_AVAILABLE


def _fallback_warning(where: str, err) -> None:
    """Warn once per process that the accelerated path handed a call to the reference path."""
    global _METAL_FAILED
    if not _METAL_FAILED:
        warnings.warn(f"HIP kernel execution failed{where}, falling back to reference path. Error: {err}",
                      RuntimeWarning, stacklevel=3)
        _METAL_FAILED = True


def _off_gpu(*ts) -> str | None:
    """None when every tensor is on a GPU, else a reason naming the first that is not."""
    for t in ts:
        if t is not None and not t.is_cuda:
            return f"the HIP path needs GPU tensors (got a tensor on {t.device})"
    return None


class MHCLayer(nn.Module):
    def __init__(
        self,
        n: int,
        C: int,
        sinkhorn_iters: int = 20,
        eps: float = 1e-5,
        use_metal: bool = True,
        threads_per_group: int | None = 256,
        identity_init: bool = True,
        auto_dispatch: bool = True,
        compile_reference: bool | None = None,
        dispatch_policy: str = "auto",
        hybrid_latency: bool = False,
        hybrid_min_C: int = 8192,
        latency_avoid_fused_n32_max_C: int = 2048,
        latency_avoid_fused_B1_min_n: int = 16,
        throughput_allow_fused_n32_min_B: int = 8,
        throughput_allow_fused_n32_min_C: int = 4096,
        throughput_allow_fused_n32_small_C: int = 512,
        fused_backward: bool = False,
        mix_kernel: str = "auto",
        *,
        use_hip: bool | None = None,
        device=None,
    ):
        super().__init__()
        # layer.py:83-102
        if n <= 0:
            raise ValueError("n must be positive")
        if C <= 0:
            raise ValueError("C must be positive")
        if dispatch_policy not in {"auto", "throughput", "latency"}:
            raise ValueError("dispatch_policy must be one of: auto, throughput, latency")
        if hybrid_min_C <= 0:
            raise ValueError("hybrid_min_C must be positive")
        if latency_avoid_fused_n32_max_C <= 0:
            raise ValueError("latency_avoid_fused_n32_max_C must be positive")
        if latency_avoid_fused_B1_min_n <= 0:
            raise ValueError("latency_avoid_fused_B1_min_n must be positive")
        if throughput_allow_fused_n32_min_B <= 0:
            raise ValueError("throughput_allow_fused_n32_min_B must be positive")
        if throughput_allow_fused_n32_min_C <= 0:
            raise ValueError("throughput_allow_fused_n32_min_C must be positive")
        if throughput_allow_fused_n32_small_C < 0:
            raise ValueError("throughput_allow_fused_n32_small_C must be >= 0")
        if mix_kernel not in {"auto", "1d", "2d"}:
            raise ValueError("mix_kernel must be one of: auto, 1d, 2d")

        self.n = int(n)
        self.C = int(C)
        self.sinkhorn_iters = int(sinkhorn_iters)
        self.eps = float(eps)
        self.auto_dispatch = bool(auto_dispatch)
        self.dispatch_policy = str(dispatch_policy)
        self.hybrid_latency = bool(hybrid_latency)
        self.hybrid_min_C = int(hybrid_min_C)
        self.latency_avoid_fused_n32_max_C = int(latency_avoid_fused_n32_max_C)
        self.latency_avoid_fused_B1_min_n = int(latency_avoid_fused_B1_min_n)
        self.throughput_allow_fused_n32_min_B = int(throughput_allow_fused_n32_min_B)
        self.throughput_allow_fused_n32_min_C = int(throughput_allow_fused_n32_min_C)
        self.throughput_allow_fused_n32_small_C = int(throughput_allow_fused_n32_small_C)
        self.fused_backward = bool(fused_backward)
        self.mix_kernel = str(mix_kernel)
        accel = bool(use_metal) if use_hip is None else bool(use_hip)
        # layer.py:121-126 (Metal availability is HIP availability here)
        if _disabled_by_env() or not accel:
            self.metal_available = torch.cuda.is_available() and _lib.LIB_PATH.exists()
            self.use_metal = False
        else:
            self.metal_available = hip_available()
            self.use_metal = self.metal_available
        self.threads_per_group = None if threads_per_group is None else int(threads_per_group)
        self.identity_init = bool(identity_init)
        if compile_reference is None:
            self.compile_reference = self.use_metal and self.auto_dispatch
        else:
            self.compile_reference = bool(compile_reference)
        self._compiled_reference = None

        # layer.py:139-153: identity-friendly init
        kw = dict(dtype=torch.float32, device=device)
        if self.identity_init:
            off = 12.0
            self.H_pre_raw = nn.Parameter(torch.full((self.n,), -off, **kw))
            self.H_post_raw = nn.Parameter(torch.full((self.n,), -off, **kw))
            self.H_res_raw = nn.Parameter(torch.full((self.n, self.n), -off, **kw) + torch.eye(self.n, **kw) * off)
        else:
            self.H_pre_raw = nn.Parameter(torch.zeros((self.n,), **kw))
            self.H_post_raw = nn.Parameter(torch.zeros((self.n,), **kw))
            self.H_res_raw = nn.Parameter(torch.zeros((self.n, self.n), **kw))
        self.rms_weight = nn.Parameter(torch.ones((self.C,), **kw))

    @property
    def use_hip(self) -> bool:
        return self.use_metal

    # ---- policy predicates (layer.py:175-244), kept with identical results
    def _should_use_metal(self, B: int, n: int, C: int) -> bool:
        if _disabled_by_env():
            return False
        if not self.use_metal:
            return False
        if n > 64:
            return False
        return True

    def _latency_policy_enabled(self) -> bool:
        return self.dispatch_policy == "latency"

    def _throughput_policy_enabled(self) -> bool:
        return self.dispatch_policy == "throughput"

    def _should_avoid_fused_latency(self, B: int, n: int, C: int) -> bool:
        if n == 32 and C <= self.latency_avoid_fused_n32_max_C:
            return True
        if B == 1 and n >= self.latency_avoid_fused_B1_min_n:
            return True
        return False

    def _should_avoid_fused_throughput(self, B: int, n: int, C: int) -> bool:
        if n != 32:
            return False
        if B < self.throughput_allow_fused_n32_min_B:
            return True
        allow_small = self.throughput_allow_fused_n32_small_C > 0 and C == self.throughput_allow_fused_n32_small_C
        allow_large = C >= self.throughput_allow_fused_n32_min_C
        return not (allow_small or allow_large)

    def _should_avoid_fused(self, B: int, n: int, C: int) -> bool:
        if not self.use_metal or not self.auto_dispatch:
            return False
        lat, thr = self._latency_policy_enabled(), self._throughput_policy_enabled()
        if not (lat or thr):
            return False
        if lat and self._should_avoid_fused_latency(B, n, C):
            return True
        if thr and self._should_avoid_fused_throughput(B, n, C):
            return True
        return False

    def _should_use_hybrid(self, B: int, n: int, C: int) -> bool:
        if not self.use_metal or not self.auto_dispatch or not self.hybrid_latency:
            return False
        if not self._latency_policy_enabled():
            return False
        return n == 32 and B == 1 and C >= self.hybrid_min_C

    def _should_use_reference_fallback(self, B: int, n: int, C: int) -> bool:
        if not self.use_metal or not self.auto_dispatch:
            return False
        if not self._should_avoid_fused(B, n, C):
            return False
        return not self._should_use_hybrid(B, n, C)

    def _should_use_fused_backward(self, B: int, n: int, C: int) -> bool:
        return bool(self.fused_backward)

    # ---- API
    def mixing_matrix(self) -> torch.Tensor:
        """Current mixing matrix M = sinkhorn(exp(H_res_raw)) (layer.py:155-173)."""
        if self.use_metal and not _disabled_by_env():
            why = _off_gpu(self.H_res_raw)
            if why is None:
                try:
                    return ops.sinkhorn_knopp_hip_autograd(self.H_res_raw, iters=self.sinkhorn_iters, eps=self.eps,
                                                           threads_per_group=self.threads_per_group)
                except RuntimeError as e:
                    why = e
            _fallback_warning(" in mixing_matrix", why)
        return ref.mixing_matrix_from_logits(self.H_res_raw, iters=self.sinkhorn_iters, eps=self.eps)

    def _reference_forward(self, x, H_pre_raw, H_post_raw, H_res_raw, rms_weight):
        return ref.mhc_forward_reference(x, H_pre_raw, H_post_raw, H_res_raw, rms_weight,
                                         sinkhorn_iters=self.sinkhorn_iters, eps=self.eps)

    def _get_reference_runner(self, x: torch.Tensor):
        """The callable that runs the reference path (layer.py:291-300).

        With ``compile_reference`` it is ``torch.compile`` of the restatement, built on first use and
        kept (about 45 s of Inductor code generation for a forward and backward on an 8-core host;
        afterwards a 256-token n=4 C=4096 step runs ~14x faster than eager).  Only CPU tensors take
        the compiled runner: for GPU tensors torch.compile would generate Triton kernels, which this
        build does not use, so GPU tensors that reach the reference path (n > 64, a library error)
        run it eagerly.
        """
        if not self.compile_reference or x.is_cuda:
            return self._reference_forward
        if self._compiled_reference is None:
            self._compiled_reference = torch.compile(self._reference_forward)
        return self._compiled_reference

    def post_combine(self, x_reshaped: torch.Tensor, y_inner_reshaped: torch.Tensor, *,
                     return_dtype: torch.dtype | None = None) -> torch.Tensor:
        """H_post * (y_inner + (M diag(H_pre)) x) on [B, n, C] views (layer.py:302-337).

        fp32 out as in the reference; ``return_dtype`` (extension) casts it, and a half type equal to
        x's dtype is written by the kernel directly.
        """
        out = None
        if self.use_metal and not _disabled_by_env():
            why = _off_gpu(x_reshaped, y_inner_reshaped, self.H_pre_raw, self.H_post_raw, self.H_res_raw)
            if why is None:
                kdt = self._kernel_out_dtype(x_reshaped, return_dtype)
                try:
                    out = ops.post_combine(x_reshaped, y_inner_reshaped, self.H_pre_raw, self.H_post_raw,
                                           self.H_res_raw, sinkhorn_iters=self.sinkhorn_iters, eps=self.eps,
                                           output_dtype=kdt)
                except RuntimeError as e:
                    why = e
            if out is None:
                _fallback_warning(" in post_combine", why)
        if out is None:
            H_pre_act, H_post_act = ref.activate_pre_post(self.H_pre_raw, self.H_post_raw)
            M = ref.mixing_matrix_from_logits(self.H_res_raw, iters=self.sinkhorn_iters, eps=self.eps)
            M_final = M * H_pre_act.reshape(1, -1)
            x_mixed = torch.einsum("ij,...jd->...id", M_final, x_reshaped.to(M_final.dtype))
            out = (y_inner_reshaped.to(x_mixed.dtype) + x_mixed) * H_post_act.reshape(1, self.n, 1)
        if return_dtype is not None and out.dtype != return_dtype:
            out = out.to(return_dtype)
        return out

    def _check(self, x: torch.Tensor):
        if x.ndim != 3:
            raise ValueError(f"x_expanded must be [B, n, C], got shape {tuple(x.shape)}")
        B, n, C = (int(s) for s in x.shape)
        if n != self.n:
            raise ValueError(f"x_expanded n={n} does not match layer n={self.n}")
        if C != self.C:
            raise ValueError(f"x_expanded C={C} does not match layer C={self.C}")
        return B, n, C

    @staticmethod
    def _kernel_out_dtype(x: torch.Tensor, return_dtype):
        # layer.py:361-364: emit a half type directly only when it matches x
        if return_dtype is not None and return_dtype == x.dtype and return_dtype in (torch.float16, torch.bfloat16):
            return return_dtype
        return None

    def forward(self, x_expanded: torch.Tensor, *, return_dtype: torch.dtype | None = None) -> torch.Tensor:
        """Run the mHC layer on x_expanded [B, n, C] (layer.py:339-435).

        The accelerated path first makes one call into the torch binding (``module_call``): it reads the
        disable switches, this layer's parameters and settings, checks the tensors' shapes, devices and
        dtypes, allocates the output and, when a gradient is needed, records the C++ autograd node whose
        backward runs the library's VJP.  At small batch the layer's latency is mostly this host code.
        It returns None whenever the general path below has something to decide (a disable switch,
        use_metal off, a shape error, tensors off the GPU, n > 64, a kernel timer, a library error).
        """
        if profiling._active is None:
            try:
                out = (ops._BINDING or ops._binding()).module_call(self, x_expanded, return_dtype)
            except (RuntimeError, ValueError, TypeError):
                out = None
            if out is not None:
                return out
        B, n, C = self._check(x_expanded)
        out = None
        if self._should_use_metal(B, n, C):
            why = _off_gpu(x_expanded, self.H_pre_raw, self.H_post_raw, self.H_res_raw, self.rms_weight)
            if why is None:
                try:
                    out = ops.mhc_layer_forward(x_expanded, self.H_pre_raw, self.H_post_raw, self.H_res_raw,
                                                self.rms_weight, sinkhorn_iters=self.sinkhorn_iters, eps=self.eps,
                                                output_dtype=self._kernel_out_dtype(x_expanded, return_dtype))
                except RuntimeError as e:
                    why = e
            if out is None:
                _fallback_warning("", why)
        if out is None:
            out = self._get_reference_runner(x_expanded)(x_expanded, self.H_pre_raw, self.H_post_raw,
                                                         self.H_res_raw, self.rms_weight)
        if return_dtype is not None and out.dtype != return_dtype:
            out = out.to(return_dtype)
        return out

    def forward_dynamic(self, x_expanded: torch.Tensor, H_pre_raw: torch.Tensor, H_post_raw: torch.Tensor,
                        H_res_raw: torch.Tensor, *, return_dtype: torch.dtype | None = None) -> torch.Tensor:
        """Per-token mappings (extension): H_pre_raw, H_post_raw [B, n]; H_res_raw [B, n, n] logits.

        Uses this layer's rms_weight, sinkhorn_iters and eps.
        """
        B, n, C = self._check(x_expanded)
        if tuple(H_pre_raw.shape) != (B, n) or tuple(H_post_raw.shape) != (B, n):
            raise ValueError(f"H_pre_raw / H_post_raw must be [B, n]=[{B}, {n}]")
        if tuple(H_res_raw.shape) != (B, n, n):
            raise ValueError(f"H_res_raw must be [B, n, n]=[{B}, {n}, {n}], got {tuple(H_res_raw.shape)}")
        out = None
        if self._should_use_metal(B, n, C):
            why = _off_gpu(x_expanded, H_pre_raw, H_post_raw, H_res_raw, self.rms_weight)
            if why is None:
                try:
                    out = ops.mhc_layer_forward_dynamic(x_expanded, H_pre_raw, H_post_raw, H_res_raw,
                                                        self.rms_weight, sinkhorn_iters=self.sinkhorn_iters,
                                                        eps=self.eps,
                                                        output_dtype=self._kernel_out_dtype(x_expanded, return_dtype))
                except RuntimeError as e:
                    why = e
            if out is None:
                _fallback_warning(" in forward_dynamic", why)
        if out is None:
            out = self._get_reference_runner(x_expanded)(x_expanded, H_pre_raw, H_post_raw, H_res_raw,
                                                         self.rms_weight)
        if return_dtype is not None and out.dtype != return_dtype:
            out = out.to(return_dtype)
        return out


class MHCRewire(nn.Module):
    """Wrap any dims -> dims module with mHC residual mixing (layer.py:438-492).

    out = H_post * (inner(H_pre * x) + (M diag(H_pre)) x), with x [..., dims]
    viewed as n streams of C = dims // n channels.  The output is fp32 as in
    the reference; ``return_dtype`` (extension, e.g. torch.bfloat16 for a
    half-precision model) selects another output dtype.
    """

    def __init__(self, inner: nn.Module, dims: int, n: int = 32, *, return_dtype: torch.dtype | None = None,
                 **mhc_kwargs):
        super().__init__()
        self.inner = inner
        self.n = n
        self.dims = dims
        self.return_dtype = return_dtype
        if dims % n != 0:
            raise ValueError(f"dims {dims} must be divisible by n={n}")
        self.mhc = MHCLayer(n=n, C=dims // n, **mhc_kwargs)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dims = x.shape[-1]
        if dims % self.n != 0:
            raise ValueError(f"input dims {dims} must be divisible by n={self.n}")
        C = dims // self.n
        x3 = x.reshape(-1, self.n, C)
        x_pre = None
        if self.mhc.use_metal and not _disabled_by_env():
            why = _off_gpu(x3, self.mhc.H_pre_raw)
            if why is None:
                try:
                    # x3 comes back through the pre-scale node, whose VJP then adds the post-combine's
                    # x gradient into its own dx pass
                    x_pre, x3 = ops.stream_scale_and_pass(x3, self.mhc.H_pre_raw)
                except RuntimeError as e:
                    why = e
            if x_pre is None:
                _fallback_warning(" in the MHCRewire pre-scale", why)
        if x_pre is None:
            H_pre_act, _ = ref.activate_pre_post(self.mhc.H_pre_raw, self.mhc.H_post_raw)
            x_pre = x3 * H_pre_act.reshape(1, self.n, 1).to(x3.dtype)
        y_inner = self.inner(x_pre.reshape(x.shape))
        if tuple(y_inner.shape) != tuple(x.shape):
            raise ValueError(
                f"inner module must preserve the shape: got {tuple(y_inner.shape)} for input {tuple(x.shape)}"
            )
        out = self.mhc.post_combine(x3, y_inner.reshape(-1, self.n, C), return_dtype=self.return_dtype)
        return out.reshape(x.shape)

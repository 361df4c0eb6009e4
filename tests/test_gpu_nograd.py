"""GPU tests of MHCLayer's fast path, in particular its no-gradient forward (inference, torch.no_grad).

Every accelerated module call makes one call into the torch binding
(``MHCLayer.forward`` -> ``module_call``); a call that needs no
gradient goes from there straight to mhc_layer_fwd.  It must give bitwise the
results of the general op path and match the oracle (reference.py:164-184),
and hand every case it does not take (tensors on another device, n > 64, a
disable switch, a library error) to the general path unchanged.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import MHCLayer, ops

pytestmark = pytest.mark.gpu


def _layer(n, C, g):
    hpre, hpost, hres, w = params(g, n, C)
    layer = MHCLayer(n=n, C=C, eps=1e-6).cuda()
    with torch.no_grad():
        for p, v in zip((layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw, layer.rms_weight),
                        (hpre, hpost, hres, w)):
            p.copy_(torch.from_numpy(v))
    return layer, (hpre, hpost, hres, w)


class _Recorder:
    """Stands in for the torch binding (ops._BINDING): records each module_call as True (a result
    without an autograd node), "grad" (a result with one), None (the call was left to the general path) or
    False (it raised, or ``fail`` was raised in its place); everything else passes through."""

    def __init__(self, real, calls, fail=None):
        self.real, self.calls, self.fail = real, calls, fail

    def __getattr__(self, name):
        return getattr(self.real, name)

    def module_call(self, *args):
        if self.fail is not None:
            self.calls.append(False)
            raise self.fail
        try:
            out = self.real.module_call(*args)
        except Exception:
            self.calls.append(False)
            raise
        self.calls.append(None if out is None else ("grad" if out.grad_fn is not None else True))
        return out


@pytest.fixture
def fast_calls(monkeypatch):
    """The module's calls into the binding: True for each no-gradient forward that returned a result."""
    calls = []
    monkeypatch.setattr(ops, "_BINDING", _Recorder(ops._binding(), calls))
    return calls


@pytest.mark.parametrize("B,n,C,dt,ret", [
    (1, 4, 4096, "bf16", torch.bfloat16),   # the B = 1 latency shape (single launch)
    (32, 4, 2048, "bf16", torch.bfloat16),  # config 1
    (32, 4, 2048, "bf16", None),            # fp32 out (the reference's default)
    (3, 8, 520, "f16", torch.float16),      # ragged C
    (300, 4, 256, "f32", None),             # more tokens than CUs: Sinkhorn launch + fused forward
    (2, 16, 1024, "bf16", torch.bfloat16),
    (1, 32, 4096, "bf16", torch.bfloat16),  # the reference's n = 32 latency rows
    (4, 2, 96, "bf16", torch.float32),      # fp32 out requested explicitly
])
def test_nograd_forward_matches_general_path_and_oracle(B, n, C, dt, ret, fast_calls):
    g = rng(300 + n + B)
    layer, (hpre, hpost, hres, w) = _layer(n, C, g)
    x = to_dtype_np(g.standard_normal((B, n, C)), dt)
    xt = dev_tensor(x, dt)
    with torch.no_grad():
        out = layer(xt, return_dtype=ret)
        assert fast_calls == [True]
        kdt = ret if ret is xt.dtype and ret in (torch.bfloat16, torch.float16) else None
        ref = ops.mhc_layer_forward(xt, layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw, layer.rms_weight,
                                    sinkhorn_iters=20, eps=1e-6, output_dtype=kdt)
        if ret is not None:
            ref = ref.to(ret)
    torch.cuda.synchronize()
    assert out.dtype == (ret or torch.float32) and out.shape == (B, n, C)
    assert torch.equal(out, ref)
    oracle = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=1e-6)
    tol = TOL["bf16" if out.dtype == torch.bfloat16 else "f16" if out.dtype == torch.float16 else dt]
    assert rel_err(np_of(out), oracle) < max(tol, 1e-5)


def test_inference_mode_and_frozen_parameters_take_the_fast_path(fast_calls):
    g = rng(11)
    layer, _ = _layer(4, 512, g)
    xt = torch.randn(8, 4, 512, device="cuda", dtype=torch.bfloat16)
    with torch.inference_mode():
        a = layer(xt, return_dtype=torch.bfloat16)
    for p in layer.parameters():
        p.requires_grad_(False)
    b = layer(xt, return_dtype=torch.bfloat16)  # grad mode on, nothing needs a gradient
    assert fast_calls == [True, True]
    assert torch.equal(a, b)


def test_gradient_calls_record_the_autograd_node(fast_calls):
    g = rng(12)
    layer, _ = _layer(4, 256, g)
    xt = torch.randn(4, 4, 256, device="cuda", dtype=torch.bfloat16)
    out = layer(xt, return_dtype=torch.bfloat16)
    assert out.requires_grad and fast_calls == ["grad"] and "LayerFn" in out.grad_fn.name()
    out.float().sum().backward()
    assert layer.H_res_raw.grad is not None


def test_disable_switch_set_after_construction_takes_the_reference_path(fast_calls, monkeypatch):
    """MHC_MLX_DISABLE_METAL=1 is read on every call (layer.py:176), also by the binding's fast path: set
    after the layer was built, the call runs the torch path."""
    g = rng(15)
    layer, (hpre, hpost, hres, w) = _layer(4, 128, g)
    x = torch.from_numpy(g.standard_normal((2, 4, 128)).astype(np.float32)).cuda()
    for name in ("MHC_MLX_DISABLE_METAL", "MHC_HIP_DISABLE"):
        monkeypatch.setenv(name, "1")
        with torch.no_grad():
            out = layer(x)
        monkeypatch.delenv(name)
        assert fast_calls[-1] is None
        ref = O.mhc_forward_reference(np_of(x), hpre, hpost, hres, w, sinkhorn_iters=20, eps=1e-6)
        assert rel_err(np_of(out), ref) < 1e-5
    with torch.no_grad():
        layer(x)
    assert fast_calls == [None, None, True]


def test_views_and_other_parameter_dtypes_take_the_fast_path(fast_calls):
    """The binding copies a non-contiguous x and converts non-fp32 parameters itself (as the general path
    does), so those calls stay on the fast path with the same results; a shape error still raises."""
    g = rng(13)
    layer, _ = _layer(4, 256, g)
    base = torch.randn(4, 4, 512, device="cuda", dtype=torch.bfloat16)
    view = base[:, :, :256]  # not contiguous
    with torch.no_grad():
        a = layer(view, return_dtype=torch.bfloat16)
        b = layer(view.contiguous(), return_dtype=torch.bfloat16)
    assert fast_calls == [True, True]
    assert torch.equal(a, b)
    layer64, _ = _layer(4, 256, rng(13))
    layer64.double()
    with torch.no_grad():
        c = layer64(view.contiguous(), return_dtype=torch.bfloat16)
    assert fast_calls == [True, True, True] and torch.equal(c, b)
    with torch.no_grad(), pytest.raises(ValueError):
        layer(torch.randn(4, 5, 256, device="cuda", dtype=torch.bfloat16))


def test_the_binding_refuses_tensors_off_the_gpu():
    """The kernels take raw device pointers: the torch binding checks that every tensor is on x's GPU
    before any launch (ValueError), with and without autograd."""
    b = ops._binding()
    x = torch.randn(2, 4, 64, device="cuda")
    p = [torch.zeros(4, device="cuda"), torch.zeros(4, device="cuda"), torch.zeros(4, 4, device="cuda"),
         torch.ones(64)]  # rms weight on the CPU
    with pytest.raises(ValueError, match="device"):
        b.layer_forward_nograd(x, *p, 20, 1e-6, 0, False)
    with pytest.raises(ValueError, match="GPU"):
        b.layer_forward_nograd(x.cpu(), *(t.cpu() for t in p), 20, 1e-6, 0, False)
    with pytest.raises(ValueError, match="device"):
        b.layer_apply(x.requires_grad_(True), *p, 20, 1e-6, 0, False, False)
    # the module's entry leaves such calls to the general path
    assert b.module_forward(x, *p, 4, 64, 20, 1e-6, None) is None
    assert b.module_forward(x.cpu(), *(t.cpu() for t in p), 4, 64, 20, 1e-6, None) is None


def test_library_error_in_the_fast_path_goes_to_the_general_path(monkeypatch):
    """A RuntimeError from the binding's forward hands the call to the general path (ops.py through
    ctypes), which gives bitwise the same result."""
    g = rng(14)
    layer, _ = _layer(4, 256, g)
    xt = torch.randn(4, 4, 256, device="cuda", dtype=torch.bfloat16)
    calls = []
    with torch.no_grad():
        want = layer(xt, return_dtype=torch.bfloat16)
        monkeypatch.setattr(ops, "_BINDING", _Recorder(ops._binding(), calls,
                                                       fail=RuntimeError("mhc_layer_fwd failed: injected")))
        got = layer(xt, return_dtype=torch.bfloat16)
    assert calls == [False] and torch.equal(got, want)


@pytest.mark.parametrize("grad_mode", ["no_grad", "inference_mode", "frozen"])
def test_nograd_n_above_64_takes_the_reference_path(grad_mode, fast_calls):
    """n > 64 is beyond the library (metal.py:827-834): like the reference layer (layer.py:175-185), the
    module runs its torch path for it, also when no gradient is needed, and never calls the library."""
    n, C, B = 65, 48, 3
    g = rng(365)
    layer, (hpre, hpost, hres, w) = _layer(n, C, g)
    x = torch.from_numpy(g.standard_normal((B, n, C)).astype(np.float32)).cuda()
    if grad_mode == "no_grad":
        with torch.no_grad():
            out = layer(x)
    elif grad_mode == "inference_mode":
        with torch.inference_mode():
            out = layer(x)
    else:
        for p in layer.parameters():
            p.requires_grad_(False)
        out = layer(x)
    assert fast_calls == [None]
    ref = O.mhc_forward_reference(np_of(x), hpre, hpost, hres, w, sinkhorn_iters=20, eps=1e-6)
    assert out.dtype == torch.float32 and out.is_cuda
    assert rel_err(np_of(out), ref) < 1e-5

"""GPU tests of the MHCLayer module contract (reference layer.py / tests).

Mirrors test_layer_forward_matches_reference (test_correctness.py:223-251),
test_latency_fallback_corner (:254-291), test_backward_matches_reference
(:294-344, here with every gradient compared), test_reference_fallback
(:346-360), test_determinism.py and test_concurrency.py.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import GRAD_TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import MHCLayer, MHCRewire, _lib, ops

pytestmark = pytest.mark.gpu


def _set(layer, hpre, hpost, hres, w):
    with torch.no_grad():
        layer.H_pre_raw.copy_(torch.from_numpy(hpre))
        layer.H_post_raw.copy_(torch.from_numpy(hpost))
        layer.H_res_raw.copy_(torch.from_numpy(hres))
        layer.rms_weight.copy_(torch.from_numpy(w))


@pytest.mark.parametrize("B,n,C", [(1, 4, 64), (2, 8, 128), (2, 16, 256), (1, 32, 256)])
def test_layer_forward_matches_reference(B, n, C):
    g = rng(100 + n)
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    hpre, hpost, hres, _ = params(g, n, C)
    w = np.ones(C, np.float32)
    hip = MHCLayer(n=n, C=C, auto_dispatch=False).cuda()
    refl = MHCLayer(n=n, C=C, use_metal=False).cuda()
    for l in (hip, refl):
        _set(l, hpre, hpost, hres, w)
    xt = dev_tensor(x, "bf16")
    y_hip, y_ref = np_of(hip(xt)), np_of(refl(xt))
    oracle = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=1e-5)
    for y in (y_hip, y_ref):
        assert np.abs(y - oracle).max() < 1e-4 and rel_err(y, oracle) < 1e-5
    assert hip(xt).dtype == torch.float32


def test_latency_policy_corner_uses_hip():
    B, n, C = 1, 32, 1024
    g = rng(7)
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    hpre, hpost, hres, w = params(g, n, C)
    auto = MHCLayer(n=n, C=C, dispatch_policy="latency", hybrid_latency=True).cuda()
    _set(auto, hpre, hpost, hres, w)
    assert auto._should_use_reference_fallback(B, n, C)
    out = np_of(auto(dev_tensor(x, "bf16")))
    oracle = O.mhc_forward_reference(x, hpre, hpost, hres, w)
    assert rel_err(out, oracle) < 1e-5


@pytest.mark.parametrize("ret", [None, torch.bfloat16, torch.float16, torch.float32])
def test_return_dtype_semantics(ret):
    n, C = 4, 256
    layer = MHCLayer(n=n, C=C, identity_init=False).cuda()
    x = torch.randn(3, n, C, device="cuda", dtype=torch.bfloat16)
    out = layer(x, return_dtype=ret)
    assert out.dtype == (torch.float32 if ret is None else ret)


def test_layer_backward_matches_oracle_all_grads():
    """Reference test_backward_matches_reference (B=1, n=4, C=16, 5 iterations), all grads."""
    B, n, C = 1, 4, 16
    g = rng(9)
    x = g.standard_normal((B, n, C)).astype(np.float32)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    hpre, hpost, hres, w = params(g, n, C)
    layer = MHCLayer(n=n, C=C, sinkhorn_iters=5).cuda()
    _set(layer, hpre, hpost, hres, w)
    xt = dev_tensor(x).requires_grad_(True)
    out = layer(xt)
    ref_out = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=5)
    assert abs(float(out.sum()) - ref_out.sum()) < 1e-4  # the reference test's loss check
    out.backward(dev_tensor(dout))
    ref = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=5)
    gots = [np_of(xt.grad), np_of(layer.H_pre_raw.grad), np_of(layer.H_post_raw.grad),
            np_of(layer.H_res_raw.grad), np_of(layer.rms_weight.grad)]
    for got, r in zip(gots, ref):
        assert rel_err(got, r) < GRAD_TOL


def test_sum_loss_gives_zero_h_res_gradient():
    """loss = sum(out): dM = 1 c^T has constant columns, so dH_res vanishes."""
    layer = MHCLayer(n=4, C=16, identity_init=False).cuda()
    with torch.no_grad():
        layer.H_res_raw.normal_()
    x = torch.randn(3, 4, 16, device="cuda")
    layer(x).sum().backward()
    assert layer.H_res_raw.grad.abs().max().item() < 1e-5


def test_env_disable_forces_reference(monkeypatch):
    monkeypatch.setenv("MHC_MLX_DISABLE_METAL", "1")
    layer = MHCLayer(n=4, C=16).cuda()
    assert layer._should_use_metal(1, 4, 16) is False
    y = layer(torch.randn(1, 4, 16, device="cuda"))
    assert y.shape == (1, 4, 16)


class _BindingSpy:
    """Stands in for the torch binding (ops._BINDING): records each call, then makes it (or raises
    ``fail`` for the names listed in ``failing``)."""

    def __init__(self, real, failing=(), fail=None):
        self.real, self.failing, self.fail, self.calls = real, set(failing), fail, []

    def __getattr__(self, name):
        fn = getattr(self.real, name)

        def call(*args):
            self.calls.append(name)
            if name in self.failing:
                raise self.fail
            return fn(*args)

        return call


def test_hip_path_is_the_one_that_runs(monkeypatch):
    """The accelerated layer must call the library (no silent torch path): the forward with gradients
    goes through the torch binding's autograd Function, whose backward runs the library's VJP."""
    spy = _BindingSpy(ops._binding())
    monkeypatch.setattr(ops, "_BINDING", spy)
    layer = MHCLayer(n=4, C=128).cuda()
    x = torch.randn(2, 4, 128, device="cuda", requires_grad=True)
    out = layer(x)
    assert spy.calls == ["module_call"] and "LayerFn" in out.grad_fn.name()
    out.sum().backward()
    assert x.grad is not None and layer.H_res_raw.grad is not None and layer.rms_weight.grad is not None
    with torch.no_grad():
        y = layer(x)
    assert spy.calls == ["module_call", "module_call"] and y.grad_fn is None


def test_gpu_layer_reports_hip_available():
    from mhc_mlx_amd import layer as L

    layer = MHCLayer(n=4, C=64)
    assert L.hip_available() is True and layer.metal_available is True and layer.use_metal is True


def test_library_failure_falls_back_once_on_gpu(monkeypatch):
    """A RuntimeError from the library runs the reference path on the same GPU tensors, warned once."""
    from mhc_mlx_amd import layer as L

    monkeypatch.setattr(L, "_METAL_FAILED", False)  # restored before the session guard checks it
    spy = _BindingSpy(ops._binding(), failing=("module_call", "layer_apply"),
                      fail=RuntimeError("mhc_layer_fwd failed (hip error 98): injected by the test"))
    monkeypatch.setattr(ops, "_BINDING", spy)
    g = rng(11)
    B, n, C = 3, 4, 128
    hpre, hpost, hres, w = params(g, n, C)
    x = g.standard_normal((B, n, C)).astype(np.float32)
    layer = MHCLayer(n=n, C=C).cuda()
    _set(layer, hpre, hpost, hres, w)
    with pytest.warns(RuntimeWarning, match="injected by the test") as rec:
        y1 = layer(dev_tensor(x))
        y2 = layer(dev_tensor(x))
    assert len(rec) == 1 and L._METAL_FAILED is True
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=layer.eps)
    assert rel_err(np_of(y1), ref) < 1e-5 and torch.equal(y1, y2)


def test_timed_path_uses_the_same_kernels(monkeypatch):
    """Under kernel_timer the layer splits its calls per kernel; results are bitwise equal."""
    from mhc_mlx_amd import kernel_timer

    torch.manual_seed(3)
    layer = MHCLayer(n=4, C=512, identity_init=False).cuda()
    x = torch.randn(33, 4, 512, device="cuda", dtype=torch.bfloat16)
    g = torch.randn_like(x)

    def run():
        xx = x.clone().requires_grad_(True)
        out = layer(xx, return_dtype=torch.bfloat16)
        grads = torch.autograd.grad(out, [xx] + list(layer.parameters()), g)
        return [out] + list(grads)

    plain = run()
    calls = []
    orig = _lib.call

    def spy(name, *args):
        calls.append(name)
        return orig(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    with kernel_timer() as kt:
        timed = run()
        stats = kt.stats()
    for k in ("mhc_sinkhorn_fwd", "mhc_fused_fwd", "mhc_fused_bwd_partials", "mhc_layer_bwd_reduce"):
        assert k in calls
    assert {"sinkhorn_fwd", "fused_fwd", "fused_bwd", "layer_bwd_reduce"} <= set(stats)
    for a, b in zip(plain, timed):
        assert torch.equal(a, b)


def test_determinism_and_state_dict():
    torch.manual_seed(42)
    a = MHCLayer(n=16, C=64, identity_init=False).cuda()
    b = MHCLayer(n=16, C=64, identity_init=False).cuda()
    b.load_state_dict(a.state_dict())
    assert list(a.state_dict().keys()) == ["H_pre_raw", "H_post_raw", "H_res_raw", "rms_weight"]
    x = torch.randn(1, 16, 64, device="cuda")
    assert torch.equal(a(x), b(x))


@pytest.mark.parametrize("T,n,C", [(300, 16, 512), (70, 32, 96), (40, 24, 48), (20, 64, 32)])
def test_backward_bitwise_reproducible(T, n, C):
    """Fixed-order sums: two fwd+bwd runs give bitwise equal gradients (n = 16 layer-wide MFMA
    backward; the 16 < n <= 64 kernels, whose outer-product blocks each belong to one wavefront)."""
    torch.manual_seed(T + n + C)
    layer = MHCLayer(n=n, C=C, eps=1e-6, identity_init=False).cuda()
    with torch.no_grad():
        for p in (layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw):
            p.normal_()
    x = torch.randn(T, n, C, device="cuda", dtype=torch.bfloat16).requires_grad_(True)
    g = torch.randn(T, n, C, device="cuda", dtype=torch.bfloat16)
    params = list(layer.parameters())
    runs = []
    for _ in range(2):
        out = layer(x, return_dtype=torch.bfloat16)
        runs.append([out] + list(torch.autograd.grad(out, [x] + params, g)))
    for a, b in zip(*runs):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, b)


@pytest.mark.parametrize("n", [32, 20])
def test_rewire_backward_bitwise_reproducible(n):
    """The post-combine VJP for 16 < n <= 64 (MHCRewire's default n = 32) is run-to-run exact."""
    torch.manual_seed(n)
    dims = 40 * n
    inner = torch.nn.Linear(dims, dims, bias=False).cuda()
    m = MHCRewire(inner, dims=dims, n=n, identity_init=False).cuda()
    with torch.no_grad():
        for p in (m.mhc.H_pre_raw, m.mhc.H_post_raw, m.mhc.H_res_raw):
            p.normal_()
    x = torch.randn(50, dims, device="cuda").requires_grad_(True)
    g = torch.randn(50, dims, device="cuda")
    prm = [x, inner.weight, m.mhc.H_pre_raw, m.mhc.H_post_raw, m.mhc.H_res_raw]
    a = torch.autograd.grad(m(x), prm, g)
    b = torch.autograd.grad(m(x), prm, g)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_mixing_matrix_doubly_stochastic_and_bomb():
    layer = MHCLayer(n=32, C=64).cuda()
    with torch.no_grad():
        layer.H_res_raw.fill_(100.0)
    M = layer.mixing_matrix()
    assert torch.isfinite(M).all()
    assert (M.sum(1) - 1).abs().max().item() <= 1e-3 and (M.sum(0) - 1).abs().max().item() <= 1e-3


def test_forward_dynamic_api():
    B, n, C = 4, 16, 64
    g = rng(3)
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    hpre, hpost, hres, w = params(g, n, C, per_token_B=B)
    layer = MHCLayer(n=n, C=C).cuda()
    with torch.no_grad():
        layer.rms_weight.copy_(torch.from_numpy(w))
    out = layer.forward_dynamic(dev_tensor(x, "bf16"), dev_tensor(hpre), dev_tensor(hpost), dev_tensor(hres),
                                return_dtype=torch.bfloat16)
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w)
    assert out.dtype == torch.bfloat16 and rel_err(np_of(out), ref) < 2e-2

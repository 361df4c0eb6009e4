"""Availability detection and the warn-once fallback of MHCLayer / MHCRewire
(mhc_mlx/layer.py:28-29, 122-126, 158-173, 306-330, 408-422), on the CPU.

Without a GPU the modules take the torch reference path without a warning,
as the reference does without Metal.  When the accelerated path is selected
but cannot run a call (CPU tensors, or a RuntimeError from the library) the
call runs the reference path and one warning is issued per process.
Results are checked against the float64 oracle.
"""

import warnings

import numpy as np
import pytest
import torch
from torch import nn

from oracle import mhc_oracle as O
from tests._helpers import np_of, rel_err

from mhc_mlx_amd import MHCLayer, MHCRewire, _lib, ops
from mhc_mlx_amd import layer as L


def _randomise(layer: MHCLayer, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in (layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw):
            p.copy_(torch.randn(p.shape, generator=g))
        layer.rms_weight.copy_(1 + 0.02 * torch.randn(layer.rms_weight.shape, generator=g))


def _ref_out(layer: MHCLayer, x: torch.Tensor) -> np.ndarray:
    return O.mhc_forward_reference(np_of(x), np_of(layer.H_pre_raw), np_of(layer.H_post_raw),
                                   np_of(layer.H_res_raw), np_of(layer.rms_weight),
                                   sinkhorn_iters=layer.sinkhorn_iters, eps=layer.eps)


@pytest.fixture
def fresh_flag(monkeypatch):
    monkeypatch.setattr(L, "_METAL_FAILED", False)


def test_no_gpu_means_reference_path_without_warning(fresh_flag, monkeypatch):
    monkeypatch.setattr(L, "_HIP_AVAILABLE", None)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    layer = MHCLayer(n=4, C=16, identity_init=False)
    assert layer.metal_available is False and layer.use_metal is False
    _randomise(layer, 0)
    x = torch.randn(3, 4, 16)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        y = layer(x)
    assert rel_err(np_of(y), _ref_out(layer, x)) < 1e-5
    assert L._METAL_FAILED is False


def test_gpu_host_without_library_raises(fresh_flag, monkeypatch, tmp_path):
    """A visible GPU with no loadable libmhc_hip.so is an installation error, not a silent fallback."""
    monkeypatch.setattr(L, "_HIP_AVAILABLE", None)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libmhc_hip.so")
    with pytest.raises(RuntimeError, match="not found"):
        MHCLayer(n=4, C=16)
    # the explicit opt-out still constructs
    assert MHCLayer(n=4, C=16, use_metal=False).use_metal is False


def _accelerated(layer):
    """Select the accelerated path as on a GPU host (this container has no GPU)."""
    layer.use_metal = True
    layer.metal_available = True
    return layer


def test_cpu_tensors_fall_back_once_with_one_warning(fresh_flag):
    layer = _accelerated(MHCLayer(n=4, C=16, identity_init=False))
    _randomise(layer, 1)
    rew = MHCRewire(nn.Linear(16, 16, bias=False), dims=16, n=4, identity_init=False)
    _accelerated(rew.mhc)
    _randomise(rew.mhc, 2)
    x = torch.randn(2, 4, 16)
    xr = torch.randn(5, 16)
    with pytest.warns(RuntimeWarning, match="falling back to reference path") as rec:
        y = layer(x)
        y2 = layer(x)
        z = rew(xr)
        m = layer.mixing_matrix()
    assert len([w for w in rec if issubclass(w.category, RuntimeWarning)]) == 1
    assert L._METAL_FAILED is True
    ref = _ref_out(layer, x)
    assert rel_err(np_of(y), ref) < 1e-5 and torch.equal(y, y2)
    mh = rew.mhc
    H_pre_act = 1.0 / (1.0 + np.exp(-np_of(mh.H_pre_raw)))
    y_inner = np_of(rew.inner(torch.from_numpy((np_of(xr).reshape(-1, 4, 4) * H_pre_act[None, :, None])
                                               .reshape(5, 16).astype(np.float32))))
    ref_z = O.post_combine(np_of(xr).reshape(-1, 4, 4), y_inner.reshape(-1, 4, 4), np_of(mh.H_pre_raw),
                           np_of(mh.H_post_raw), np_of(mh.H_res_raw), sinkhorn_iters=mh.sinkhorn_iters, eps=mh.eps)
    assert rel_err(np_of(z).reshape(-1, 4, 4), ref_z) < 1e-5
    assert rel_err(np_of(m), O.mixing_matrix_from_logits(np_of(layer.H_res_raw), iters=layer.sinkhorn_iters,
                                                         eps=layer.eps)) < 1e-5


def test_library_failure_falls_back_once(fresh_flag, monkeypatch):
    """A RuntimeError from the library (e.g. a HIP error) runs the reference path, warned once."""
    calls = []

    def failing(*a, **k):
        calls.append(1)
        raise _lib.MHCError("mhc_layer_fwd: HIP error 98: invalid device function")

    monkeypatch.setattr(ops, "mhc_layer_forward", failing)
    monkeypatch.setattr(L, "_off_gpu", lambda *ts: None)
    layer = _accelerated(MHCLayer(n=4, C=16, identity_init=False))
    _randomise(layer, 3)
    x = torch.randn(2, 4, 16, requires_grad=True)
    with pytest.warns(RuntimeWarning, match="invalid device function") as rec:
        y = layer(x)
        y2 = layer(x)
    assert len(calls) == 2 and len(rec) == 1 and L._METAL_FAILED is True
    assert rel_err(np_of(y), _ref_out(layer, x)) < 1e-5 and torch.equal(y, y2)
    # the fallback result carries autograd like the reference path
    y.sum().backward()
    assert x.grad is not None and layer.H_res_raw.grad is not None


def test_argument_errors_are_not_swallowed(fresh_flag, monkeypatch):
    def bad(*a, **k):
        raise ValueError("x must be bfloat16 when output_dtype is bfloat16")

    monkeypatch.setattr(ops, "mhc_layer_forward", bad)
    monkeypatch.setattr(L, "_off_gpu", lambda *ts: None)
    layer = _accelerated(MHCLayer(n=4, C=16))
    with pytest.raises(ValueError, match="bfloat16"):
        layer(torch.randn(1, 4, 16))
    assert L._METAL_FAILED is False


def test_env_disable_is_silent(fresh_flag, monkeypatch):
    monkeypatch.setenv("MHC_MLX_DISABLE_METAL", "1")
    layer = MHCLayer(n=4, C=16, identity_init=False)
    assert layer.use_metal is False
    _randomise(layer, 4)
    x = torch.randn(2, 4, 16)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        y = layer(x)
    assert rel_err(np_of(y), _ref_out(layer, x)) < 1e-5


def test_nograd_cpu_call_takes_the_general_path(fresh_flag):
    """The no-gradient fast path takes GPU tensors only; a CPU call under no_grad still falls back once."""
    layer = _accelerated(MHCLayer(n=4, C=16, identity_init=False))
    _randomise(layer, 4)
    x = torch.randn(2, 4, 16)
    assert ops.layer_forward_nograd(x, layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw, layer.rms_weight,
                                    20, 1e-5, torch.float32) is None
    with torch.no_grad(), pytest.warns(RuntimeWarning, match="falling back to reference path") as rec:
        y = layer(x)
    assert len(rec) == 1 and L._METAL_FAILED is True
    assert rel_err(np_of(y), _ref_out(layer, x)) < 1e-5


def test_compile_reference_compiles_the_cpu_reference_once(fresh_flag, monkeypatch):
    """compile_reference (layer.py:133-137, 291-300): the reference path of a CPU call runs
    torch.compile of the restatement, built on the first such call and reused; without the flag
    the restatement runs as is.  The real compiled runner is checked against the oracle."""
    made = []
    real_compile = torch.compile

    def counting_compile(fn, *a, **k):
        made.append(fn)
        return real_compile(fn, *a, **k)

    monkeypatch.setattr(torch, "compile", counting_compile)
    plain = MHCLayer(n=4, C=16, identity_init=False, use_metal=False)
    assert plain.compile_reference is False
    _randomise(plain, 3)
    x = torch.randn(3, 4, 16)
    plain(x)
    assert made == []

    layer = MHCLayer(n=4, C=16, identity_init=False, use_metal=False, compile_reference=True)
    _randomise(layer, 3)
    with torch.no_grad():
        y = layer(x)
        y2 = layer(x)
    assert len(made) == 1 and layer._get_reference_runner(x) is layer._compiled_reference
    assert rel_err(np_of(y), _ref_out(layer, x)) < 1e-5 and torch.equal(y, y2)
    hp = torch.randn(3, 4)
    hr = torch.randn(3, 4, 4)
    with torch.no_grad():
        yd = layer.forward_dynamic(x, hp, hp, hr)
    assert len(made) == 1
    ref_d = O.mhc_forward_reference(np_of(x), np_of(hp), np_of(hp), np_of(hr), np_of(layer.rms_weight),
                                    sinkhorn_iters=layer.sinkhorn_iters, eps=layer.eps)
    assert rel_err(np_of(yd), ref_d) < 1e-5

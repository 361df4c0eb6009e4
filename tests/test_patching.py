"""AutoPatcher on torch models (CPU): the reference's tests/test_patching.py and
tests/test_quantized.py restated for torch modules, plus the torch containers.

Numerics here use the layer's torch path (``use_metal=False``), compared with
the float64 oracle of MHCRewire(Linear); the HIP path of patched models is
covered by tests/test_gpu_patching.py.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O

from mhc_mlx_amd import AutoPatcher, MHCRewire


def test_autopatcher_custom_block():
    """Reference test_autopatcher_custom_block: only the square layers are rewired."""
    dims, n = 64, 4

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.linear1 = torch.nn.Linear(dims, dims)
            self.linear2 = torch.nn.Linear(dims, dims * 2)
            self.linear3 = torch.nn.Linear(dims * 2, dims)
            self.linear4 = torch.nn.Linear(dims, dims)

    model = Block()
    assert AutoPatcher.patch(model, n_streams=n, verbose=True, use_metal=False) == 2
    assert isinstance(model.linear1, MHCRewire) and isinstance(model.linear4, MHCRewire)
    assert not isinstance(model.linear2, MHCRewire) and not isinstance(model.linear3, MHCRewire)
    y = model.linear1(torch.randn(1, dims))
    assert y.shape == (1, dims)


def test_autopatcher_list_containers():
    """Reference test_autopatcher_list_container, with torch's registered containers."""
    dims, n = 64, 4

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = torch.nn.ModuleList([torch.nn.Linear(dims, dims), torch.nn.Linear(dims, 32)])
            self.seq = torch.nn.Sequential(torch.nn.Linear(dims, dims), torch.nn.ReLU(), torch.nn.Linear(dims, dims))
            self.heads = torch.nn.ModuleDict({"a": torch.nn.Linear(dims, dims), "b": torch.nn.Linear(dims, 8)})

    model = Model()
    assert AutoPatcher.patch(model, n_streams=n, verbose=False) == 4
    assert isinstance(model.layers[0], MHCRewire) and not isinstance(model.layers[1], MHCRewire)
    assert isinstance(model.seq[0], MHCRewire) and isinstance(model.seq[2], MHCRewire)
    assert isinstance(model.heads["a"], MHCRewire) and not isinstance(model.heads["b"], MHCRewire)


def test_patch_rules():
    n = 8
    assert not AutoPatcher._is_patchable(torch.nn.Linear(60, 60), n)      # 60 % 8 != 0
    assert AutoPatcher._is_patchable(torch.nn.Linear(64, 64, bias=False), n)
    assert not AutoPatcher._is_patchable(torch.nn.Linear(64, 32), n)
    assert not AutoPatcher._is_patchable(torch.nn.Conv1d(64, 64, 1), n)
    assert not AutoPatcher._is_patchable(torch.nn.LazyLinear(64), n)     # width unknown until first call
    assert AutoPatcher._get_dims(torch.nn.Linear(48, 48)) == 48
    assert AutoPatcher._get_dims(torch.nn.ReLU()) == 0


def test_root_is_not_replaced_and_patch_is_idempotent(capsys):
    lin = torch.nn.Linear(32, 32)
    assert AutoPatcher.patch(lin, n_streams=4) == 0       # the root module itself is never rewired
    model = torch.nn.Sequential(torch.nn.Linear(32, 32))
    assert AutoPatcher.patch(model, n_streams=4) == 1
    assert AutoPatcher.patch(model, n_streams=4) == 0     # the wrapped inner layer is left alone
    assert isinstance(model[0], MHCRewire) and isinstance(model[0].inner, torch.nn.Linear)
    out = capsys.readouterr().out
    assert "[AutoPatcher] Rewiring 0 (dims=32, streams=4)" in out and "Patched 1 layers." in out


def test_kwargs_reach_the_layer_and_half_models_keep_their_dtype():
    model = torch.nn.Sequential(torch.nn.Linear(64, 64).to(torch.bfloat16))
    AutoPatcher.patch(model, n_streams=4, verbose=False, sinkhorn_iters=7, eps=1e-6, use_metal=False)
    rw = model[0]
    assert rw.mhc.sinkhorn_iters == 7 and rw.mhc.eps == 1e-6 and rw.mhc.n == 4 and rw.mhc.C == 16
    assert rw.return_dtype == torch.bfloat16
    assert rw.mhc.H_pre_raw.dtype == torch.float32        # mHC parameters stay fp32 (layer.py:139-153)
    y = model(torch.randn(3, 64, dtype=torch.bfloat16))
    assert y.dtype == torch.bfloat16
    fp32 = torch.nn.Sequential(torch.nn.Linear(64, 64))
    AutoPatcher.patch(fp32, n_streams=4, verbose=False, use_metal=False)
    assert fp32[0].return_dtype is None and fp32(torch.randn(2, 64)).dtype == torch.float32


def test_patched_forward_matches_oracle():
    dims, n, T = 64, 4, 5
    g = np.random.default_rng(0)
    lin = torch.nn.Linear(dims, dims, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy((0.05 * g.standard_normal((dims, dims))).astype(np.float32)))
    model = torch.nn.Sequential(lin)
    AutoPatcher.patch(model, n_streams=n, verbose=False, use_metal=False, identity_init=False)
    hpre, hpost = g.standard_normal(n).astype(np.float32), g.standard_normal(n).astype(np.float32)
    hres = g.standard_normal((n, n)).astype(np.float32)
    with torch.no_grad():
        model[0].mhc.H_pre_raw.copy_(torch.from_numpy(hpre))
        model[0].mhc.H_post_raw.copy_(torch.from_numpy(hpost))
        model[0].mhc.H_res_raw.copy_(torch.from_numpy(hres))
    x = g.standard_normal((T, dims)).astype(np.float32)
    got = model(torch.from_numpy(x)).detach().numpy()
    ref, _ = O.rewire_linear_forward(x, lin.weight.detach().numpy(), hpre, hpost, hres, 20, 1e-5)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5


def test_quantized_linear_rewire():
    """Reference test_quantized_linear_rewire: a quantized Linear is wrapped, and only the mHC
    parameters train (torch's dynamic-quantized Linear holds no trainable parameters)."""
    nnqd = pytest.importorskip("torch.ao.nn.quantized.dynamic")
    dims, n = 512, 16
    q = nnqd.Linear(dims, dims)
    assert AutoPatcher._is_patchable(q, n) and AutoPatcher._get_dims(q) == dims
    model = torch.nn.Sequential(q)
    assert AutoPatcher.patch(model, n_streams=n, verbose=False, use_metal=False) == 1
    rw = model[0]
    y = rw(torch.randn(1, dims))
    assert y.shape == (1, dims)
    trainable = {k for k, p in rw.named_parameters() if p.requires_grad}
    assert trainable and all(k.startswith("mhc.") for k in trainable)
    with pytest.warns(UserWarning):   # torch warns that quantized::linear_dynamic has no autograd kernel
        y.sum().backward()
    assert rw.mhc.H_pre_raw.grad is not None and rw.mhc.H_res_raw.grad is not None

"""CPU counterparts of tests/test_gpu_reference_suites.py on the explicit
torch path (use_metal=False, layer.py:122-126): the module semantics of the
reference's test_vision.py and test_determinism.py, checked against the
float64 oracle.  The HIP kernels are exercised by the GPU file.
"""

import io
import pickle

import numpy as np
import torch
from torch import nn

from oracle import mhc_oracle as O
from tests._helpers import np_of, rel_err

from mhc_mlx_amd import MHCLayer, MHCRewire


class _NHWCConv(nn.Module):
    def __init__(self, c: int):
        super().__init__()
        self.conv = nn.Conv2d(c, c, kernel_size=3, padding=1)

    def forward(self, x):
        return self.conv(x.permute(0, 3, 1, 2)).permute(0, 2, 3, 1)


def _randomise(layer: MHCLayer, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in (layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw):
            p.copy_(torch.randn(p.shape, generator=g))


def test_conv2d_rewire_torch_path():
    """test_vision.py:5-23 on the torch path: [B, H, W, C] in and out, mix applied, oracle parity."""
    torch.manual_seed(0)
    B, H, W, C, n = 2, 8, 8, 64, 16
    inner = _NHWCConv(C)
    model = MHCRewire(inner, dims=C, n=n, use_metal=False)
    _randomise(model.mhc, 1)
    x = torch.randn(B, H, W, C)
    seen = {}
    hook = inner.register_forward_hook(lambda m, i, o: seen.__setitem__("y", o.detach()))
    y = model(x)
    hook.remove()
    assert y.shape == (B, H, W, C)
    assert not torch.equal(y, inner(x))
    k = C // n
    mh = model.mhc
    ref = O.post_combine(np_of(x).reshape(-1, n, k), np_of(seen["y"]).reshape(-1, n, k), np_of(mh.H_pre_raw),
                         np_of(mh.H_post_raw), np_of(mh.H_res_raw), sinkhorn_iters=mh.sinkhorn_iters, eps=mh.eps)
    assert rel_err(np_of(y).reshape(-1, n, k), ref) < 1e-5


def test_pickling_and_seed_determinism_torch_path():
    """test_determinism.py:7-47: same seed, same parameters and output; pickling keeps them."""
    layers = []
    for _ in range(2):
        torch.manual_seed(42)
        layer = MHCLayer(n=16, C=64, identity_init=False, use_metal=False)
        _randomise(layer, 42)
        layers.append(layer)
    x = torch.randn(1, 16, 64)
    assert torch.equal(layers[0](x), layers[1](x))
    buf = io.BytesIO()
    pickle.dump(layers[0], buf)
    buf.seek(0)
    loaded = pickle.load(buf)  # written by this test
    for (k1, v1), (k2, v2) in zip(layers[0].state_dict().items(), loaded.state_dict().items()):
        assert k1 == k2 and torch.equal(v1, v2), k1
    assert torch.equal(loaded(x), layers[0](x))
    ref = O.mhc_forward_reference(np_of(x), np_of(loaded.H_pre_raw), np_of(loaded.H_post_raw),
                                  np_of(loaded.H_res_raw), np_of(loaded.rms_weight),
                                  sinkhorn_iters=loaded.sinkhorn_iters, eps=loaded.eps)
    assert rel_err(np_of(loaded(x)), ref) < 1e-5
    assert np.isfinite(np_of(loaded(x))).all()

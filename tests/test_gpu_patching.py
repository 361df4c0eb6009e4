"""AutoPatcher on the GPU: a patched mock Llama block (examples/patch_llama_mock.py of
the reference) runs its rewired layers through the HIP kernels, forward and
backward, and agrees with the float64 oracle layer by layer."""

import copy

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import np_of, rel_err

from mhc_mlx_amd import AutoPatcher, MHCRewire, kernel_timer

pytestmark = pytest.mark.gpu


class Attention(torch.nn.Module):
    def __init__(self, dims):
        super().__init__()
        self.wq = torch.nn.Linear(dims, dims, bias=False)
        self.wk = torch.nn.Linear(dims, dims, bias=False)
        self.wv = torch.nn.Linear(dims, dims, bias=False)
        self.wo = torch.nn.Linear(dims, dims, bias=False)

    def forward(self, x):
        q, k, v = self.wq(x), self.wk(x), self.wv(x)
        s = torch.softmax((q.float() @ k.float().transpose(1, 2).contiguous()) / x.shape[-1] ** 0.5, dim=-1)
        return self.wo((s @ v.float()).to(x.dtype))


class MLP(torch.nn.Module):
    def __init__(self, dims, hidden):
        super().__init__()
        self.w1 = torch.nn.Linear(dims, hidden, bias=False)
        self.w2 = torch.nn.Linear(hidden, dims, bias=False)
        self.w3 = torch.nn.Linear(dims, hidden, bias=False)

    def forward(self, x):
        return self.w2(torch.nn.functional.silu(self.w1(x)) * self.w3(x))


class Block(torch.nn.Module):
    def __init__(self, dims, hidden):
        super().__init__()
        self.attention_norm = torch.nn.RMSNorm(dims)
        self.attention = Attention(dims)
        self.ffn_norm = torch.nn.RMSNorm(dims)
        self.feed_forward = MLP(dims, hidden)

    def forward(self, x):
        h = x + self.attention(self.attention_norm(x))
        return h + self.feed_forward(self.ffn_norm(h))


def _randomise(model, seed):
    g = torch.Generator().manual_seed(seed)
    for m in model.modules():
        if isinstance(m, MHCRewire):
            with torch.no_grad():
                for p in (m.mhc.H_pre_raw, m.mhc.H_post_raw, m.mhc.H_res_raw):
                    p.copy_(torch.randn(p.shape, generator=g))


def test_patched_block_uses_the_hip_kernels_and_matches_torch_path():
    dims, hidden, n = 256, 512, 4
    torch.manual_seed(0)
    block = Block(dims, hidden).cuda()
    ref_block = copy.deepcopy(block)
    assert AutoPatcher.patch(block, n_streams=n, verbose=False) == 4          # wq, wk, wv, wo
    assert AutoPatcher.patch(ref_block, n_streams=n, verbose=False, use_metal=False) == 4
    _randomise(block, 1)
    _randomise(ref_block, 1)
    x = torch.randn(2, 16, dims, device="cuda")
    xr = x.clone().requires_grad_(True)
    x.requires_grad_(True)
    with kernel_timer() as kt:
        y = block(x)
        y.square().sum().backward()
        names = set(kt.stats())
    assert {"stream_scale_fwd", "stream_mix_add_fwd", "stream_mix_add_bwd", "stream_scale_bwd"} <= names
    yr = ref_block(xr)
    yr.square().sum().backward()
    assert rel_err(np_of(y), np_of(yr)) < 1e-5
    assert rel_err(np_of(x.grad), np_of(xr.grad)) < 1e-5
    for (na, a), (nb, b) in zip(block.named_parameters(), ref_block.named_parameters()):
        assert na == nb
        if na.endswith("mhc.rms_weight"):   # MHCRewire does not use the RMSNorm weight (layer.py:469-492)
            assert a.grad is None and b.grad is None
            continue
        assert rel_err(np_of(a.grad), np_of(b.grad)) < 1e-5, na


def test_patched_linear_matches_oracle():
    dims, n, T = 512, 16, 8
    g = np.random.default_rng(3)
    model = torch.nn.Sequential(torch.nn.Linear(dims, dims, bias=False)).cuda()
    W = (0.02 * g.standard_normal((dims, dims))).astype(np.float32)
    with torch.no_grad():
        model[0].weight.copy_(torch.from_numpy(W))
    AutoPatcher.patch(model, n_streams=n, verbose=False, identity_init=False)
    hpre, hpost = g.standard_normal(n).astype(np.float32), g.standard_normal(n).astype(np.float32)
    hres = g.standard_normal((n, n)).astype(np.float32)
    rw = model[0]
    with torch.no_grad():
        rw.mhc.H_pre_raw.copy_(torch.from_numpy(hpre))
        rw.mhc.H_post_raw.copy_(torch.from_numpy(hpost))
        rw.mhc.H_res_raw.copy_(torch.from_numpy(hres))
    x = g.standard_normal((T, dims)).astype(np.float32)
    out = model(torch.from_numpy(x).cuda())
    ref, _ = O.rewire_linear_forward(x, W, hpre, hpost, hres)
    assert rel_err(np_of(out), ref) < 1e-5


def test_patched_bf16_model_trains():
    dims, hidden, n = 256, 512, 8
    torch.manual_seed(1)
    block = Block(dims, hidden).cuda().to(torch.bfloat16)
    AutoPatcher.patch(block, n_streams=n, verbose=False)
    assert block.attention.wq.return_dtype == torch.bfloat16
    assert block.attention.wq.mhc.H_res_raw.device.type == "cuda"
    x = torch.randn(2, 8, dims, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    y = block(x)
    assert y.dtype == torch.bfloat16 and torch.isfinite(y.float()).all()
    y.float().square().mean().backward()
    for name, p in block.named_parameters():
        if name.endswith("mhc.rms_weight"):
            continue
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), name

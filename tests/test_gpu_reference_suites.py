"""GPU restatements of the reference's vision, stress, determinism and
concurrency tests, checked against the float64 oracle.

- tests/test_vision.py:5-47 (MHCRewire around a Conv2d on [B, H, W, C] with
  n=16, and around a ViT block on [B, L, D] with n=32);
- tests/test_stress.py:36-111 (B=1, n=8, C=4096 fp16 forward; seed sweep);
- tests/test_determinism.py:7-47 (same seed, same layer and output; pickling);
- tests/test_concurrency.py:10-58 (four processes running fwd+bwd at once).

MLX's random streams are not available, so the inputs come from this build's
seeded generators; the reference's assertions are kept and each result is
also compared with the oracle.
"""

import io
import multiprocessing as mp
import pickle

import numpy as np
import pytest
import torch
from torch import nn

from oracle import mhc_oracle as O
from tests._helpers import dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import MHCLayer, MHCRewire, ops

pytestmark = pytest.mark.gpu


class _NHWCConv(nn.Module):
    """MLX's Conv2d takes channels-last input; torch's takes NCHW."""

    def __init__(self, c: int):
        super().__init__()
        self.conv = nn.Conv2d(c, c, kernel_size=3, padding=1)

    def forward(self, x):
        return self.conv(x.permute(0, 3, 1, 2)).permute(0, 2, 3, 1)


class _ViTBlock(nn.Module):
    def __init__(self, d: int):
        super().__init__()
        self.norm = nn.LayerNorm(d)
        self.linear = nn.Linear(d, d)

    def forward(self, x):
        return self.linear(self.norm(x))


def _randomise(layer: MHCLayer, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in (layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw):
            p.copy_(torch.randn(p.shape, generator=g))


def _check_rewire_against_oracle(model: MHCRewire, x: torch.Tensor, n: int):
    """out == H_post * (inner(H_pre x) + M diag(H_pre) x) with the inner output captured."""
    seen = {}
    hook = model.inner.register_forward_hook(lambda m, i, o: seen.__setitem__("y", o.detach()))
    y = model(x)
    hook.remove()
    C = x.shape[-1] // n
    x3 = np_of(x).reshape(-1, n, C)
    y3 = np_of(seen["y"]).reshape(-1, n, C)
    mh = model.mhc
    ref = O.post_combine(x3, y3, np_of(mh.H_pre_raw), np_of(mh.H_post_raw), np_of(mh.H_res_raw),
                         sinkhorn_iters=mh.sinkhorn_iters, eps=mh.eps)
    assert rel_err(np_of(y).reshape(-1, n, C), ref) < 1e-5
    return y


def test_conv2d_rewire():
    """test_vision.py:5-23: Conv2d wrapped on a 4-D input, n=16."""
    torch.manual_seed(0)
    B, H, W, C, n = 2, 32, 32, 64, 16
    inner = _NHWCConv(C).cuda()
    model = MHCRewire(inner, dims=C, n=n).cuda()
    _randomise(model.mhc, 1)
    x = torch.randn(B, H, W, C, device="cuda")
    y = _check_rewire_against_oracle(model, x, n)
    assert y.shape == (B, H, W, C)
    assert not torch.equal(y, inner(x))  # the mHC mix is applied


def test_vision_transformer_block_rewire():
    """test_vision.py:25-43: a LayerNorm + Linear block on [B, L, D], n=32 (16 < n <= 64 kernels)."""
    torch.manual_seed(1)
    B, L, D, n = 2, 196, 256, 32
    model = MHCRewire(_ViTBlock(D), dims=D, n=n).cuda()
    _randomise(model.mhc, 2)
    x = torch.randn(B, L, D, device="cuda")
    y = _check_rewire_against_oracle(model, x, n)
    assert y.shape == (B, L, D)
    (y.float().square().mean()).backward()
    # rms_weight belongs to the wrapped MHCLayer but not to the post-combine
    used = list(model.inner.parameters()) + [model.mhc.H_pre_raw, model.mhc.H_post_raw, model.mhc.H_res_raw]
    for p in used:
        assert p.grad is not None and torch.isfinite(p.grad).all()


def test_large_c_forward_fp16():
    """test_stress.py:36-75: B=1, n=8, C=4096 fp16, 10 Sinkhorn iterations, fp16 out, |err| < 5e-2."""
    g = rng(321)
    B, n, C = 1, 8, 4096
    x = to_dtype_np(g.standard_normal((B, n, C)), "f16")
    hpre, hpost, hres, _ = params(g, n, C)
    w = np.ones(C, np.float32)
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=10, eps=1e-5)
    a, p = O.activate_pre_post(hpre, hpost, np.float32)
    M = O.mixing_matrix_from_logits(hres, iters=10, eps=1e-5, dtype=np.float32)
    out = ops.mhc_forward_fused_hip(dev_tensor(x, "f16"), dev_tensor(M), dev_tensor(a), dev_tensor(p),
                                    dev_tensor(w), eps=1e-5, output_dtype=torch.float16)
    assert out.dtype == torch.float16
    got = np_of(out)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() < 5e-2
    assert rel_err(got, ref) < 5e-3  # the fp16 bar of test_correctness.py:52-96


@pytest.mark.parametrize("seed", [1, 7, 13])
def test_seed_sweep_bf16(seed):
    """test_stress.py:78-111: B=2, n=4, C=256 bf16, 10 iterations; finite, and within the bf16 bar."""
    g = rng(seed)
    B, n, C = 2, 4, 256
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    hpre, hpost, hres, _ = params(g, n, C)
    w = np.ones(C, np.float32)
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=10, eps=1e-5)
    a, p = O.activate_pre_post(hpre, hpost, np.float32)
    M = O.mixing_matrix_from_logits(hres, iters=10, eps=1e-5, dtype=np.float32)
    out = ops.mhc_forward_fused_hip(dev_tensor(x, "bf16"), dev_tensor(M), dev_tensor(a), dev_tensor(p),
                                    dev_tensor(w), eps=1e-5)
    got = np_of(out)
    assert np.isfinite(got).all()
    assert rel_err(got, ref) < 1e-5  # fp32 output by default (layer.py:361-364)


def test_initialization_determinism():
    """test_determinism.py:7-26: the same seed gives the same parameters and output."""
    n, C = 16, 64
    layers = []
    for _ in range(2):
        torch.manual_seed(42)
        layer = MHCLayer(n=n, C=C, identity_init=False).cuda()
        _randomise(layer, 42)
        layers.append(layer)
    for (k1, v1), (k2, v2) in zip(layers[0].state_dict().items(), layers[1].state_dict().items()):
        assert k1 == k2 and torch.equal(v1, v2), k1
    x = torch.randn(1, n, C, device="cuda")
    assert torch.equal(layers[0](x), layers[1](x))


def test_pickling():
    """test_determinism.py:29-47: a layer survives pickling with its parameters, and still runs."""
    n, C = 16, 64
    layer = MHCLayer(n=n, C=C).cuda()
    _randomise(layer, 3)
    buf = io.BytesIO()
    pickle.dump(layer, buf)
    buf.seek(0)
    loaded = pickle.load(buf)  # written by this test
    for (k1, v1), (k2, v2) in zip(layer.state_dict().items(), loaded.state_dict().items()):
        assert k1 == k2 and torch.equal(v1, v2), k1
    x = torch.randn(2, n, C, device="cuda")
    assert torch.equal(layer(x), loaded(x))


def _stress_proc(proc_id: int, n_iters: int, q) -> None:
    try:
        torch.manual_seed(proc_id)
        B, n, C = 2, 32, 512
        layer = MHCLayer(n=n, C=C).cuda()
        for _ in range(n_iters):
            x = torch.randn(B, n, C, device="cuda")
            loss = layer(x).sum()
            grads = torch.autograd.grad(loss, list(layer.parameters()))
            assert all(torch.isfinite(gr).all() for gr in grads)
        torch.cuda.synchronize()
        q.put((proc_id, "ok"))
    except Exception as e:  # reported to the parent, which fails the test
        q.put((proc_id, repr(e)))


def test_multiprocess_fwd_bwd():
    """test_concurrency.py:40-55: four processes run MHCLayer(n=32, C=512) fwd+bwd 50 times at once."""
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    procs = [ctx.Process(target=_stress_proc, args=(i, 50, q)) for i in range(4)]
    try:
        for p in procs:
            p.start()
        for p in procs:
            p.join(timeout=240)  # each child imports torch first
        for p in procs:
            assert p.exitcode == 0, p.exitcode
        results = dict(q.get(timeout=5) for _ in procs)
    finally:
        for p in procs:
            if p.is_alive():
                p.kill()
                p.join()
    assert results == {i: "ok" for i in range(4)}, results

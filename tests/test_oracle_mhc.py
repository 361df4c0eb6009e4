"""CPU: pin the oracle's fused forward, backward and MHCRewire restatements.

Independent checks:
* brute force: scalar loops over (b, i, c) restating reference.py:72-184
* identity init gives out ~= x (reference test_identity_mapping_n4);
  M = I with H_post -> 0 gives x; the mix term is linear in x
* backward: torch.autograd (float64) of the package's torch restatement
  (reference.py restated in torch) and central finite differences
* MHCRewire: the explicit (non-folded) formulation of layer.py:332-337 and
  its autograd; weight-folding equivalence (reference test_folding.py)
"""

import math

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O


def _brute_forward(x, hpre, hpost, hres, w, iters, eps):
    B, n, C = x.shape
    a = [1 / (1 + math.exp(-v)) for v in hpre]
    p = [2 / (1 + math.exp(-v)) for v in hpost]
    M = O.mixing_matrix_from_logits(hres, iters, eps)
    out = np.zeros((B, n, C))
    for b in range(B):
        y = [sum(a[i] * x[b, i, c] for i in range(n)) for c in range(C)]
        inv = 1.0 / math.sqrt(sum(v * v for v in y) / C + eps)
        for i in range(n):
            for c in range(C):
                out[b, i, c] = sum(M[i, j] * x[b, j, c] for j in range(n)) + p[i] * y[c] * inv * w[c]
    return out


def _params(seed, n, C):
    g = np.random.default_rng(seed)
    return g.standard_normal(n), g.standard_normal(n), g.standard_normal((n, n)), 1 + 0.02 * g.standard_normal(C)


@pytest.mark.parametrize("B,n,C", [(1, 4, 8), (2, 3, 5), (2, 1, 7)])
def test_forward_vs_brute_force(B, n, C):
    hpre, hpost, hres, w = _params(B + n + C, n, C)
    x = np.random.default_rng(1).standard_normal((B, n, C))
    got = O.mhc_forward_reference(x, hpre, hpost, hres, w, 20, 1e-5)
    assert np.allclose(got, _brute_forward(x, hpre, hpost, hres, w, 20, 1e-5), atol=1e-12)


def test_identity_init_passthrough():
    n, C = 4, 64
    x = np.random.default_rng(123).standard_normal((2, n, C))
    out = O.mhc_forward_reference(x, np.full(n, -12.0), np.full(n, -12.0),
                                  np.full((n, n), -12.0) + np.eye(n) * 12.0, np.ones(C))
    assert np.abs(out - x).max() < 1e-4


def test_identity_mix_and_linearity():
    g = np.random.default_rng(2)
    B, n, C = 2, 4, 16
    x1, x2 = g.standard_normal((2, B, n, C))
    M = np.eye(n)
    a = np.full(n, 0.3)
    p = np.zeros(n)
    assert np.allclose(O.mhc_forward_fused_reference(x1, M, a, p, np.ones(C)), x1)
    Mr = g.random((n, n))
    mix = lambda v: O.stream_mix_ref(v, Mr)
    assert np.allclose(mix(2 * x1 + 3 * x2), 2 * mix(x1) + 3 * mix(x2))


def test_per_token_equals_static_per_token():
    g = np.random.default_rng(3)
    B, n, C = 3, 4, 8
    x = g.standard_normal((B, n, C))
    hpre, hpost, hres = g.standard_normal((B, n)), g.standard_normal((B, n)), g.standard_normal((B, n, n))
    w = g.standard_normal(C)
    out = O.mhc_forward_reference(x, hpre, hpost, hres, w)
    for b in range(B):
        assert np.allclose(out[b], O.mhc_forward_reference(x[b:b + 1], hpre[b], hpost[b], hres[b], w)[0])


def test_bf16_round_is_rne():
    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -2.5e-3, 3.0e38, np.inf], np.float32)
    t = torch.tensor(vals).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_round(vals), t)


# ------------------------------------------------------------------ backward

def _torch_grads(x, hpre, hpost, hres, w, dout, iters, eps):
    from mhc_mlx_amd import reference as R

    ts = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, hpre, hpost, hres, w)]
    out = R.mhc_forward_reference(*ts, sinkhorn_iters=iters, eps=eps)
    return [g.numpy() for g in torch.autograd.grad(out, ts, torch.tensor(dout, dtype=torch.float64))]


@pytest.mark.parametrize("B,n,C", [(2, 4, 16), (3, 3, 7), (2, 8, 5), (1, 1, 9)])
def test_backward_vs_torch_autograd(B, n, C):
    g = np.random.default_rng(B * 100 + n * 10 + C)
    x = g.standard_normal((B, n, C))
    dout = g.standard_normal((B, n, C))
    hpre, hpost, hres, w = _params(7 + n, n, C)
    got = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, 20, 1e-5)
    ref = _torch_grads(x, hpre, hpost, hres, w, dout, 20, 1e-5)
    for a, b in zip(got, ref):
        assert np.allclose(a, b, atol=1e-11, rtol=1e-9)


def test_per_token_backward_vs_torch_autograd():
    g = np.random.default_rng(11)
    B, n, C = 3, 5, 6
    x = g.standard_normal((B, n, C))
    dout = g.standard_normal((B, n, C))
    hpre, hpost, hres = g.standard_normal((B, n)), g.standard_normal((B, n)), g.standard_normal((B, n, n))
    w = 1 + 0.1 * g.standard_normal(C)
    got = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, 20, 1e-5)
    ref = _torch_grads(x, hpre, hpost, hres, w, dout, 20, 1e-5)
    for a, b in zip(got, ref):
        assert np.allclose(a, b, atol=1e-11, rtol=1e-9)


def test_backward_vs_finite_differences():
    g = np.random.default_rng(12)
    B, n, C = 2, 3, 4
    x = g.standard_normal((B, n, C))
    dout = g.standard_normal((B, n, C))
    hpre, hpost, hres, w = _params(13, n, C)
    args = [x, hpre, hpost, hres, w]
    got = O.mhc_backward_reference(*args, dout, 6, 1e-5)
    h = 1e-6
    for k, arr in enumerate(args):
        fd = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            ap, am = [a.copy() for a in args], [a.copy() for a in args]
            ap[k][idx] += h
            am[k][idx] -= h
            fd[idx] = ((O.mhc_forward_reference(*ap, 6, 1e-5) - O.mhc_forward_reference(*am, 6, 1e-5)) * dout).sum() / (2 * h)
        assert np.allclose(got[k], fd, atol=1e-7), k


def test_fused_backward_activated_contract():
    """Grads w.r.t. activated H chain to raw grads through s(1-s) and 2 s(1-s)."""
    g = np.random.default_rng(14)
    B, n, C = 2, 4, 8
    x, dout = g.standard_normal((2, B, n, C))
    hpre, hpost, hres, w = _params(15, n, C)
    a, p = O.activate_pre_post(hpre, hpost)
    M = O.mixing_matrix_from_logits(hres, 20)
    _, dM, dA, dP, _ = O.mhc_fused_backward(x, M, a, p, w, dout)
    _, dpre, dpost, dres, _ = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout)
    assert np.allclose(dpre, dA * a * (1 - a))
    s = p / 2
    assert np.allclose(dpost, dP * 2 * s * (1 - s))
    assert np.allclose(dres, O.sinkhorn_knopp_vjp(hres, dM, 20))


# ------------------------------------------------------------------ MHCRewire

def _torch_post_combine(x, y, hpre, hpost, hres, iters, eps):
    from mhc_mlx_amd import reference as R

    a, p = R.activate_pre_post(hpre, hpost)
    M = R.mixing_matrix_from_logits(hres, iters, eps)
    Mf = M * a.reshape(1, -1)
    return (y + torch.einsum("ij,bjd->bid", Mf, x)) * p.reshape(1, -1, 1)


def test_post_combine_and_backward_vs_torch():
    g = np.random.default_rng(16)
    B, n, C = 3, 4, 6
    x, y, dout = g.standard_normal((3, B, n, C))
    hpre, hpost, hres, _ = _params(17, n, C)
    ts = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, y, hpre, hpost, hres)]
    out = _torch_post_combine(*ts, 20, 1e-5)
    assert np.allclose(out.detach().numpy(), O.post_combine(x, y, hpre, hpost, hres))
    ref = torch.autograd.grad(out, ts, torch.tensor(dout))
    got = O.post_combine_backward(x, y, hpre, hpost, hres, dout)
    for a, b in zip(got, ref):
        assert np.allclose(a, b.numpy(), atol=1e-11)


def test_rewire_linear_backward_vs_torch():
    g = np.random.default_rng(18)
    T, n, C = 3, 4, 5
    dims = n * C
    x = g.standard_normal((T, dims))
    W = 0.1 * g.standard_normal((dims, dims))
    dout = g.standard_normal((T, dims))
    hpre, hpost, hres, _ = _params(19, n, C)
    ts = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, W, hpre, hpost, hres)]
    from mhc_mlx_amd import reference as R

    a, _ = R.activate_pre_post(ts[2], ts[3])
    x3 = ts[0].reshape(T, n, C)
    y = ((x3 * a.reshape(1, n, 1)).reshape(T, dims) @ ts[1].T).reshape(T, n, C)
    out = _torch_post_combine(x3, y, ts[2], ts[3], ts[4], 20, 1e-5).reshape(T, dims)
    o, _ = O.rewire_linear_forward(x, W, hpre, hpost, hres)
    assert np.allclose(out.detach().numpy(), o)
    ref = torch.autograd.grad(out, ts, torch.tensor(dout))
    got = O.rewire_linear_backward(x, W, hpre, hpost, hres, dout)
    for a_, b_ in zip(got, ref):
        assert np.allclose(a_, b_.numpy(), atol=1e-10)

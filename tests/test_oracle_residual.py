"""CPU: pin the oracle's residual_add_agg and its VJP (utils.py:4-24).

Independent checks:
* brute force: scalar loops over (b, i, c) restating residual_add_agg.metal:39-66
* res = 0 reduces y_agg to stream_aggregate (reference.py:72-86), which is
  pinned separately; the op is symmetric in (x, res); a one-hot H_pre picks
  out one stream of x + res
* backward: torch.autograd (float64) of an independent torch formulation
  and central finite differences
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O


def _brute(x, res, h):
    B, n, C = x.shape
    out = np.zeros((B, n, C))
    y = np.zeros((B, C))
    for b in range(B):
        for c in range(C):
            acc = 0.0
            for i in range(n):
                v = float(x[b, i, c]) + float(res[b, i, c])
                out[b, i, c] = v
                acc += v * float(h[i])
            y[b, c] = acc
    return out, y


@pytest.mark.parametrize("B,n,C", [(1, 4, 8), (2, 3, 5), (3, 1, 7), (2, 6, 3)])
def test_forward_vs_brute_force(B, n, C):
    g = np.random.default_rng(B * 100 + n * 10 + C)
    x, res, h = g.standard_normal((B, n, C)), g.standard_normal((B, n, C)), g.standard_normal(n)
    out, y = O.residual_add_agg(x, res, h)
    bo, by = _brute(x, res, h)
    assert np.allclose(out, bo, atol=1e-13) and np.allclose(y, by, atol=1e-12)


def test_zero_residual_is_stream_aggregate():
    g = np.random.default_rng(3)
    x, h = g.standard_normal((4, 5, 33)), g.standard_normal(5)
    out, y = O.residual_add_agg(x, np.zeros_like(x), h)
    assert np.array_equal(out, x)
    assert np.allclose(y, O.stream_aggregate(x, h), atol=1e-13)


def test_symmetric_and_one_hot():
    g = np.random.default_rng(4)
    x, res = g.standard_normal((2, 4, 9)), g.standard_normal((2, 4, 9))
    h = g.standard_normal(4)
    a = O.residual_add_agg(x, res, h)
    b = O.residual_add_agg(res, x, h)
    assert np.allclose(a[0], b[0]) and np.allclose(a[1], b[1])
    for k in range(4):
        e = np.zeros(4)
        e[k] = 1.0
        _, y = O.residual_add_agg(x, res, e)
        assert np.allclose(y, x[:, k] + res[:, k], atol=1e-14)


def _torch_loss(x, res, h, dout, dy):
    val = x + res
    y = (val * h[None, :, None]).sum(dim=1)
    return (val * dout).sum() + (y * dy).sum()


@pytest.mark.parametrize("which", ["both", "out_only", "y_only"])
def test_backward_vs_torch_autograd(which):
    g = np.random.default_rng(5)
    B, n, C = 3, 4, 11
    x, res, h = g.standard_normal((B, n, C)), g.standard_normal((B, n, C)), g.standard_normal(n)
    dout = g.standard_normal((B, n, C)) if which != "y_only" else None
    dy = g.standard_normal((B, C)) if which != "out_only" else None
    tx, tr, th = (torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, res, h))
    td = torch.zeros((B, n, C), dtype=torch.float64) if dout is None else torch.tensor(dout)
    ty = torch.zeros((B, C), dtype=torch.float64) if dy is None else torch.tensor(dy)
    _torch_loss(tx, tr, th, td, ty).backward()
    dx, dres, dh = O.residual_add_agg_backward(x, res, h, dout, dy)
    assert np.allclose(dx, tx.grad.numpy(), atol=1e-12)
    assert np.allclose(dres, tr.grad.numpy(), atol=1e-12)
    assert np.allclose(dh, th.grad.numpy(), atol=1e-11)


def test_backward_finite_differences():
    g = np.random.default_rng(6)
    B, n, C = 2, 3, 4
    x, res, h = g.standard_normal((B, n, C)), g.standard_normal((B, n, C)), g.standard_normal(n)
    dout, dy = g.standard_normal((B, n, C)), g.standard_normal((B, C))

    def loss(x_, r_, h_):
        o, y = O.residual_add_agg(x_, r_, h_)
        return float((o * dout).sum() + (y * dy).sum())

    dx, _, dh = O.residual_add_agg_backward(x, res, h, dout, dy)
    step = 1e-6
    for idx in [(0, 0, 0), (1, 2, 3), (0, 1, 2)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += step
        xm[idx] -= step
        assert abs((loss(xp, res, h) - loss(xm, res, h)) / (2 * step) - dx[idx]) < 1e-7
    for k in range(n):
        hp, hm = h.copy(), h.copy()
        hp[k] += step
        hm[k] -= step
        assert abs((loss(x, res, hp) - loss(x, res, hm)) / (2 * step) - dh[k]) < 1e-6

"""CPU: pin the oracle's Sinkhorn forward and VJP (no GPU).

Independent checks (never a retyped formula):
* brute force: scalar pure-Python loops restating reference.py:20-48, 58-69
* closed forms: rank-1 (additive) logits -> 1/n after one iteration;
  constant logits -> 1/n; identity init -> I; the 2x2 limit
  sqrt(ad)/(sqrt(ad)+sqrt(bc)); a doubly-stochastic exp(H) is a fixed point
* invariances: per-row logit shifts; unit column sums after the last step
* VJP: torch.autograd (float64) of the package's torch restatement, central
  finite differences, zero row sums, dM = 1 c^T -> 0
"""

import math

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O


def _brute_sinkhorn(H, iters, eps):
    n = len(H)
    mx = [max(r) for r in H]
    P = [[math.exp(H[i][j] - mx[i]) for j in range(n)] for i in range(n)]
    for _ in range(iters):
        for i in range(n):
            s = sum(P[i])
            sc = 1.0 / s if s > eps else 1.0
            P[i] = [v * sc for v in P[i]]
        for j in range(n):
            s = sum(P[i][j] for i in range(n))
            sc = 1.0 / s if s > eps else 0.0
            for i in range(n):
                P[i][j] *= sc
    return np.array(P)


@pytest.mark.parametrize("n", [1, 2, 3, 4, 6])
@pytest.mark.parametrize("iters", [0, 1, 3, 20])
def test_sinkhorn_vs_brute_force(n, iters):
    H = np.random.default_rng(n * 10 + iters).standard_normal((n, n))
    assert np.allclose(O.mixing_matrix_from_logits(H, iters=iters), _brute_sinkhorn(H.tolist(), iters, 1e-5),
                       atol=1e-14, rtol=1e-12)


def test_sinkhorn_masks_vs_brute_force():
    H = np.random.default_rng(4).standard_normal((5, 5))
    H[:, 1] = -40.0
    H[2, :] = -45.0
    H[2, 1] = 0.0
    for eps in (1e-5, 1e-3):
        ref = _brute_sinkhorn(H.tolist(), 20, eps)
        assert np.allclose(O.mixing_matrix_from_logits(H, iters=20, eps=eps), ref, atol=1e-14)
    # a column with only e^-40 mass falls below eps and is zeroed
    H2 = np.random.default_rng(5).standard_normal((4, 4))
    H2[:, 2] = -40.0
    M2 = O.mixing_matrix_from_logits(H2, iters=20, eps=1e-5)
    assert np.allclose(M2, _brute_sinkhorn(H2.tolist(), 20, 1e-5), atol=1e-14)
    assert np.abs(M2[:, 2]).max() == 0.0


def test_rank_one_logits_give_uniform_after_one_iteration():
    g = np.random.default_rng(1)
    a, b = g.standard_normal(5), g.standard_normal(5)
    M = O.mixing_matrix_from_logits(a[:, None] + b[None, :], iters=1)
    assert np.allclose(M, 1.0 / 5, atol=1e-15)


def test_constant_logits_bomb():
    M = O.mixing_matrix_from_logits(np.full((32, 32), 100.0), iters=20, dtype=np.float32)
    assert np.isfinite(M).all() and np.allclose(M, 1.0 / 32, atol=1e-7)


def test_identity_init():
    n = 8
    M = O.mixing_matrix_from_logits(np.full((n, n), -12.0) + np.eye(n) * 12.0, iters=20)
    assert np.abs(M - np.eye(n)).max() < 1e-4


def test_two_by_two_limit():
    H = np.array([[0.3, -0.7], [1.1, 0.2]])
    a, b, c, d = np.exp(H).ravel()
    p = math.sqrt(a * d) / (math.sqrt(a * d) + math.sqrt(b * c))
    M = O.mixing_matrix_from_logits(H, iters=200)
    assert np.allclose(M, [[p, 1 - p], [1 - p, p]], atol=1e-12)


def test_doubly_stochastic_fixed_point():
    # exp(H) with H = log(D) for a doubly-stochastic D stays D
    D = np.array([[0.2, 0.5, 0.3], [0.5, 0.1, 0.4], [0.3, 0.4, 0.3]])
    M = O.mixing_matrix_from_logits(np.log(D), iters=7)
    assert np.allclose(M, D, atol=1e-14)


def test_row_shift_invariance_and_column_sums():
    g = np.random.default_rng(2)
    H = g.standard_normal((3, 6, 6))
    s = g.standard_normal((3, 6, 1)) * 5
    M1 = O.mixing_matrix_from_logits(H, 20)
    M2 = O.mixing_matrix_from_logits(H + s, 20)
    assert np.allclose(M1, M2, atol=1e-13)
    assert np.allclose(M1.sum(-2), 1.0, atol=1e-13)


def test_batched_equals_per_matrix():
    H = np.random.default_rng(3).standard_normal((4, 5, 5))
    Mb = O.mixing_matrix_from_logits(H, 20)
    for k in range(4):
        assert np.array_equal(Mb[k], O.mixing_matrix_from_logits(H[k], 20))


def test_reference_raises_on_non_square():
    with pytest.raises(ValueError, match="square"):
        O.mixing_matrix_from_logits(np.zeros((3, 4)))


# ------------------------------------------------------------------ VJP

def _torch_vjp(H, dM, iters, eps):
    from mhc_mlx_amd import reference as R

    Ht = torch.tensor(H, dtype=torch.float64, requires_grad=True)
    M = R.mixing_matrix_from_logits(Ht, iters=iters, eps=eps)
    (g,) = torch.autograd.grad(M, Ht, torch.tensor(dM, dtype=torch.float64))
    return g.numpy()


@pytest.mark.parametrize("n,iters", [(1, 3), (2, 5), (4, 20), (7, 10), (16, 20)])
def test_vjp_vs_torch_autograd(n, iters):
    g = np.random.default_rng(100 + n)
    H = g.standard_normal((3, n, n))
    dM = g.standard_normal((3, n, n))
    got = O.sinkhorn_knopp_vjp(H, dM, iters=iters)
    ref = _torch_vjp(H, dM, iters, 1e-5)
    assert np.allclose(got, ref, atol=1e-12, rtol=1e-9)


def test_vjp_with_masks_vs_finite_differences():
    """Masked steps are constant scales (1 for rows, 0 for columns).

    Plain autograd of the reference graph is NaN here: once a column is
    zeroed its later sums are exactly 0 and where()'s unused branch 1/0 feeds
    0 * inf into the backward.  The oracle (and the kernels) differentiate the
    piecewise-constant masks, which finite differences confirm away from the
    eps thresholds.
    """
    g = np.random.default_rng(5)
    n, iters = 5, 6
    H = g.standard_normal((n, n))
    H[:, 3] = -40.0
    dM = g.standard_normal((n, n))
    for eps in (1e-5, 1e-3):
        got = O.sinkhorn_knopp_vjp(H, dM, iters, eps)
        h = 1e-6
        fd = np.zeros_like(H)
        for i in range(n):
            for j in range(n):
                Hp, Hm = H.copy(), H.copy()
                Hp[i, j] += h
                Hm[i, j] -= h
                fd[i, j] = ((O.mixing_matrix_from_logits(Hp, iters, eps)
                             - O.mixing_matrix_from_logits(Hm, iters, eps)) * dM).sum() / (2 * h)
        assert np.allclose(got, fd, atol=1e-8)
        assert np.abs(got[:, 3]).max() < 1e-12  # only e^-40-sized entries reach column 3


def test_vjp_vs_finite_differences():
    g = np.random.default_rng(6)
    n, iters = 4, 8
    H = g.standard_normal((n, n))
    dM = g.standard_normal((n, n))
    got = O.sinkhorn_knopp_vjp(H, dM, iters=iters)
    h = 1e-6
    fd = np.zeros_like(H)
    for i in range(n):
        for j in range(n):
            Hp, Hm = H.copy(), H.copy()
            Hp[i, j] += h
            Hm[i, j] -= h
            fd[i, j] = ((O.mixing_matrix_from_logits(Hp, iters) - O.mixing_matrix_from_logits(Hm, iters)) * dM).sum() / (2 * h)
    assert np.allclose(got, fd, atol=1e-8)


def test_vjp_invariants():
    g = np.random.default_rng(7)
    H = g.standard_normal((5, 5))
    dM = g.standard_normal((5, 5))
    assert np.abs(O.sinkhorn_knopp_vjp(H, dM, 20).sum(-1)).max() < 1e-12
    c = g.standard_normal(5)
    assert np.abs(O.sinkhorn_knopp_vjp(H, np.ones((5, 1)) * c[None, :], 20)).max() < 1e-12

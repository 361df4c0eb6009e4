"""Write the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The reference (svdrecbd/mhc-mlx) stores no golden vectors and cannot run in
this environment (it needs MLX), so two kinds of fixtures are kept:

* closed forms, computed here from the mathematics and not from the oracle:
  rank-1 logits (M = 1/n after one iteration), constant logits (the 100.0
  input of tests/test_stability.py:20 of the reference: M = 1/n), the 2 x 2
  limit p = sqrt(ad) / (sqrt(ad) + sqrt(bc)), and a doubly-stochastic exp(H)
  (a fixed point: M = exp(H));
* regression vectors from the float64 oracle (oracle/mhc_oracle.py, pinned
  by tests/test_oracle_*.py) for the BASELINE config-0 recipe, the
  deterministic arange recipe of tests/test_correctness.py:147-156 of the
  reference, a small backward with every gradient, a mini config 3
  (per-token parameters), a small residual_add_agg and a small MHCRewire
  post-combine / pre-scale, each with its gradients.

Inputs are seeded numpy draws; every file is a plain .npz (no pickles).
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import mhc_oracle as O  # noqa: E402


def closed_forms():
    out = {}
    g = np.random.default_rng(11)
    # rank-1 logits: exp(a_i + b_j) is an outer product, one row+column step gives 1/n
    for n in (4, 5):
        a, b = g.standard_normal(n), g.standard_normal(n)
        out[f"rank1_n{n}_H"] = a[:, None] + b[None, :]
        out[f"rank1_n{n}_M"] = np.full((n, n), 1.0 / n)
    # constant logits
    out["const100_n32_H"] = np.full((32, 32), 100.0, np.float32)
    out["const100_n32_M"] = np.full((32, 32), 1.0 / 32)
    # 2x2 limit
    H = np.array([[0.3, -0.7], [1.1, 0.2]])
    a, b, c, d = np.exp(H).ravel()
    p = math.sqrt(a * d) / (math.sqrt(a * d) + math.sqrt(b * c))
    out["two_by_two_H"] = H
    out["two_by_two_M"] = np.array([[p, 1 - p], [1 - p, p]])
    # doubly-stochastic fixed point (a convex combination of permutations)
    P1 = np.eye(4)
    P2 = np.roll(np.eye(4), 1, axis=1)
    P3 = np.roll(np.eye(4), 2, axis=1)
    D = 0.5 * P1 + 0.3 * P2 + 0.2 * P3 + 0.0
    D = 0.9 * D + 0.1 / 4  # strictly positive, still doubly stochastic
    out["fixed_point_H"] = np.log(D).astype(np.float64)
    out["fixed_point_M"] = D
    return out


def cfg0():
    g = np.random.default_rng(0)
    x = g.standard_normal((1, 4, 512)).astype(np.float32)
    hpre = g.standard_normal(4).astype(np.float32)
    hpost = g.standard_normal(4).astype(np.float32)
    hres = g.standard_normal((4, 4)).astype(np.float32)
    w = (1.0 + 0.02 * g.standard_normal(512)).astype(np.float32)
    out = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=1e-6)
    M = O.mixing_matrix_from_logits(hres, iters=20, eps=1e-6)
    return dict(x=x, hpre=hpre, hpost=hpost, hres=hres, w=w, out=out, M=M, iters=20, eps=1e-6)


def arange_kat():
    B, n, C = 2, 4, 129
    hpre = (np.arange(n, dtype=np.float32) * 0.1) - 0.2
    hpost = (np.arange(n, dtype=np.float32) * 0.07) - 0.1
    hres = (np.arange(n * n, dtype=np.float32).reshape(n, n) * 0.01) - 0.05
    w = np.ones(C, np.float32)
    x = np.arange(B * n * C, dtype=np.float32).reshape(B, n, C) * 0.001
    out = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=10, eps=1e-5)
    return dict(x=x, hpre=hpre, hpost=hpost, hres=hres, w=w, out=out, iters=10, eps=1e-5)


def bwd_small():
    g = np.random.default_rng(5)
    B, n, C = 2, 4, 16
    x = g.standard_normal((B, n, C)).astype(np.float32)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    hpre, hpost = g.standard_normal(n).astype(np.float32), g.standard_normal(n).astype(np.float32)
    hres = g.standard_normal((n, n)).astype(np.float32)
    w = (1.0 + 0.02 * g.standard_normal(C)).astype(np.float32)
    out = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=5, eps=1e-5)
    dx, dpre, dpost, dres, dw = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=5, eps=1e-5)
    return dict(x=x, dout=dout, hpre=hpre, hpost=hpost, hres=hres, w=w, out=out, dx=dx, dpre=dpre, dpost=dpost,
                dres=dres, dw=dw, iters=5, eps=1e-5)


def cfg3_mini():
    g = np.random.default_rng(6)
    T, n, C = 8, 16, 32
    x = g.standard_normal((T, n, C)).astype(np.float32)
    dout = g.standard_normal((T, n, C)).astype(np.float32)
    hpre = g.standard_normal((T, n)).astype(np.float32)
    hpost = g.standard_normal((T, n)).astype(np.float32)
    hres = g.standard_normal((T, n, n)).astype(np.float32)
    w = (1.0 + 0.02 * g.standard_normal(C)).astype(np.float32)
    out = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=1e-6)
    dx, dpre, dpost, dres, dw = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=1e-6)
    return dict(x=x, dout=dout, hpre=hpre, hpost=hpost, hres=hres, w=w, out=out, dx=dx, dpre=dpre, dpost=dpost,
                dres=dres, dw=dw, iters=20, eps=1e-6)


def residual_mini():
    """residual_add_agg (utils.py:4-24): bf16-representable inputs, odd C, every gradient."""
    g = np.random.default_rng(7)
    B, n, C = 3, 4, 129
    x = O.bf16_round(g.standard_normal((B, n, C)).astype(np.float32))
    res = O.bf16_round(g.standard_normal((B, n, C)).astype(np.float32))
    h = O.sigmoid(g.standard_normal(n)).astype(np.float32)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    dy = g.standard_normal((B, C)).astype(np.float32)
    out, y_agg = O.residual_add_agg(x, res, h)
    dx, dres, dh = O.residual_add_agg_backward(x, res, h, dout, dy)
    return dict(x=x, res=res, h=h, dout=dout, dy=dy, out=out, y_agg=y_agg, dx=dx, dres=dres, dh=dh)


def rewire_mini():
    """MHCRewire post-combine and pre-scale (layer.py:302-337, 476-480): bf16-representable x and
    y_inner, every gradient of both."""
    g = np.random.default_rng(8)
    B, n, C = 3, 4, 72
    x = O.bf16_round(g.standard_normal((B, n, C)).astype(np.float32))
    y = O.bf16_round(g.standard_normal((B, n, C)).astype(np.float32))
    hpre = g.standard_normal(n).astype(np.float32)
    hpost = g.standard_normal(n).astype(np.float32)
    hres = g.standard_normal((n, n)).astype(np.float32)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    dscale = g.standard_normal((B, n, C)).astype(np.float32)
    out = O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)
    dx, dy, dpre, dpost, dres = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    a = O.sigmoid(hpre.astype(np.float64))
    xs = x * a[None, :, None]

    def scale_vjp(d):
        d = d.astype(np.float64)
        return d * a[None, :, None], np.einsum("bic,bic->i", d, x.astype(np.float64)) * a * (1.0 - a)

    # a bf16 output takes its cotangent in bf16: the expected gradients for that rounding too
    dxs, dpre_s = scale_vjp(dscale)
    dxs16, dpre_s16 = scale_vjp(O.bf16_round(dscale))
    return dict(x=x, y=y, hpre=hpre, hpost=hpost, hres=hres, dout=dout, dscale=dscale, out=out, dx=dx, dy=dy,
                dpre=dpre, dpost=dpost, dres=dres, x_scaled=xs, dx_scaled=dxs, dpre_scaled=dpre_s,
                dx_scaled_bf16=dxs16, dpre_scaled_bf16=dpre_s16)


FIXTURES = {
    "sinkhorn_closed_forms.npz": closed_forms,
    "cfg0_fwd.npz": cfg0,
    "arange_kat.npz": arange_kat,
    "bwd_small.npz": bwd_small,
    "cfg3_mini.npz": cfg3_mini,
    "residual_mini.npz": residual_mini,
    "rewire_mini.npz": rewire_mini,
}


def main() -> None:
    for name, fn in FIXTURES.items():
        np.savez_compressed(HERE / name, **fn())
        print("wrote", HERE / name)


if __name__ == "__main__":
    main()

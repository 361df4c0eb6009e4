"""The HIP path against the golden fixtures of tests/golden/ (GPU)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from tests._helpers import GRAD_TOL, dev_tensor, np_of, rel_err

from mhc_mlx_amd import ops

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("key,iters", [("rank1_n4", 1), ("rank1_n5", 1), ("const100_n32", 20),
                                       ("two_by_two", 200), ("fixed_point", 7)])
def test_sinkhorn_closed_forms(key, iters):
    z = load("sinkhorn_closed_forms.npz")
    M = ops.sinkhorn_knopp_hip(dev_tensor(z[f"{key}_H"]), iters=iters, eps=1e-5)
    assert np.abs(np_of(M) - z[f"{key}_M"]).max() < 2e-6


def _grads_of(z, per_token):
    ps = [dev_tensor(z[k]).requires_grad_(True) for k in ("hpre", "hpost", "hres", "w")]
    xt = dev_tensor(z["x"]).requires_grad_(True)
    it, eps = int(z["iters"]), float(z["eps"])
    f = ops.mhc_layer_forward_dynamic if per_token else ops.mhc_layer_forward
    out = f(xt, *ps, sinkhorn_iters=it, eps=eps)
    out.backward(dev_tensor(z["dout"]))
    return out, [xt.grad] + [p.grad for p in ps]


def test_cfg0_forward():
    z = load("cfg0_fwd.npz")
    out = ops.mhc_layer_forward(*(dev_tensor(z[k]) for k in ("x", "hpre", "hpost", "hres", "w")),
                                sinkhorn_iters=int(z["iters"]), eps=float(z["eps"]))
    assert rel_err(np_of(out), z["out"]) < 1e-5
    M = ops.sinkhorn_knopp_hip(dev_tensor(z["hres"]), iters=int(z["iters"]), eps=float(z["eps"]))
    assert rel_err(np_of(M), z["M"]) < 1e-5


@pytest.mark.parametrize("dt,tol", [("f32", 1e-5), ("bf16", 2e-2), ("f16", 5e-3)])
def test_arange_kat(dt, tol):
    z = load("arange_kat.npz")
    xt = dev_tensor(z["x"], dt)
    out = ops.mhc_layer_forward(xt, *(dev_tensor(z[k]) for k in ("hpre", "hpost", "hres", "w")),
                                sinkhorn_iters=int(z["iters"]), eps=float(z["eps"]),
                                output_dtype=None if dt == "f32" else xt.dtype)
    # the half-precision runs see x rounded to dt; the reference test compares them with the
    # fp32 reference output at these tolerances too (test_correctness.py:138-179)
    assert rel_err(np_of(out), z["out"]) < tol


@pytest.mark.parametrize("name,per_token", [("bwd_small.npz", False), ("cfg3_mini.npz", True)])
def test_backward_fixtures(name, per_token):
    z = load(name)
    out, grads = _grads_of(z, per_token)
    assert rel_err(np_of(out), z["out"]) < 1e-5
    for k, g in zip(["dx", "dpre", "dpost", "dres", "dw"], grads):
        assert rel_err(np_of(g), z[k]) < GRAD_TOL, (k, rel_err(np_of(g), z[k]))


@pytest.mark.parametrize("dt,tol", [("f32", 1e-5), ("bf16", 1e-5)])
def test_residual_fixture(dt, tol):
    """The fixture's inputs are bf16-representable: both dtypes see the same values."""
    z = load("residual_mini.npz")
    xt = dev_tensor(z["x"], dt).requires_grad_(True)
    rt = dev_tensor(z["res"], dt).requires_grad_(True)
    ht = dev_tensor(z["h"]).requires_grad_(True)
    out, y = ops.residual_add_agg_hip(xt, rt, ht)
    assert rel_err(np_of(out), z["out"]) < tol and rel_err(np_of(y), z["y_agg"]) < tol
    torch.autograd.backward([out, y], [dev_tensor(z["dout"]), dev_tensor(z["dy"])])
    assert rel_err(np_of(ht.grad), z["dh"]) < 1e-5
    gtol = 1e-5 if dt == "f32" else 2e-2
    assert rel_err(np_of(xt.grad), z["dx"]) < gtol and rel_err(np_of(rt.grad), z["dres"]) < gtol


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rewire_fixture(dt):
    """MHCRewire post-combine and pre-scale against rewire_mini.npz (bf16-representable x and
    y_inner: both dtypes see the same values; fp32 cotangents)."""
    z = load("rewire_mini.npz")
    xt = dev_tensor(z["x"], dt).requires_grad_(True)
    yt = dev_tensor(z["y"], dt).requires_grad_(True)
    ps = [dev_tensor(z[k]).requires_grad_(True) for k in ("hpre", "hpost", "hres")]
    out = ops.post_combine(xt, yt, *ps, sinkhorn_iters=20, eps=1e-5)
    assert rel_err(np_of(out), z["out"]) < 1e-5
    out.backward(dev_tensor(z["dout"]))
    for name, got in zip(["dx", "dy", "dpre", "dpost", "dres"], [xt.grad, yt.grad] + [p.grad for p in ps]):
        tol = (1e-5 if dt == "f32" else 2e-2) if name in ("dx", "dy") else GRAD_TOL
        assert rel_err(np_of(got), z[name]) < tol, (name, rel_err(np_of(got), z[name]))
    xs = dev_tensor(z["x"], dt).requires_grad_(True)
    hs = dev_tensor(z["hpre"]).requires_grad_(True)
    sc = ops.stream_scale(xs, hs)
    assert rel_err(np_of(sc), z["x_scaled"]) < (1e-6 if dt == "f32" else 1e-2)
    sc.backward(dev_tensor(z["dscale"]))  # cast to the output's dtype by autograd
    sfx = "" if dt == "f32" else "_bf16"
    assert rel_err(np_of(xs.grad), z["dx_scaled" + sfx]) < (1e-6 if dt == "f32" else 1e-2)
    assert rel_err(np_of(hs.grad), z["dpre_scaled" + sfx]) < 1e-5

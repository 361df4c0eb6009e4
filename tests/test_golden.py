"""Golden fixtures of tests/golden/ against the oracle (CPU).

Closed-form fixtures pin the Sinkhorn restatement independently of it;
the oracle-generated fixtures pin the oracle against accidental change
(regenerate with tests/golden/make_golden.py only after a deliberate one).
"""

from pathlib import Path

import numpy as np
import pytest

from oracle import mhc_oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("key,iters", [("rank1_n4", 1), ("rank1_n5", 1), ("const100_n32", 20),
                                       ("two_by_two", 200), ("fixed_point", 7)])
def test_oracle_sinkhorn_closed_forms(key, iters):
    z = load("sinkhorn_closed_forms.npz")
    M = O.mixing_matrix_from_logits(z[f"{key}_H"].astype(np.float64), iters=iters, eps=1e-5)
    assert np.abs(M - z[f"{key}_M"]).max() < 1e-12


def test_oracle_reproduces_cfg0():
    z = load("cfg0_fwd.npz")
    out = O.mhc_forward_reference(z["x"], z["hpre"], z["hpost"], z["hres"], z["w"],
                                  sinkhorn_iters=int(z["iters"]), eps=float(z["eps"]))
    assert np.allclose(out, z["out"], rtol=1e-12, atol=0)
    assert np.allclose(O.mixing_matrix_from_logits(z["hres"], 20, float(z["eps"])), z["M"], rtol=1e-12, atol=0)


def test_oracle_reproduces_arange_kat():
    z = load("arange_kat.npz")
    out = O.mhc_forward_reference(z["x"], z["hpre"], z["hpost"], z["hres"], z["w"],
                                  sinkhorn_iters=int(z["iters"]), eps=float(z["eps"]))
    assert np.allclose(out, z["out"], rtol=1e-12, atol=0)


@pytest.mark.parametrize("name", ["bwd_small.npz", "cfg3_mini.npz"])
def test_oracle_reproduces_backward_fixtures(name):
    z = load(name)
    it, eps = int(z["iters"]), float(z["eps"])
    out = O.mhc_forward_reference(z["x"], z["hpre"], z["hpost"], z["hres"], z["w"], sinkhorn_iters=it, eps=eps)
    assert np.allclose(out, z["out"], rtol=1e-12, atol=1e-15)
    grads = O.mhc_backward_reference(z["x"], z["hpre"], z["hpost"], z["hres"], z["w"], z["dout"],
                                     sinkhorn_iters=it, eps=eps)
    for k, g in zip(["dx", "dpre", "dpost", "dres", "dw"], grads):
        assert np.allclose(g, z[k], rtol=1e-10, atol=1e-14), k


def test_oracle_reproduces_residual_fixture():
    z = load("residual_mini.npz")
    out, y = O.residual_add_agg(z["x"], z["res"], z["h"])
    assert np.allclose(out, z["out"], rtol=1e-12, atol=0) and np.allclose(y, z["y_agg"], rtol=1e-12, atol=1e-15)
    for k, g in zip(["dx", "dres", "dh"], O.residual_add_agg_backward(z["x"], z["res"], z["h"], z["dout"], z["dy"])):
        assert np.allclose(g, z[k], rtol=1e-12, atol=1e-14), k


def test_oracle_reproduces_rewire_fixture():
    z = load("rewire_mini.npz")
    out = O.post_combine(z["x"], z["y"], z["hpre"], z["hpost"], z["hres"], 20, 1e-5)
    assert np.allclose(out, z["out"], rtol=1e-12, atol=1e-15)
    grads = O.post_combine_backward(z["x"], z["y"], z["hpre"], z["hpost"], z["hres"], z["dout"], 20, 1e-5)
    for k, g in zip(["dx", "dy", "dpre", "dpost", "dres"], grads):
        assert np.allclose(g, z[k], rtol=1e-12, atol=1e-14), k

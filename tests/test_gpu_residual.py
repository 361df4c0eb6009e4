"""GPU parity: residual_add_agg (utils.py:4-24, metal.py:1673-1731) and its VJP.

The forward is compared with the float64 oracle at fp32 1e-5 relative (the
reference tests' fp32 tolerance) for y_agg and for an fp32 out; a half out
is compared with the oracle's value rounded to that type (RNE), which the
kernel must reproduce to the type's last bit up to one ulp.  Shapes cover
ragged channel tails (C not a multiple of 8), n = 1 and the maximum n = 64,
every input / output dtype pair and T = 0.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import TORCH_DT, dev_tensor, np_of, rel_err, rng, to_dtype_np

from mhc_mlx_amd import ops, residual_add_agg
from mhc_mlx_amd import metal as metal_names

pytestmark = pytest.mark.gpu


def _inputs(B, n, C, dt, seed):
    g = rng(seed)
    x = to_dtype_np(g.standard_normal((B, n, C)), dt)
    res = to_dtype_np(g.standard_normal((B, n, C)), dt)
    h = O.sigmoid(g.standard_normal(n)).astype(np.float32)
    return x, res, h


@pytest.mark.parametrize("B,n,C", [(3, 4, 64), (2, 4, 129), (5, 1, 8), (2, 8, 1000), (2, 16, 24), (2, 17, 9),
                                   (2, 32, 40), (1, 64, 16), (4, 3, 1), (1, 4, 4096)])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_forward_matches_oracle(B, n, C, dt):
    x, res, h = _inputs(B, n, C, dt, 7 + B * 31 + n * 7 + C)
    out, y = ops.residual_add_agg_hip(dev_tensor(x, dt), dev_tensor(res, dt), dev_tensor(h))
    ro, ry = O.residual_add_agg(x, res, h)
    assert out.dtype == torch.float32 and y.dtype == torch.float32
    assert tuple(out.shape) == (B, n, C) and tuple(y.shape) == (B, C)
    assert rel_err(np_of(out), ro) < 1e-6
    assert rel_err(np_of(y), ry) < 1e-5


@pytest.mark.parametrize("xdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("odt", ["bf16", "f16"])
def test_half_output_is_rounded_sum(xdt, odt):
    B, n, C = 3, 4, 136
    x, res, h = _inputs(B, n, C, xdt, 11)
    out, y = ops.residual_add_agg_hip(dev_tensor(x, xdt), dev_tensor(res, xdt), dev_tensor(h),
                                      output_dtype=TORCH_DT[odt])
    assert out.dtype == TORCH_DT[odt]
    ro, ry = O.residual_add_agg(x, res, h, dtype=np.float32)
    # out is fp32(x + res) rounded once to the output type (RNE)
    assert np.array_equal(np_of(out), to_dtype_np(ro, odt).astype(np.float64))
    # y_agg comes from the unrounded fp32 sum
    assert rel_err(np_of(y), O.residual_add_agg(x, res, h)[1]) < 1e-5


def test_mixed_input_dtypes_are_promoted():
    B, n, C = 2, 4, 32
    x, res, h = _inputs(B, n, C, "bf16", 12)
    out, y = ops.residual_add_agg_hip(dev_tensor(x, "bf16"), dev_tensor(res, "f32"), dev_tensor(h))
    ro, ry = O.residual_add_agg(x, res, h)
    assert rel_err(np_of(out), ro) < 1e-6 and rel_err(np_of(y), ry) < 1e-5


@pytest.mark.parametrize("B,n,C", [(3, 4, 64), (2, 4, 129), (2, 8, 1000), (2, 17, 9), (1, 64, 16), (4, 1, 3)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("which", ["both", "out_only", "y_only"])
def test_backward_matches_oracle(B, n, C, dt, which):
    x, res, h = _inputs(B, n, C, dt, 13 + B + n + C)
    g = rng(14 + n)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    dy = g.standard_normal((B, C)).astype(np.float32)
    xt, rt = dev_tensor(x, dt).requires_grad_(True), dev_tensor(res, dt).requires_grad_(True)
    ht = dev_tensor(h).requires_grad_(True)
    out, y = ops.residual_add_agg_hip(xt, rt, ht)
    if which == "both":
        torch.autograd.backward([out, y], [dev_tensor(dout), dev_tensor(dy)])
        rd, rdy = dout, dy
    elif which == "out_only":
        out.backward(dev_tensor(dout))
        rd, rdy = dout, None
    else:
        y.backward(dev_tensor(dy))
        rd, rdy = None, dy
    rdx, rdres, rdh = O.residual_add_agg_backward(x, res, h, rd, rdy)
    gtol = 1e-5 if dt == "f32" else 2e-2
    assert xt.grad.dtype == xt.dtype and rt.grad.dtype == rt.dtype
    assert rel_err(np_of(xt.grad), rdx) < gtol
    assert rel_err(np_of(rt.grad), rdres) < gtol
    if which == "out_only":
        assert float(ht.grad.abs().max()) == 0.0
    else:
        assert rel_err(np_of(ht.grad), rdh) < 1e-5


def test_backward_half_upstream_gradient():
    """dout in the output's half type (output_dtype=bf16) reaches the kernel without a cast."""
    B, n, C = 2, 4, 256
    x, res, h = _inputs(B, n, C, "bf16", 15)
    dout = to_dtype_np(rng(16).standard_normal((B, n, C)), "bf16")
    xt, rt = dev_tensor(x, "bf16").requires_grad_(True), dev_tensor(res, "bf16").requires_grad_(True)
    ht = dev_tensor(h).requires_grad_(True)
    out, y = ops.residual_add_agg_hip(xt, rt, ht, output_dtype=torch.bfloat16)
    (out.float() * dev_tensor(dout)).sum().backward()
    rdx, _, _ = O.residual_add_agg_backward(x, res, h, dout, None)
    assert rel_err(np_of(xt.grad), rdx) < 2e-2


def test_backward_is_deterministic():
    B, n, C = 512, 4, 512
    x, res, h = _inputs(B, n, C, "bf16", 17)
    dy = dev_tensor(rng(18).standard_normal((B, C)))
    grads = []
    for _ in range(3):
        ht = dev_tensor(h).requires_grad_(True)
        _, y = ops.residual_add_agg_hip(dev_tensor(x, "bf16"), dev_tensor(res, "bf16"), ht)
        y.backward(dy)
        grads.append(ht.grad.clone())
    assert all(torch.equal(grads[0], gg) for gg in grads[1:])


def test_empty_batch():
    x = torch.empty((0, 4, 64), device="cuda", dtype=torch.bfloat16, requires_grad=True)
    ht = torch.rand(4, device="cuda", requires_grad=True)
    out, y = ops.residual_add_agg_hip(x, x.detach().clone(), ht)
    assert tuple(out.shape) == (0, 4, 64) and tuple(y.shape) == (0, 64)
    y.sum().backward()
    assert float(ht.grad.abs().max()) == 0.0


def test_reference_names_and_errors():
    assert metal_names.residual_add_agg_metal is ops.residual_add_agg_hip
    x = torch.randn(2, 4, 8, device="cuda")
    h = torch.rand(4, device="cuda")
    o1, y1 = residual_add_agg(x, x, h)
    assert torch.equal(o1, 2 * x)
    with pytest.raises(ValueError, match="x must be"):
        ops.residual_add_agg_hip(x[0], x[0], h)
    with pytest.raises(ValueError, match="res must match"):
        ops.residual_add_agg_hip(x, x[:1], h)
    with pytest.raises(ValueError, match="threads_per_group"):
        ops.residual_add_agg_hip(x, x, h, threads_per_group=0)
    with pytest.raises(ValueError, match="H_pre"):
        ops.residual_add_agg_hip(x, x, h[:3])
    with pytest.raises(ValueError, match="output_dtype"):
        ops.residual_add_agg_hip(x, x, h, output_dtype=torch.int32)
    with pytest.raises(ValueError, match="MAX_N"):
        ops.residual_add_agg_hip(torch.zeros(1, 65, 4, device="cuda"), torch.zeros(1, 65, 4, device="cuda"),
                                 torch.zeros(65, device="cuda"))


"""GPU parity: MHCRewire kernels (post-combine, pre-scale, stream_mix_add).

Mirrors tests/test_rewire.py and tests/test_folding.py of the reference,
plus gradient comparisons with the float64 oracle.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import GRAD_TOL, TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import MHCRewire, ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,n,C", [(3, 4, 64), (2, 16, 16), (2, 32, 16), (4, 3, 10), (2, 8, 1024)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_post_combine_matches_oracle(B, n, C, xdt):
    g = rng(40 + B + n + C)
    x = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    y = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    hpre, hpost, hres, _ = params(g, n, C)
    xt = dev_tensor(x, xdt).requires_grad_(True)
    yt = dev_tensor(y, xdt).requires_grad_(True)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres)]
    out = ops.post_combine(xt, yt, *ps, sinkhorn_iters=20, eps=1e-5)
    assert out.dtype == torch.float32
    ref = O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)
    assert rel_err(np_of(out), ref) < 1e-5
    out.backward(dev_tensor(dout))
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    gots = [np_of(xt.grad), np_of(yt.grad)] + [np_of(t.grad) for t in ps]
    for name, got, r in zip(["dx", "dy", "dH_pre", "dH_post", "dH_res"], gots, refs):
        tol = (1e-5 if xdt == "f32" else 2e-2) if name in ("dx", "dy") else GRAD_TOL
        assert rel_err(got, r) < tol, (name, B, n, C, xdt, rel_err(got, r))


@pytest.mark.parametrize("gdt", ["bf16", "f32"])
def test_post_combine_bf16_with_bf16_or_fp32_grad(gdt):
    """bf16 x and y with a bf16 gradient (8-channel items) or an fp32 one (4-channel items)."""
    B, n, C = 5, 4, 256
    g = rng(47)
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    y = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt)
    hpre, hpost, hres, _ = params(g, n, C)
    xt = dev_tensor(x, "bf16").requires_grad_(True)
    yt = dev_tensor(y, "bf16").requires_grad_(True)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres)]
    out = ops.post_combine(xt, yt, *ps, sinkhorn_iters=20, eps=1e-5)
    out.backward(dev_tensor(dout, gdt))
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    gots = [np_of(xt.grad), np_of(yt.grad)] + [np_of(t.grad) for t in ps]
    for name, got, r in zip(["dx", "dy", "dH_pre", "dH_post", "dH_res"], gots, refs):
        tol = 2e-2 if name in ("dx", "dy") else GRAD_TOL
        assert rel_err(got, r) < tol, (name, gdt, rel_err(got, r))


@pytest.mark.parametrize("gdt", ["bf16", "f32"])
def test_rewire_kernels_walk_several_items_per_thread(gdt, knobs):
    """One workgroup per CU: each thread walks many (token, chunk) items and, with three
    chunks per token (C = 24), the chunk index wraps between the items of a thread."""
    for env in ("MHC_MIX_FWD_GRID", "MHC_MIX_BWD_GRID", "MHC_SCALE_FWD_GRID", "MHC_SCALE_BWD_GRID"):
        knobs(env, 1)
    B, n, C = 30000, 4, 24
    g = rng(48)
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    y = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt)
    hpre, hpost, hres, _ = params(g, n, C)
    xt = dev_tensor(x, "bf16").requires_grad_(True)
    yt = dev_tensor(y, "bf16").requires_grad_(True)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres)]
    out = ops.post_combine(xt, yt, *ps, sinkhorn_iters=20, eps=1e-5)
    assert rel_err(np_of(out), O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)) < 1e-5
    out.backward(dev_tensor(dout, gdt))
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    gots = [np_of(xt.grad), np_of(yt.grad)] + [np_of(t.grad) for t in ps]
    for name, got, r in zip(["dx", "dy", "dH_pre", "dH_post", "dH_res"], gots, refs):
        tol = 2e-2 if name in ("dx", "dy") else GRAD_TOL
        assert rel_err(got, r) < tol, (name, gdt, rel_err(got, r))
    # pre-scale on the same walk
    ht = dev_tensor(hpre).requires_grad_(True)
    xs = dev_tensor(x, "bf16").requires_grad_(True)
    sc = ops.stream_scale(xs, ht)
    a = O.sigmoid(hpre)
    assert rel_err(np_of(sc), x * a[None, :, None]) < 1e-2
    sc.backward(dev_tensor(dout, "bf16"))
    d16 = to_dtype_np(dout, "bf16").astype(np.float64)
    assert rel_err(np_of(xs.grad), d16 * a[None, :, None]) < 1e-2
    assert rel_err(np_of(ht.grad), np.einsum("bic,bic->i", d16, x) * a * (1 - a)) < GRAD_TOL


def _post_combine_run(x, y, dout, hpre, hpost, hres, xdt, gdt, odt):
    xt = dev_tensor(x, xdt).requires_grad_(True)
    yt = dev_tensor(y, xdt).requires_grad_(True)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres)]
    out = ops.post_combine(xt, yt, *ps, sinkhorn_iters=20, eps=1e-5,
                           output_dtype=None if odt == "f32" else xt.dtype)
    out.backward(dev_tensor(dout, gdt).to(out.dtype))
    return [out.detach().clone(), xt.grad.clone(), yt.grad.clone()] + [t.grad.clone() for t in ps]


@pytest.mark.parametrize("B,n,C", [(5, 32, 128), (3, 24, 64), (2, 17, 192), (4, 32, 1024)])
@pytest.mark.parametrize("xdt,gdt,odt", [("bf16", "f32", "f32"), ("bf16", "bf16", "bf16"), ("f16", "f32", "f32"),
                                         ("f32", "f32", "f32")])
def test_post_combine_mfma_above_16_streams(B, n, C, xdt, gdt, odt, knobs):
    """16 < n <= 32 with C a multiple of 64 runs on the fp32 matrix cores (mix32.hip): forward and every
    gradient against the float64 oracle, per element for the 16-bit outputs (one rounding of the fp32
    result), and against the generic kernels (MHC_MIX32 = 0) to fp32 rounding."""
    g = rng(600 + B + n + C)
    x = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    y = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt if odt == "f32" else odt)
    hpre, hpost, hres, _ = params(g, n, C)
    got = _post_combine_run(x, y, dout, hpre, hpost, hres, xdt, gdt, odt)
    ref_out = O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    names = ["out", "dx", "dy", "dH_pre", "dH_post", "dH_res"]
    for name, t, r in zip(names, got, [ref_out] + list(refs)):
        v = np_of(t)
        if name in ("out", "dx", "dy") and t.dtype != torch.float32:
            ulp = 2.0 ** -8 if t.dtype == torch.bfloat16 else 2.0 ** -11
            assert (np.abs(v - r) <= ulp * np.abs(r) + 1e-5 * np.abs(r).max()).all(), name
        else:
            assert rel_err(v, r) < (1e-5 if name in ("out", "dx", "dy") else GRAD_TOL), (name, rel_err(v, r))
    knobs("MHC_MIX32", 0)
    gen = _post_combine_run(x, y, dout, hpre, hpost, hres, xdt, gdt, odt)
    for name, a, b in zip(names, got, gen):
        # two roundings of fp32 values that agree to fp32 rounding: at most one 16-bit ulp apart
        half_ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}.get(a.dtype, 1e-5)
        assert rel_err(np_of(a), np_of(b)) < half_ulp, name


@pytest.mark.parametrize("B,n,C", [(4, 64, 64), (3, 64, 128), (2, 64, 1024), (2, 48, 64), (3, 33, 128)])
@pytest.mark.parametrize("xdt,gdt,odt", [("bf16", "f32", "f32"), ("bf16", "bf16", "bf16"), ("f16", "f32", "f32"),
                                         ("f32", "f32", "f32")])
def test_post_combine_mfma_above_32_streams(B, n, C, xdt, gdt, odt, knobs):
    """32 < n <= 64 with C a multiple of 64: the forward runs on the fp32 matrix cores (mix64_fwd_kernel,
    rows past n through the buffer range check), and at n = 64 the VJP too (mix64_bwd_kernel).  Forward
    and every gradient against the float64 oracle (16-bit outputs per element, within one rounding of the
    fp32 result), and against the generic kernels (MHC_MIX32 = 0) to fp32 rounding."""
    g = rng(700 + B + n + C)
    x = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    y = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt if odt == "f32" else odt)
    hpre, hpost, hres, _ = params(g, n, C)
    got = _post_combine_run(x, y, dout, hpre, hpost, hres, xdt, gdt, odt)
    ref_out = O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    names = ["out", "dx", "dy", "dH_pre", "dH_post", "dH_res"]
    for name, t, r in zip(names, got, [ref_out] + list(refs)):
        v = np_of(t)
        if name in ("out", "dx", "dy") and t.dtype != torch.float32:
            ulp = 2.0 ** -8 if t.dtype == torch.bfloat16 else 2.0 ** -11
            assert (np.abs(v - r) <= ulp * np.abs(r) + 1e-5 * np.abs(r).max()).all(), name
        else:
            assert rel_err(v, r) < (1e-5 if name in ("out", "dx", "dy") else GRAD_TOL), (name, rel_err(v, r))
    knobs("MHC_MIX32", 0)
    gen = _post_combine_run(x, y, dout, hpre, hpost, hres, xdt, gdt, odt)
    for name, a, b in zip(names, got, gen):
        half_ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}.get(a.dtype, 1e-5)
        assert rel_err(np_of(a), np_of(b)) < half_ulp, name


@pytest.mark.parametrize("gdt", ["bf16", "f32"])
def test_post_combine_mfma64_walks_several_items_per_wave(gdt, knobs):
    """One workgroup per CU for the n = 64 MFMA post-combine: each wave walks several (token, slab) items,
    so the VJP's S / Yd sums run across items and are added over the waves at the end; a second run is
    bitwise identical."""
    knobs("MHC_MIX_FWD_GRID", 1)
    knobs("MHC_MIX_BWD_GRID", 1)
    B, n, C = 1500, 64, 128
    g = rng(51)
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    y = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt)
    hpre, hpost, hres, _ = params(g, n, C)
    runs = [_post_combine_run(x, y, dout, hpre, hpost, hres, "bf16", gdt, "f32") for _ in range(2)]
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    assert rel_err(np_of(runs[0][0]), O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)) < 1e-5
    for name, t, r in zip(["dx", "dy", "dH_pre", "dH_post", "dH_res"], runs[0][1:], refs):
        tol = 1e-2 if name in ("dx", "dy") else GRAD_TOL
        assert rel_err(np_of(t), r) < tol, (name, rel_err(np_of(t), r))


@pytest.mark.parametrize("gdt", ["bf16", "f32"])
def test_post_combine_mfma_walks_several_items_per_wave(gdt, knobs):
    """One workgroup per CU for the n = 32 MFMA post-combine: each wave walks several (token, slab) items,
    so the backward's S / Yd sums run across items; a second run is bitwise identical."""
    knobs("MHC_MIX_FWD_GRID", 1)
    knobs("MHC_MIX_BWD_GRID", 1)
    B, n, C = 3000, 32, 128
    g = rng(49)
    x = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    y = to_dtype_np(g.standard_normal((B, n, C)), "bf16")
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt)
    hpre, hpost, hres, _ = params(g, n, C)
    runs = [_post_combine_run(x, y, dout, hpre, hpost, hres, "bf16", gdt, "f32") for _ in range(2)]
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    assert rel_err(np_of(runs[0][0]), O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)) < 1e-5
    for name, t, r in zip(["dx", "dy", "dH_pre", "dH_post", "dH_res"], runs[0][1:], refs):
        tol = 1e-2 if name in ("dx", "dy") else GRAD_TOL
        assert rel_err(np_of(t), r) < tol, (name, rel_err(np_of(t), r))


@pytest.mark.parametrize("n,C", [(4, 64), (16, 16), (32, 8), (3, 9), (32, 64), (20, 128)])
def test_stream_mix_add_matches_reference_semantics(n, C):
    """stream_mix_add_metal: out = M x + y_dist (fp32); VJP dx = M^T g, dM = sum g x^T, dy = g."""
    B = 3
    g = rng(60 + n)
    x = g.standard_normal((B, n, C)).astype(np.float32)
    yd = g.standard_normal((B, n, C)).astype(np.float32)
    M = g.random((n, n)).astype(np.float32)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    xt, Mt, yt = (dev_tensor(v).requires_grad_(True) for v in (x, M, yd))
    out = ops.stream_mix_add_hip_autograd(xt, Mt, yt)
    assert rel_err(np_of(out), np.einsum("ij,bjc->bic", M, x) + yd) < 1e-5
    out.backward(dev_tensor(dout))
    assert rel_err(np_of(xt.grad), np.einsum("ij,bic->bjc", M, dout)) < 1e-5
    assert rel_err(np_of(Mt.grad), np.einsum("bic,bjc->ij", dout, x)) < 1e-5
    assert rel_err(np_of(yt.grad), dout) == 0.0


@pytest.mark.parametrize("n,C", [(4, 64), (16, 16), (64, 8), (5, 11)])
def test_stream_scale_matches_oracle(n, C):
    B = 4
    g = rng(70 + n)
    x = g.standard_normal((B, n, C)).astype(np.float32)
    hpre = g.standard_normal(n).astype(np.float32)
    dout = g.standard_normal((B, n, C)).astype(np.float32)
    xt, ht = dev_tensor(x).requires_grad_(True), dev_tensor(hpre).requires_grad_(True)
    out = ops.stream_scale(xt, ht)
    a = O.sigmoid(hpre)
    assert rel_err(np_of(out), x * a[None, :, None]) < 1e-6
    out.backward(dev_tensor(dout))
    assert rel_err(np_of(xt.grad), dout * a[None, :, None]) < 1e-6
    ref_dh = np.einsum("bic,bic->i", dout, x) * a * (1 - a)
    assert rel_err(np_of(ht.grad), ref_dh) < 1e-5


@pytest.mark.parametrize("T,n,C,dt", [(300, 4, 1024, "bf16"), (64, 32, 512, "f16"), (64, 32, 128, "bf16"),
                                      (20, 4, 100, "f16"), (10, 3, 64, "f32")])
def test_stream_scale_passthrough_adds_the_second_gradient(T, n, C, dt):
    """stream_scale_and_pass returns (a_i x_i, x); the VJP writes dx = a_i g_i + g_pass in one pass (the
    flat kernel with its accumulator for aligned 16-bit data with C a multiple of 512, the per-stream
    kernel otherwise): one rounding of the fp32 result for 16-bit x.  With only the pass-through used,
    dx is its gradient unchanged."""
    g = rng(7300 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre = g.standard_normal(n).astype(np.float32)
    g1 = to_dtype_np(g.standard_normal((T, n, C)), dt)
    g2 = to_dtype_np(g.standard_normal((T, n, C)), dt)
    a = O.sigmoid(hpre)
    xt, ht = dev_tensor(x, dt).requires_grad_(True), dev_tensor(hpre).requires_grad_(True)
    xp, xpass = ops.stream_scale_and_pass(xt, ht)
    assert xpass.data_ptr() == xt.data_ptr() and torch.equal(xpass, xt)
    assert rel_err(np_of(xp), x * a[None, :, None]) < (1e-6 if dt == "f32" else TOL[dt])
    torch.autograd.backward([xp, xpass], [dev_tensor(g1, dt), dev_tensor(g2, dt)])
    ref = g1 * a[None, :, None] + g2
    got = np_of(xt.grad)
    if dt == "f32":
        assert rel_err(got, ref) < 1e-6
    else:
        ulp = 2.0 ** -8 if dt == "bf16" else 2.0 ** -11
        assert (np.abs(got - ref) <= ulp * np.abs(ref) + 1e-6 * np.abs(ref).max()).all()
    assert rel_err(np_of(ht.grad), np.einsum("bic,bic->i", g1, x) * a * (1 - a)) < GRAD_TOL
    xt2 = dev_tensor(x, dt).requires_grad_(True)
    _, xpass2 = ops.stream_scale_and_pass(xt2, ht)
    xpass2.backward(dev_tensor(g2, dt))
    assert torch.equal(xt2.grad, dev_tensor(g2, dt))


@pytest.mark.parametrize("dims,n,T", [(64, 4, 3), (256, 16, 2), (512, 32, 2), (4096, 4, 16), (4096, 32, 8)])
def test_rewire_linear_matches_oracle(dims, n, T):
    g = rng(dims + n)
    torch.manual_seed(dims)
    lin = torch.nn.Linear(dims, dims, bias=False).cuda()
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy((0.02 * g.standard_normal((dims, dims))).astype(np.float32)))
    model = MHCRewire(lin, dims=dims, n=n).cuda()
    hpre, hpost, hres, _ = params(g, n, dims // n)
    with torch.no_grad():
        model.mhc.H_pre_raw.copy_(torch.from_numpy(hpre))
        model.mhc.H_post_raw.copy_(torch.from_numpy(hpost))
        model.mhc.H_res_raw.copy_(torch.from_numpy(hres))
    x = g.standard_normal((T, dims)).astype(np.float32)
    dout = g.standard_normal((T, dims)).astype(np.float32)
    xt = dev_tensor(x).requires_grad_(True)
    out = model(xt)
    W = lin.weight.detach().cpu().numpy()
    ref_out, _ = O.rewire_linear_forward(x, W, hpre, hpost, hres)
    # the inner GEMM runs in torch (TF32 off by default on ROCm fp32 GEMMs)
    assert rel_err(np_of(out), ref_out) < 1e-5
    out.backward(dev_tensor(dout))
    dx, dW, dpre, dpost, dres = O.rewire_linear_backward(x, W, hpre, hpost, hres, dout)
    assert rel_err(np_of(xt.grad), dx) < 1e-5
    assert rel_err(np_of(lin.weight.grad), dW) < 1e-5
    assert rel_err(np_of(model.mhc.H_pre_raw.grad), dpre) < GRAD_TOL
    assert rel_err(np_of(model.mhc.H_post_raw.grad), dpost) < GRAD_TOL
    assert rel_err(np_of(model.mhc.H_res_raw.grad), dres) < GRAD_TOL


def test_rewire_folded_equals_explicit():
    """Reference test_weight_folding_correctness: same params, same output (<1e-5)."""
    dims, n = 256, 16
    torch.manual_seed(42)
    lin = torch.nn.Linear(dims, dims).cuda()

    class NoFold(torch.nn.Module):
        def __init__(self, l):
            super().__init__()
            self.l = l

        def forward(self, x):
            return self.l(x)

    a = MHCRewire(lin, dims=dims, n=n).cuda()
    b = MHCRewire(NoFold(lin), dims=dims, n=n).cuda()
    b.mhc.load_state_dict(a.mhc.state_dict())
    x = torch.randn(1, dims, device="cuda")
    assert (a(x) - b(x)).abs().max().item() < 1e-5


def test_rewire_shapes_and_errors():
    dims, n = 512, 16
    model = MHCRewire(torch.nn.Linear(dims, dims), dims=dims, n=n).cuda()
    y = model(torch.randn(2, dims, device="cuda"))
    assert y.shape == (2, dims) and model.mhc.n == n and model.mhc.C == dims // n
    bad = MHCRewire(torch.nn.Linear(dims, 256), dims=dims, n=32).cuda()
    with pytest.raises(ValueError):
        bad(torch.randn(1, dims, device="cuda"))
    blk = MHCRewire(torch.nn.Sequential(torch.nn.RMSNorm(1024), torch.nn.Linear(1024, 1024)), dims=1024, n=32).cuda()
    assert blk(torch.randn(1, 16, 1024, device="cuda")).shape == (1, 16, 1024)


@pytest.mark.parametrize("T,n,C,xdt,odt", [(300, 4, 1024, "bf16", "bf16"), (7, 32, 128, "bf16", "f32"),
                                           (5, 3, 24, "f16", "f16"), (9, 4, 64, "f32", "f32"),
                                           (4, 5, 12, "bf16", "bf16")])
def test_stream_scale_flat_matches_per_stream(T, n, C, xdt, odt, knobs):
    """The pre-scale as one flat elementwise pass (16-byte chunks, the stream of each chunk from its row;
    the default for whole aligned chunks) is bitwise the per-stream kernel (MHC_SCALE_FWD_FLAT=0), and both
    match x * sigmoid(h).  C = 12 at 16-bit (not a whole number of 8-channel chunks) takes the per-stream
    kernel either way."""
    g = rng(7700 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), xdt)
    hpre = g.standard_normal(n).astype(np.float32)
    xt, ht = dev_tensor(x, xdt), dev_tensor(hpre)
    outs = []
    for flat in (1, 0):
        knobs("MHC_SCALE_FWD_FLAT", flat)
        with torch.no_grad():
            o = ops.stream_scale(xt, ht)
            if odt == "f32" and o.dtype != torch.float32:
                o = o.float()
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = x * O.sigmoid(hpre)[None, :, None]
    assert rel_err(np_of(outs[0]), ref) < {"bf16": 2 ** -8, "f16": 2 ** -11, "f32": 1e-6}[xdt]


@pytest.mark.parametrize("T,n,C,xdt", [(300, 4, 1024, "bf16"), (64, 2, 1024, "f16"), (33, 8, 512, "bf16"),
                                       (20, 4, 2048, "bf16"), (5, 3, 128, "bf16")])
def test_stream_scale_vjp_flat_matches_per_stream(T, n, C, xdt, knobs):
    """The pre-scale VJP as a flat pass (16-bit x and dout, 8-channel chunks, each thread's chunks in one
    stream) gives dx bitwise equal to the per-stream kernel's (MHC_SCALE_BWD_FLAT=0) and dH_pre within
    fp32 summation order of it; both match the oracle.  The last shape (8 chunks per row) takes the
    per-stream kernel either way."""
    g = rng(7800 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), xdt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), xdt)
    hpre = g.standard_normal(n).astype(np.float32)
    res = []
    for flat in (1, 0):
        knobs("MHC_SCALE_BWD_FLAT", flat)
        xt, ht = dev_tensor(x, xdt).requires_grad_(True), dev_tensor(hpre).requires_grad_(True)
        ops.stream_scale(xt, ht).backward(dev_tensor(dout, xdt))
        res.append((xt.grad, ht.grad))
    torch.cuda.synchronize()
    assert torch.equal(res[0][0], res[1][0])
    assert rel_err(np_of(res[0][1]), np_of(res[1][1])) < 1e-5
    a = O.sigmoid(hpre)
    ref_dh = np.einsum("bic,bic->i", dout.astype(np.float64), x.astype(np.float64)) * a * (1 - a)
    assert rel_err(np_of(res[0][1]), ref_dh) < 1e-5
    assert rel_err(np_of(res[0][0]), dout * a[None, :, None]) < {"bf16": 2 ** -8, "f16": 2 ** -11}[xdt]


@pytest.mark.parametrize("B,n,C", [(4, 64, 64), (3, 48, 128), (2, 40, 96), (5, 64, 256), (3, 33, 32), (2, 36, 45),
                                   (3, 64, 2)])
@pytest.mark.parametrize("xdt,gdt,odt", [("bf16", "bf16", "bf16"), ("bf16", "f32", "f32"), ("f16", "f16", "f16"),
                                         ("f16", "f32", "f32")])
def test_post_combine_generic_mfma_sums(B, n, C, xdt, gdt, odt, knobs):
    """32 < n <= 64 on the generic post-combine kernels (MHC_MIX32 = 0: the MFMA mix kernels off): with
    16-bit x and dout of x's dtype or fp32 and C a multiple of 32, the VJP's sums S = G X^T run on MFMA
    (fp32 dout split into three 16-bit terms) and Yd as wave dot products.  Every gradient matches the
    oracle, and the VALU sums (MHC_GEN_MFMA=0) to fp32 summation order; dx and dy are bitwise the same
    either way."""
    knobs("MHC_MIX32", 0)
    g = rng(650 + B + n + C)
    x = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    y = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt if odt == "f32" else odt)
    hpre, hpost, hres, _ = params(g, n, C)
    got = _post_combine_run(x, y, dout, hpre, hpost, hres, xdt, gdt, odt)
    # the forward too (generic kernel, one channel per thread)
    fwd = O.post_combine(x, y, hpre, hpost, hres, 20, 1e-5)
    o = np_of(got[0])
    if got[0].dtype == torch.float32:
        assert rel_err(o, fwd) < 1e-5
    else:
        ulp = 2.0 ** -8 if got[0].dtype == torch.bfloat16 else 2.0 ** -11
        assert (np.abs(o - fwd) <= ulp * np.abs(fwd) + 1e-5 * np.abs(fwd).max()).all()
    refs = O.post_combine_backward(x, y, hpre, hpost, hres, dout, 20, 1e-5)
    names = ["dx", "dy", "dH_pre", "dH_post", "dH_res"]
    for name, t, r in zip(names, got[1:], refs):
        v = np_of(t)
        if name in ("dx", "dy") and t.dtype != torch.float32:
            ulp = 2.0 ** -8 if t.dtype == torch.bfloat16 else 2.0 ** -11
            assert (np.abs(v - r) <= ulp * np.abs(r) + 1e-5 * np.abs(r).max()).all(), name
        else:
            assert rel_err(v, r) < (1e-5 if name in ("dx", "dy") else GRAD_TOL), (name, rel_err(v, r))
    knobs("MHC_GEN_MFMA", 0)
    valu = _post_combine_run(x, y, dout, hpre, hpost, hres, xdt, gdt, odt)
    assert torch.equal(got[1], valu[1]) and torch.equal(got[2], valu[2])
    for name, a, b in zip(names[2:], got[3:], valu[3:]):
        assert rel_err(np_of(a), np_of(b)) < 1e-5, name

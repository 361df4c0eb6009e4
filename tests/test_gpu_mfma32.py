"""GPU parity of the 16 < n <= 32 MFMA kernels (csrc/mfma32.hip) against the float64 oracle.

The forward covers n = 17 to 32, C from one 128-channel slab to 4096 (one, two and four slabs per wave),
16-bit x with 16-bit or fp32 output, layer-wide and per-token parameters; the backward covers
layer-wide parameters with 16-bit x and dout up to C = 1024, and above it up to C = 8192 at n = 32
(2 to 8 slabs per wave, x and g read again after the RMS barrier) and 5120 below n = 32, and per-token
parameters up to C = 1024.  With the grid knobs at a few workgroups every workgroup walks many tokens.
Shapes outside these ranges (odd C, fp32 x, fp32 dout, per-token backward above C = 1024) take the
generic kernels and are covered by tests/test_gpu_fused.py.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import GRAD_TOL, TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import ops

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _ulp_bound(got, ref, dt):
    """One rounding to the output dtype (2^-9 / 2^-12 relative) with a factor of two, plus a floor."""
    ulp = {"bf16": 2.0 ** -8, "f16": 2.0 ** -11}[dt]
    err = np.abs(got - ref)
    bound = ulp * np.abs(ref) + 1e-6
    assert (err <= bound).all(), float((err / bound).max())


@pytest.mark.parametrize("T,n,C", [(5, 32, 128), (40, 32, 512), (7, 24, 384), (9, 17, 256), (3, 32, 1024),
                                   (4, 32, 2048), (6, 20, 1280),
                                   # C above 2048: a runtime loop over each wave's slabs, x read again after
                                   # the RMS barrier, y kept in LDS; 17 and 18 slabs split over 1 and 3 waves
                                   (3, 32, 4096), (300, 32, 3072), (2, 24, 4096), (5, 20, 3072), (2, 32, 8192),
                                   (3, 24, 6144), (1, 32, 16384), (4, 32, 2176), (3, 20, 2304)])
@pytest.mark.parametrize("xdt,odt", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16")])
@pytest.mark.parametrize("per_token", [False, True])
def test_mfma32_forward(T, n, C, xdt, odt, per_token, knobs):
    knobs("MHC_FWD_GRID", 1)  # fewer workgroups than tokens: each walks several
    g = rng(3200 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), xdt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T if per_token else None)
    xt = dev_tensor(x, xdt)
    ps = [dev_tensor(v) for v in (hpre, hpost, hres, w)]
    fn = ops.mhc_layer_forward_dynamic if per_token else ops.mhc_layer_forward
    with torch.no_grad():
        out = fn(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=None if odt == "f32" else xt.dtype)
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    got = np_of(out)
    assert rel_err(got, ref) < (1e-5 if odt == "f32" else TOL[odt]), rel_err(got, ref)
    if odt != "f32":
        _ulp_bound(got, ref, odt)


@pytest.mark.parametrize("T,n,C,settings", [(3, 32, 4096, {"MHC_MF32_FWD_LOOP": 0}),
                                            (5, 24, 3072, {"MHC_MF32_FWD_LOOP": 0}),
                                            (4, 32, 4096, {"MHC_MF32_FWD_WAVES": 8}),
                                            (3, 32, 3072, {"MHC_MF32_FWD_WAVES": 1}),
                                            (2, 20, 8192, {"MHC_MF32_FWD_WAVES": 2})])
@pytest.mark.parametrize("odt", ["bf16", "f32"])
def test_mfma32_forward_other_splits(T, n, C, settings, odt, knobs):
    """C above 2048 with the four-slab register variant (MHC_MF32_FWD_LOOP=0, C <= 4096) and with the
    runtime-loop variant on 8, 1 and 2 waves per workgroup."""
    for k, v in settings.items():
        knobs(k, v)
    test_mfma32_forward(T, n, C, "bf16", odt, True, knobs)
    test_mfma32_forward(T, n, C, "bf16", odt, False, knobs)


@pytest.mark.parametrize("T,n,C", [(5, 32, 128), (300, 32, 512), (40, 24, 256), (33, 17, 640), (7, 32, 1024),
                                   (64, 28, 384),
                                   # n = 32 above C = 1024: 2 .. 8 slabs per wave on 3 to 8 waves, the
                                   # one-slab-ahead variant up to C = 3072 (C = 1408 has no split); n < 32
                                   # there: up to 5 slabs per wave, rows beyond n through the buffer range check
                                   (3, 32, 1152), (9, 32, 1536), (2, 32, 1408), (4, 32, 2048), (5, 32, 2560),
                                   (17, 32, 3072), (2, 32, 3584), (3, 32, 4096), (2, 32, 8192), (4, 24, 2048),
                                   (11, 20, 3072), (3, 17, 4096), (5, 28, 1536)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_mfma32_backward_layer_wide(T, n, C, dt, knobs):
    _backward_layer_wide(T, n, C, dt, knobs)


@pytest.mark.parametrize("T,C,settings", [(6, 2048, {"MHC_MF32_WAVES": 4}), (5, 4096, {"MHC_MF32_WAVES": 8}),
                                           (4, 3072, {"MHC_MF32_WAVES": 2}), (6, 2048, {"MHC_BWD_PIPE": 0}),
                                           (7, 3072, {"MHC_BWD_PIPE": 0})])
def test_mfma32_backward_other_splits(T, C, settings, knobs):
    """Other splits of the same shapes: 4 waves of 4 slabs (pipelined), 8 of 4 and 3 of 8 (not pipelined), and
    the unpipelined kernel at 2 and 3 slabs per wave (MHC_BWD_PIPE = 0)."""
    for name, value in settings.items():
        knobs(name, value)
    _backward_layer_wide(T, 32, C, "bf16", knobs)


def _backward_layer_wide(T, n, C, dt, knobs):
    knobs("MHC_BWD_GRID", 3)
    g = rng(3300 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C)
    runs = []
    for _ in range(2):
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = dev_tensor(x, dt).requires_grad_(True)
        out = ops.mhc_layer_forward(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dev_tensor(dout, dt))
        runs.append([out.detach(), xt.grad] + [p.grad for p in ps])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    ref_out = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    _ulp_bound(np_of(runs[0][0]), ref_out, dt)
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    _ulp_bound(np_of(runs[0][1]), refs[0], dt)
    for name, got, r in zip(["dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], runs[0][2:], refs[1:]):
        assert rel_err(np_of(got), r) < GRAD_TOL, (name, rel_err(np_of(got), r))


@pytest.mark.parametrize("T,n,C", [(5, 32, 128), (300, 32, 512), (40, 24, 256), (33, 17, 640), (7, 32, 1024),
                                   (64, 28, 384), (9, 20, 896)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("grid", [None, 3])
@pytest.mark.parametrize("legacy", [0, 1])
def test_mfma32_backward_per_token(T, n, C, dt, grid, legacy, knobs):
    """Per-token parameters at 16 < n <= 32 on MFMA, C a multiple of 128 up to 1024: whole tokens per
    wave (mf64_bwd_pt_kernel with two 16-row blocks, the default) or, with MHC_BWD_LEGACY=1, one
    workgroup per token (mf32_bwd_pt_kernel: the token's parameters split by wave 0 one token ahead into
    one of two LDS blocks, the token's dM, dh_pre, dh_post summed across the waves through their slab
    buffers): against the oracle (every gradient), against the generic kernel (MHC_BWD_MFMA=0), and
    bitwise between two runs; with MHC_BWD_GRID=3 each workgroup walks many tokens, so both parameter
    blocks are used."""
    if grid is not None:
        knobs("MHC_BWD_GRID", grid)
    knobs("MHC_BWD_LEGACY", legacy)
    knobs("MHC_SK_BLK_RECORD", 0)
    g = rng(3500 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T)

    def run():
        xt = dev_tensor(x, dt).requires_grad_(True)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        out = ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dev_tensor(dout, dt))
        return [xt.grad] + [p.grad for p in ps]

    a, b = run(), run()
    knobs("MHC_BWD_MFMA", 0)
    gen = run()
    torch.cuda.synchronize()
    for name, u, v in zip(("dx", "dH_pre", "dH_post", "dH_res", "d_w"), a, b):
        assert torch.equal(u, v), (name, _where_unequal(u, v))
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    _ulp_bound(np_of(a[0]), refs[0], dt)
    for name, got, ref in zip(("dH_pre", "dH_post", "dH_res", "d_w"), a[1:], refs[1:]):
        assert rel_err(np_of(got), ref) < GRAD_TOL, (name, rel_err(np_of(got), ref))
    assert rel_err(np_of(a[0]), np_of(gen[0])) < TOL[dt]
    for got, ref in zip(a[1:], gen[1:]):
        assert rel_err(np_of(got), np_of(ref)) < 1e-5


@pytest.mark.parametrize("T,n,C", [(64, 64, 512), (30, 40, 256), (9, 64, 1024), (20, 48, 768)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_mfma64_backward_g_through_lds_is_bitwise(T, n, C, dt, knobs):
    """With one slab per wave the 32 < n <= 64 layer backward keeps G in LDS across the RMS barrier and
    splits M^T per lane (GL); MHC_BWD_PIPE=0 reads G again from memory and takes M^T from the workgroup's
    LDS copy.  The operands and every sum are the same, so all gradients are bitwise equal."""
    knobs("MHC_SK_BLK_RECORD", 0)
    g = rng(6700 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C)

    def run():
        xt = dev_tensor(x, dt).requires_grad_(True)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        out = ops.mhc_layer_forward(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dev_tensor(dout, dt))
        return [xt.grad] + [p.grad for p in ps]

    a = run()
    knobs("MHC_BWD_PIPE", 0)
    b = run()
    torch.cuda.synchronize()
    for name, u, v in zip(("dx", "dH_pre", "dH_post", "dH_res", "d_w"), a, b):
        assert torch.equal(u, v), (name, _where_unequal(u, v))
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    _ulp_bound(np_of(a[0]), refs[0], dt)


@pytest.mark.parametrize("T,n,C", [(5, 64, 128), (300, 64, 512), (40, 48, 256), (33, 33, 640), (7, 64, 1024),
                                   (9, 40, 2048), (3, 64, 4096),
                                   # 16 < n <= 32 above C = 1024, beyond the n <= 32 per-token kernel
                                   (6, 32, 2048), (4, 24, 1536), (3, 17, 4096)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("grid", [None, 3])
def test_mfma64_backward_per_token(T, n, C, dt, grid, knobs):
    """Per-token parameters at 32 < n <= 64 on MFMA (mf64_bwd_pt_kernel: whole tokens per wave, the
    token's dM, dh_pre and dh_post written from the wave's own sums, dx with the token's M^T split per
    lane), C a multiple of 128 up to 4096: against the oracle (every gradient), against the generic
    kernel (MHC_BWD_MFMA=0; the two paths' parameter sums differ in their last bits, so the MFMA kernel
    ran), and bitwise between two runs; with MHC_BWD_GRID=3 each wave walks many tokens."""
    if grid is not None:
        knobs("MHC_BWD_GRID", grid)
    knobs("MHC_SK_BLK_RECORD", 0)
    g = rng(3600 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T)

    def run():
        xt = dev_tensor(x, dt).requires_grad_(True)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        out = ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dev_tensor(dout, dt))
        return [xt.grad] + [p.grad for p in ps]

    a, b = run(), run()
    knobs("MHC_BWD_MFMA", 0)
    gen = run()
    torch.cuda.synchronize()
    for name, u, v in zip(("dx", "dH_pre", "dH_post", "dH_res", "d_w"), a, b):
        assert torch.equal(u, v), (name, _where_unequal(u, v))
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    _ulp_bound(np_of(a[0]), refs[0], dt)
    for name, got, ref in zip(("dH_pre", "dH_post", "dH_res", "d_w"), a[1:], refs[1:]):
        assert rel_err(np_of(got), ref) < GRAD_TOL, (name, rel_err(np_of(got), ref))
    assert rel_err(np_of(a[0]), np_of(gen[0])) < TOL[dt]
    for got, ref in zip(a[1:], gen[1:]):
        assert rel_err(np_of(got), np_of(ref)) < 1e-5
    assert not all(torch.equal(u, v) for u, v in zip(a[1:], gen[1:]))


def test_mfma32_matches_the_generic_kernels(knobs):
    """The MFMA kernels and the VALU kernels they replace agree to rounding on the same inputs."""
    T, n, C = 64, 32, 512
    g = rng(3400)
    x = dev_tensor(to_dtype_np(g.standard_normal((T, n, C)), "bf16"), "bf16")
    dout = dev_tensor(to_dtype_np(g.standard_normal((T, n, C)), "bf16"), "bf16")
    hpre, hpost, hres, w = params(g, n, C)
    res = {}
    for mf in (1, 0):
        knobs("MHC_FWD_MFMA", mf)
        knobs("MHC_BWD_MFMA", mf)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = x.clone().requires_grad_(True)
        out = ops.mhc_layer_forward(xt, *ps, eps=EPS, output_dtype=torch.bfloat16)
        out.backward(dout)
        res[mf] = [out.detach(), xt.grad] + [p.grad for p in ps]
    for name, a, b in zip(["out", "dx", "dpre", "dpost", "dres", "dw"], res[1], res[0]):
        # out and dx: one bf16 rounding of fp32 values that differ in the last bits
        tol = 2.0 ** -8 if name in ("out", "dx") else GRAD_TOL
        assert rel_err(np_of(a), np_of(b)) < tol, (name, rel_err(np_of(a), np_of(b)))


@pytest.mark.parametrize("T,n,C", [(1, 32, 256), (1, 32, 4096), (32, 32, 512), (32, 32, 2048), (256, 32, 1024),
                                   (1, 24, 8192), (7, 20, 3072), (2, 17, 128)])
@pytest.mark.parametrize("xdt,odt", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16")])
def test_single_launch_layer_forward_matches_two_launches(T, n, C, xdt, odt, knobs):
    """Layer-wide 16 < n <= 32 with at most one token per CU: the Sinkhorn projection runs inside the
    forward kernel (one launch, M written by workgroup 0).  Out and M are bitwise those of the
    projection kernel followed by the forward (MHC_FWD_SKF=0), and match the oracle."""
    g = rng(3300 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), xdt)
    hpre, hpost, hres, w = params(g, n, C)
    xt = dev_tensor(x, xdt)
    ps = [dev_tensor(v) for v in (hpre, hpost, hres, w)]
    odtype = torch.float32 if odt == "f32" else xt.dtype
    res = []
    for skf in (1, 0):
        knobs("MHC_FWD_SKF", skf)
        out, M = ops._layer_fwd(xt, *ps, 20, EPS, odtype, False)
        res.append((out, M))
    torch.cuda.synchronize()
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(res[0][0]), ref) < (1e-5 if odt == "f32" else TOL[odt])
    assert rel_err(np_of(res[0][1]), O.mixing_matrix_from_logits(hres, iters=20, eps=EPS)) < 1e-5


@pytest.mark.parametrize("T,n,C", [(5, 64, 128), (40, 64, 512), (7, 48, 384), (9, 33, 256), (3, 64, 1024),
                                   (4, 64, 2048), (2, 40, 4096), (1, 64, 8192), (300, 64, 256), (6, 56, 1280)])
@pytest.mark.parametrize("xdt,odt", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16")])
@pytest.mark.parametrize("grid", [None, 1])
def test_mfma64_forward(T, n, C, xdt, odt, grid, knobs):
    """32 < n <= 64 with layer-wide parameters on MFMA (mf64_fwd_loop_kernel: two 32-stream halves chained
    per contraction, four 16-row blocks of M), C a multiple of 128 up to 8192, against the oracle; with
    MHC_FWD_GRID=1 every workgroup walks several tokens."""
    if grid is not None:
        knobs("MHC_FWD_GRID", grid)
    g = rng(6400 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), xdt)
    hpre, hpost, hres, w = params(g, n, C)
    xt = dev_tensor(x, xdt)
    ps = [dev_tensor(v) for v in (hpre, hpost, hres, w)]
    with torch.no_grad():
        out = ops.mhc_layer_forward(xt, *ps, sinkhorn_iters=20, eps=EPS,
                                    output_dtype=None if odt == "f32" else xt.dtype)
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    got = np_of(out)
    assert rel_err(got, ref) < (1e-5 if odt == "f32" else TOL[odt]), rel_err(got, ref)
    if odt != "f32":
        _ulp_bound(got, ref, odt)


@pytest.mark.parametrize("T,n,C", [(5, 64, 128), (40, 64, 512), (7, 48, 384), (3, 64, 1024), (2, 40, 4096),
                                   (1, 64, 8192), (300, 64, 256), (6, 56, 1280)])
@pytest.mark.parametrize("xdt,odt", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16")])
@pytest.mark.parametrize("grid", [None, 1])
def test_mfma64_forward_per_token(T, n, C, xdt, odt, grid, knobs):
    """32 < n <= 64 with per-token parameters on MFMA (mf64_fwd_loop_kernel<PT>: the token's a split per
    lane, its M and p split by the workgroup into LDS buffers of the token's parity), against the
    oracle; with MHC_FWD_GRID=1 every workgroup walks several tokens, so both buffers are reused.  An
    fp32 output differs in its last bits from the generic kernel's (MHC_FWD_MFMA=0), so the MFMA kernel
    ran."""
    if grid is not None:
        knobs("MHC_FWD_GRID", grid)
    g = rng(6500 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), xdt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T)
    xt = dev_tensor(x, xdt)
    ps = [dev_tensor(v) for v in (hpre, hpost, hres, w)]
    run = lambda: ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=EPS,
                                                output_dtype=None if odt == "f32" else xt.dtype)
    with torch.no_grad():
        out = run()
        knobs("MHC_FWD_MFMA", 0)
        gen = run()
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    got = np_of(out)
    assert rel_err(got, ref) < (1e-5 if odt == "f32" else TOL[odt]), rel_err(got, ref)
    assert rel_err(got, np_of(gen)) < (1e-5 if odt == "f32" else TOL[odt])
    if odt != "f32":
        _ulp_bound(got, ref, odt)
    else:
        assert not torch.equal(out, gen)


@pytest.mark.parametrize("T,n,C,per_token", [(50, 64, 256, False), (20, 48, 512, False), (33, 33, 96, False),
                                             (300, 40, 128, False), (16, 24, 160, True), (9, 64, 64, True),
                                             (12, 32, 224, True), (7, 20, 40, False)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_generic_backward_mfma_parameter_sums(T, n, C, per_token, dt, knobs):
    """The generic backward (n > 32, per-token n > 16, and C that the n <= 32 MFMA kernels do not take)
    forms dM = G X^T on MFMA for 16-bit x == dout with C a multiple of 32 (MHC_GEN_MFMA=0: the VALU
    outer-product blocks).  dx is bitwise the same either way (the dx pass is shared), every parameter
    gradient agrees to fp32 summation order, and both match the oracle."""
    g = rng(6500 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T if per_token else None)
    fn = ops.mhc_layer_forward_dynamic if per_token else ops.mhc_layer_forward
    res = []
    for mf in (1, 0):
        knobs("MHC_GEN_MFMA", mf)
        knobs("MHC_SK_BLK_RECORD", 0)  # the same (recomputing) Sinkhorn VJP both times
        xt = dev_tensor(x, dt).requires_grad_(True)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        out = fn(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dev_tensor(dout, dt))
        res.append([xt.grad] + [p.grad for p in ps])
    torch.cuda.synchronize()
    assert torch.equal(res[0][0], res[1][0])
    for a, b in zip(res[0][1:], res[1][1:]):
        assert rel_err(np_of(a), np_of(b)) < 1e-5
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(res[0][0]), refs[0]) < TOL[dt]
    for got, ref in zip(res[0][1:], refs[1:]):
        assert rel_err(np_of(got), ref) < GRAD_TOL


def _where_unequal(u, v, k=8):
    """How many elements of two runs differ, and the first k positions with both values."""
    d = (u != v).nonzero()
    return int(d.shape[0]), [(tuple(i.tolist()), float(u[tuple(i)]), float(v[tuple(i)])) for i in d[:k]]


@pytest.mark.parametrize("T,n,C", [(64, 64, 512), (300, 64, 1024), (20, 48, 512), (9, 33, 2048), (5, 64, 4096),
                                   (40, 40, 768), (50, 64, 128), (33, 40, 256), (17, 64, 384), (4, 64, 8192),
                                   (3, 37, 6272),
                                   # 16 < n < 32 above C = 5120, beyond the n <= 32 layer-wide kernels
                                   (3, 24, 6144), (2, 20, 8192)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("grid", [None, 2])
def test_mfma64_backward(T, n, C, dt, grid, knobs):
    """32 < n <= 64 layer-wide backward on MFMA (mf64_bwd_kernel: dM = G X^T in 16 x 16 blocks and the
    parameter dot products before the RMS barrier, dx = M^T G on MFMA in two 32-stream halves after
    it), C a multiple of 128 from 128 to 8192 (one to eight waves, one to seven slabs per wave),
    against the oracle for every gradient and against the generic backward (MHC_BWD_MFMA=0); with
    MHC_BWD_GRID=2 each workgroup walks many tokens.  Two runs are bitwise equal."""
    if grid is not None:
        knobs("MHC_BWD_GRID", grid)
    knobs("MHC_SK_BLK_RECORD", 0)
    g = rng(6600 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C)

    def run():
        xt = dev_tensor(x, dt).requires_grad_(True)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        out = ops.mhc_layer_forward(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dev_tensor(dout, dt))
        return [xt.grad] + [p.grad for p in ps]

    a, b = run(), run()
    knobs("MHC_BWD_MFMA", 0)
    gen = run()
    torch.cuda.synchronize()
    for name, u, v in zip(("dx", "dH_pre", "dH_post", "dH_res", "d_w"), a, b):
        assert torch.equal(u, v), (name, _where_unequal(u, v))
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(a[0]), refs[0]) < TOL[dt]
    _ulp_bound(np_of(a[0]), refs[0], dt)
    for got, ref in zip(a[1:], refs[1:]):
        assert rel_err(np_of(got), ref) < GRAD_TOL
    for got, other in zip(a[1:], gen[1:]):
        assert rel_err(np_of(got), np_of(other)) < 1e-5
    # the MFMA kernel ran: its parameter sums associate differently from the generic kernel's
    assert not all(torch.equal(u, v) for u, v in zip(a[1:], gen[1:]))

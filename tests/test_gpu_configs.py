"""GPU parity at the benchmark configurations and on every kernel path they use.

* Config 0 (x [1,4,512] fp32) and config 1 (x [32,4,2048] bf16) are small
  enough for the float64 oracle at full size.
* Shapes that reach the full-tile kernels (two chunks per thread, T >= CU
  count) and the multi-row parameter reduction (more than 64 partial rows),
  at sizes the oracle finishes in about a second.
* Config 2 (32768 x 4 x 4096 bf16, fwd+bwd) and config 3 (16384 x 16 x 1024
  bf16, per-token parameters) at full size, through properties that do not
  need the oracle to see every token: tokens are independent, so out / dx
  (and the per-token parameter gradients) of a random sample of tokens must
  match the oracle run on those tokens alone; the layer-wide parameter
  gradients are sums over tokens and are compared with a float64 torch
  reference of the same sums computed on the GPU in chunks, then chained
  through the oracle's sigmoid and Sinkhorn VJP; the mixing matrices must be
  doubly stochastic to the oracle's own residual; a second run must be
  bitwise identical.
* Config 4 (MHCRewire(Linear(4096, 4096)), n=4, 8192 tokens) against a
  float64 formulation of layer.py:332-337 fed with the wrapped GEMM's own
  input, output and gradients.

Parameter gradients are held at GRAD_TOL (1e-5 relative) for every input
dtype, as fp32 values are in the reference tests.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import GRAD_TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import MHCLayer, MHCRewire, ops

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _layer_from(hpre, hpost, hres, w, n, C):
    layer = MHCLayer(n=n, C=C, sinkhorn_iters=20, eps=EPS).cuda()
    with torch.no_grad():
        layer.H_pre_raw.copy_(torch.from_numpy(hpre))
        layer.H_post_raw.copy_(torch.from_numpy(hpost))
        layer.H_res_raw.copy_(torch.from_numpy(hres))
        layer.rms_weight.copy_(torch.from_numpy(w))
    return layer


def _fwd_bwd(layer, x, dout):
    xt = x.clone().requires_grad_(True)
    out = layer(xt, return_dtype=x.dtype)
    grads = torch.autograd.grad(out, [xt] + list(layer.parameters()), dout)
    return out, grads


# --------------------------------------------------------------- configs 0 and 1


def test_config0_forward_fp32():
    """x [1,4,512] fp32 N(0,1), seed 0, eps 1e-6."""
    g = rng(0)
    x = g.standard_normal((1, 4, 512)).astype(np.float32)
    hpre, hpost, hres, w = params(g, 4, 512)
    layer = _layer_from(hpre, hpost, hres, w, 4, 512)
    out = layer(dev_tensor(x))
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    assert out.dtype == torch.float32
    assert rel_err(np_of(out), ref) < 1e-5


def test_config1_forward_bf16():
    """x [32,4,2048] bf16 with bf16 output (latency regime)."""
    g = rng(1)
    x = to_dtype_np(g.standard_normal((32, 4, 2048)), "bf16")
    hpre, hpost, hres, w = params(g, 4, 2048)
    layer = _layer_from(hpre, hpost, hres, w, 4, 2048)
    out = layer(dev_tensor(x, "bf16"), return_dtype=torch.bfloat16)
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    got = np_of(out)
    assert rel_err(got, ref) < 2e-2
    assert (np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6).all()


# ----------------------------------------------------- full-tile kernel paths


@pytest.mark.parametrize("T,n,C,dt", [(300, 4, 1024, "bf16"), (300, 4, 1024, "f32"), (300, 8, 512, "bf16"),
                                      (600, 4, 1024, "bf16"), (40, 4, 2048, "f16"),
                                      (700, 16, 1024, "bf16"), (300, 16, 512, "f16"), (50, 16, 128, "bf16"),
                                      (300, 16, 2048, "bf16"),
                                      # n = 8 with 16-byte chunks: 512-thread workgroups at C = 4096
                                      (200, 8, 4096, "bf16"), (100, 8, 2048, "f16")])
def test_full_tile_paths_fwd_bwd(T, n, C, dt):
    """T >= CU count (two chunks per thread), C a multiple of the tile, > 64 partial rows."""
    g = rng(T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C)
    layer = _layer_from(hpre, hpost, hres, w, n, C)
    xt = dev_tensor(x, dt)
    out, grads = _fwd_bwd(layer, xt, dev_tensor(dout, dt))
    ref = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    tol = {"f32": 1e-5, "bf16": 2e-2, "f16": 5e-3}[dt]
    assert rel_err(np_of(out), ref) < tol
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], grads, refs):
        t = tol if name == "dx" else GRAD_TOL
        assert rel_err(np_of(got), r) < t, (name, rel_err(np_of(got), r))


# -------------------------------------------------------- full-size helpers


def _param_grads_f64(x, g, a, p, M, w, chunk=2048):
    """Layer-wide sums of the VJP in float64 on the GPU (same equations as the oracle)."""
    T, n, C = x.shape
    a, p, w = a.double(), p.double(), w.double()
    dM = torch.zeros(n, n, dtype=torch.float64, device=x.device)
    dA = torch.zeros(n, dtype=torch.float64, device=x.device)
    dP = torch.zeros(n, dtype=torch.float64, device=x.device)
    dw = torch.zeros(C, dtype=torch.float64, device=x.device)
    for s in range(0, T, chunk):
        xf = x[s:s + chunk].double()
        gf = g[s:s + chunk].double()
        y = (xf * a[None, :, None]).sum(1)
        inv = torch.rsqrt((y * y).mean(-1) + EPS)
        dyn = (gf * p[None, :, None]).sum(1)
        d_r = (dyn * y * w).sum(-1)
        dy = dyn * inv[:, None] * w - ((inv ** 3) / C * d_r)[:, None] * y
        for i in range(n):
            for j in range(n):
                dM[i, j] += (gf[:, i] * xf[:, j]).sum()
        dA += (dy[:, None, :] * xf).sum((0, 2))
        dP += (gf * (y * inv[:, None] * w)[:, None, :]).sum((0, 2))
        dw += (dyn * y * inv[:, None]).sum(0)
    return dM.cpu().numpy(), dA.cpu().numpy(), dP.cpu().numpy(), dw.cpu().numpy()


def _bf16_bound(got, ref):
    """|got - ref| <= 2^-8 |ref| + 1e-6 everywhere: the error of one bf16 rounding (2^-9 relative) with
    a factor of two for the fp32 arithmetic before it, plus an absolute floor for values near zero."""
    err = np.abs(got - ref)
    bound = 2.0 ** -8 * np.abs(ref) + 1e-6
    assert (err <= bound).all(), float((err / bound).max())


def _sample(T, k, seed):
    return np.sort(np.random.default_rng(seed).choice(T, size=k, replace=False))


# --------------------------------------------------------------- config 2


def test_config2_full_size_fwd_bwd():
    """32768 tokens x 4 streams x 4096 channels, bf16, all gradients."""
    T, n, C = 32768, 4, 4096
    g = rng(2)
    hpre, hpost, hres, w = params(g, n, C)
    layer = _layer_from(hpre, hpost, hres, w, n, C)
    gen = torch.Generator("cuda").manual_seed(2)
    x = torch.randn(T, n, C, device="cuda", dtype=torch.bfloat16, generator=gen)
    dout = torch.randn(T, n, C, device="cuda", dtype=torch.bfloat16, generator=gen)
    out, grads = _fwd_bwd(layer, x, dout)
    dx, d_pre, d_post, d_res, d_w = grads

    # token-local outputs on a sample of tokens vs the oracle on those tokens
    idx = _sample(T, 48, 20)
    xs, gs = np_of(x[idx]).astype(np.float32), np_of(dout[idx]).astype(np.float32)
    ref = O.mhc_forward_reference(xs, hpre, hpost, hres, w, sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(out[idx]), ref) < 2e-2
    rdx = O.mhc_backward_reference(xs, hpre, hpost, hres, w, gs, sinkhorn_iters=20, eps=EPS)[0]
    assert rel_err(np_of(dx[idx]), rdx) < 2e-2
    # one bf16 rounding of an fp32 result, element by element
    _bf16_bound(np_of(out[idx]), ref)
    _bf16_bound(np_of(dx[idx]), rdx)

    # layer-wide sums vs float64 on the GPU, chained through the oracle
    a, p = O.activate_pre_post(hpre, hpost)
    M = O.mixing_matrix_from_logits(hres, iters=20, eps=EPS)
    dM, dA, dP, dw = _param_grads_f64(x, dout, torch.from_numpy(a).cuda(), torch.from_numpy(p).cuda(),
                                      torch.from_numpy(M).cuda(), torch.from_numpy(w).cuda())
    s_pre, s_post = O.sigmoid(hpre), O.sigmoid(hpost)
    assert rel_err(np_of(d_pre), dA * s_pre * (1 - s_pre)) < GRAD_TOL
    assert rel_err(np_of(d_post), dP * 2 * s_post * (1 - s_post)) < GRAD_TOL
    assert rel_err(np_of(d_w), dw) < GRAD_TOL
    assert rel_err(np_of(d_res), O.sinkhorn_knopp_vjp(hres, dM, iters=20, eps=EPS)) < GRAD_TOL

    # the mixing matrix and a bitwise rerun
    Mg = np_of(layer.mixing_matrix())
    assert rel_err(Mg, M) < 1e-5
    assert O.ds_residual(Mg) <= max(1e-5, O.ds_residual(M) + 1e-6)
    out2, grads2 = _fwd_bwd(layer, x, dout)
    assert torch.equal(out, out2)
    for u, v in zip(grads, grads2):
        assert torch.equal(u, v)


# --------------------------------------------------------------- config 3


def test_config3_full_size_dynamic_fwd_bwd():
    """16384 tokens x 16 streams x 1024 channels, bf16, per-token H (batched Sinkhorn over 16384 matrices)."""
    T, n, C = 16384, 16, 1024
    g = rng(3)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T)
    layer = MHCLayer(n=n, C=C, sinkhorn_iters=20, eps=EPS).cuda()
    with torch.no_grad():
        layer.rms_weight.copy_(torch.from_numpy(w))
    gen = torch.Generator("cuda").manual_seed(3)
    x = torch.randn(T, n, C, device="cuda", dtype=torch.bfloat16, generator=gen)
    dout = torch.randn(T, n, C, device="cuda", dtype=torch.bfloat16, generator=gen)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres)]
    xt = x.clone().requires_grad_(True)
    out = layer.forward_dynamic(xt, *ps, return_dtype=torch.bfloat16)
    grads = torch.autograd.grad(out, [xt] + ps + [layer.rms_weight], dout)
    dx, d_pre, d_post, d_res, d_w = grads

    # everything but d_w is token-local: sample tokens vs the oracle
    idx = _sample(T, 32, 30)
    xs, gs = np_of(x[idx]).astype(np.float32), np_of(dout[idx]).astype(np.float32)
    hp, hq, hr = hpre[idx], hpost[idx], hres[idx]
    ref = O.mhc_forward_reference(xs, hp, hq, hr, w, sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(out[idx]), ref) < 2e-2
    refs = O.mhc_backward_reference(xs, hp, hq, hr, w, gs, sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(dx[idx]), refs[0]) < 2e-2
    _bf16_bound(np_of(out[idx]), ref)
    _bf16_bound(np_of(dx[idx]), refs[0])
    assert rel_err(np_of(d_pre[idx]), refs[1]) < GRAD_TOL
    assert rel_err(np_of(d_post[idx]), refs[2]) < GRAD_TOL
    assert rel_err(np_of(d_res[idx]), refs[3]) < GRAD_TOL

    # d_w sums every token: float64 reference on the GPU with per-token a, p
    a, p = O.activate_pre_post(hpre, hpost)
    at, pt = torch.from_numpy(a).cuda(), torch.from_numpy(p).cuda()
    wt = torch.from_numpy(w).cuda().double()
    dw = torch.zeros(C, dtype=torch.float64, device="cuda")
    for s in range(0, T, 2048):
        xf, gf = x[s:s + 2048].double(), dout[s:s + 2048].double()
        y = (xf * at[s:s + 2048, :, None]).sum(1)
        inv = torch.rsqrt((y * y).mean(-1) + EPS)
        dyn = (gf * pt[s:s + 2048, :, None]).sum(1)
        dw += (dyn * y * inv[:, None]).sum(0)
    assert rel_err(np_of(d_w), dw.cpu().numpy()) < GRAD_TOL

    # all 16384 mixing matrices: doubly stochastic to the oracle's residual
    Mg = ops.sinkhorn_knopp_hip(dev_tensor(hres), iters=20, eps=EPS)
    Mo = O.mixing_matrix_from_logits(hres[idx], iters=20, eps=EPS)
    assert rel_err(np_of(Mg[idx]), Mo) < 1e-5
    Mh = np_of(Mg)
    res = max(np.abs(Mh.sum(-1) - 1).max(), np.abs(Mh.sum(-2) - 1).max())
    Mall = O.mixing_matrix_from_logits(hres, iters=20, eps=EPS)
    res_o = max(np.abs(Mall.sum(-1) - 1).max(), np.abs(Mall.sum(-2) - 1).max())
    assert res <= max(1e-5, res_o + 1e-6), (res, res_o)


# --------------------------------------------------------------- config 4


def test_config4_rewire_linear_full_size():
    """MHCRewire(Linear(4096, 4096, bias=False), dims=4096, n=4): C = 1024 per the API (layer.py:464-467).

    The reference is the float64 formulation of layer.py:332-337 and 476-480, fed with the wrapped GEMM's
    own input, output and gradients (captured by module hooks), so that everything this library computes
    is compared at fp32 rounding: the post-combine output (fp32) at 1e-5, the parameter gradients
    (sums over 8192 x 1024 products) at 1e-5, the pre-scale output and the cotangent handed to the GEMM
    within one bf16 rounding, and dx (bf16) within the rounding of its two terms.  The GEMM's own
    gradient (torch, bf16) is checked at bf16 tolerance.
    """
    T, dims, n = 8192, 4096, 4
    C = dims // n
    torch.manual_seed(4)
    inner = torch.nn.Linear(dims, dims, bias=False).cuda().to(torch.bfloat16)
    with torch.no_grad():
        inner.weight.normal_(0.0, 0.02)
    m = MHCRewire(inner, dims=dims, n=n, eps=EPS, identity_init=False).cuda()
    with torch.no_grad():
        for prm in (m.mhc.H_pre_raw, m.mhc.H_post_raw, m.mhc.H_res_raw):
            prm.normal_()
    seen = {}

    def fwd_hook(mod, inp, out):
        seen["x_pre"], seen["y"] = inp[0].detach(), out.detach()

    def bwd_hook(mod, gin, gout):
        seen["dx_pre"], seen["dy"] = gin[0].detach(), gout[0].detach()

    hooks = [inner.register_forward_hook(fwd_hook), inner.register_full_backward_hook(bwd_hook)]
    x = torch.randn(T, dims, device="cuda", dtype=torch.bfloat16).requires_grad_(True)
    g = torch.randn(T, dims, device="cuda", dtype=torch.float32)
    try:
        out = m(x)
        gx, gw, gpre, gpost, gres = torch.autograd.grad(
            out, [x, inner.weight, m.mhc.H_pre_raw, m.mhc.H_post_raw, m.mhc.H_res_raw], g)
    finally:
        for h in hooks:
            h.remove()
    assert out.dtype == torch.float32

    f64 = torch.float64
    hp, hq, hr = (np_of(t) for t in (m.mhc.H_pre_raw, m.mhc.H_post_raw, m.mhc.H_res_raw))
    a_np, p_np = O.activate_pre_post(hp, hq)
    a, p = torch.from_numpy(a_np).cuda(), torch.from_numpy(p_np).cuda()
    M = torch.from_numpy(O.mixing_matrix_from_logits(hr, iters=20, eps=EPS)).cuda()
    Mf = M * a[None, :]
    x3 = x.detach().to(f64).reshape(T, n, C)

    # pre-scale: one bf16 rounding of a_i x_i
    xp = (x3 * a[None, :, None]).reshape(T, dims)
    assert ((seen["x_pre"].to(f64) - xp).abs() <= 2.0 ** -8 * xp.abs() + 1e-30).all()

    # post-combine on the GEMM's output: fp32 rounding
    y = seen["y"].to(f64).reshape(T, n, C)
    mixed = torch.stack([sum(Mf[i, j] * x3[:, j] for j in range(n)) for i in range(n)], 1)
    ref = (p[None, :, None] * (y + mixed)).reshape(T, dims)
    assert rel_err(np_of(out), ref.cpu().numpy()) < 1e-5

    # gradients: sums in float64 from the same tensors
    g3 = g.to(f64).reshape(T, n, C)
    pg = p[None, :, None] * g3
    assert ((seen["dy"].to(f64).reshape(T, n, C) - pg).abs() <= 2.0 ** -8 * pg.abs() + 1e-30).all()
    dP = (g3 * (y + mixed)).sum((0, 2))
    dMf = torch.stack([torch.stack([(pg[:, i] * x3[:, j]).sum() for j in range(n)]) for i in range(n)])
    dM = dMf * a[None, :]
    dxp = seen["dx_pre"].to(f64).reshape(T, n, C)
    dA = (dMf * M).sum(0) + (dxp * x3).sum((0, 2))
    s_pre, s_post = torch.sigmoid(torch.from_numpy(hp).cuda()), torch.sigmoid(torch.from_numpy(hq).cuda())
    assert rel_err(np_of(gpre), (dA * s_pre * (1 - s_pre)).cpu().numpy()) < 1e-5
    assert rel_err(np_of(gpost), (dP * 2 * s_post * (1 - s_post)).cpu().numpy()) < 1e-5
    rres = O.sinkhorn_knopp_vjp(hr, dM.cpu().numpy(), iters=20, eps=EPS)
    assert rel_err(np_of(gres), rres) < 1e-5
    # dx = a_j dx_pre_j + sum_i Mf_ij p_i g_i, each term and the sum rounded to bf16 at most once
    t1 = a[None, :, None] * dxp
    t2 = torch.stack([sum(Mf[i, j] * pg[:, i] for i in range(n)) for j in range(n)], 1)
    err = (gx.to(f64).reshape(T, n, C) - (t1 + t2)).abs()
    assert (err <= 2.0 ** -7 * (t1.abs() + t2.abs()) + 1e-30).all()
    # the GEMM's weight gradient (torch, bf16 output)
    rgw = seen["dy"].to(f64).t() @ seen["x_pre"].to(f64)
    assert rel_err(np_of(gw), rgw.cpu().numpy()) < 1e-2


@pytest.mark.parametrize("T,C,dt", [(300, 1024, "bf16"), (40, 256, "bf16"), (70, 512, "f16"), (3, 1024, "bf16"),
                                   (50, 384, "bf16"), (20, 128, "f16"), (9, 768, "bf16"), (1500, 256, "bf16"),
                                   # two slabs per wave with 5-8 waves (C up to 2048)
                                   (300, 2048, "bf16"), (40, 1280, "f16")])
def test_per_token_n16_mfma_path(T, C, dt):
    """Per-token n=16 with C a multiple of 128 (the MFMA kernels: one or two 128-channel slabs per wave;
    T = 1500 exceeds the persistent backward grid, so workgroups walk several tokens), all gradients."""
    n = 16
    g = rng(7000 + T + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
    xt = dev_tensor(x, dt).requires_grad_(True)
    out = ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
    tol = {"bf16": 2e-2, "f16": 5e-3}[dt]
    assert rel_err(np_of(out), O.mhc_forward_reference(x, hpre, hpost, hres, w, 20, EPS)) < tol
    out.backward(dev_tensor(dout, dt))
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    gots = [xt.grad] + [p.grad for p in ps]
    for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], gots, refs):
        t = tol if name == "dx" else GRAD_TOL
        assert rel_err(np_of(got), r) < t, (name, rel_err(np_of(got), r))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_per_token_n16_activated_c_abi(dt):
    """mhc_fused_bwd through the C ABI with per-token M and activated H (h_mode ACTIVATED): the
    op-level VJP contract (gradients w.r.t. M and the activated H, metal.py:2857) on the MFMA kernel."""
    import ctypes

    from mhc_mlx_amd import _lib

    T, n, C = 600, 16, 512
    g = rng(7100)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    a = O.sigmoid(g.standard_normal((T, n))).astype(np.float32)
    p = (2 * O.sigmoid(g.standard_normal((T, n)))).astype(np.float32)
    M = O.mixing_matrix_from_logits(g.standard_normal((T, n, n)), 20, EPS).astype(np.float32)
    w = (1 + 0.02 * g.standard_normal(C)).astype(np.float32)
    xt, gt = dev_tensor(x, dt), dev_tensor(dout, dt)
    Mt, at, pt, wt = (dev_tensor(v) for v in (M, a, p, w))
    dx = torch.empty_like(xt)
    dM = torch.empty((T, n, n), device="cuda")
    da = torch.empty((T, n), device="cuda")
    dp = torch.empty((T, n), device="cuda")
    dw = torch.empty((C,), device="cuda")
    nb = _lib.query("mhc_fused_bwd_workspace_bytes", T, n, C, 1)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    code = {"bf16": _lib.DTYPE_BF16, "f16": _lib.DTYPE_F16}[dt]
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    _lib.call("mhc_fused_bwd", P(xt), code, P(gt), code, P(Mt), n * n, P(at), P(pt), n, _lib.H_ACTIVATED, P(wt),
              P(dx), code, P(dM), P(da), P(dp), P(dw), P(ws), nb, T, n, C, ctypes.c_float(EPS),
              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    rdx, rdM, rda, rdp, rdw = O.mhc_fused_backward(x, M, a, p, w, dout, eps=EPS)
    tol = {"bf16": 2e-2, "f16": 5e-3}[dt]
    assert rel_err(np_of(dx), rdx) < tol
    for name, got, r in (("dM", dM, rdM), ("dH_pre", da, rda), ("dH_post", dp, rdp), ("d_w", dw, rdw)):
        assert rel_err(np_of(got), r) < GRAD_TOL, (name, rel_err(np_of(got), r))


@pytest.mark.parametrize("T,C", [(300, 1024), (37, 256)])
def test_per_token_n16_recorded_sinkhorn_state(T, C, knobs):
    """Per-token n = 16 with gradients records the Sinkhorn VJP state in the forward
    (mhc_sinkhorn_fwd_record) and the backward uses it (mhc_sinkhorn_bwd_recorded); with
    MHC_SK16_RECORD=0 the backward recomputes it.  Both give bitwise the same output and gradients."""
    from mhc_mlx_amd import kernel_timer

    n = 16
    g = rng(7300 + T)
    x = to_dtype_np(g.standard_normal((T, n, C)), "bf16")
    dout = dev_tensor(to_dtype_np(g.standard_normal((T, n, C)), "bf16"), "bf16")
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T)
    results = []
    for rec in ("1", "0"):
        knobs("MHC_SK16_RECORD", int(rec))
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = dev_tensor(x, "bf16").requires_grad_(True)
        out = ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dout)
        results.append([out.detach(), xt.grad] + [p.grad for p in ps])
    for name, a, b in zip(["out", "dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], *results):
        assert torch.equal(a, b), name
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, np_of(dout), sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(results[0][4]), refs[3]) < GRAD_TOL
    # without gradients nothing is recorded: the forward is the plain one (and identical)
    knobs("MHC_SK16_RECORD", 1)
    with torch.no_grad():
        ps = [dev_tensor(v) for v in (hpre, hpost, hres, w)]
        out_ng = ops.mhc_layer_forward_dynamic(dev_tensor(x, "bf16"), *ps, sinkhorn_iters=20, eps=EPS,
                                               output_dtype=torch.bfloat16)
    assert torch.equal(out_ng, results[0][0])


@pytest.mark.parametrize("T,n,C,per_token", [(300, 32, 512, False), (64, 24, 1024, False), (40, 48, 256, False),
                                             (37, 32, 256, True), (20, 20, 384, True)])
def test_block_sinkhorn_recorded_state_in_the_layer(T, n, C, per_token, knobs):
    """16 < n <= 64 with gradients: the layer's Sinkhorn forward records the VJP state and the
    backward reads it (layer-wide: partial sums, reduction, recorded VJP); with MHC_SK_BLK_RECORD=0
    the backward is mhc_layer_bwd, which recomputes it.  Both give bitwise the same output and
    gradients, and dH_res_raw matches the oracle."""
    g = rng(7400 + T + n)
    x = to_dtype_np(g.standard_normal((T, n, C)), "bf16")
    dout = dev_tensor(to_dtype_np(g.standard_normal((T, n, C)), "bf16"), "bf16")
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T if per_token else None)
    fn = ops.mhc_layer_forward_dynamic if per_token else ops.mhc_layer_forward
    results = []
    for rec in (1, 0):
        knobs("MHC_SK_BLK_RECORD", rec)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = dev_tensor(x, "bf16").requires_grad_(True)
        out = fn(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
        out.backward(dout)
        results.append([out.detach(), xt.grad] + [p.grad for p in ps])
    knobs("MHC_SK_BLK_RECORD", None)
    for name, a, b in zip(["out", "dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], *results):
        assert torch.equal(a, b), name
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, np_of(dout), sinkhorn_iters=20, eps=EPS)
    assert rel_err(np_of(results[0][4]), refs[3]) < GRAD_TOL


def test_per_token_n16_valu_fallback(knobs):
    """The VALU kernels that serve n = 16 when the MFMA kernels decline (here forced off through
    their knobs) give the same parity."""
    knobs("MHC_FWD_MFMA", 0)
    knobs("MHC_BWD_MFMA", 0)
    T, n, C, dt = 40, 16, 512, "bf16"
    g = rng(7200)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
    xt = dev_tensor(x, dt).requires_grad_(True)
    out = ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=EPS, output_dtype=xt.dtype)
    assert rel_err(np_of(out), O.mhc_forward_reference(x, hpre, hpost, hres, w, 20, EPS)) < 2e-2
    out.backward(dev_tensor(dout, dt))
    refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=EPS)
    gots = [xt.grad] + [p.grad for p in ps]
    for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], gots, refs):
        assert rel_err(np_of(got), r) < (2e-2 if name == "dx" else GRAD_TOL), name

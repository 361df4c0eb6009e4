"""GPU parity: fused forward / backward (static and per-token parameters).

Forward cases follow tests/test_correctness.py:52-179 of the reference
((2,4,128) at fp32/fp16/bf16 tolerances 1e-5/5e-3/2e-2, n=16 bf16, odd
C=129 with arange inputs) and add the shapes this library dispatches
differently: n not a power of two, the runtime-n kernels (n > 16) and the
two-pass path for tiles larger than the register budget.  The reference
never compares gradients (test_correctness.py:343-344); here every gradient
is compared with the float64 oracle.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import GRAD_TOL, TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import ops

pytestmark = pytest.mark.gpu

FWD_SHAPES = [
    (2, 4, 128), (2, 4, 129), (1, 4, 512), (3, 3, 64), (2, 1, 40), (2, 2, 24), (2, 8, 128),
    (2, 5, 72), (2, 16, 64), (2, 16, 256), (1, 32, 256), (2, 24, 40), (1, 64, 64), (2, 4, 20000),
    # full-tile forward with two chunks per thread (more than 512 chunks: 4-channel chunks
    # with fp32 output at C = 3072 / 4096, 8-channel chunks at C = 8192); n = 8 with two chunks
    # per thread is bounded at 512 threads, so C = 16384 with 16-bit output takes the general kernel
    (2, 4, 4096), (2, 8, 3072), (1, 4, 8192), (2, 8, 8192), (1, 8, 16384),
    # n = 16 with C a multiple of 128: the MFMA forward (one or two 128-channel slabs per wave)
    (3, 16, 128), (2, 16, 384), (2, 16, 1024), (1, 16, 2048),
]


def _inputs(B, n, C, xdt, seed):
    g = rng(seed)
    x = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    hpre, hpost, hres, w = params(g, n, C)
    return x, hpre, hpost, hres, w


@pytest.mark.parametrize("B,n,C", FWD_SHAPES)
@pytest.mark.parametrize("xdt,odt", [("f32", "f32"), ("bf16", "f32"), ("bf16", "bf16"), ("f16", "f16")])
def test_fused_forward_matches_oracle(B, n, C, xdt, odt):
    x, hpre, hpost, hres, w = _inputs(B, n, C, xdt, 100 + B * 31 + n * 7 + C)
    a, p = O.activate_pre_post(hpre, hpost, np.float32)
    M = O.mixing_matrix_from_logits(hres, iters=20, eps=1e-5, dtype=np.float32)
    ref = O.mhc_forward_fused_reference(x, M, a, p, w, eps=1e-5)
    out = ops.mhc_forward_fused_hip(dev_tensor(x, xdt), dev_tensor(M), dev_tensor(a), dev_tensor(p),
                                    dev_tensor(w), eps=1e-5,
                                    output_dtype=None if odt == "f32" else dev_tensor(x, xdt).dtype)
    assert out.dtype == {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[odt]
    got = np_of(out)
    assert rel_err(got, ref) < TOL[odt], (B, n, C, xdt, odt, rel_err(got, ref))
    if odt != "f32":
        # one rounding of the output: within 1 ulp of the rounded oracle
        ulp = 2.0 ** -8 if odt == "bf16" else 2.0 ** -11
        assert (np.abs(got - ref) <= ulp * np.abs(ref) + 1e-6).all()


def test_fused_forward_arange_kat_half_output():
    """Reference test_fused_forward_half_output (test_correctness.py:138-179)."""
    B, n, C = 2, 4, 129
    H_pre_raw = (np.arange(n, dtype=np.float32) * 0.1) - 0.2
    H_post_raw = (np.arange(n, dtype=np.float32) * 0.07) - 0.1
    H_res_raw = (np.arange(n * n, dtype=np.float32).reshape(n, n) * 0.01) - 0.05
    w = np.ones(C, np.float32)
    a, p = O.activate_pre_post(H_pre_raw, H_post_raw, np.float32)
    M = O.mixing_matrix_from_logits(H_res_raw, iters=10, eps=1e-5, dtype=np.float32)
    for dt, tol in (("f16", 5e-3), ("bf16", 2e-2)):
        x = to_dtype_np(np.arange(B * n * C, dtype=np.float32).reshape(B, n, C) * 0.001, dt)
        ref = O.mhc_forward_reference(x, H_pre_raw, H_post_raw, H_res_raw, w, sinkhorn_iters=10, eps=1e-5)
        xt = dev_tensor(x, dt)
        out = ops.mhc_forward_fused_hip(xt, dev_tensor(M), dev_tensor(a), dev_tensor(p), dev_tensor(w),
                                        eps=1e-5, output_dtype=xt.dtype)
        assert np.abs(np_of(out) - ref).max() < tol


def test_identity_mapping_n4():
    """Reference test_identity_mapping_n4: identity init gives out ~= x (1e-4)."""
    B, n, C = 2, 4, 64
    x = to_dtype_np(rng(123).standard_normal((B, n, C)), "bf16")
    hpre = np.full(n, -12.0, np.float32)
    hpost = np.full(n, -12.0, np.float32)
    hres = (np.full((n, n), -12.0) + np.eye(n) * 12.0).astype(np.float32)
    w = np.ones(C, np.float32)
    out = ops.mhc_layer_forward(dev_tensor(x, "bf16"), dev_tensor(hpre), dev_tensor(hpost), dev_tensor(hres),
                                dev_tensor(w), sinkhorn_iters=20, eps=1e-5)
    assert np.abs(np_of(out) - x).max() < 1e-4


# ------------------------------------------------------------------ backward

BWD_SHAPES = [(2, 4, 128), (3, 4, 129), (2, 3, 64), (2, 8, 96), (2, 16, 64), (2, 5, 40), (2, 24, 48),
              (1, 32, 64), (2, 4, 20000),
              # n = 16, C a multiple of 128 up to 1024: the MFMA backward with layer-wide
              # parameters for 16-bit x == dout (one or two slabs per wave, 64-512 threads)
              (3, 16, 128), (5, 16, 256), (4, 16, 384), (3, 16, 512), (2, 16, 1024)]


def _bwd_case(B, n, C, xdt, gdt, seed, per_token=False):
    g = rng(seed)
    x = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=B if per_token else None)
    return x, dout, hpre, hpost, hres, w


def _grad_tol(dt):
    return 1e-5 if dt == "f32" else TOL[dt]


@pytest.mark.parametrize("B,n,C", BWD_SHAPES)
@pytest.mark.parametrize("xdt,gdt", [("f32", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16")])
def test_fused_backward_activated_matches_oracle(B, n, C, xdt, gdt):
    """Op-level VJP (metal.py:2787-2857): grads w.r.t. x, M, activated H, w."""
    x, dout, hpre, hpost, hres, w = _bwd_case(B, n, C, xdt, gdt, 500 + B * 13 + n * 5 + C)
    a, p = O.activate_pre_post(hpre, hpost, np.float32)
    M = O.mixing_matrix_from_logits(hres, iters=20, eps=1e-5, dtype=np.float32)
    ts = [dev_tensor(v).requires_grad_(True) for v in (M, a, p, w)]
    xt = dev_tensor(x, xdt).requires_grad_(True)
    out = ops.mhc_forward_fused_hip_autograd(xt, *ts[:3], ts[3], eps=1e-5)
    out.backward(dev_tensor(dout, gdt).to(out.dtype))
    ref = O.mhc_fused_backward(x, M, a, p, w, dout, eps=1e-5)
    names = ["dx", "dM", "dH_pre", "dH_post", "d_w"]
    gots = [np_of(xt.grad)] + [np_of(t.grad) for t in ts]
    tol_x = _grad_tol(xdt)
    for name, got, r in zip(names, gots, ref):
        tol = tol_x if name == "dx" else GRAD_TOL
        assert rel_err(got, r) < tol, (name, B, n, C, xdt, gdt, rel_err(got, r))


@pytest.mark.parametrize("B,n,C", [(2, 4, 128), (2, 16, 64), (2, 24, 48), (2, 4, 20000)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_layer_backward_raw_matches_oracle(B, n, C, xdt):
    """Whole-layer VJP from raw logits, through sigmoid and 20 Sinkhorn iterations."""
    x, dout, hpre, hpost, hres, w = _bwd_case(B, n, C, xdt, xdt, 900 + n + C)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
    xt = dev_tensor(x, xdt).requires_grad_(True)
    out = ops.mhc_layer_forward(xt, *ps, sinkhorn_iters=20, eps=1e-5,
                                output_dtype=None if xdt == "f32" else xt.dtype)
    out.backward(dev_tensor(dout, xdt))
    ref = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=1e-5)
    gots = [np_of(xt.grad)] + [np_of(t.grad) for t in ps]
    for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], gots, ref):
        tol = _grad_tol(xdt) if name == "dx" else GRAD_TOL
        assert rel_err(got, r) < tol, (name, B, n, C, xdt, rel_err(got, r))


@pytest.mark.parametrize("B,n,C", [(6, 4, 96), (5, 16, 64), (4, 8, 33), (3, 24, 40), (3, 3, 16), (4, 16, 256),
                                   (3, 16, 1024),
                                   # C beyond the layer-wide kernel's one chunk per thread: the general kernel
                                   (2, 4, 20000), (2, 8, 5000)])
@pytest.mark.parametrize("xdt", ["f32", "bf16", "f16"])
def test_dynamic_per_token_matches_oracle(B, n, C, xdt):
    """Per-token H_pre/H_post [B, n] and H_res [B, n, n] (forward and all gradients)."""
    x, dout, hpre, hpost, hres, w = _bwd_case(B, n, C, xdt, xdt, 1300 + B + n + C, per_token=True)
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
    xt = dev_tensor(x, xdt).requires_grad_(True)
    out = ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=1e-5,
                                        output_dtype=None if xdt == "f32" else xt.dtype)
    ref_out = O.mhc_forward_reference(x, hpre, hpost, hres, w, sinkhorn_iters=20, eps=1e-5)
    assert rel_err(np_of(out), ref_out) < TOL[xdt]
    out.backward(dev_tensor(dout, xdt))
    ref = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=1e-5)
    gots = [np_of(xt.grad)] + [np_of(t.grad) for t in ps]
    for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], gots, ref):
        tol = _grad_tol(xdt) if name == "dx" else GRAD_TOL
        assert rel_err(got, r) < tol, (name, B, n, C, xdt, rel_err(got, r))


@pytest.mark.parametrize("B,n,C,xdt,gdt", [(64, 4, 4096, "bf16", "bf16"), (48, 8, 2048, "bf16", "bf16"),
                                           (40, 4, 1024, "bf16", "f32"), (30, 8, 512, "f16", "f32"),
                                           (25, 3, 200, "f32", "f32")])
@pytest.mark.parametrize("legacy", [0, 1])
def test_per_token_backward_with_many_tokens_per_workgroup(B, n, C, xdt, gdt, legacy, knobs):
    """Per-token n <= 8 with MHC_BWD_GRID = 3: every workgroup walks many tokens, so the per-token reset
    of the parameter sums and the reuse of the LDS reduction run.  n = 4, C = 4096 bf16 is the full-tile
    variant of the benchmarked shape; fp32 dout comes with the default fp32 output.  MHC_BWD_LEGACY = 1
    sends the same shapes to the general backward kernel.  A second run is bitwise identical."""
    knobs("MHC_BWD_GRID", 3)
    knobs("MHC_BWD_LEGACY", legacy)
    x, dout, hpre, hpost, hres, w = _bwd_case(B, n, C, xdt, gdt, 1700 + B + n + C, per_token=True)
    runs = []
    for _ in range(2):
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = dev_tensor(x, xdt).requires_grad_(True)
        out = ops.mhc_layer_forward_dynamic(xt, *ps, sinkhorn_iters=20, eps=1e-5,
                                            output_dtype=xt.dtype if gdt == xdt and xdt != "f32" else None)
        out.backward(dev_tensor(dout, gdt))
        runs.append([xt.grad.clone()] + [t.grad.clone() for t in ps])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    ref = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=1e-5)
    for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], runs[0], ref):
        tol = _grad_tol(xdt) if name == "dx" else GRAD_TOL
        assert rel_err(np_of(got), r) < tol, (name, rel_err(np_of(got), r))


@pytest.mark.parametrize("B,n,C,xdt,per_token,spw", [
    (64, 4, 4096, "bf16", False, None), (5, 4, 4096, "bf16", False, None), (1, 4, 2048, "f16", False, None),
    (37, 16, 1024, "bf16", True, None), (37, 16, 1024, "bf16", True, 1), (9, 16, 2048, "f16", True, None),
    (21, 16, 512, "bf16", False, 1), (21, 16, 512, "f16", False, None)])
@pytest.mark.parametrize("grid", [3, 100])
def test_pipelined_loads_match_unpipelined(B, n, C, xdt, per_token, spw, grid, knobs):
    """MHC_BWD_PIPE = 1 (the next token's x and dout loaded during this token's dx pass) against 0 at one
    grid: the same sums in the same order, so every gradient is bitwise equal.  Grid 3 walks many tokens per
    workgroup; grid 100 leaves workgroups without a token when B < 100."""
    knobs("MHC_BWD_GRID", grid)
    if spw is not None:
        knobs("MHC_BWD_SPW", spw)
    x, dout, hpre, hpost, hres, w = _bwd_case(B, n, C, xdt, xdt, 2100 + B + n + C, per_token=per_token)
    runs = []
    for pipe in (1, 0):
        knobs("MHC_BWD_PIPE", pipe)
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = dev_tensor(x, xdt).requires_grad_(True)
        fwd = ops.mhc_layer_forward_dynamic if per_token else ops.mhc_layer_forward
        out = fwd(xt, *ps, sinkhorn_iters=20, eps=1e-5, output_dtype=xt.dtype)
        out.backward(dev_tensor(dout, xdt))
        runs.append([xt.grad.clone()] + [t.grad.clone() for t in ps])
    for name, a, b in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], *runs):
        assert torch.equal(a, b), name
    if B * n * C <= 64 * 16 * 1024:
        ref = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=1e-5)
        for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], runs[0], ref):
            tol = _grad_tol(xdt) if name == "dx" else GRAD_TOL
            assert rel_err(np_of(got), r) < tol, (name, rel_err(np_of(got), r))


def test_backward_is_deterministic():
    B, n, C = 64, 4, 1024
    x, dout, hpre, hpost, hres, w = _bwd_case(B, n, C, "bf16", "bf16", 77)
    grads = []
    for _ in range(2):
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = dev_tensor(x, "bf16").requires_grad_(True)
        ops.mhc_layer_forward(xt, *ps, output_dtype=torch.bfloat16).backward(dev_tensor(dout, "bf16"))
        grads.append([xt.grad.clone()] + [t.grad.clone() for t in ps])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_fused_rejects_bad_arguments():
    x = torch.zeros(2, 4, 8, device="cuda")
    M = torch.zeros(4, 4, device="cuda")
    h = torch.zeros(4, device="cuda")
    w = torch.ones(8, device="cuda")
    with pytest.raises(ValueError, match="x must be"):
        ops.mhc_forward_fused_hip(x[0], M, h, h, w)
    with pytest.raises(ValueError, match="rms_weight must be shape"):
        ops.mhc_forward_fused_hip(x, M, h, h, torch.ones(7, device="cuda"))
    with pytest.raises(ValueError, match="x must be bfloat16"):
        ops.mhc_forward_fused_hip(x, M, h, h, w, output_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors"):
        ops.mhc_forward_fused_hip(x.cpu(), M, h, h, w)


@pytest.mark.parametrize("T,C", [(1000, 4096), (700, 1024), (300, 2048), (257, 512)])
@pytest.mark.parametrize("xdt,odt", [("bf16", "bf16"), ("f16", "f16"), ("bf16", "f32")])
def test_pipelined_forward_matches_per_token_workgroups(T, C, xdt, odt, knobs):
    """n = 4 full tiles: the pipelined forward (MHC_FWD_PIPE: persistent grid, the next token's loads
    issued before the RMS barrier) is bitwise the one-token-per-workgroup kernel, with one and three
    workgroups per CU (several tokens per workgroup), and matches the oracle."""
    n = 4
    x, hpre, hpost, hres, w = _inputs(T, n, C, xdt, 4400 + T + C)
    a, p = O.activate_pre_post(hpre, hpost, np.float32)
    M = O.mixing_matrix_from_logits(hres, iters=20, eps=1e-5, dtype=np.float32)
    xt = dev_tensor(x, xdt)
    outs = []
    for pipe in (0, 1, 3):
        knobs("MHC_FWD_PIPE", pipe)
        outs.append(ops.mhc_forward_fused_hip(xt, dev_tensor(M), dev_tensor(a), dev_tensor(p), dev_tensor(w),
                                              eps=1e-5, output_dtype=None if odt == "f32" else xt.dtype))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = O.mhc_forward_fused_reference(x, M, a, p, w, eps=1e-5)
    assert rel_err(np_of(outs[1]), ref) < TOL[odt]

"""mhc_layer_bwd_noalloc (the workspace in the library's fixed device array)
against mhc_layer_bwd with a caller workspace, through the C ABI.

Two calls in a row on one GPU, the second with a smaller input, so the
second runs on what the first left in the array.  The two entry points run
the same kernels with the same partial-row counts, so their results are
bitwise equal; the smaller shapes are also checked against the float64
oracle.
"""

import ctypes

import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import GRAD_TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import _lib

pytestmark = pytest.mark.gpu

EPS = 1e-6
ITERS = 20
P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
CODE = {"bf16": _lib.DTYPE_BF16, "f32": _lib.DTYPE_F32}


def _case(T, n, C, dt, per_token, seed):
    g = rng(seed)
    x = to_dtype_np(g.standard_normal((T, n, C)), dt)
    dout = to_dtype_np(g.standard_normal((T, n, C)), dt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T if per_token else None)
    return x, dout, hpre, hpost, hres, w


def _run(T, n, C, dt, per_token, seed, noalloc):
    x, dout, hpre, hpost, hres, w = _case(T, n, C, dt, per_token, seed)
    xt, gt = dev_tensor(x, dt), dev_tensor(dout, dt)
    hp, hq, hr, wt = (dev_tensor(v) for v in (hpre, hpost, hres, w))
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    M = torch.empty_like(hr)
    out = torch.empty_like(xt)
    _lib.call("mhc_layer_fwd", P(xt), CODE[dt], P(hp), P(hq), P(hr), P(wt), P(out), CODE[dt], P(M), T, n, C,
              int(per_token), ITERS, ctypes.c_float(EPS), s)
    dx = torch.empty_like(xt)
    grads = [torch.empty_like(hp), torch.empty_like(hq), torch.empty_like(hr), torch.empty_like(wt)]
    common = (P(xt), CODE[dt], P(gt), CODE[dt], P(hp), P(hq), P(hr), P(M), P(wt), P(dx)) + tuple(P(t) for t in grads)
    if noalloc:
        _lib.call("mhc_layer_bwd_noalloc", *common, T, n, C, int(per_token), ITERS, ctypes.c_float(EPS), s)
    else:
        nb = _lib.query("mhc_layer_bwd_workspace_bytes", T, n, C, int(per_token), ITERS)
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        _lib.call("mhc_layer_bwd", *common, P(ws), nb, T, n, C, int(per_token), ITERS, ctypes.c_float(EPS), s)
    torch.cuda.synchronize()
    return [dx] + grads


# (T, n, C, dtype, per_token): the first is config 2's layer shape at 4096 tokens (35 MB of workspace on a
# 256-CU GPU), the second a smaller one run on what the first left in the array.
PAIRS = [
    ((4096, 4, 4096, "bf16", False), (300, 4, 1000, "bf16", False)),
    ((2000, 16, 1024, "bf16", True), (37, 8, 256, "f32", True)),
    ((1000, 32, 512, "bf16", False), (5, 4, 64, "f32", False)),
    ((500, 64, 1024, "bf16", False), (7, 48, 512, "bf16", False)),
    # config 3 (per-token n = 16 at 16384 tokens): the block-layout Sinkhorn VJP needs no workspace
    ((16384, 16, 1024, "bf16", True), (300, 16, 512, "bf16", True)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_the_workspace_entry_point(first, second):
    for k, shape in enumerate((first, second)):
        print("noalloc case", shape, flush=True)
        seed = 9100 + 17 * k + shape[0]
        ref = _run(*shape, seed, noalloc=False)
        got = _run(*shape, seed, noalloc=True)
        for name, a, b in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], got, ref):
            assert torch.equal(a, b), (shape, name)
        T, n, C, dt, pt = shape
        if T * n * C <= 2_000_000:
            x, dout, hpre, hpost, hres, w = _case(T, n, C, dt, pt, seed)
            refs = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, ITERS, EPS)
            assert rel_err(np_of(got[0]), refs[0]) < (2e-2 if dt == "bf16" else 1e-5)
            for name, a, r in zip(["dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], got[1:], refs[1:]):
                assert rel_err(np_of(a), r) < GRAD_TOL, name


def test_noalloc_rejects_shapes_beyond_its_array():
    """Per-token n = 16 at 16384 tokens with 300 Sinkhorn iterations: more than the block layout's
    32 VJP checkpoints, so the VJP keeps 256 bytes of state per matrix and iteration in its workspace,
    1.2 GB, more than the 64 MiB array.  The call is rejected on the host before anything is launched.
    (At 20 iterations config 3 needs no Sinkhorn workspace and fits.)"""
    T, n, C, iters = 16384, 16, 1024, 300
    assert _lib.query("mhc_layer_bwd_workspace_bytes", T, n, C, 1, iters) > 64 << 20
    # real buffers of the call's own sizes, so nothing out of bounds could be touched even if the host
    # check were missing; the call must still be rejected before any launch
    dev = "cuda"
    x = torch.zeros((T, n, C), dtype=torch.bfloat16, device=dev)
    g = torch.zeros_like(x)
    dx = torch.empty_like(x)
    hpre, hpost = torch.zeros((T, n), device=dev), torch.zeros((T, n), device=dev)
    hres, M = torch.zeros((T, n, n), device=dev), torch.zeros((T, n, n), device=dev)
    w = torch.ones(C, device=dev)
    dpre, dpost, dres, dw = (torch.empty_like(t) for t in (hpre, hpost, hres, w))
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    before = dx.clone()
    rc = _lib.load().mhc_layer_bwd_noalloc(P(x), 1, P(g), 1, P(hpre), P(hpost), P(hres), P(M), P(w), P(dx),
                                           P(dpre), P(dpost), P(dres), P(dw), T, n, C, 1, iters,
                                           ctypes.c_float(EPS), None)
    torch.cuda.synchronize()
    assert rc == -1
    assert torch.equal(dx, before)
    assert "mhc_layer_bwd with a workspace" in _lib.last_error()

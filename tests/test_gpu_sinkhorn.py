"""GPU parity: batched Sinkhorn-Knopp forward and VJP vs the oracle.

Mirrors the reference's tests/test_correctness.py:33-49 (n=4/20 iters tol
1e-5; n=16/10 iters tol 1e-4 there, 1e-5 here), tests/test_stability.py
(logits all 100.0, n=32) and tests/test_stress.py:17-31 (eps 1e-3 / 1e-6),
plus eps-mask cases and the doubly-stochastic residual criterion.
"""

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import dev_tensor, np_of, rel_err, rng

from mhc_mlx_amd import ops

pytestmark = pytest.mark.gpu


def _fwd(H: np.ndarray, iters: int, eps: float) -> np.ndarray:
    return np_of(ops.sinkhorn_knopp_hip(dev_tensor(H), iters=iters, eps=eps))


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8, 12, 16, 24, 32, 64])
@pytest.mark.parametrize("iters", [0, 1, 5, 20])
def test_sinkhorn_fwd_matches_oracle(n, iters):
    g = rng(1000 + n * 7 + iters)
    batch = 5
    H = g.standard_normal((batch, n, n)).astype(np.float32)
    got = _fwd(H, iters, 1e-5)
    ref = O.mixing_matrix_from_logits(H, iters=iters, eps=1e-5)
    assert np.isfinite(got).all()
    assert rel_err(got, ref, 1.0) < 1e-5, (n, iters, rel_err(got, ref, 1.0))


@pytest.mark.parametrize("n,iters,tol", [(4, 20, 1e-5), (16, 10, 1e-5)])
def test_sinkhorn_single_matrix_reference_tolerances(n, iters, tol):
    H = rng(0).standard_normal((n, n)).astype(np.float32)
    got = _fwd(H, iters, 1e-5)
    ref = O.mixing_matrix_from_logits(H, iters=iters, eps=1e-5)
    assert got.shape == (n, n)
    assert rel_err(got, ref, 1.0) < tol


@pytest.mark.parametrize("eps", [1e-3, 1e-6])
def test_sinkhorn_eps_extremes(eps):
    H = rng(123).standard_normal((8, 8)).astype(np.float32)
    got = _fwd(H, 20, eps)
    ref = O.mixing_matrix_from_logits(H, iters=20, eps=eps)
    assert np.isfinite(got).all()
    assert rel_err(got, ref, 1.0) < 1e-5


def test_sinkhorn_bomb_logits_n32():
    H = np.full((32, 32), 100.0, dtype=np.float32)
    got = _fwd(H, 20, 1e-5)
    assert np.isfinite(got).all()
    assert np.abs(got.sum(1) - 1).max() <= 1e-3 and np.abs(got.sum(0) - 1).max() <= 1e-3
    assert np.abs(got - 1.0 / 32).max() < 1e-6


def test_sinkhorn_identity_init():
    n = 8
    H = (np.full((n, n), -12.0) + np.eye(n) * 12.0).astype(np.float32)
    got = _fwd(H, 20, 1e-5)
    assert np.abs(got - np.eye(n)).max() < 1e-4


def test_sinkhorn_masked_columns_and_rows():
    # column 2 is ~e^-40 after the row-max shift: its sum falls below eps and
    # the reference zeroes it; row 3 then carries (almost) nothing.
    n = 6
    g = rng(7)
    H = g.standard_normal((3, n, n)).astype(np.float32)
    H[:, :, 2] = -40.0
    H[1, 3, :] = -45.0
    H[1, 3, 2] = 0.0
    for eps in (1e-5, 1e-3):
        got = _fwd(H, 20, eps)
        ref = O.mixing_matrix_from_logits(H.astype(np.float64), iters=20, eps=eps)
        assert rel_err(got, ref, 1.0) < 1e-5


@pytest.mark.parametrize("n,batch", [(4, 16384), (16, 1024)])
def test_sinkhorn_ds_residual(n, batch):
    """Row/column-sum residual: <= max(1e-5, oracle(fp32) residual + 1e-6)."""
    H = rng(5 + n).standard_normal((batch, n, n)).astype(np.float32)
    got = _fwd(H, 20, 1e-6)
    ref32 = O.mixing_matrix_from_logits(H, iters=20, eps=1e-6, dtype=np.float32)
    assert O.ds_residual(got) <= max(1e-5, O.ds_residual(ref32) + 1e-6)
    # column sums are exactly normalised by the last step
    assert np.abs(got.sum(-2) - 1).max() < 1e-5


# ------------------------------------------------------------------ VJP

@pytest.mark.parametrize("n", [1, 2, 3, 4, 7, 8, 16, 24, 32, 64])
@pytest.mark.parametrize("iters", [1, 5, 20])
def test_sinkhorn_vjp_matches_oracle(n, iters):
    g = rng(3000 + n * 3 + iters)
    batch = 3
    H = g.standard_normal((batch, n, n)).astype(np.float32)
    dM = g.standard_normal((batch, n, n)).astype(np.float32)
    Ht = dev_tensor(H).requires_grad_(True)
    M = ops.sinkhorn_knopp_hip_autograd(Ht, iters=iters, eps=1e-5)
    M.backward(dev_tensor(dM))
    got = np_of(Ht.grad)
    ref = O.sinkhorn_knopp_vjp(H, dM, iters=iters, eps=1e-5)
    assert rel_err(got, ref, 1e-3) < 1e-5, (n, iters, rel_err(got, ref, 1e-3))
    # row sums of dH vanish (row-shift invariance)
    assert np.abs(got.sum(-1)).max() < 1e-4 * max(1.0, np.abs(dM).max())


def test_sinkhorn_vjp_masked_columns():
    n = 6
    g = rng(11)
    H = g.standard_normal((2, n, n)).astype(np.float32)
    H[:, :, 4] = -40.0
    dM = g.standard_normal((2, n, n)).astype(np.float32)
    Ht = dev_tensor(H).requires_grad_(True)
    ops.sinkhorn_knopp_hip_autograd(Ht, iters=20, eps=1e-5).backward(dev_tensor(dM))
    ref = O.sinkhorn_knopp_vjp(H.astype(np.float64), dM, iters=20, eps=1e-5)
    got = np_of(Ht.grad)
    assert rel_err(got, ref, 1.0) < 1e-5


def test_sinkhorn_vjp_long_iterations_use_workspace():
    # 4 * iters * 64 floats per wave exceeds the LDS budget: global state path
    n, iters = 64, 80
    g = rng(21)
    H = g.standard_normal((2, n, n)).astype(np.float32)
    dM = g.standard_normal((2, n, n)).astype(np.float32)
    from mhc_mlx_amd import _lib
    assert _lib.query("mhc_sinkhorn_bwd_workspace_bytes", 2, n, iters) > 0
    Ht = dev_tensor(H).requires_grad_(True)
    ops.sinkhorn_knopp_hip_autograd(Ht, iters=iters, eps=1e-5).backward(dev_tensor(dM))
    ref = O.sinkhorn_knopp_vjp(H, dM, iters=iters, eps=1e-5)
    got = np_of(Ht.grad)
    assert rel_err(got, ref, 1e-3) < 1e-5


def test_sinkhorn_vjp_constant_column_cotangent_is_zero():
    # dM = 1 c^T: column sums of M are fixed to 1, so the gradient vanishes
    n = 5
    H = rng(2).standard_normal((n, n)).astype(np.float32)
    c = rng(3).standard_normal(n).astype(np.float32)
    dM = np.ones((n, 1), np.float32) * c[None, :]
    Ht = dev_tensor(H).requires_grad_(True)
    ops.sinkhorn_knopp_hip_autograd(Ht, iters=20, eps=1e-5).backward(dev_tensor(dM))
    assert np.abs(np_of(Ht.grad)).max() < 1e-5


def test_sinkhorn_rejects_bad_shapes():
    with pytest.raises(ValueError, match="square"):
        ops.sinkhorn_knopp_hip(torch.zeros(3, 4, device="cuda"))
    with pytest.raises(ValueError, match="MAX_N_ALLOWED"):
        ops.sinkhorn_knopp_hip(torch.zeros(65, 65, device="cuda"))


# ------------------------------------------------ n = 16 batched kernels
# (default: the 4 x 4-block layout, 16 lanes per matrix, VJP state recomputed in registers in segments of
# 9 iterations; MHC_SK16_CPL = 4 / 2: four / eight lanes per matrix, VJP state in the workspace)

@pytest.mark.parametrize("batch", [1, 15, 17, 64, 65, 1000])
def test_sinkhorn16_batches_and_tails(batch):
    """Batches that leave waves and workgroups partly empty."""
    g = rng(4000 + batch)
    H = (2.0 * g.standard_normal((batch, 16, 16))).astype(np.float32)
    dM = g.standard_normal((batch, 16, 16)).astype(np.float32)
    got = _fwd(H, 20, 1e-6)
    ref = O.mixing_matrix_from_logits(H, iters=20, eps=1e-6)
    assert rel_err(got, ref, 1.0) < 1e-5
    Ht = dev_tensor(H).requires_grad_(True)
    ops.sinkhorn_knopp_hip_autograd(Ht, iters=20, eps=1e-6).backward(dev_tensor(dM))
    rg = O.sinkhorn_knopp_vjp(H, dM, iters=20, eps=1e-6)
    assert rel_err(np_of(Ht.grad), rg, 1e-3) < 1e-5


def test_sinkhorn16_masked_rows_and_columns():
    """Eps masks (reference.py:37-46): a column below eps is zeroed, a masked row passes its
    gradient through unchanged."""
    g = rng(4100)
    H = g.standard_normal((40, 16, 16)).astype(np.float32)
    H[::3, :, 5] = -40.0                       # a masked column in every third matrix
    H[1::3, 7, :] = -45.0                      # a row that is all tiny ...
    H[1::3, 7, 0] = 0.0                        # ... except one entry (its max)
    dM = g.standard_normal((40, 16, 16)).astype(np.float32)
    for eps in (1e-5, 1e-3):
        got = _fwd(H, 20, eps)
        ref = O.mixing_matrix_from_logits(H.astype(np.float64), iters=20, eps=eps)
        assert rel_err(got, ref, 1.0) < 1e-5, eps
        Ht = dev_tensor(H).requires_grad_(True)
        ops.sinkhorn_knopp_hip_autograd(Ht, iters=20, eps=eps).backward(dev_tensor(dM))
        rg = O.sinkhorn_knopp_vjp(H.astype(np.float64), dM, iters=20, eps=eps)
        assert rel_err(np_of(Ht.grad), rg, 1.0) < 1e-5, eps


def test_sinkhorn16_vjp_in_place_c_abi():
    """mhc_sinkhorn_bwd with dM and dlogits the same buffer (as the per-token layer backward uses
    it) and iters = 0 (the VJP of exp and the row-max shift alone)."""
    import ctypes

    from mhc_mlx_amd import _lib

    g = rng(4200)
    B = 200
    H = g.standard_normal((B, 16, 16)).astype(np.float32)
    dM = g.standard_normal((B, 16, 16)).astype(np.float32)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for iters in (0, 1, 20):
        Ht, buf = dev_tensor(H), dev_tensor(dM)
        nb = _lib.query("mhc_sinkhorn_bwd_workspace_bytes", B, 16, iters)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
        _lib.call("mhc_sinkhorn_bwd", P(Ht), P(buf), P(buf), B, 16, iters, ctypes.c_float(1e-6), P(ws), nb, s)
        rg = O.sinkhorn_knopp_vjp(H, dM, iters=iters, eps=1e-6)
        assert rel_err(np_of(buf), rg, 1e-3) < 1e-5, iters


@pytest.mark.parametrize("B,iters,cpl_fwd,cpl_bwd", [(200, 20, "4", "4"), (33, 1, "4", "2"), (65, 0, "2", "4"),
                                                   (1000, 20, "2", "2"), (200, 20, "0", "0"), (1000, 20, "0", "0"),
                                                   (77, 19, "0", "0"), (50, 37, "0", "0"), (33, 1, "0", "4"),
                                                   (65, 9, "4", "0")])
def test_sinkhorn16_recorded_state_matches_recompute(B, iters, cpl_fwd, cpl_bwd, knobs):
    """mhc_sinkhorn_fwd_record / mhc_sinkhorn_bwd_recorded (always the block layout: the forward records
    each iteration's row and column sums and the scales at each VJP segment's start, and the VJP rebuilds
    the scales from them with the forward's own products) give bitwise the results of mhc_sinkhorn_fwd /
    mhc_sinkhorn_bwd in the block layout (MHC_SK16_CPL 0, whose VJP recomputes its segments from LDS
    checkpoints).  With the lanes-per-matrix layouts (4 / 2) selected for the unrecorded calls the sums
    associate differently (last-bit differences), so those cases are held to the oracle's tolerance.
    The state buffer is deliberately not 256-byte aligned; masked rows and columns included."""
    knobs("MHC_SK16_RECORD", 1)
    import ctypes

    from mhc_mlx_amd import _lib

    g = rng(4300 + B + iters)
    H = (2.0 * g.standard_normal((B, 16, 16))).astype(np.float32)
    H[::5, :, 3] = -40.0
    dM = g.standard_normal((B, 16, 16)).astype(np.float32)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    eps = ctypes.c_float(1e-5)
    Ht = dev_tensor(H)
    knobs("MHC_SK16_CPL", int(cpl_fwd))
    M_plain = torch.empty_like(Ht)
    _lib.call("mhc_sinkhorn_fwd", P(Ht), P(M_plain), B, 16, iters, eps, s)
    nst = _lib.query("mhc_sinkhorn_state_bytes", B, 16, iters)
    nseg = -(-iters // 5)
    assert nst == B * 128 * max(1, iters + max(nseg - 1, 0)) + 256
    st_buf = torch.empty(nst + 64, dtype=torch.uint8, device="cuda")
    st = st_buf[48:]  # 48 bytes past the allocation's start
    M_rec = torch.empty_like(Ht)
    _lib.call("mhc_sinkhorn_fwd_record", P(Ht), P(M_rec), P(st), nst, B, 16, iters, eps, s)
    if cpl_fwd == "0":
        assert torch.equal(M_rec, M_plain)
    else:
        assert rel_err(np_of(M_rec), np_of(M_plain), 1.0) < 2e-6
    knobs("MHC_SK16_CPL", int(cpl_bwd))
    d_rec = dev_tensor(dM)
    _lib.call("mhc_sinkhorn_bwd_recorded", P(Ht), P(d_rec), P(d_rec), P(st), nst, B, 16, iters, eps, s)
    nb = _lib.query("mhc_sinkhorn_bwd_workspace_bytes", B, 16, iters)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    d_plain = dev_tensor(dM)
    _lib.call("mhc_sinkhorn_bwd", P(Ht), P(d_plain), P(d_plain), B, 16, iters, eps, P(ws), nb, s)
    if cpl_bwd == "0":
        assert torch.equal(d_rec, d_plain)
    rg = O.sinkhorn_knopp_vjp(H.astype(np.float64), dM, iters=iters, eps=1e-5)
    assert rel_err(np_of(d_rec), rg, 1.0) < 1e-5
    assert rel_err(np_of(d_plain), rg, 1.0) < 1e-5


@pytest.mark.parametrize("iters", [300, 4, 6, 11])
def test_sinkhorn16_recorded_vjp_any_iteration_count(iters):
    """The recorded VJP keeps no state in LDS, so it runs at iteration counts beyond the block layout's 32
    LDS checkpoints (300: the unrecorded VJP takes the four-lanes-per-matrix kernel there), and at counts
    around its 5-iteration segments.  Against the oracle (the 300-iteration VJP, a long product of steps,
    at 1e-4); matrices past a multiple of four (the last wave's idle lane groups) included."""
    import ctypes

    from mhc_mlx_amd import _lib

    B = 37
    g = rng(4700 + iters)
    H = (2.0 * g.standard_normal((B, 16, 16))).astype(np.float32)
    H[::4, :, 5] = -40.0
    dM = g.standard_normal((B, 16, 16)).astype(np.float32)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    eps = ctypes.c_float(1e-5)
    Ht = dev_tensor(H)
    nst = _lib.query("mhc_sinkhorn_state_bytes", B, 16, iters)
    st = torch.empty(nst, dtype=torch.uint8, device="cuda")
    M = torch.empty_like(Ht)
    _lib.call("mhc_sinkhorn_fwd_record", P(Ht), P(M), P(st), nst, B, 16, iters, eps, s)
    d = dev_tensor(dM)
    _lib.call("mhc_sinkhorn_bwd_recorded", P(Ht), P(d), P(d), P(st), nst, B, 16, iters, eps, s)
    H64 = H.astype(np.float64)
    assert rel_err(np_of(M), O.mixing_matrix_from_logits(H64, iters=iters, eps=1e-5), 1.0) < 1e-5
    rg = O.sinkhorn_knopp_vjp(H64, dM, iters=iters, eps=1e-5)
    assert rel_err(np_of(d), rg, 1.0) < (1e-4 if iters > 100 else 1e-5)


@pytest.mark.parametrize("iters", [0, 1, 8, 9, 10, 17, 18, 19, 20, 28, 37, 300])
def test_sinkhorn16_block_layout_iteration_counts(iters):
    """The block layout's VJP at iteration counts around its 9-iteration segments (segments aligned to the
    end, the first one shorter), with masked columns; 300 iterations need more than its 32 checkpoints and
    take the four-lanes-per-matrix VJP instead.  Forward and VJP against the oracle; the VJP of 300
    iterations is a long product of steps and is held at 1e-4."""
    B = 37
    g = rng(4500 + iters)
    H = (2.0 * g.standard_normal((B, 16, 16))).astype(np.float32)
    H[::4, :, 2] = -40.0
    dM = g.standard_normal((B, 16, 16)).astype(np.float32)
    got = _fwd(H, iters, 1e-5)
    assert rel_err(got, O.mixing_matrix_from_logits(H.astype(np.float64), iters=iters, eps=1e-5), 1.0) < 1e-5
    Ht = dev_tensor(H).requires_grad_(True)
    ops.sinkhorn_knopp_hip_autograd(Ht, iters=iters, eps=1e-5).backward(dev_tensor(dM))
    rg = O.sinkhorn_knopp_vjp(H.astype(np.float64), dM, iters=iters, eps=1e-5)
    assert rel_err(np_of(Ht.grad), rg, 1.0) < (1e-4 if iters > 100 else 1e-5)


@pytest.mark.parametrize("cpl", [4, 2])
def test_sinkhorn16_layouts_agree(cpl, knobs):
    """The block layout (default) and the lanes-per-matrix layouts compute the same iterations with the sums
    associated differently: M and the VJP agree to fp32 rounding."""
    B = 300
    g = rng(4600 + cpl)
    H = (2.0 * g.standard_normal((B, 16, 16))).astype(np.float32)
    dM = g.standard_normal((B, 16, 16)).astype(np.float32)
    res = {}
    for layout in (0, cpl):
        knobs("MHC_SK16_CPL", layout)
        Ht = dev_tensor(H).requires_grad_(True)
        M = ops.sinkhorn_knopp_hip_autograd(Ht, iters=20, eps=1e-6)
        M.backward(dev_tensor(dM))
        res[layout] = (np_of(M), np_of(Ht.grad))
    assert rel_err(res[0][0], res[cpl][0], 1.0) < 2e-6
    assert rel_err(res[0][1], res[cpl][1], 1.0) < 1e-5


@pytest.mark.parametrize("B,n,iters", [(1, 32, 20), (1, 24, 20), (5, 32, 3), (1, 64, 20), (3, 48, 1), (9, 17, 0),
                                       (1, 32, 90), (700, 32, 20), (700, 64, 20), (300, 48, 5)])
def test_sinkhorn_blk_recorded_state_matches_recompute(B, n, iters):
    """16 < n <= 64: mhc_sinkhorn_fwd_record / mhc_sinkhorn_bwd_recorded give bitwise the results of
    mhc_sinkhorn_fwd / mhc_sinkhorn_bwd (the forward records the same state the VJP otherwise
    recomputes into LDS or its workspace: 90 iterations at n = 32 and n = 64 exceed one wave's LDS
    share), and both match the oracle.  The state buffer is deliberately not 256-byte aligned; masked
    rows and columns included; the VJP runs in place (dM aliasing dH) as the layer's per-token
    backward calls it."""
    import ctypes

    from mhc_mlx_amd import _lib

    g = rng(4400 + B + n + iters)
    H = (2.0 * g.standard_normal((B, n, n))).astype(np.float32)
    H[::3, :, 1] = -40.0
    dM = g.standard_normal((B, n, n)).astype(np.float32)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    eps = ctypes.c_float(1e-5)
    Ht = dev_tensor(H)
    M_plain = torch.empty_like(Ht)
    _lib.call("mhc_sinkhorn_fwd", P(Ht), P(M_plain), B, n, iters, eps, s)
    nst = _lib.query("mhc_sinkhorn_state_bytes", B, n, iters)
    npow = 32 if n <= 32 else 64
    assert nst == B * max(iters, 1) * 6 * npow * 4 + 256
    st_buf = torch.empty(nst + 64, dtype=torch.uint8, device="cuda")
    st = st_buf[48:]
    M_rec = torch.empty_like(Ht)
    _lib.call("mhc_sinkhorn_fwd_record", P(Ht), P(M_rec), P(st), nst, B, n, iters, eps, s)
    assert torch.equal(M_rec, M_plain)
    d_rec = dev_tensor(dM)
    _lib.call("mhc_sinkhorn_bwd_recorded", P(Ht), P(d_rec), P(d_rec), P(st), nst, B, n, iters, eps, s)
    nb = _lib.query("mhc_sinkhorn_bwd_workspace_bytes", B, n, iters)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    d_plain = torch.empty_like(Ht)
    _lib.call("mhc_sinkhorn_bwd", P(Ht), P(dev_tensor(dM)), P(d_plain), B, n, iters, eps, P(ws), nb, s)
    torch.cuda.synchronize()
    assert torch.equal(d_rec, d_plain)
    rm = O.mixing_matrix_from_logits(H.astype(np.float64), iters=iters, eps=1e-5)
    assert rel_err(np_of(M_rec), rm, 1.0) < 1e-5
    rg = O.sinkhorn_knopp_vjp(H.astype(np.float64), dM, iters=iters, eps=1e-5)
    assert rel_err(np_of(d_rec), rg, 1.0) < 1e-5


def test_sinkhorn16_identity_init_and_bomb():
    n = 16
    Hi = (np.full((n, n), -12.0) + np.eye(n) * 12.0).astype(np.float32)
    assert np.abs(_fwd(np.stack([Hi] * 20), 20, 1e-5) - np.eye(n)).max() < 1e-4
    Hb = np.full((20, n, n), 100.0, np.float32)
    got = _fwd(Hb, 20, 1e-5)
    assert np.isfinite(got).all() and np.abs(got - 1.0 / n).max() < 1e-6


@pytest.mark.parametrize("n,batch,iters", [(64, 1, 20), (48, 7, 1), (33, 2, 0), (64, 3, 32), (40, 1, 5),
                                           (64, 1, 33), (64, 5000, 20)])
def test_sinkhorn_workgroup_kernels_match_one_wave_kernels(n, batch, iters, knobs):
    """32 < n <= 64 runs on one four-wave workgroup per matrix (column sums through LDS; MHC_SK_WG=0
    keeps one wave per matrix).  Forward and VJP agree with the one-wave
    kernels to summation order and with the oracle, with masked rows and columns; above 32 iterations
    (the recomputed state no longer fits the workgroup's LDS) both sides take the one-wave kernels and
    agree bitwise."""
    g = rng(4600 + n + batch + iters)
    H = (2.0 * g.standard_normal((batch, n, n))).astype(np.float32)
    H[::2, :, 3] = -40.0
    H[:, 5, :] = -30.0
    dM = g.standard_normal((batch, n, n)).astype(np.float32)

    def run():
        Ht = dev_tensor(H).requires_grad_(True)
        M = ops.sinkhorn_knopp_hip_autograd(Ht, iters=iters, eps=1e-5)
        M.backward(dev_tensor(dM))
        return M.detach(), Ht.grad

    M1, d1 = run()
    knobs("MHC_SK_WG", 0)
    M0, d0 = run()
    torch.cuda.synchronize()
    if iters > 32:
        assert torch.equal(M1, M0) and torch.equal(d1, d0)
    assert rel_err(np_of(M1), np_of(M0), 1.0) < 1e-6
    assert rel_err(np_of(d1), np_of(d0), 1e-3) < 1e-5
    rm = O.mixing_matrix_from_logits(H.astype(np.float64), iters=iters, eps=1e-5)
    assert rel_err(np_of(M1), rm, 1.0) < 1e-5
    rg = O.sinkhorn_knopp_vjp(H.astype(np.float64), dM, iters=iters, eps=1e-5)
    assert rel_err(np_of(d1), rg, 1e-3) < 1e-5

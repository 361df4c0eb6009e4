"""GPU parity of the tile backward (bwd_tile_kernel), the kernel that takes every n <= 16 shape the
specialised backward kernels do not: fp32 and mixed dtypes above n = 8, n that is not 4, 8 or 16,
C beyond the register-resident kernels and rows without vector alignment.

The shapes cover one-tile tokens (staged in LDS by the first pass) and tokens of several tiles with a
partial last one, partial chunks (C not a multiple of the chunk width), every NMAX (4, 8, 16) with
n below it, layer-wide and per-token parameters, and MHC_BWD_GRID = 2 so that each workgroup walks
several tokens (the layer-wide sums accumulate across tokens, the per-token ones are reset).  Every
gradient is compared with the float64 oracle of the whole layer (mhc_mlx/metal.py:2787-2857 through
reference.py:148-184), and a second run must be bitwise identical.  n = 1 is not among the shapes:
the RMS norm is scale-invariant, so its one H_pre gradient is zero up to the eps term and a relative
bound would measure only the rounding of a cancelling sum.
"""

import pytest
import torch

from oracle import mhc_oracle as O
from tests._helpers import GRAD_TOL, TOL, dev_tensor, np_of, params, rel_err, rng, to_dtype_np

from mhc_mlx_amd import ops

pytestmark = pytest.mark.gpu

# (B, n, C, x dtype, dout dtype); comments name the tile layout each shape takes
SHAPES = [
    (3, 2, 77, "f32", "f32"),        # NMAX 4, one tile, partial chunk
    (4, 3, 202, "bf16", "bf16"),     # NMAX 4, one tile, rows not 16-byte aligned
    (2, 4, 1020, "bf16", "bf16"),    # NMAX 4, one tile (C % 8 != 0 keeps it off the layer-wide kernel)
    (2, 2, 1030, "f32", "f32"),      # NMAX 4, two tiles, partial chunks
    (2, 4, 20000, "bf16", "f32"),    # NMAX 4, 20 tiles
    (3, 5, 100, "f16", "f16"),       # NMAX 8, one tile
    (2, 8, 96, "bf16", "bf16"),      # NMAX 8, one tile
    (2, 7, 2500, "bf16", "f32"),     # NMAX 8, three tiles, partial last tile
    (2, 8, 4096, "f32", "f32"),      # NMAX 8, four tiles
    (3, 9, 33, "f16", "f32"),        # NMAX 16, one tile, partial chunk
    (2, 16, 64, "f32", "f32"),       # NMAX 16, one tile
    (2, 12, 2048, "bf16", "bf16"),   # NMAX 16, four tiles
    (2, 16, 1000, "f32", "f32"),     # NMAX 16, two tiles
    (2, 16, 4096, "bf16", "bf16"),   # NMAX 16, eight tiles (beyond the MFMA kernel's C <= 2048)
]


def _grad_tol(dt):
    return 1e-5 if dt == "f32" else TOL[dt]


def _run(x, dout, hpre, hpost, hres, w, xdt, gdt, per_token):
    ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
    xt = dev_tensor(x, xdt).requires_grad_(True)
    f = ops.mhc_layer_forward_dynamic if per_token else ops.mhc_layer_forward
    out = f(xt, *ps, sinkhorn_iters=20, eps=1e-5, output_dtype=xt.dtype if gdt == xdt and xdt != "f32" else None)
    out.backward(dev_tensor(dout, gdt))
    return [xt.grad.clone()] + [t.grad.clone() for t in ps]


@pytest.mark.parametrize("B,n,C,xdt,gdt", SHAPES)
@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("grid", [0, 2])
def test_tile_backward_matches_oracle(B, n, C, xdt, gdt, per_token, grid, knobs):
    if grid:
        knobs("MHC_BWD_GRID", grid)
    g = rng(2100 + B * 7 + n * 31 + C)
    x = to_dtype_np(g.standard_normal((B, n, C)), xdt)
    dout = to_dtype_np(g.standard_normal((B, n, C)), gdt)
    hpre, hpost, hres, w = params(g, n, C, per_token_B=B if per_token else None)
    print(f"case B={B} n={n} C={C} {xdt}/{gdt} per_token={per_token} grid={grid}", flush=True)
    first = _run(x, dout, hpre, hpost, hres, w, xdt, gdt, per_token)
    again = _run(x, dout, hpre, hpost, hres, w, xdt, gdt, per_token)
    for a, b in zip(first, again):
        assert torch.equal(a, b)
    ref = O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, sinkhorn_iters=20, eps=1e-5)
    for name, got, r in zip(["dx", "dH_pre_raw", "dH_post_raw", "dH_res_raw", "d_w"], first, ref):
        tol = _grad_tol(xdt) if name == "dx" else GRAD_TOL
        assert rel_err(np_of(got), r) < tol, (name, rel_err(np_of(got), r))

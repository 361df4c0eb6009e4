"""Run-to-run determinism of every kernel family on its main shapes.

Each path (the n = 4 and n = 8 layer-wide full tiles, n = 4 per-token, the n = 16 MFMA kernels per-token and
layer-wide, the n = 32 MFMA kernels at one, two and four slabs per wave and the runtime-loop forward above C = 2048
(C = 4096, 8192, and per-token n = 24 at C = 3072), n = 24, the 32 < n <= 64 MFMA kernels at n = 48 and 64,
and MHCRewire's post-combine at n = 4, 32 and 64) runs forward and backward five times on the same inputs; every output and gradient must
be bitwise equal to the first run's.  The kernels use fixed-order reductions, so any difference is a defect:
a race, or a register or memory hazard that depends on timing.  Parity with the oracle is covered by the
other test files; this file checks that the values do not move between runs.
"""

import pytest
import torch

from tests._helpers import dev_tensor, params, rng, to_dtype_np

from mhc_mlx_amd import MHCRewire, ops

pytestmark = pytest.mark.gpu

REPS = 5


def _assert_reruns_equal(run):
    first = run()
    for rep in range(1, REPS):
        cur = run()
        diff = [i for i, (a, b) in enumerate(zip(first, cur)) if not torch.equal(a, b)]
        assert not diff, f"run {rep}: outputs {diff} differ from run 0"  # stops at the first mismatching run


@pytest.mark.parametrize("T,n,C,per_token", [(4096, 4, 4096, False), (4096, 4, 4096, True), (2048, 8, 2048, False),
                                             (2048, 16, 1024, True), (2048, 16, 2048, False),
                                             (2048, 32, 512, False), (512, 32, 2048, False),
                                             (512, 32, 4096, False), (256, 32, 8192, False), (512, 24, 1024, False),
                                             (300, 24, 3072, True),
                                             # 32 < n <= 64 on MFMA (mf64_fwd_loop_kernel, mf64_bwd_kernel)
                                             (4096, 64, 512, False), (1024, 64, 2048, False),
                                             (2048, 48, 1024, False)])
def test_layer_reruns_are_bitwise_equal(T, n, C, per_token):
    g = rng(7100 + T + n + C)
    x = to_dtype_np(g.standard_normal((T, n, C)), "bf16")
    dout = dev_tensor(to_dtype_np(g.standard_normal((T, n, C)), "bf16"), "bf16")
    hpre, hpost, hres, w = params(g, n, C, per_token_B=T if per_token else None)
    fn = ops.mhc_layer_forward_dynamic if per_token else ops.mhc_layer_forward

    def run():
        ps = [dev_tensor(v).requires_grad_(True) for v in (hpre, hpost, hres, w)]
        xt = dev_tensor(x, "bf16").requires_grad_(True)
        out = fn(xt, *ps, sinkhorn_iters=20, eps=1e-5, output_dtype=xt.dtype)
        out.backward(dout)
        return [out.detach(), xt.grad] + [p.grad for p in ps]

    _assert_reruns_equal(run)


@pytest.mark.parametrize("n,T", [(4, 2048), (32, 2048), (64, 8192)])
def test_rewire_reruns_are_bitwise_equal(n, T):
    """MHCRewire(Linear(4096, 4096)): n = 64 runs the post-combine's generic MFMA sums at C = 64."""
    dims = 4096
    dev = torch.device("cuda")
    torch.manual_seed(7200 + n)
    inner = torch.nn.Linear(dims, dims, bias=False).to(dev).to(torch.bfloat16)
    m = MHCRewire(inner, dims=dims, n=n, eps=1e-5, identity_init=False).to(dev)
    x = torch.randn(T, dims, device=dev, dtype=torch.bfloat16)
    g = torch.randn(T, dims, device=dev, dtype=torch.float32)

    def run():
        xi = x.clone().requires_grad_(True)
        out = m(xi)
        grads = torch.autograd.grad(out, [xi, m.mhc.H_pre_raw, m.mhc.H_post_raw, m.mhc.H_res_raw], g)
        return [out.detach()] + list(grads)

    _assert_reruns_equal(run)

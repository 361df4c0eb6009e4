"""HIP-graph capture of the C ABI's layer forward and allocation-free backward.

A caller that captures (the case `mhc_layer_bwd_noalloc` exists for) keeps
every buffer outside the capture: inputs, outputs and gradients are
allocated first, the calls run once eagerly on the capturing stream (which
also performs the library's one-time per-device queries), and only the
kernel launches are recorded.  Each replay must reproduce the eager results
bitwise, with eager work on the default stream between replays.  No autograd
and no tensor allocation take part in the capture.
"""

import ctypes

import pytest
import torch

from tests._helpers import dev_tensor, params, rng, to_dtype_np

from mhc_mlx_amd import _lib

pytestmark = pytest.mark.gpu

EPS = 1e-6
ITERS = 20
P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731


@pytest.mark.parametrize("T,n,C,per_token", [(32, 4, 2048, False), (300, 4, 1024, False), (9, 16, 64, True),
                                             (64, 32, 512, False), (1, 4, 4096, False), (1, 32, 4096, False),
                                             (40, 64, 512, False)])
def test_graph_replays_of_the_c_abi_match_eager(T, n, C, per_token):
    print("graph case", T, n, C, per_token, flush=True)
    g = rng(9300 + T + n + C)
    x = dev_tensor(to_dtype_np(g.standard_normal((T, n, C)), "bf16"), "bf16")
    dout = dev_tensor(to_dtype_np(g.standard_normal((T, n, C)), "bf16"), "bf16")
    hp, hq, hr, w = (dev_tensor(v) for v in params(g, n, C, per_token_B=T if per_token else None))
    out, M, dx = torch.empty_like(x), torch.empty_like(hr), torch.empty_like(x)
    grads = [torch.empty_like(hp), torch.empty_like(hq), torch.empty_like(hr), torch.empty_like(w)]
    bf16 = _lib.DTYPE_BF16

    def launch():
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.call("mhc_layer_fwd", P(x), bf16, P(hp), P(hq), P(hr), P(w), P(out), bf16, P(M), T, n, C,
                  int(per_token), ITERS, ctypes.c_float(EPS), s)
        _lib.call("mhc_layer_bwd_noalloc", P(x), bf16, P(dout), bf16, P(hp), P(hq), P(hr), P(M), P(w), P(dx),
                  *(P(t) for t in grads), T, n, C, int(per_token), ITERS, ctypes.c_float(EPS), s)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = [t.clone() for t in [out, M, dx] + grads]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        launch()
    for rep in range(4):
        for t in [out, M, dx] + grads:
            t.fill_(float("nan"))  # replays must rewrite every output
        graph.replay()
        torch.cuda.synchronize()
        _ = (x.float().sum() + dout.float().sum()).item()  # eager work between replays
        for name, a, b in zip(["out", "M", "dx", "dH_pre", "dH_post", "dH_res", "d_w"], [out, M, dx] + grads,
                              eager):
            assert torch.equal(a, b), (rep, name)

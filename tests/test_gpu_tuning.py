"""The gfx950 tuner (python -m mhc_mlx_amd.tune) on the GPU: it writes a file that loads, picks
candidate values, and results do not depend on the launch shape chosen."""

import json

import pytest
import torch

from tests._helpers import np_of, rel_err

from mhc_mlx_amd import _lib, ops, tune, tuning

pytestmark = pytest.mark.gpu


def test_tuner_writes_a_loadable_file(tmp_path, monkeypatch, knobs):
    out = tmp_path / "mhc_tuning.json"
    assert tune.main(["--out", str(out), "--scale", "0.05", "--only", "residual_add_agg", "sinkhorn_16"]) == 0
    cfg = json.loads(out.read_text())
    for op in ("residual_add_agg", "sinkhorn_16"):
        env, cands = tuning.KNOBS[op]
        assert cfg[op][env] in cands
        assert set(cfg["_timings_us"][op]) == {str(c) for c in cands}
    for env, _ in tuning.KNOBS.values():
        monkeypatch.delenv(env, raising=False)
        knobs(env, None)
    tuning.load([str(out)])
    assert _lib.get_knob("MHC_RES_GRID") == cfg["residual_add_agg"]["MHC_RES_GRID"]


@pytest.mark.parametrize("op", ["residual_add_agg", "stream_mix_add", "mhc_fused_n16", "sinkhorn_16"])
def test_results_do_not_depend_on_the_knob(op, knobs):
    runs = {}
    env, cands = tuning.KNOBS[op]
    g = torch.Generator("cuda").manual_seed(1)
    if op == "residual_add_agg":
        x = torch.randn(300, 4, 512, device="cuda", dtype=torch.bfloat16, generator=g)
        h = torch.rand(4, device="cuda", generator=g)
        fn = lambda: ops.residual_add_agg_hip(x, x.flip(0), h)  # noqa: E731
    elif op == "stream_mix_add":
        x = torch.randn(300, 4, 256, device="cuda", dtype=torch.bfloat16, generator=g)
        p = [torch.randn(s, device="cuda", generator=g) for s in ((4,), (4,), (4, 4))]
        fn = lambda: (ops.post_combine(x, x.flip(0), *p),)  # noqa: E731
    else:
        x = torch.randn(200, 16, 1024, device="cuda", dtype=torch.bfloat16, generator=g)
        p = [torch.randn(200, 16, device="cuda", generator=g), torch.randn(200, 16, device="cuda", generator=g),
             torch.randn(200, 16, 16, device="cuda", generator=g), torch.ones(1024, device="cuda")]
        fn = lambda: (ops.mhc_layer_forward_dynamic(x, *p),)  # noqa: E731
    for v in cands:
        knobs(env, v)
        with torch.no_grad():
            runs[v] = [t.clone() for t in fn()]
    ref = runs[cands[0]]
    for v, got in runs.items():
        for a, b in zip(got, ref):
            if op in ("sinkhorn_16", "mhc_fused_n16"):
                # other lane layouts: the Sinkhorn sums associate differently, so M and the fp32
                # output agree to fp32 rounding
                assert a.dtype == torch.float32
                assert rel_err(np_of(a), np_of(b)) < 1e-6, v
            else:
                assert torch.equal(a, b), v

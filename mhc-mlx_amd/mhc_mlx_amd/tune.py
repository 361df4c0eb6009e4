"""Measure the library's launch-shape knobs on this GPU and write a tuning file.

    python -m mhc_mlx_amd.tune [--out mhc_tuning.json] [--scale 1.0]

The gfx950 counterpart of the reference's ``scripts/tune.py`` (tune.py:50-103):
for every op in ``tuning.KNOBS`` each candidate value of its knob is set in
the library's knob table (``mhc_set_knob``), the
op's representative workload is timed with HIP events on the current stream
(warm-up, then the mean of timed calls, as tune.py:12-24), and the fastest
value is kept.  The file is written in the format ``tuning.load`` reads;
timings and the device name go under ``_``-prefixed keys.
"""

from __future__ import annotations

import argparse
import json
import sys

import torch

from . import _lib, ops
from .tuning import KNOBS


def _time_us(fn, warmup: int = 3, iters: int = 10) -> float:
    for _ in range(warmup):
        fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters * 1e3


def workloads(scale: float = 1.0, dev="cuda"):
    """op name -> a callable running that op's representative workload once."""
    bf = torch.bfloat16
    g = torch.Generator(dev).manual_seed(0)
    T4 = max(64, int(8192 * scale))
    T16 = max(64, int(4096 * scale))
    x4 = torch.randn(T4, 4, 4096, device=dev, dtype=bf, generator=g)
    r4 = torch.randn(T4, 4, 4096, device=dev, dtype=bf, generator=g)
    h4 = torch.rand(4, device=dev, generator=g)
    xm = torch.randn(T4, 4, 1024, device=dev, dtype=bf, generator=g).requires_grad_(True)
    ym = torch.randn(T4, 4, 1024, device=dev, dtype=bf, generator=g).requires_grad_(True)
    pm = [torch.randn(s, device=dev, generator=g).requires_grad_(True) for s in ((4,), (4,), (4, 4))]
    gm = torch.randn(T4, 4, 1024, device=dev, generator=g)
    gs = torch.randn(T4, 4, 1024, device=dev, dtype=bf, generator=g)
    x16 = torch.randn(T16, 16, 1024, device=dev, dtype=bf, generator=g).requires_grad_(True)
    d16 = torch.randn(T16, 16, 1024, device=dev, dtype=bf, generator=g)
    p16 = [torch.randn(T16, 16, device=dev, generator=g).requires_grad_(True),
           torch.randn(T16, 16, device=dev, generator=g).requires_grad_(True),
           torch.randn(T16, 16, 16, device=dev, generator=g).requires_grad_(True)]
    w16 = torch.ones(1024, device=dev).requires_grad_(True)
    xl = torch.randn(T4, 4, 4096, device=dev, dtype=bf, generator=g).requires_grad_(True)
    pl = [torch.randn(s, device=dev, generator=g).requires_grad_(True) for s in ((4,), (4,), (4, 4), (4096,))]

    def mix_fwd():
        with torch.no_grad():
            ops.post_combine(xm, ym, *pm)

    def mix_bwd():
        torch.autograd.grad(ops.post_combine(xm, ym, *pm), [xm, ym] + pm, gm)

    def scale_fwd():
        with torch.no_grad():
            ops.stream_scale(xm, pm[0])

    def scale_bwd():
        torch.autograd.grad(ops.stream_scale(xm, pm[0]), [xm, pm[0]], gs)

    def n16_fwd():
        with torch.no_grad():
            ops.mhc_layer_forward_dynamic(x16, *p16, w16, output_dtype=bf)

    def n16_step():
        out = ops.mhc_layer_forward_dynamic(x16, *p16, w16, output_dtype=bf)
        torch.autograd.grad(out, [x16] + p16 + [w16], d16)

    def layer_fwd():
        with torch.no_grad():
            ops.mhc_layer_forward(xl, *pl, output_dtype=bf)

    def layer_step():
        out = ops.mhc_layer_forward(xl, *pl, output_dtype=bf)
        torch.autograd.grad(out, [xl] + pl, xl.detach())

    return {
        "residual_add_agg": lambda: ops.residual_add_agg_hip(x4, r4, h4, output_dtype=bf),
        "stream_mix_add": mix_fwd,
        "stream_mix_add_bwd": mix_bwd,
        "stream_scale": scale_fwd,
        "stream_scale_bwd": scale_bwd,
        "mhc_fused_n16": n16_fwd,
        "mhc_fused_bwd_n16": n16_step,
        "sinkhorn_16": n16_step,
        "mhc_fused": layer_fwd,
        "mhc_fused_bwd": layer_step,
    }


def tune(scale: float = 1.0, only: list[str] | None = None, log=print) -> dict:
    """Time every candidate of every knob; returns the tuning-file content."""
    if not torch.cuda.is_available():
        raise RuntimeError("mhc_mlx_amd.tune needs a GPU")
    runs = workloads(scale)
    result: dict = {"_device": torch.cuda.get_device_name(0), "_timings_us": {}}
    for op, (env, candidates) in KNOBS.items():
        if only and op not in only:
            continue
        prev = _lib.get_knob(env)
        times = {}
        try:
            for v in candidates:
                _lib.set_knob(env, v)
                times[v] = _time_us(runs[op])
                log(f"  {op:20s} {env}={v:<5d} {times[v]:10.1f} us")
        finally:
            _lib.set_knob(env, prev)
        best = min(times, key=times.get)
        log(f"  -> {op}: {env}={best}")
        result[op] = {env: best}
        result["_timings_us"][op] = {str(k): round(t, 2) for k, t in times.items()}
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", default="mhc_tuning.json")
    ap.add_argument("--scale", type=float, default=1.0, help="workload size relative to the defaults")
    ap.add_argument("--only", nargs="*", default=None, help="tune only these ops")
    args = ap.parse_args(argv)
    cfg = tune(args.scale, args.only)
    with open(args.out, "w") as f:
        json.dump(cfg, f, indent=2, sort_keys=True)
    print(f"wrote {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())

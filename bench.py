"""Benchmark: fused mHC forward + backward on one MI355X.

Workload: MHCLayer(n=4, C=4096) on 32768 tokens (B=8 x T=4096 flattened),
bf16 activations with bf16 output (return_dtype=bf16) and a bf16 upstream
gradient; one step = forward + backward with gradients for x, H_pre_raw,
H_post_raw, H_res_raw (through 20 Sinkhorn iterations) and rms_weight.
Synthetic seeded data; random parameters drawn as in the BASELINE recipe.

Prints one JSON line (rank 0): tokens/s over the timed steps, the HBM
roofline of the dominant kernel (fused backward) from HIP events recorded
around its launches during the timed steps, the forward latency at B=32 and
B=1, and the CPU baseline (the numpy oracle, fp32, one thread, on a bounded
token sample of the same workload).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "mhc-mlx_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
METRIC = "mHC fwd+bwd tokens/s & % HBM peak (n=4,C=4096,bf16); B=1 fwd latency µs"


def _params(g, n, C):
    import numpy as np

    return (g.standard_normal(n).astype(np.float32), g.standard_normal(n).astype(np.float32),
            g.standard_normal((n, n)).astype(np.float32), (1 + 0.02 * g.standard_normal(C)).astype(np.float32))


def _layer(n, C, dev, g, eps):
    import torch

    from mhc_mlx_amd import MHCLayer

    hpre, hpost, hres, w = _params(g, n, C)
    layer = MHCLayer(n=n, C=C, sinkhorn_iters=20, eps=eps).to(dev)
    with torch.no_grad():
        layer.H_pre_raw.copy_(torch.from_numpy(hpre))
        layer.H_post_raw.copy_(torch.from_numpy(hpost))
        layer.H_res_raw.copy_(torch.from_numpy(hres))
        layer.rms_weight.copy_(torch.from_numpy(w))
    return layer


def _fwd_latency_us(n, C, B, dev, reps=200):
    import numpy as np
    import torch

    g = np.random.default_rng(1)
    layer = _layer(n, C, dev, g, 1e-6)
    x = torch.randn(B, n, C, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        for _ in range(20):
            layer(x, return_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            layer(x, return_dtype=torch.bfloat16)
            e.record()
            e.synchronize()
            ts.append(s.elapsed_time(e) * 1e3)
    return statistics.median(ts)


def _cpu_baseline(n, C, budget_s=12.0, chunk=64):
    """Oracle (numpy fp32 restatement of reference.py + its VJP) on token chunks."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import mhc_oracle as O

    g = np.random.default_rng(0)
    hpre, hpost, hres, w = _params(g, n, C)
    x = O.bf16_round(g.standard_normal((chunk, n, C)).astype(np.float32))
    dout = O.bf16_round(g.standard_normal((chunk, n, C)).astype(np.float32))
    done = 0
    t0 = time.perf_counter()
    with threadpool_limits(limits=1):
        while time.perf_counter() - t0 < budget_s:
            O.mhc_forward_reference(x, hpre, hpost, hres, w, 20, 1e-6, dtype=np.float32)
            O.mhc_backward_reference(x, hpre, hpost, hres, w, dout, 20, 1e-6, dtype=np.float32)
            done += chunk
    dt = time.perf_counter() - t0
    return {"value": done / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{done} tokens of config 2 ({chunk}-token chunks, n={n}, C={C}, bf16-rounded "
                      f"inputs, fp32 numpy fwd+bwd incl. 20-iteration Sinkhorn VJP) in {dt:.1f}s"}


def _traffic():
    """HBM bytes per fused-backward launch from the committed rocprofv3 --pmc summary (None if absent)."""
    p = ROOT / "profiles" / "cfg2_fused_bwd_traffic.md"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def _copy_probe(mib: int, reps: int = 5) -> int:
    """Plain copy of a known size (read mib MiB, write mib MiB per launch).

    Run under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, its counters give the
    factor that turns those counters into bytes for this device.
    """
    import torch

    nbytes = mib << 20
    src = torch.ones(nbytes // 4, device="cuda:0", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": nbytes, "copy_probe_bytes_written": nbytes, "launches": reps,
                      "kernel": "torch.mul(src, 1.0, out=dst) fp32"}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=32768)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-latency", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain fp32 copy of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.copy_probe_mib > 0:
        return _copy_probe(args.copy_probe_mib)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU per box; the mHC path shards by token "
                                   "(see DESIGN.md) and has no multi-GPU benchmark", "n_gpus": args.gpus}))
        return 2

    import numpy as np
    import torch

    from mhc_mlx_amd import _lib, kernel_timer

    _lib.load()
    dev = torch.device("cuda:0")
    T, n, C = args.tokens, 4, 4096
    g = np.random.default_rng(0)
    layer = _layer(n, C, dev, g, 1e-6)
    x = torch.randn(T, n, C, device=dev, dtype=torch.bfloat16, generator=torch.Generator(dev).manual_seed(0))
    dout = torch.randn(T, n, C, device=dev, dtype=torch.bfloat16, generator=torch.Generator(dev).manual_seed(1))
    x.requires_grad_(True)
    params = [layer.H_pre_raw, layer.H_post_raw, layer.H_res_raw, layer.rms_weight]

    def step():
        out = layer(x, return_dtype=torch.bfloat16)
        return torch.autograd.grad(out, [x] + params, dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    with kernel_timer() as kt:
        t_start = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t_start.record()
        for _ in range(args.steps):
            step()
        t_end.record()
        torch.cuda.synchronize()
        stats = kt.stats()
    ms_total = t_start.elapsed_time(t_end)
    ms_step = ms_total / args.steps
    tokens_per_s = T * args.steps / (ms_total / 1e3)

    elems = T * n * C
    bytes_fwd = 2 * elems * 2          # read x, write out (bf16)
    bytes_bwd = 3 * elems * 2          # read x, read dout, write dx (bf16)
    bwd_ms = stats["fused_bwd"]["mean_ms"]
    achieved = bytes_bwd / (bwd_ms / 1e3) / 1e9
    fwd_ms = stats["fused_fwd"]["mean_ms"]

    result = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "mHC fwd+bwd, config 2", "tokens": T, "n": n, "C": C,
                   "io_dtype": "bf16", "sinkhorn_iters": 20, "eps": 1e-6, "parallelism": "none (1 GPU)"},
        "step_hbm_frac": (bytes_fwd + bytes_bwd) / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": _traffic(),
                     "kernel": "fused_bwd_kernel", "algorithmic_bytes_per_launch": bytes_bwd},
        "kernels_ms": {k: round(v["mean_ms"], 4) for k, v in stats.items()},
        "fused_fwd_hbm_frac": bytes_fwd / (fwd_ms / 1e3) / 1e9 / HBM_PEAK_GBS,
    }
    del x, dout
    torch.cuda.empty_cache()
    if not args.no_latency:
        result["fwd_latency_us_B32_C2048"] = _fwd_latency_us(4, 2048, 32, dev)
        result["fwd_latency_us_B1_C4096"] = _fwd_latency_us(4, 4096, 1, dev)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = _cpu_baseline(n, C)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Per-kernel HIP event timing for the ops in this package.

``with kernel_timer() as kt:`` makes every op record a start/end
``torch.cuda.Event`` pair around its library call, on the stream the call
enqueues on (torch's current stream).  ``kt.stats()`` synchronises and returns
per-name launch counts and durations.  With no active timer the ops pay one
global lookup.
"""

from __future__ import annotations

import contextlib
import statistics
from collections import defaultdict

_active = None


class KernelTimer:
    def __init__(self):
        self._pairs = defaultdict(list)
        self.enabled = True

    @contextlib.contextmanager
    def record(self, name: str):
        if not self.enabled:
            yield
            return
        import torch

        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        try:
            yield
        finally:
            end.record()
            self._pairs[name].append((start, end))

    def clear(self) -> None:
        self._pairs.clear()

    def stats(self) -> dict:
        import torch

        torch.cuda.synchronize()
        out = {}
        for name, pairs in self._pairs.items():
            ms = [s.elapsed_time(e) for s, e in pairs]
            out[name] = {
                "count": len(ms),
                "mean_ms": statistics.fmean(ms),
                "median_ms": statistics.median(ms),
                "min_ms": min(ms),
                "max_ms": max(ms),
            }
        return out


@contextlib.contextmanager
def kernel_timer():
    """Activate a KernelTimer for the ops of this package (not thread-safe)."""
    global _active
    prev = _active
    timer = KernelTimer()
    _active = timer
    try:
        yield timer
    finally:
        _active = prev


def timed(name: str):
    t = _active
    if t is None:
        return contextlib.nullcontext()
    return t.record(name)

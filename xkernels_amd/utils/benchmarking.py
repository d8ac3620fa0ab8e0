"""GPU timing with HIP events (the reference's utils/benchmarking.py:94-141
reports the floor over repeats plus p10 / p90; same statistics here)."""
from __future__ import annotations

import statistics
from collections.abc import Callable

import torch


def time_ms(fn: Callable[[], object], *, iters: int = 20, warmup: int = 3,
            stream: torch.cuda.Stream | None = None) -> list[float]:
    """Per-iteration milliseconds of ``fn`` measured with events on ``stream``."""
    s = stream or torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        starts[i].record(s)
        fn()
        ends[i].record(s)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in zip(starts, ends)]


def benchmark_repeat(fn: Callable[[], object], *, n_repeat: int = 5, iters: int = 20,
                     warmup: int = 3) -> dict[str, float]:
    """Median of per-repeat medians; ``ms`` is the floor (min over repeats)."""
    meds = []
    for _ in range(n_repeat):
        meds.append(statistics.median(time_ms(fn, iters=iters, warmup=warmup)))
    meds.sort()
    q = lambda f: meds[min(len(meds) - 1, int(round(f * (len(meds) - 1))))]  # noqa: E731
    return {"ms": meds[0], "median": statistics.median(meds), "p10": q(0.1), "p90": q(0.9),
            "spread_ratio": (q(0.9) / q(0.1)) if q(0.1) > 0 else float("nan"),
            "n_repeat": n_repeat}

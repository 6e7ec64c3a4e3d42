"""Latency statistics and timing harnesses.

`bench` and `summarize_latencies` keep the reference's signatures, return
keys and order statistics (exq/eval/bench.py:15-46 and :96-113), so scripts
written against the reference read the same numbers.  `bench` times with the
host clock around a device synchronisation, as the reference does; for
kernels of a few microseconds that clock mostly measures launch and sync
overhead, so `bench_events` times each call with HIP events recorded on the
current stream (optionally replaying a HIP graph of the call) and returns the
same keys.
"""
from __future__ import annotations

import math
import statistics
import time
from typing import Callable


def latency_stats(times_ms: list[float]) -> dict:
    """p50 / p75 / p95 / p99 / mean / std / ci95 / n of a list of latencies
    (ms), with the reference's indexing into the sorted list
    (exq/eval/bench.py:36-46): p50 = t[n // 2], p75 = t[int(0.75 (n - 1))],
    p95 = t[int(0.95 (n - 1))], p99 = t[min(int(0.99 (n - 1)), n - 1)], std the
    sample standard deviation, ci95 = 1.96 std / sqrt(n)."""
    t = sorted(float(v) for v in times_ms)
    n = len(t)
    if n == 0:
        raise ValueError("latency_stats needs at least one measurement")
    std = statistics.stdev(t) if n > 1 else 0.0
    return {
        "p50": t[n // 2],
        "p75": t[int(0.75 * (n - 1))],
        "p95": t[int(0.95 * (n - 1))],
        "p99": t[min(int(0.99 * (n - 1)), n - 1)],
        "mean": statistics.mean(t),
        "std": std,
        "ci95": 1.96 * std / math.sqrt(n) if n > 1 else 0.0,
        "n": n,
    }


def _sync():
    import torch
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def bench(fn: Callable, n_warmup: int = 20, n_runs: int = 100) -> dict:
    """Warm up, then time `n_runs` calls of `fn` with the host clock between
    device synchronisations (exq/eval/bench.py:15-46).  Returns latency_stats
    of the per-call times in ms."""
    if n_runs < 1:
        raise ValueError("n_runs must be >= 1")
    for _ in range(n_warmup):
        fn()
    _sync()
    times = []
    for _ in range(n_runs):
        _sync()
        t0 = time.perf_counter()
        fn()
        _sync()
        times.append((time.perf_counter() - t0) * 1000.0)
    return latency_stats(times)


def bench_events(fn: Callable, n_warmup: int = 20, n_runs: int = 100,
                 graph: bool = False) -> dict:
    """Time `n_runs` calls of `fn` on the GPU with a pair of HIP events per
    call on the current stream (no host clock, no synchronisation between
    calls).  With graph=True, `fn` is captured once into a HIP graph (after
    the warm-up, outside the capture) and each timed call is one replay.
    Returns latency_stats of the per-call times in ms."""
    import torch
    if n_runs < 1:
        raise ValueError("n_runs must be >= 1")
    if not torch.cuda.is_available():
        raise RuntimeError("bench_events times on a GPU; use bench() on the host")
    call = fn
    if graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(max(1, n_warmup)):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        call = g.replay
    for _ in range(n_warmup):
        call()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n_runs)]
    for a, b in ev:
        a.record()
        call()
        b.record()
    torch.cuda.synchronize()
    return latency_stats([a.elapsed_time(b) for a, b in ev])


def summarize_latencies(times: list[float]) -> dict:
    """tpot_p50 / p95 / p99 / mean / std / ci95, memory_gb and n_runs of a list
    of per-token latencies (ms), with the reference's indexing
    (exq/eval/bench.py:96-113): p95 = t[int(0.95 n)], p99 = t[min(int(0.99 n),
    n - 1)].  An empty list gives an empty dict."""
    if not times:
        return {}
    t = sorted(float(v) for v in times)
    n = len(t)
    mem_gb = 0.0
    try:
        import torch
        if torch.cuda.is_available():
            mem_gb = torch.cuda.max_memory_allocated() / 1e9
    except ImportError:  # pragma: no cover - torch is a dependency
        pass
    std = statistics.stdev(t) if n > 1 else 0.0
    return {
        "tpot_p50": t[n // 2],
        "tpot_p95": t[min(int(0.95 * n), n - 1)],
        "tpot_p99": t[min(int(0.99 * n), n - 1)],
        "tpot_mean": statistics.mean(t),
        "tpot_std": std,
        "tpot_ci95": 1.96 * std / math.sqrt(n) if n > 1 else 0.0,
        "memory_gb": mem_gb,
        "n_runs": n,
    }

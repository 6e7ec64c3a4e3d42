"""Benchmark helpers with the reference's interface (exq/eval/bench.py)."""
from exq_amd.eval.bench import bench, bench_events, latency_stats, summarize_latencies

__all__ = ["bench", "bench_events", "latency_stats", "summarize_latencies"]

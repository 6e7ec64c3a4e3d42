"""The reference's benchmark statistics (exq/eval/bench.py:15-46, 96-113):
known answers that pin its order-statistic indexing, invariances, the host
harness on the CPU."""
import math
import random
import statistics

import pytest

from exq_amd.eval import bench, latency_stats, summarize_latencies


def test_latency_stats_known_answers():
    # ten samples 0..9: p50 = t[5], p75 = t[int(6.75)] = t[6], p95 = t[int(8.55)] = t[8],
    # p99 = t[int(8.91)] = t[8]  (an index of int(q * n) would give 7 / 9 / 9)
    st = latency_stats([float(v) for v in range(10)])
    assert (st["p50"], st["p75"], st["p95"], st["p99"]) == (5.0, 6.0, 8.0, 8.0)
    assert st["mean"] == 4.5 and st["n"] == 10
    # sample standard deviation of 0..9: sqrt(82.5 / 9)
    assert st["std"] == pytest.approx(math.sqrt(82.5 / 9), rel=1e-12)
    assert st["ci95"] == pytest.approx(1.96 * math.sqrt(82.5 / 9) / math.sqrt(10), rel=1e-12)
    # 1..100: p50 = 51, p75 = t[74] = 75, p95 = t[94] = 95, p99 = t[98] = 99
    st = latency_stats([float(v) for v in range(1, 101)])
    assert (st["p50"], st["p75"], st["p95"], st["p99"]) == (51.0, 75.0, 95.0, 99.0)


def test_latency_stats_order_and_single_value():
    vals = [0.3, 7.5, 1.25, 9.0, 2.0, 2.0, 4.75]
    shuffled = vals[:]
    random.Random(3).shuffle(shuffled)
    assert latency_stats(vals) == latency_stats(shuffled)
    assert latency_stats(vals)["std"] == pytest.approx(statistics.stdev(vals))
    one = latency_stats([2.5])
    assert one == {"p50": 2.5, "p75": 2.5, "p95": 2.5, "p99": 2.5, "mean": 2.5, "std": 0.0,
                   "ci95": 0.0, "n": 1}
    with pytest.raises(ValueError):
        latency_stats([])


def test_summarize_latencies_known_answers():
    # twenty samples 0..19: tpot_p95 = t[int(19.0)] = 19, tpot_p99 = t[min(19, 19)] = 19
    st = summarize_latencies([float(v) for v in range(20)])
    assert st["tpot_p50"] == 10.0 and st["tpot_p95"] == 19.0 and st["tpot_p99"] == 19.0
    assert st["tpot_mean"] == 9.5 and st["n_runs"] == 20
    assert st["tpot_ci95"] == pytest.approx(1.96 * statistics.stdev(range(20)) / math.sqrt(20))
    assert summarize_latencies([]) == {}


def test_bench_host_harness_calls_and_keys():
    calls = []
    st = bench(lambda: calls.append(1), n_warmup=3, n_runs=7)
    assert len(calls) == 10
    assert set(st) == {"p50", "p75", "p95", "p99", "mean", "std", "ci95", "n"}
    assert st["n"] == 7 and 0.0 <= st["p50"] <= st["p95"] <= st["p99"]
    with pytest.raises(ValueError):
        bench(lambda: None, n_runs=0)

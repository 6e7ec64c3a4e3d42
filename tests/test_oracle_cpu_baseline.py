"""Pins of the timed CPU baseline (oracle/cpu_baseline.py): its torch dequant
equals the numpy oracle's bit for bit, and its per-(token, k) loop computes
the same layer as oracle.moe.moe_layer, so the timed CPU path is the layer."""
import numpy as np
import torch

from oracle import cpu_baseline, moe, quant


def _layer(E=6, H=256, I=128, T=5, k=2, seed=3):
    rng = np.random.default_rng(seed)
    w13 = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float16)
    w2 = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float16)
    p13, s13 = quant.pack_experts_int4(w13)
    p2, s2 = quant.pack_experts_int4(w2)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    wts = rng.random((T, k)).astype(np.float32)
    return x, p13, s13, p2, s2, ids, wts


def test_torch_dequant_equals_oracle_bitwise():
    _, p13, s13, p2, s2, _, _ = _layer()
    a = cpu_baseline.dequant_int4_torch(torch.from_numpy(p13), torch.from_numpy(s13)).numpy()
    assert np.array_equal(a, quant.dequant_int4(p13, s13))
    b = cpu_baseline.dequant_int4_torch(torch.from_numpy(p2), torch.from_numpy(s2)).numpy()
    assert np.array_equal(b, quant.dequant_int4(p2, s2))


def test_loop_equals_oracle_layer():
    x, p13, s13, p2, s2, ids, wts = _layer()
    d13, d2 = quant.dequant_int4(p13, s13), quant.dequant_int4(p2, s2)
    used = sorted(set(ids.reshape(-1).tolist()))
    w13 = {e: torch.from_numpy(d13[e]) for e in used}
    w2 = {e: torch.from_numpy(d2[e]) for e in used}
    got = cpu_baseline.moe_layer_loop(torch.from_numpy(x), w13, w2, torch.from_numpy(ids),
                                      torch.from_numpy(wts)).numpy()
    ref = moe.moe_layer(x, d13, d2, ids, wts, accum=np.float64)
    assert moe.rel_l2(got, ref) < 1e-5
    # a dropped k-term or a swapped gate/up would be far outside that bound
    bad = cpu_baseline.moe_layer_loop(torch.from_numpy(x), w13, w2,
                                      torch.from_numpy(ids[:, :1]),
                                      torch.from_numpy(wts[:, :1])).numpy()
    assert moe.rel_l2(bad, ref) > 1e-2


def test_time_cpu_layer_reports_percentiles():
    x, p13, s13, p2, s2, ids, wts = _layer(T=2)
    t = lambda a: torch.from_numpy(a)  # noqa: E731
    r = cpu_baseline.time_cpu_layer(t(x), t(p13), t(s13), t(p2), t(s2), t(ids), t(wts),
                                    "predequantized", reps=5, warmup=1, threads=1)
    assert r["reps"] == 5 and r["p5_us"] <= r["p50_us"] <= r["p95_us"]

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


def test_torch_int8_dequant_equals_oracle_bitwise():
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, size=(3, 40, 72), dtype=np.int8)
    sc = (rng.random((3, 40)) * 0.01 + 1e-4).astype(np.float16)
    a = cpu_baseline.dequant_int8_torch(torch.from_numpy(q), torch.from_numpy(sc)).numpy()
    assert np.array_equal(a, quant.dequant_int8(q, sc))


def test_loop_with_shared_experts_equals_oracle_layer():
    x, p13, s13, p2, s2, ids, wts = _layer(seed=7)
    rng = np.random.default_rng(8)
    sh13 = (rng.standard_normal((2, 2 * 128, 256)) * 0.02).astype(np.float32)
    sh2 = (rng.standard_normal((2, 256, 128)) * 0.02).astype(np.float32)
    d13, d2 = quant.dequant_int4(p13, s13), quant.dequant_int4(p2, s2)
    used = sorted(set(ids.reshape(-1).tolist()))
    w13 = {e: torch.from_numpy(d13[e]) for e in used}
    w2 = {e: torch.from_numpy(d2[e]) for e in used}
    shared = tuple((torch.from_numpy(sh13[s]), torch.from_numpy(sh2[s])) for s in range(2))
    t = lambda a: torch.from_numpy(a)  # noqa: E731
    got = cpu_baseline.moe_layer_loop(t(x), w13, w2, t(ids), t(wts), shared).numpy()
    ref = moe.moe_layer(x, d13, d2, ids, wts, shared_w13=sh13, shared_w2=sh2, accum=np.float64)
    assert moe.rel_l2(got, ref) < 1e-5
    # one shared expert left out is far outside that bound
    bad = cpu_baseline.moe_layer_loop(t(x), w13, w2, t(ids), t(wts), shared[:1]).numpy()
    assert moe.rel_l2(bad, ref) > 1e-2
    # a dropped slot (-1) contributes nothing, as in the oracle
    ids2 = ids.copy()
    ids2[0, 0] = -1
    got2 = cpu_baseline.moe_layer_loop(t(x), w13, w2, t(ids2), t(wts), shared).numpy()
    ref2 = moe.moe_layer(x, d13, d2, ids2, wts, shared_w13=sh13, shared_w2=sh2, accum=np.float64)
    assert moe.rel_l2(got2, ref2) < 1e-5


def test_bank_dequantisers_follow_tiers():
    rng = np.random.default_rng(11)
    E, S, H, I = 4, 1, 256, 128
    w13 = (rng.standard_normal((E + S, 2 * I, H)) * 0.02).astype(np.float16)
    w2 = (rng.standard_normal((E + S, H, I)) * 0.02).astype(np.float16)
    tier = [2, 1, 0, 2, 0]          # routed 0..3, shared 4
    index = [0, 0, 0, 1, 1]
    p13, s13 = quant.pack_experts_int4(w13[[0, 3]])
    p2, s2 = quant.pack_experts_int4(w2[[0, 3]])
    q13, qs13 = quant.quantize_int8(w13[[1]])
    q2, qs2 = quant.quantize_int8(w2[[1]])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    tensors = {"n_experts": E,
               "int4_w13": t(p13), "int4_w13_scales": t(s13),
               "int4_w2": t(p2), "int4_w2_scales": t(s2),
               "int8_w13": t(q13), "int8_w13_scales": t(qs13),
               "int8_w2": t(q2), "int8_w2_scales": t(qs2),
               "bf16_w13": t(w13[[2, 4]].astype(np.float32)).to(torch.bfloat16),
               "bf16_w2": t(w2[[2, 4]].astype(np.float32)).to(torch.bfloat16)}
    routed, shared = cpu_baseline.bank_deq(tier, index, tensors, used=[0, 1, 2, 3])
    assert sorted(routed) == [0, 1, 2, 3] and len(shared) == 1
    a, b = routed[3]()
    assert np.array_equal(a.numpy(), quant.dequant_int4(p13[1], s13[1]))
    assert np.array_equal(b.numpy(), quant.dequant_int4(p2[1], s2[1]))
    a, _ = routed[1]()
    assert np.array_equal(a.numpy(), quant.dequant_int8(q13[0], qs13[0]))
    a, _ = routed[2]()
    assert np.array_equal(a.numpy(), tensors["bf16_w13"][0].float().numpy())
    a, _ = shared[0]()
    assert np.array_equal(a.numpy(), tensors["bf16_w13"][1].float().numpy())


def test_budget_caps_reps_for_slow_calls(monkeypatch):
    x, p13, s13, p2, s2, ids, wts = _layer(T=2)
    t = lambda a: torch.from_numpy(a)  # noqa: E731
    clock = iter(range(0, 10 ** 6, 2))  # every call seems to take 2 s
    monkeypatch.setattr(cpu_baseline.time, "perf_counter", lambda: next(clock))
    r = cpu_baseline.time_cpu_experts(t(x), cpu_baseline.int4_deq(t(p13), t(s13), t(p2), t(s2)),
                                      t(ids), t(wts), reps=20, warmup=0, threads=1, budget_s=9)
    assert r["reps"] == 4


def test_grouped_variant_equals_loop():
    """The context-only grouped variant computes the same layer as the
    reference loop (dropped slots, shared experts and repeated experts too)."""
    x, p13, s13, p2, s2, ids, wts = _layer(E=5, T=9, k=3, seed=11)
    ids = ids.copy()
    ids[2, 1] = -1
    rng = np.random.default_rng(12)
    sh13 = torch.from_numpy((rng.standard_normal((1, 256, 256)) * 0.02).astype(np.float32))
    sh2 = torch.from_numpy((rng.standard_normal((1, 256, 128)) * 0.02).astype(np.float32))
    d13, d2 = quant.dequant_int4(p13, s13), quant.dequant_int4(p2, s2)
    w13 = {e: torch.from_numpy(d13[e]) for e in range(5)}
    w2 = {e: torch.from_numpy(d2[e]) for e in range(5)}
    t = lambda a: torch.from_numpy(a)  # noqa: E731
    shared = ((sh13[0], sh2[0]),)
    a = cpu_baseline.moe_layer_loop(t(x), w13, w2, t(ids), t(wts), shared).numpy()
    b = cpu_baseline.moe_layer_grouped(t(x), w13, w2, t(ids), t(wts), shared).numpy()
    assert moe.rel_l2(b, a) < 1e-5
    r = cpu_baseline.time_cpu_layer(t(x), t(p13), t(s13), t(p2), t(s2), t(ids), t(wts),
                                    "grouped", reps=3, warmup=1, threads=1)
    assert r["variant"] == "grouped" and r["reps"] == 3

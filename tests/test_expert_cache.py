"""Two-tier expert weight cache (exq_amd.runtime.ExpertWeightCache), the
counterpart of exq/runtime/__init__.py:35-106 and the prefetch loop at
146-166.  The CPU tests cover placement by plan, hit/miss counting, the
priority filter of the static schedule and the LRU bound; the GPU test
prefetches packed INT4 experts on a side stream and runs the fused layer on
them with no host synchronisation in between."""
import numpy as np
import pytest
import torch

from exq_amd.runtime import ExpertWeightCache


def _w(seed, shape=(4, 8)):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g)


def test_placement_by_plan():
    plan = {"0:0": "BF16", "0:1": "INT8", "0:2": "INT4"}
    c = ExpertWeightCache(plan, device="cpu")
    assert not c.has_offloaded_weights
    for e in range(4):  # expert 3 is not in the plan: INT4, the default
        c.register_expert(0, e, _w(e))
    assert c.is_gpu_resident(0, 0) and c.is_gpu_resident(0, 1)
    assert not c.is_gpu_resident(0, 2) and not c.is_gpu_resident(0, 3)
    assert c.has_offloaded_weights
    s = c.stats
    assert (s["gpu_resident"], s["cpu_stored"]) == (2, 2)
    assert torch.equal(c.get(0, 0), _w(0))
    assert c.get(0, 2) is None  # cold and not prefetched: a miss
    assert (c.hits, c.misses) == (1, 1) and c.stats["hit_rate"] == 0.5


def test_prefetch_then_get_tuple_weights():
    c = ExpertWeightCache({}, device="cpu")
    w = (_w(1), _w(2, (3,)).to(torch.float16), torch.arange(5, dtype=torch.uint8))
    c.register_expert(2, 7, w)
    assert c.get(2, 7) is None
    c.prefetch(2, 7, None)
    c.prefetch(2, 7, None)  # already resident: nothing more
    c.prefetch(5, 5, None)  # not registered: ignored
    c.sync_prefetches(None)
    got = c.get(2, 7)
    assert isinstance(got, tuple) and len(got) == 3
    for x, y in zip(got, w):
        assert x.dtype == y.dtype and torch.equal(x, y)
    assert c.stats["gpu_resident"] == 1 and c.stats["cpu_stored"] == 1


def test_issue_prefetches_priority_filter():
    c = ExpertWeightCache({"1:0": "BF16"}, device="cpu")
    assert c.issue_prefetches({0: [(1, 1, 0)]}, None) == 0  # nothing offloaded yet
    for e in range(4):
        c.register_expert(1, e, _w(10 + e))
    table = {0: [(1, 1, 0), (1, 2, 2)], 3: [(1, 3, 1), (1, 0, 0)]}
    # HIGH (0) and MEDIUM (1) targets are issued; LOW (2) is skipped
    assert c.issue_prefetches(table, None) == 3
    assert c.is_gpu_resident(1, 1) and c.is_gpu_resident(1, 3)
    assert not c.is_gpu_resident(1, 2)


def test_capacity_evicts_least_recently_used():
    one = 4 * 8 * 4
    c = ExpertWeightCache({"0:9": "BF16"}, device="cpu", capacity_bytes=2 * one)
    c.register_expert(0, 9, _w(9))  # hot: outside the bound, never dropped
    for e in range(3):
        c.register_expert(0, e, _w(e))
    c.prefetch(0, 0, None)
    c.prefetch(0, 1, None)
    assert c.get(0, 0) is not None  # expert 0 is now the most recently used
    c.prefetch(0, 2, None)          # drops expert 1
    assert c.evictions == 1
    assert c.is_gpu_resident(0, 0) and c.is_gpu_resident(0, 2) and c.is_gpu_resident(0, 9)
    assert c.get(0, 1) is None
    c.prefetch(0, 1, None)          # comes back from the host copy, drops expert 0
    assert torch.equal(c.get(0, 1), _w(1)) and not c.is_gpu_resident(0, 0)
    small = ExpertWeightCache({}, device="cpu", capacity_bytes=one - 1)
    small.register_expert(0, 0, _w(0))
    with pytest.raises(ValueError, match="capacity_bytes"):
        small.prefetch(0, 0, None)


def test_reregister_moves_between_tiers():
    plan = {"0:0": "INT4"}
    c = ExpertWeightCache(plan, device="cpu")
    c.register_expert(0, 0, _w(0))
    c.prefetch(0, 0, None)
    plan["0:0"] = "BF16"
    c.register_expert(0, 0, _w(1))
    assert torch.equal(c.get(0, 0), _w(1)) and not c.has_offloaded_weights


@pytest.mark.gpu
def test_prefetched_int4_experts_feed_fused_layer(device):
    """Cold packed experts prefetched on a side stream; the current stream
    assembles the bank from get() and runs the layer: bitwise equal to the
    layer on the original bank."""
    from exq_amd import synth
    from exq_amd.kernels import fused_experts, pack_experts_int4
    E, H, I, T, k = 8, 256, 128, 5, 2
    w13, w2 = synth.expert_weights_gpu(E, I, H, 41, device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).to(device)
    ids = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)).to(device)
    wts = torch.softmax(torch.randn(T, k, device=device), dim=-1)
    ref = fused_experts(x, p13, s13, p2, s2, wts, ids)

    plan = {"3:0": "BF16", "3:1": "INT8"}  # experts 0 and 1 hot, the rest cold
    cache = ExpertWeightCache(plan, device=device)
    for e in range(E):
        cache.register_expert(3, e, (p13[e], s13[e], p2[e], s2[e]))
    assert cache.stats["gpu_resident"] == 2 and cache.stats["cpu_stored"] == E - 2
    assert all(t.is_pinned() for t in cache._host[(3, 5)])
    side = torch.cuda.Stream(device)
    for e in range(E):
        cache.prefetch(3, e, side)
    parts = [cache.get(3, e) for e in range(E)]  # the current stream waits per copy
    bank = [torch.stack([p[j] for p in parts]) for j in range(4)]
    out = fused_experts(x, *bank, wts, ids)
    torch.cuda.synchronize(device)
    assert torch.equal(out, ref)
    cache.sync_prefetches(side)
    assert cache.stats["hits"] == E and cache.stats["misses"] == 0


@pytest.mark.gpu
def test_bounded_cache_evicts_and_refetches_on_gpu(device):
    """LRU bound on the device: a dropped expert comes back from its pinned
    host copy bit-identical, and the device bytes never exceed the bound."""
    E, shape = 6, (64, 256)
    ws = [torch.randn(shape, generator=torch.Generator().manual_seed(e)).to(torch.bfloat16)
          for e in range(E)]
    one = ws[0].numel() * ws[0].element_size()
    cache = ExpertWeightCache({}, device=device, capacity_bytes=3 * one)
    for e in range(E):
        cache.register_expert(0, e, ws[e])
    side = torch.cuda.Stream(device)
    for rnd in range(2):
        for e in range(E):
            cache.prefetch(0, e, side)
            assert cache.device_bytes <= 3 * one
            got = cache.get(0, e)
            assert torch.equal(got.cpu(), ws[e])
    cache.sync_prefetches(side)
    assert cache.evictions == 2 * E - 3
    assert cache.stats["gpu_resident"] == 3 and cache.stats["hits"] == 2 * E

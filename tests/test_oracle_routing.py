"""Pins of the routing oracle: brute force on tiny inputs, a hand-derived
padded layout and the structural invariants."""
import numpy as np
import pytest

from oracle import routing


def _brute_sort(ids):
    flat = [int(v) for v in np.asarray(ids).reshape(-1)]
    return sorted(range(len(flat)), key=lambda s: (flat[s], s))


@pytest.mark.parametrize("T,k,E,seed", [(1, 1, 4, 0), (3, 2, 4, 1), (7, 3, 5, 2), (16, 8, 64, 3)])
def test_sort_matches_brute_force(T, k, E, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    order, ends, max_tok = routing.sort_tokens_by_expert(ids, E)
    assert order.tolist() == _brute_sort(ids)
    flat = ids.reshape(-1).tolist()
    counts = [flat.count(e) for e in range(E)]
    assert ends.tolist() == [0] + list(np.cumsum(counts))
    assert max_tok == max(counts)
    # invariants: monotone ends, segment e holds only expert e, ascending slots
    assert np.all(np.diff(ends) >= 0) and ends[-1] == T * k
    for e in range(E):
        seg = order[ends[e]:ends[e + 1]]
        assert all(flat[s] == e for s in seg) and list(seg) == sorted(seg)


def test_dispatch_sorted_ids():
    ids = np.array([[3, 1], [1, 0], [3, 2]])
    order, sids, ends = routing.dispatch(ids, 4)
    assert order.tolist() == [3, 1, 2, 5, 0, 4]
    assert sids.tolist() == [0, 1, 1, 2, 3, 3]
    assert ends.tolist() == [0, 1, 3, 4, 6]


def test_align_hand_derived_layout():
    # ids = [[2,0],[2,1]], E = 3 passed as num_experts = E + 1 = 4, B = 4.
    # buckets (id+1): b1 = {slot1}, b2 = {slot3}, b3 = {slot0, slot2}
    sorted_ids, expert_ids, ntpp, cumsum = routing.moe_align_block_size(
        np.array([[2, 0], [2, 1]]), 4, 4)
    assert cumsum.tolist() == [0, 0, 4, 8, 12]
    assert ntpp.tolist() == [12]
    assert sorted_ids.tolist() == [1, 4, 4, 4, 3, 4, 4, 4, 0, 2, 4, 4, 4, 4, 4, 4]
    assert expert_ids.tolist() == [0, 1, 2, -1]


def test_align_filtered_ids_go_to_bucket_zero():
    sorted_ids, expert_ids, ntpp, cumsum = routing.moe_align_block_size(
        np.array([[-1, 1], [0, -1]]), 3, 2)
    assert cumsum.tolist() == [0, 2, 4, 6]
    assert sorted_ids[:6].tolist() == [0, 3, 2, 4, 1, 4]
    assert expert_ids[:3].tolist() == [-1, 0, 1]


@pytest.mark.parametrize("T,k,E,B,seed", [(1, 8, 64, 16, 0), (16, 8, 64, 16, 1),
                                          (5, 2, 8, 4, 2), (64, 8, 128, 16, 3)])
def test_align_then_build_ends_equals_canonical_sort(T, k, E, B, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    sorted_ids, expert_ids, ntpp, cumsum = routing.moe_align_block_size(ids, E + 1, B)
    n = T * k
    assert len(sorted_ids) == n + (E + 1) * (B - 1)
    # closed form: padded bucket sizes are multiples of B covering each count
    counts = np.bincount(ids.reshape(-1) + 1, minlength=E + 1)
    assert np.all(np.diff(cumsum) % B == 0)
    assert np.all(np.diff(cumsum) >= counts) and np.all(np.diff(cumsum) < counts + B)
    ends, order = routing.build_ends_from_slots(sorted_ids, ids.reshape(-1), n, E)
    ref_order, ref_ends, _ = routing.sort_tokens_by_expert(ids, E)
    assert ends.tolist() == ref_ends.tolist()
    assert order.tolist() == ref_order.tolist()


def test_build_ends_keeps_order_of_appearance():
    # slots listed out of ascending order inside an expert keep that order
    sorted_ids = np.array([2, 0, 9, 1, 9], dtype=np.int32)
    flat = np.array([1, 0, 1], dtype=np.int32)
    ends, order = routing.build_ends_from_slots(sorted_ids, flat, 3, 2)
    assert ends.tolist() == [0, 1, 3]
    assert order.tolist() == [1, 2, 0]


def test_softmax_topk_brute_force():
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((6, 10)).astype(np.float32)
    lg[0, 3] = lg[0, 7] = 5.0  # tie -> lower id first
    ids, w = routing.route_softmax_topk(lg, 3, renormalize=True)
    for t in range(6):
        p = np.exp(lg[t] - lg[t].max())
        p /= p.sum()
        ref = sorted(range(10), key=lambda e: (-p[e], e))[:3]
        assert ids[t].tolist() == ref
        assert abs(w[t].sum() - 1.0) < 1e-6
    assert ids[0, 0] == 3 and ids[0, 1] == 7


@pytest.mark.parametrize("T,k,E,B,seed", [(16, 8, 64, 16, 7), (3, 2, 5, 4, 8)])
def test_align_contract_the_reference_consumer_relies_on(T, k, E, B, seed):
    """What the reference's call site and consumer fix about the padded layout
    (sglang_backend.py:102-109 sizes the buffers n + (E+1)(B-1) and
    ceil(./B); exq_dispatch.cu:83-96 counts an entry only when slot < n_active):
    every padding entry is >= n_active, every real slot appears exactly once,
    and the block count covers num_tokens_post_pad.  The +1 bucket shift and
    the expert_ids fill past the end are sgl_kernel conventions outside this
    contract."""
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    n = T * k
    sorted_ids, expert_ids, ntpp, cumsum = routing.moe_align_block_size(ids, E + 1, B)
    assert len(sorted_ids) == n + (E + 1) * (B - 1)
    assert len(expert_ids) == -(-len(sorted_ids) // B)
    real = sorted_ids[sorted_ids < n]
    assert sorted(real.tolist()) == list(range(n))
    pad_mask = np.ones(len(sorted_ids), bool)
    pad_mask[np.isin(sorted_ids, real)] = False
    assert np.all(sorted_ids[pad_mask] >= n)
    assert int(ntpp[0]) <= len(sorted_ids) and int(ntpp[0]) % B == 0
    # every block before num_tokens_post_pad names the expert of its real slots
    flat = ids.reshape(-1)
    for blk in range(int(ntpp[0]) // B):
        ent = sorted_ids[blk * B:(blk + 1) * B]
        ent = ent[ent < n]
        assert all(flat[s] == expert_ids[blk] for s in ent)

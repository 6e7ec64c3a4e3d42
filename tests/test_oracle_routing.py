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


def _rounded_softmax_tie_rows():
    """Rows whose distinct logits give bit-equal fp32 softmax values.

    0.001 and the next float32 after it differ by 1.2e-10, far below the
    spacing of float32 near 3.0 (2.4e-7), so l - max rounds to one value for
    both and their probabilities are equal: a tie that ranking on the logits
    would split."""
    a = np.float32(0.001)
    b = np.nextafter(a, np.float32(1.0))
    assert a != b
    rows = [np.array([3.0, a, b, -1.0], np.float32),     # tie inside the top 3
            np.array([3.0, b, a, -1.0], np.float32)]     # larger logit holds the lower id
    wide = np.full(64, -5.0, np.float32)                 # tie at the 8th (last) place:
    wide[50:56] = 2.0                                    # seven clear winners (with 63),
    wide[9], wide[20] = a, b                             # then 9 and 20 tie
    wide[63] = 3.0
    rows.append(wide)
    return rows


@pytest.mark.parametrize("k", [1, 2, 3, 8])
def test_softmax_topk_matches_torch_on_rounded_ties(k):
    """The reference routes with torch.topk(F.softmax(logits)) (triton_emitter.py:273-277):
    the ranking is on the rounded fp32 probabilities, so distinct logits with equal
    probabilities are a tie.  torch.topk does not fix the order of equal values (on
    this CPU build, six equal values at ids 50..55 come back as 53 first); the oracle
    orders a tie by the lower id, a deterministic refinement of torch's result.  So:
    the chosen probabilities equal torch's bit for bit, a tie is listed in ascending
    id order, and where torch's ids are unambiguous they are equal."""
    import torch
    for row in _rounded_softmax_tie_rows():
        if k > row.size:
            continue
        lg = row[None, :]
        p = torch.softmax(torch.from_numpy(lg), dim=-1)
        t_w, t_ids = torch.topk(p, k, dim=-1)
        ids, w = routing.route_softmax_topk(lg, k, renormalize=False)
        # torch's exp and its multiply by 1/sum differ from numpy's exp and divide
        # by a few ulp; the ranking of the rounded values is what must agree
        np.testing.assert_allclose(w, t_w.numpy(), rtol=1e-6, atol=0)
        pr = p.numpy()[0]
        assert ids[0].tolist() == sorted(range(row.size), key=lambda e: (-pr[e], e))[:k]
        if len(set(pr[ids[0]].tolist())) == k and pr[ids[0][-1]] not in np.delete(pr, ids[0]):
            assert ids.tolist() == t_ids.numpy().astype(np.int64).tolist()
    a_row, _, wide = _rounded_softmax_tie_rows()
    # the 4-expert row: torch's own answer, and the lower id at the k-th place
    assert routing.route_softmax_topk(a_row[None], 3, False)[0].tolist() == [[0, 1, 2]]
    assert torch.topk(torch.softmax(torch.from_numpy(a_row[None]), -1), 3)[1].tolist() == [[0, 1, 2]]
    assert routing.route_softmax_topk(a_row[None], 2, False)[0].tolist() == [[0, 1]]
    assert routing.route_softmax_topk(wide[None], 8, False)[0].tolist() == [
        [63, 50, 51, 52, 53, 54, 55, 9]]


def test_softmax_topk_matches_torch_on_random_rows():
    """Ids equal torch.topk over torch's fp32 softmax on seeded rows of every
    config's width, Zipf-biased and plain."""
    import torch
    from exq_amd import synth
    for name in ("olmoe", "qwen3", "deepseek_v2_lite", "mixtral"):
        cfg = synth.CONFIGS[name]
        lg = synth.router_logits(cfg, 256, synth.seed_for(cfg) + 3)
        p = torch.softmax(torch.from_numpy(lg), dim=-1)
        tw, t_ids = torch.topk(p, cfg.top_k, dim=-1)
        ids, w = routing.route_softmax_topk(lg, cfg.top_k, renormalize=False)
        assert np.array_equal(ids, t_ids.numpy().astype(np.int64))
        np.testing.assert_allclose(w, tw.numpy(), rtol=2e-6, atol=0)

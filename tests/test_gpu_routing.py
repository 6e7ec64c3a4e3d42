"""Routing preparation on the GPU vs the oracle: bit-exact."""
import numpy as np
import pytest
import torch

from oracle import routing
from tests._helpers import banner

pytestmark = pytest.mark.gpu


def _ids(T, k, E, seed, dtype=torch.int64, invalid=0):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]) if T else \
        np.zeros((0, k), np.int64)
    if invalid:
        flat = ids.reshape(-1)
        flat[rng.choice(flat.size, size=min(invalid, flat.size), replace=False)] = -1
    return ids, torch.from_numpy(ids).to(dtype)


CASES = [(1, 8, 64), (16, 8, 64), (64, 8, 128), (5, 2, 8), (1, 1, 1), (4096, 2, 8),
         (2048, 6, 64), (300, 8, 1000)]
# above 2048 items or 1023 experts: the multi-block sort (several work-groups,
# each recounting every item); up to 4095 experts
WIDE = [(2048, 8, 64), (4096, 8, 128), (64, 8, 3000), (333, 8, 4095), (9000, 2, 1500),
        (257, 8, 8)]


@pytest.mark.parametrize("T,k,E", CASES + WIDE)
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_dispatch_bit_exact(T, k, E, dtype, device):
    from exq_amd.kernels.exq_dispatch import dispatch
    banner(f"dispatch T={T} k={k} E={E} {dtype}")
    ids, t = _ids(T, k, E, T * 31 + E)
    n = T * k
    so = torch.empty(n, dtype=torch.int64, device=device)
    si = torch.empty(n, dtype=torch.int64, device=device)
    ends = torch.empty(E + 1, dtype=torch.int32, device=device)
    dispatch(t.to(device), so, si, ends, E)
    r_so, r_si, r_ends = routing.dispatch(ids, E)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(si.cpu().numpy(), r_si)
    assert np.array_equal(ends.cpu().numpy(), r_ends)


@pytest.mark.parametrize("T,k,E", CASES[:6] + [(2048, 8, 64), (64, 8, 2000), (600, 4, 1100)])
@pytest.mark.parametrize("B", [16, 4])
def test_align_then_build_ends_bit_exact(T, k, E, B, device):
    from exq_amd.kernels.exq_dispatch import build_ends_from_slots, moe_align_block_size
    banner(f"align+build_ends T={T} k={k} E={E} B={B}")
    ids, t = _ids(T, k, E, 7 + T + E)
    n = T * k
    nb = E + 1
    cap = n + nb * (B - 1)
    sorted_ids = torch.full((cap,), -7, dtype=torch.int32, device=device)
    blk = torch.empty((cap + B - 1) // B, dtype=torch.int32, device=device)
    ntpp = torch.empty(1, dtype=torch.int32, device=device)
    cs = torch.empty(nb + 1, dtype=torch.int32, device=device)
    moe_align_block_size(t.to(device), nb, B, sorted_ids, blk, ntpp, cs, True)
    r = routing.moe_align_block_size(ids, nb, B)
    assert np.array_equal(sorted_ids.cpu().numpy(), r[0])
    assert np.array_equal(blk.cpu().numpy(), r[1])
    assert np.array_equal(ntpp.cpu().numpy(), r[2])
    assert np.array_equal(cs.cpu().numpy(), r[3])
    flat = t.reshape(-1).to(torch.int32).to(device)
    ends = torch.full((E + 1,), 99, dtype=torch.int32, device=device)  # not pre-zeroed
    so = torch.empty(n, dtype=torch.int64, device=device)
    build_ends_from_slots(sorted_ids, flat, ends, so, n, E)
    r_ends, r_so = routing.build_ends_from_slots(r[0], ids.reshape(-1), n, E)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    assert np.array_equal(so.cpu().numpy(), r_so)
    c_so, c_ends, _ = routing.sort_tokens_by_expert(ids, E)  # the canonical stable order
    assert np.array_equal(so.cpu().numpy(), c_so) and np.array_equal(ends.cpu().numpy(), c_ends)


def test_align_filtered_ids(device):
    from exq_amd.kernels.exq_dispatch import moe_align_block_size
    banner("align filtered ids")
    ids, t = _ids(33, 4, 16, 5, invalid=20)
    nb, B = 17, 8
    cap = ids.size + nb * (B - 1)
    out = [torch.empty(cap, dtype=torch.int32, device=device),
           torch.empty((cap + B - 1) // B, dtype=torch.int32, device=device),
           torch.empty(1, dtype=torch.int32, device=device),
           torch.empty(nb + 1, dtype=torch.int32, device=device)]
    moe_align_block_size(t.to(device), nb, B, *out, True)
    r = routing.moe_align_block_size(ids, nb, B)
    for a, b in zip(out, r):
        assert np.array_equal(a.cpu().numpy(), b)


def test_empty_and_repeatable(device):
    from exq_amd.kernels.exq_dispatch import dispatch
    banner("dispatch empty + repeat")
    so = torch.empty(0, dtype=torch.int64, device=device)
    ends = torch.full((9,), 5, dtype=torch.int32, device=device)
    dispatch(torch.empty(0, 8, dtype=torch.int64, device=device), so, so.clone(), ends, 8)
    assert ends.cpu().tolist() == [0] * 9
    ids, t = _ids(64, 8, 128, 3)
    outs = []
    for _ in range(3):
        so = torch.empty(512, dtype=torch.int64, device=device)
        si = torch.empty(512, dtype=torch.int64, device=device)
        e = torch.empty(129, dtype=torch.int32, device=device)
        dispatch(t.to(device), so, si, e, 128)
        outs.append(so.cpu())
    assert all(torch.equal(outs[0], o) for o in outs[1:])


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_wide_sort_skewed_prefill_batch(dtype, device):
    """A DeepSeek-V2-Lite prefill chunk (2048 tokens x top-6 = 12,288 slots, and
    the same with top-8 for 16,384) with Zipf-skewed ids: many slots per bucket
    in every block.  dispatch, sort_tokens_by_expert (with the row gather),
    align and build_ends are bit-exact with the oracle."""
    from exq_amd import synth
    from exq_amd.kernels import sort_tokens_by_expert
    from exq_amd.kernels.exq_dispatch import build_ends_from_slots, dispatch, moe_align_block_size
    cfg = synth.CONFIGS["deepseek_v2_lite"]
    for k in (6, 8):
        banner(f"wide sort skewed T=2048 k={k} {dtype}")
        c = synth.MoeConfig("wide", cfg.config_id, cfg.hidden, cfg.inter, cfg.n_experts, k,
                            False)
        ids, _ = synth.routing(c, 2048)
        E, n = cfg.n_experts, ids.size
        t = torch.from_numpy(ids).to(dtype).to(device)
        so = torch.empty(n, dtype=torch.int64, device=device)
        si = torch.empty(n, dtype=torch.int64, device=device)
        ends = torch.full((E + 1,), -3, dtype=torch.int32, device=device)
        dispatch(t.reshape(-1), so, si, ends, E)
        r_so, r_si, r_ends = routing.dispatch(ids, E)
        assert np.array_equal(so.cpu().numpy(), r_so)
        assert np.array_equal(si.cpu().numpy(), r_si)
        assert np.array_equal(ends.cpu().numpy(), r_ends)
        x = torch.randn(2048, 256, dtype=torch.bfloat16, device=device)
        o, sh, e2, mt = sort_tokens_by_expert(t, x, E)
        c_so, c_ends, c_mt = routing.sort_tokens_by_expert(ids, E)
        assert np.array_equal(o.cpu().numpy(), c_so) and np.array_equal(e2.cpu().numpy(), c_ends)
        assert mt == c_mt
        assert torch.equal(sh, x[o // k])
        nb, B = E + 1, 16
        cap = n + nb * (B - 1)
        sid = torch.full((cap,), -7, dtype=torch.int32, device=device)
        blk = torch.full(((cap + B - 1) // B,), -9, dtype=torch.int32, device=device)
        ntpp = torch.empty(1, dtype=torch.int32, device=device)
        cs = torch.empty(nb + 1, dtype=torch.int32, device=device)
        moe_align_block_size(t, nb, B, sid, blk, ntpp, cs, True)
        r = routing.moe_align_block_size(ids, nb, B)
        for got, want in zip((sid, blk, ntpp, cs), r):
            assert np.array_equal(got.cpu().numpy(), want)
        e3 = torch.full((E + 1,), 99, dtype=torch.int32, device=device)
        so3 = torch.empty(n, dtype=torch.int64, device=device)
        build_ends_from_slots(sid, t.reshape(-1).to(torch.int32), e3, so3, n, E)
        assert np.array_equal(so3.cpu().numpy(), c_so) and np.array_equal(e3.cpu().numpy(), c_ends)

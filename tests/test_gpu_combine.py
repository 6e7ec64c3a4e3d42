"""The decode layer's combine on the GPU vs the fp32 oracle.

The combine computes out[t] = the sum over token t's slots (ascending) of
weight x the slot's down-projection row, with each slot's k-splits summed
first.  It runs in two places:
- inside the down kernel, by the last work-group of each column block, with
  one, two or three k-splits;
- as a separate launch, with four or more splits or from 32 tokens on.

Each shape below takes one of these paths.  It runs with int32 / int64 ids,
fp32 / bf16 / fp16 router weights and dropped or out-of-range ids.
Tolerance: relative L2 error <= 0.5 %.  Every path repeats bitwise."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from tests._helpers import assert_close_rel, banner, oracle_int4_layer

pytestmark = pytest.mark.gpu
TOL = 5e-3
E, K_TOP, H = 4, 2, 512

# (intermediate size, tokens).  With 4 experts of hidden size 512, top-2 and a
# few tokens, the down kernel has far fewer units than resident work-groups.
# It then splits each contraction over I / 512 work-groups (at least four
# k-blocks each):
#   I = 512 / 1024 / 1536 give one / two / three splits, combined in-kernel;
#   I = 2048 gives four splits, combined by the separate launch;
#   40 tokens take the separate launch whatever the split count.
SHAPES = [(512, 3), (1024, 3), (1536, 3), (2048, 3), (1024, 40)]
W_DTYPES = [torch.float32, torch.bfloat16, torch.float16]
ID_DTYPES = [torch.int64, torch.int32]


@pytest.mark.parametrize("I,T", SHAPES)
def test_combine_paths_dtypes_and_dropped_ids(I, T, device):
    from exq_amd.kernels import fused_experts, pack_experts_int4
    cfg = synth.MoeConfig(f"combine_{I}", 35, H, I, E, K_TOP, True, zipf=False)
    banner(f"combine I={I} T={T}")
    w13, w2 = synth.expert_weights_gpu(E, I, H, 800 + I, device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    del w13, w2
    ids, w = synth.routing(cfg, T, 0)
    ids = ids.copy()
    ids[0, 1] = -1         # dropped
    ids[T - 1, 0] = E + 3  # out of range: dropped too
    x = torch.from_numpy(synth.hidden_np(T, H, 5 + T)).to(torch.bfloat16).to(device)
    for wd in W_DTYPES:
        tw = torch.from_numpy(w).to(wd).to(device)
        ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, tw.float().cpu().numpy())
        outs = []
        for idd in ID_DTYPES:
            tid = torch.from_numpy(ids).to(idd).to(device)
            out = fused_experts(x, p13, s13, p2, s2, tw, tid)
            assert_close_rel(out, ref, TOL, f"combine I={I} T={T} w={wd} ids={idd}")
            assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid), out)
            outs.append(out)
        # the ids' width changes nothing
        assert torch.equal(outs[0], outs[1])
    # a token with every slot dropped gets zeros
    allbad = np.full_like(ids, -1)
    allbad[1:] = ids[1:]
    tid = torch.from_numpy(allbad).to(device)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device), tid)
    assert torch.count_nonzero(out[0]) == 0
    ref = oracle_int4_layer(x, p13, s13, p2, s2, allbad, w)
    assert_close_rel(out, ref, TOL, f"combine I={I} T={T} token 0 dropped")


@pytest.mark.parametrize("I,T,E,k", [(512, 3, 16, 12), (512, 40, 32, 20)])
def test_combine_more_slots_than_one_batch(I, T, E, k, device):
    """More slots per token than one load batch holds.  The in-kernel combine
    takes eight slots per batch, so top-12 at three tokens takes two batches.
    The combine launch takes 16 (slot, split) items per batch, so top-20 at
    40 tokens takes two."""
    from exq_amd.kernels import fused_experts, pack_experts_int4
    cfg = synth.MoeConfig(f"combine_k{k}", 36, H, I, E, k, True, zipf=False)
    banner(f"combine top-{k} T={T}")
    w13, w2 = synth.expert_weights_gpu(E, I, H, 900 + k, device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    del w13, w2
    ids, w = synth.routing(cfg, T, 0)
    ids = ids.copy()
    ids[0, k - 1] = -1  # dropped, in the second batch
    ids[1, 3] = -1
    x = torch.from_numpy(synth.hidden_np(T, H, 6 + T)).to(torch.bfloat16).to(device)
    for wd in (torch.float32, torch.bfloat16):
        tw = torch.from_numpy(w).to(wd).to(device)
        tid = torch.from_numpy(ids).to(device)
        out = fused_experts(x, p13, s13, p2, s2, tw, tid)
        ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, tw.float().cpu().numpy())
        assert_close_rel(out, ref, TOL, f"combine top-{k} T={T} w={wd}")
        assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid), out)


@pytest.mark.parametrize("I,T", [(512, 3), (1536, 3), (1024, 40)])
def test_combine_shared_experts(I, T, device):
    """Shared experts (every token, weight 1, slots k .. k + S - 1) through
    both combines.  The bank has 8 INT4 routed experts, top-2 routing and two
    INT4 shared experts: one and three k-splits in-kernel at three tokens, and
    the combine launch at 40 tokens."""
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    from tests.test_gpu_mixed import _oracle
    E, S, k = 8, 2, 2
    cfg = synth.MoeConfig(f"combine_shared_{I}", 37, H, I, E, k, True, zipf=False)
    banner(f"combine shared I={I} T={T}")
    w13, w2 = synth.expert_weights_gpu(E, I, H, 950 + I, device)
    s13, s2 = synth.expert_weights_gpu(S, I, H, 960 + I, device)
    bank = MixedExpertBank.from_weights(w13, w2, [2] * E, shared_w13=s13, shared_w2=s2,
                                        shared_tier=2)
    del w13, w2, s13, s2
    ids, w = synth.routing(cfg, T, 0)
    ids = ids.copy()
    ids[0, 0] = -1  # a dropped routed slot: the shared slots still count
    x = torch.from_numpy(synth.hidden_np(T, H, 8 + T)).to(torch.bfloat16).to(device)
    tid = torch.from_numpy(ids).to(device)
    tw = torch.from_numpy(w).to(device)
    out = fused_experts_mixed(x, bank, tw, tid)
    assert_close_rel(out, _oracle(bank, x, ids, w), TOL, f"combine shared I={I} T={T}")
    assert torch.equal(fused_experts_mixed(x, bank, tw, tid), out)

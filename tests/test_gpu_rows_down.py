"""The decode layer's down projection by output rows (batches of one or two
tokens, k + shared >= 4, T * (k + shared) <= 64), against the oracle:
several top-k (up to the 64-slot limit), dropped ids, bf16 and f16
activations, int32 / int64 ids and f32 / bf16 / f16 router weights, group
sizes 128 and 256, an intermediate size whose 32-k chunks do not divide
evenly over 32 lanes (I = 1280: 40 chunks), mixed BF16 / INT8 / INT4 banks
with shared experts, and top-k below the kernel's minimum (which runs the
tiled down kernel).  Each layer is also
computed twice and compared bitwise.  Tolerance: relative L2 <= 0.5 %."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import moe, quant
from tests._helpers import assert_close_rel, banner

pytestmark = pytest.mark.gpu

TOL = 5e-3

# (E, H, I, group size, k, T, activation dtype, drop fraction)
CASES = [
    (128, 2048, 768, 128, 8, 1, torch.bfloat16, 0.0),    # Qwen3 layer shape
    (64, 2048, 1024, 128, 8, 2, torch.bfloat16, 0.0),    # OLMoE layer shape
    (16, 256, 256, 128, 4, 1, torch.float16, 0.0),       # the minimum top-k
    (16, 256, 256, 128, 3, 1, torch.bfloat16, 0.0),      # below it: tiled down kernel
    (40, 512, 1280, 128, 6, 2, torch.bfloat16, 0.2),     # 40 chunks, dropped ids
    (40, 512, 1280, 256, 6, 1, torch.float16, 0.0),      # group size 256
    (96, 256, 384, 128, 32, 2, torch.bfloat16, 0.1),     # 64 slots, the limit
    (128, 256, 512, 128, 32, 1, torch.float16, 0.5),     # half the slots dropped
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_rows_down(case, device):
    from exq_amd.kernels import fused_experts, pack_experts_int4
    E, H, I, g, k, T, act, drop = CASES[case]
    banner(f"rows down E={E} H={H} I={I} g={g} k={k} T={T} {act} drop={drop}")
    rng = np.random.default_rng(900 + case)
    w13, w2 = synth.expert_weights_gpu(E, I, H, 900 + case, device)
    p13, s13 = pack_experts_int4(w13, group_size=g)
    p2, s2 = pack_experts_int4(w2, group_size=g)
    del w13, w2
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    if drop:
        ids[rng.random(ids.shape) < drop] = -1
    w = rng.random((T, k)).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(act).to(device)
    # id and router-weight dtypes vary over the cases (the kernel reads either)
    ids_dt = (torch.int64, torch.int32)[case % 2]
    w_dt = (torch.float32, torch.bfloat16, torch.float16)[case % 3]
    tid = torch.from_numpy(ids).to(ids_dt).to(device)
    tw = torch.from_numpy(w).to(w_dt).to(device)
    w = tw.float().cpu().numpy()  # the weights as the kernel reads them
    out = fused_experts(x, p13, s13, p2, s2, tw, tid)
    again = fused_experts(x, p13, s13, p2, s2, tw, tid)
    assert torch.equal(out, again), "rows-down layer is not bitwise repeatable"
    used = np.unique(ids[ids >= 0])
    d13 = np.zeros((E, 2 * I, H), np.float32)
    d2 = np.zeros((E, H, I), np.float32)
    for e in used:
        d13[e] = quant.dequant_int4(p13[e].cpu().numpy(), s13[e].cpu().numpy())
        d2[e] = quant.dequant_int4(p2[e].cpu().numpy(), s2[e].cpu().numpy())
    ref = moe.moe_layer(x.float().cpu().numpy(), d13, d2, ids, w)
    if not used.size:
        assert torch.count_nonzero(out) == 0
        return
    assert_close_rel(out, ref, TOL, f"rows down case {case}")


# mixed banks: (E, H, I, k, T, n_shared, tiers (None = from synth.mixed_tiers), act)
MIXED = [
    (16, 512, 256, 4, 1, 0, [1] * 8 + [2] * 4 + [0] * 4, torch.bfloat16),   # mostly INT8
    (16, 512, 1280, 6, 2, 2, None, torch.bfloat16),                         # shared experts, 40 chunks
    (64, 2048, 1408, 6, 1, 2, [2] * 64, torch.bfloat16),                    # DeepSeek-V2-Lite shape
    (16, 512, 256, 5, 2, 1, [0] * 6 + [1] * 5 + [2] * 5, torch.float16),
]


@pytest.mark.parametrize("case", range(len(MIXED)))
def test_rows_down_mixed(case, device):
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    from tests.test_gpu_mixed import _oracle
    E, H, I, k, T, S, tiers, act = MIXED[case]
    banner(f"rows down mixed E={E} H={H} I={I} k={k} T={T} shared={S} {act}")
    rng = np.random.default_rng(950 + case)
    w13, w2 = synth.expert_weights_gpu(E, I, H, 950 + case, device)
    sh13 = sh2 = None
    if S:
        sh13, sh2 = synth.expert_weights_gpu(S, I, H, 960 + case, device)
    tiers = tiers if tiers is not None else synth.mixed_tiers(E, 950 + case)
    bank = MixedExpertBank.from_weights(w13, w2, tiers, act_dtype=act, shared_w13=sh13,
                                        shared_w2=sh2, shared_tier=0)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    w = rng.random((T, k)).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(act).to(device)
    tid, tw = torch.from_numpy(ids).to(device), torch.from_numpy(w).to(device)
    out = fused_experts_mixed(x, bank, tw, tid)
    assert torch.equal(out, fused_experts_mixed(x, bank, tw, tid))
    assert_close_rel(out, _oracle(bank, x, ids, w), TOL, f"rows down mixed case {case}")

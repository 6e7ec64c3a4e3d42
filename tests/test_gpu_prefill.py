"""The tiled INT4 prefill kernel (128-row token groups x 128 weight rows) on
the GPU vs the fp32 dequantise-then-matmul oracle.  Covers several token
groups per expert, ragged last groups, one expert taking every row, f16 and
bf16 activations, the sorted-row GEMM on both kernels (N % 128 == 0 tiles,
N = 96 does not), group size 256 (the untiled kernel), and mixed tiers where
BF16 / INT8 groups and INT4 groups run on different kernels in one layer.
Tolerance: relative L2 <= 0.5%."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import moe, quant, routing
from tests._helpers import assert_close_rel, banner, oracle_int4_layer

pytestmark = pytest.mark.gpu

TOL = 5e-3

WIDE = synth.MoeConfig("prefill_wide", 41, 1024, 512, 8, 2, True)
# two experts, both on every token: far more than 512 rows per expert, so the
# INT4 tiles are 128 rows x 128 weight rows (fewer rows per expert take the
# 64 x 256 tiles, as WIDE does)
FEW = synth.MoeConfig("prefill_few", 47, 1024, 512, 2, 2, True, zipf=False)
# More than 512 rows per expert with 256-row tiles available: the INT4 tiles
# are 128 rows x 256 weight rows with scaled weight operands.  ODD: three scale
# groups in the down projection (I = 384), an odd count for the kernel's
# two-groups-per-iteration loop; ONE: a single group (I = 128).
PS_ODD = synth.MoeConfig("prefill_ps_odd", 49, 512, 384, 2, 2, True, zipf=False)
PS_ONE = synth.MoeConfig("prefill_ps_one", 50, 256, 128, 2, 2, True, zipf=False)


def _pack(E, I, H, seed, device, group_size=128):
    from exq_amd.kernels import pack_experts_int4
    w13, w2 = synth.expert_weights_gpu(E, I, H, seed, device)
    p13, s13 = pack_experts_int4(w13, group_size=group_size)
    p2, s2 = pack_experts_int4(w2, group_size=group_size)
    return p13, s13, p2, s2


def _hidden(T, H, seed, device, dtype):
    return torch.from_numpy(synth.hidden_np(T, H, seed)).to(dtype).to(device)


@pytest.mark.parametrize("cfg,T,dtype", [(WIDE, 300, torch.bfloat16), (WIDE, 300, torch.float16),
                                         (WIDE, 1100, torch.bfloat16), (FEW, 1100, torch.bfloat16),
                                         (FEW, 1100, torch.float16),
                                         (PS_ODD, 700, torch.bfloat16), (PS_ODD, 700, torch.float16),
                                         (PS_ONE, 600, torch.bfloat16), (PS_ONE, 600, torch.float16)])
def test_prefill_fused_zipf_routing(cfg, T, dtype, device):
    from exq_amd.kernels import fused_experts
    banner(f"prefill fused {cfg.name} T={T} {dtype}")
    p13, s13, p2, s2 = _pack(cfg.n_experts, cfg.inter, cfg.hidden, 900, device)
    ids, w = synth.routing(cfg, T)
    counts = np.bincount(ids.reshape(-1), minlength=cfg.n_experts)
    assert counts.max() > 128  # several token groups for the busiest expert
    x = _hidden(T, cfg.hidden, 901 + T, device, dtype)
    so = torch.empty(T * cfg.top_k, dtype=torch.int64, device=device)
    ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=device)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device), sort_order_out=so,
                        expert_ends_out=ends)
    torch.cuda.synchronize()
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, cfg.n_experts)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"prefill fused {cfg.name} T={T} {dtype}")


def test_prefill_one_expert_takes_all_rows(device):
    """Every row on one expert: 600 rows = nine full 64-row groups + 24 (and,
    at 128 rows per group, four + 88)."""
    from exq_amd.kernels import fused_experts
    cfg = WIDE
    banner("prefill one expert")
    T = 300
    p13, s13, p2, s2 = _pack(cfg.n_experts, cfg.inter, cfg.hidden, 910, device)
    ids = np.full((T, 2), 5, dtype=np.int64)
    ids[:, 1] = 5
    rng = np.random.default_rng(11)
    w = rng.random((T, 2)).astype(np.float32)
    x = _hidden(T, cfg.hidden, 912, device, torch.bfloat16)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device))
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, "prefill one expert")


def _split_ids(T, dropped):
    """Top-2 ids of T = 1024 tokens with row counts on both sides of the
    per-expert tile switch (kI4BigMinRows = 384 rows): expert 0 exactly 384
    (three full 128-row groups), expert 1 383 (six 64-row groups, the last
    ragged), expert 2 700 (five 128-row groups + 60), expert 3 257, expert 4
    300, experts 6-7 none, and the last 24 tokens' second ids on expert 5 or
    dropped (-1)."""
    ids = np.empty((T, 2), dtype=np.int64)
    ids[:384, 0] = 0
    ids[384:767, 0] = 1
    ids[767:, 0] = 3
    ids[:700, 1] = 2
    ids[700:1000, 1] = 4
    ids[1000:, 1] = -1 if dropped else 5
    counts = np.bincount(ids[ids >= 0], minlength=8)
    assert counts.tolist() == [384, 383, 700, 257, 300, 0 if dropped else 24, 0, 0]
    return ids


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_per_expert_tile_shape(dtype, device):
    """Experts averaging under 512 rows take the 64 x 256 INT4 tiles; those
    with at least 384 rows take 128-row groups on the 128 x 256 scaled-operand
    tiles, in the same launch.  Boundary counts 383 / 384, a ragged big
    group and empty experts; sort order and boundaries bit-exact."""
    from exq_amd.kernels import fused_experts
    T, E = 1024, 8
    banner(f"prefill per-expert tile shape {dtype}")
    p13, s13, p2, s2 = _pack(E, 512, 1024, 980, device)
    ids = _split_ids(T, dropped=False)
    w = np.random.default_rng(981).random((T, 2)).astype(np.float32)
    x = _hidden(T, 1024, 982, device, dtype)
    so = torch.empty(T * 2, dtype=torch.int64, device=device)
    ends = torch.empty(E + 1, dtype=torch.int32, device=device)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device), sort_order_out=so,
                        expert_ends_out=ends)
    torch.cuda.synchronize()
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, E)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"prefill per-expert tile shape {dtype}")


@pytest.mark.parametrize("act", [torch.bfloat16, torch.float16])
def test_prefill_per_expert_tile_shape_mixed_bank(act, device):
    """The same split in a mixed bank: the big INT4 expert 2 and the small
    INT4 experts 1, 3 and 4 share a launch with the BF16 experts 0 and 6
    (expert 0 at exactly 384 rows is BF16 here); INT8 expert 5 is idle and 24
    ids are dropped."""
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    T, E = 1024, 8
    banner(f"prefill per-expert tile shape mixed bank {act}")
    w13, w2 = synth.expert_weights_gpu(E, 512, 1024, 983, device)
    bank = MixedExpertBank.from_weights(w13, w2, [0, 2, 2, 2, 2, 1, 0, 2], act_dtype=act)
    ids = _split_ids(T, dropped=True)
    w = np.random.default_rng(984).random((T, 2)).astype(np.float32)
    x = _hidden(T, 1024, 985, device, act)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device))
    from tests.test_gpu_mixed import _oracle
    assert_close_rel(out, _oracle(bank, x, ids, w), TOL,
                     f"prefill per-expert tile shape mixed bank {act}")


def test_prefill_per_expert_tile_shape_none_big(device):
    """A batch of 512 tokens (the per-expert switch is on) whose experts all stay
    below 384 rows: the 128 x 256 range of the combined launch is empty and every
    INT4 group takes the 64 x 256 tiles."""
    from exq_amd.kernels import fused_experts
    cfg = synth.MoeConfig("prefill_none_big", 52, 1024, 512, 32, 2, True, zipf=False)
    T = 512
    banner("prefill per-expert tile shape, no big expert")
    p13, s13, p2, s2 = _pack(cfg.n_experts, cfg.inter, cfg.hidden, 986, device)
    ids, w = synth.routing(cfg, T)
    counts = np.bincount(ids.reshape(-1), minlength=cfg.n_experts)
    assert counts.max() < 384 and T * cfg.top_k < 512 * cfg.n_experts
    x = _hidden(T, cfg.hidden, 987, device, torch.bfloat16)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device))
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, "prefill per-expert tile shape, no big expert")


def test_prefill_group_size_256_untiled(device):
    """group_size 256 is not tiled: the 64-row grouped kernel runs instead."""
    from exq_amd.kernels import fused_experts
    cfg = WIDE
    banner("prefill group 256")
    T = 200
    p13, s13, p2, s2 = _pack(cfg.n_experts, cfg.inter, cfg.hidden, 920, device, group_size=256)
    assert s13.shape[-1] == cfg.hidden // 256
    ids, w = synth.routing(cfg, T)
    x = _hidden(T, cfg.hidden, 921, device, torch.bfloat16)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device))
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, "prefill group 256")


@pytest.mark.parametrize("N", [256, 96])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_sorted_int4_gemm(N, dtype, device):
    from exq_amd.kernels import moe_int4_forward, pack_experts_int4
    banner(f"prefill sorted gemm N={N} {dtype}")
    E, K, T, k = 8, 512, 300, 2
    cfg = synth.MoeConfig("sorted", 43, K, N, E, k, True)
    rng = np.random.default_rng(N)
    w = torch.from_numpy((rng.standard_normal((E, N, K)) * 0.02).astype(np.float32)).to(device)
    p, s = pack_experts_int4(w)
    ids, _ = synth.routing(cfg, T)
    x = _hidden(T, K, 930, device, dtype)
    out = moe_int4_forward(x, p, s, torch.from_numpy(ids).to(device), E)
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, E)
    a = moe.gather_hidden(x.float().cpu().numpy(), r_so, k)
    ref = moe.grouped_gemm_sorted(a, quant.dequant_int4(p.cpu().numpy(), s.cpu().numpy()), r_ends)
    assert_close_rel(out, ref, TOL, f"sorted gemm N={N} {dtype}")


@pytest.mark.parametrize("act", [torch.bfloat16, torch.float16])
def test_prefill_mixed_tiers(act, device):
    """BF16 / INT8 token groups on the grouped kernel, INT4 on the tiled one."""
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner(f"prefill mixed tiers {act}")
    T = 400
    cfg = synth.MoeConfig("mix_prefill", 44, 512, 256, 16, 4, False)
    w13, w2 = synth.expert_weights_gpu(16, 256, 512, 71, device)
    tiers = synth.mixed_tiers(16, 71)
    assert set(tiers) == {0, 1, 2}
    bank = MixedExpertBank.from_weights(w13, w2, tiers, act_dtype=act)
    ids, w = synth.routing(cfg, T)
    x = _hidden(T, 512, 940, device, act)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device))
    from tests.test_gpu_mixed import _oracle
    assert_close_rel(out, _oracle(bank, x, ids, w), TOL, f"prefill mixed {act}")


@pytest.mark.parametrize("act", [torch.bfloat16, torch.float16])
def test_prefill_mixed_tiers_large_experts(act, device):
    """A mixed bank with more than 512 rows per routed expert: its INT4
    experts take the 128 x 256 scaled-operand tiles beside the BF16 tiles and
    the grouped INT8 kernel."""
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner(f"prefill mixed tiers large experts {act}")
    T, E = 1100, 8
    cfg = synth.MoeConfig("mix_prefill_big", 51, 512, 256, E, 4, False)
    assert T * cfg.top_k >= 512 * E
    w13, w2 = synth.expert_weights_gpu(E, 256, 512, 73, device)
    tiers = [2, 0, 2, 1, 2, 2, 1, 2]
    bank = MixedExpertBank.from_weights(w13, w2, tiers, act_dtype=act)
    ids, w = synth.routing(cfg, T)
    x = _hidden(T, 512, 960, device, act)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device))
    from tests.test_gpu_mixed import _oracle
    assert_close_rel(out, _oracle(bank, x, ids, w), TOL, f"prefill mixed large experts {act}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_sorted_bf16_gemm_tiled(dtype, device):
    """Unquantised sorted-row GEMM with N % 128 == 0 runs on the BF16 tiled
    kernel; a masked expert's rows stay zero."""
    from exq_amd.kernels import moe_grouped_gemm
    banner(f"prefill grouped gemm tiled {dtype}")
    rng = np.random.default_rng(5)
    E, N, K, T, k = 8, 256, 384, 300, 2
    W = torch.from_numpy((rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)).to(dtype)
    cfg = synth.MoeConfig("sorted_bf", 45, K, N, E, k, True)
    ids, _ = synth.routing(cfg, T)
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(dtype)
    mask = torch.ones(E, dtype=torch.int32)
    mask[3] = 0
    out = moe_grouped_gemm(x.to(device), W.to(device), torch.from_numpy(ids).to(device), E,
                           expert_mask=mask.to(device))
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, E)
    a = moe.gather_hidden(x.float().numpy(), r_so, k)
    Wm = W.float().numpy().copy()
    Wm[3] = 0
    ref = moe.grouped_gemm_sorted(a, Wm, r_ends)
    assert_close_rel(out, ref, TOL, f"grouped gemm tiled {dtype}")


def test_prefill_mixed_mostly_int8_strided_grid(device):
    """Mostly INT8 experts next to INT4 and BF16 ones at a large batch: the
    grouped kernel's grid (capped while the tiled kernels run) strides over
    more units than it has work-groups."""
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner("prefill mixed mostly int8")
    T, E = 2000, 16
    cfg = synth.MoeConfig("mix_int8", 46, 512, 512, E, 4, False)
    w13, w2 = synth.expert_weights_gpu(E, 512, 512, 72, device)
    tiers = [1] * E
    tiers[3] = 2
    tiers[9] = 0
    bank = MixedExpertBank.from_weights(w13, w2, tiers)
    ids, w = synth.routing(cfg, T)
    int8_rows = sum(int((ids == e).sum()) for e in range(E) if tiers[e] == 1)
    assert int8_rows // 64 * (512 // 16) > 2048  # more gate/up units than the capped grid
    x = _hidden(T, 512, 950, device, torch.bfloat16)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device))
    from tests.test_gpu_mixed import _oracle
    assert_close_rel(out, _oracle(bank, x, ids, w), TOL, "prefill mixed mostly int8")


@pytest.mark.parametrize("T", [300, 9000])
def test_prefill_routing_plan_sizes(T, device):
    """The fused layer's routing plan above one work-group: 2,400 slots take the
    one-launch plan (every block recounts all slots), 72,000 slots the
    three-launch plan through the workspace (per-block counts, offsets,
    scatter).  sort_order / expert_ends are bit-exact; the output is within
    0.5 % of the oracle on 64 sampled tokens."""
    from exq_amd.kernels import fused_experts
    cfg = synth.MoeConfig("plan_sizes", 48, 256, 128, 16, 8, True)
    banner(f"prefill routing plan T={T} ({T * cfg.top_k} slots)")
    p13, s13, p2, s2 = _pack(cfg.n_experts, cfg.inter, cfg.hidden, 930, device)
    ids, w = synth.routing(cfg, T)
    x = _hidden(T, cfg.hidden, 931, device, torch.bfloat16)
    so = torch.empty(T * cfg.top_k, dtype=torch.int64, device=device)
    ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=device)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device), sort_order_out=so,
                        expert_ends_out=ends)
    torch.cuda.synchronize()
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, cfg.n_experts)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    rows = np.sort(np.random.default_rng(T).choice(T, size=64, replace=False))
    ref = oracle_int4_layer(x[torch.from_numpy(rows).to(device)], p13, s13, p2, s2, ids[rows],
                            w[rows])
    assert_close_rel(out[torch.from_numpy(rows).to(device)], ref, TOL,
                     f"prefill routing plan T={T} (64 rows)")

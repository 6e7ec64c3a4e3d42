"""Mixed-precision (BF16 / INT8 / INT4) dispatch and shared experts on the
GPU vs the oracle (each tier dequantised by its own rule).  Tolerance:
relative L2 <= 0.5%."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import moe, quant
from tests._helpers import assert_close_rel, banner

pytestmark = pytest.mark.gpu

TOL = 5e-3


def _dequant_bank(bank, e):
    """Float weights (w13, w2) of expert e as the bank stores them."""
    t = int(bank.tier[e].item())
    i = int(bank.index[e].item())
    if t == 0:
        return bank.bf16_w13[i].float().cpu().numpy(), bank.bf16_w2[i].float().cpu().numpy()
    if t == 1:
        return (quant.dequant_int8(bank.int8_w13[i].cpu().numpy(), bank.int8_w13_scales[i].cpu().numpy()),
                quant.dequant_int8(bank.int8_w2[i].cpu().numpy(), bank.int8_w2_scales[i].cpu().numpy()))
    return (quant.dequant_int4(bank.int4_w13[i].cpu().numpy(), bank.int4_w13_scales[i].cpu().numpy()),
            quant.dequant_int4(bank.int4_w2[i].cpu().numpy(), bank.int4_w2_scales[i].cpu().numpy()))


def _oracle(bank, x, ids, w):
    E, S = bank.n_experts, bank.n_shared
    parts = [_dequant_bank(bank, e) for e in range(E + S)]
    w13 = np.stack([p[0] for p in parts[:E]])
    w2 = np.stack([p[1] for p in parts[:E]])
    sh13 = np.stack([p[0] for p in parts[E:]]) if S else None
    sh2 = np.stack([p[1] for p in parts[E:]]) if S else None
    return moe.moe_layer(x.float().cpu().numpy(), w13, w2, ids, w, sh13, sh2)


@pytest.mark.parametrize("T", [1, 7, 32, 100])
@pytest.mark.parametrize("act", [torch.bfloat16, torch.float16])
def test_mixed_tiers_small(T, act, device):
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner(f"mixed small T={T} {act}")
    cfg = synth.MoeConfig("mix_small", 7, 512, 256, 16, 4, False)
    w13, w2 = synth.expert_weights_gpu(16, 256, 512, 70, device)
    tiers = synth.mixed_tiers(16, 70)
    assert set(tiers) == {0, 1, 2}
    bank = MixedExpertBank.from_weights(w13, w2, tiers, act_dtype=act)
    ids, w = synth.routing(cfg, T)
    x = torch.from_numpy(synth.hidden_np(T, 512, T)).to(act).to(device)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device))
    assert_close_rel(out, _oracle(bank, x, ids, w), TOL, f"mixed small T={T} {act}")


def test_mixed_olmoe_shape(device):
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner("mixed olmoe T=32")
    cfg = synth.CONFIGS["mixed_olmoe"]
    w13, w2 = synth.expert_weights_gpu(64, 1024, 2048, synth.seed_for(cfg), device)
    tiers = synth.mixed_tiers(64, synth.seed_for(cfg))
    bank = MixedExpertBank.from_weights(w13, w2, tiers)
    del w13, w2
    ids, w = synth.routing(cfg, 32)
    x = torch.from_numpy(synth.hidden_np(32, 2048, 5)).to(torch.bfloat16).to(device)
    so = torch.empty(32 * 8, dtype=torch.int64, device=device)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device), sort_order_out=so)
    from oracle import routing
    assert np.array_equal(so.cpu().numpy(), routing.sort_tokens_by_expert(ids, 64)[0])
    used = np.unique(ids)
    E = 64
    ref_parts = {int(e): _dequant_bank(bank, int(e)) for e in used}
    remap = {int(e): i for i, e in enumerate(used)}
    w13d = np.stack([ref_parts[int(e)][0] for e in used])
    w2d = np.stack([ref_parts[int(e)][1] for e in used])
    ids_c = np.vectorize(remap.get)(ids)
    ref = moe.moe_layer(x.float().cpu().numpy(), w13d, w2d, ids_c, w)
    assert_close_rel(out, ref, TOL, "mixed olmoe T=32")
    assert E == bank.n_experts


@pytest.mark.parametrize("T", [1, 2])
def test_mixed_tiers_split_contraction(T, device):
    """BF16, INT8 and INT4 down projections with their 13-k-block contraction
    split three ways (few active experts); fixed-order split sums repeat
    bitwise."""
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner(f"mixed split T={T}")
    E = 8
    cfg = synth.MoeConfig("mix_split", 32, 512, 1664, E, 2, True, zipf=False)
    w13, w2 = synth.expert_weights_gpu(E, 1664, 512, 73, device)
    tiers = [0, 1, 2, 0, 1, 2, 1, 2]
    for act in (torch.bfloat16, torch.float16):
        bank = MixedExpertBank.from_weights(w13, w2, tiers, act_dtype=act)
        for seed in range(3):  # different expert pairs
            ids, w = synth.routing(cfg, T)
            ids = (ids + seed * 3) % E
            ids[0, :] = [seed % E, (seed + 1) % E]
            x = torch.from_numpy(synth.hidden_np(T, 512, 40 + seed)).to(act).to(device)
            tid = torch.from_numpy(ids).to(device)
            tw = torch.from_numpy(w).to(device)
            out = fused_experts_mixed(x, bank, tw, tid)
            assert_close_rel(out, _oracle(bank, x, ids, w), TOL, f"mixed split {act} {seed}")
            assert torch.equal(fused_experts_mixed(x, bank, tw, tid), out)


@pytest.mark.parametrize("T", [1, 16, 64, 200])
def test_shared_experts_deepseek_shape(T, device):
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner(f"deepseek shared T={T}")
    cfg = synth.CONFIGS["deepseek_v2_lite"]
    w13, w2 = synth.expert_weights_gpu(64, 1408, 2048, synth.seed_for(cfg), device)
    s13, s2 = synth.expert_weights_gpu(2, 1408, 2048, synth.seed_for(cfg) + 500, device)
    bank = MixedExpertBank.from_weights(w13, w2, [2] * 64, shared_w13=s13, shared_w2=s2,
                                        shared_tier=0)
    del w13, w2
    ids, w = synth.routing(cfg, T)
    x = torch.from_numpy(synth.hidden_np(T, 2048, T)).to(torch.bfloat16).to(device)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device))
    used = np.unique(ids)
    remap = {int(e): i for i, e in enumerate(used)}
    parts = [_dequant_bank(bank, int(e)) for e in used]
    sh = [_dequant_bank(bank, 64 + s) for s in range(2)]
    ref = moe.moe_layer(x.float().cpu().numpy(), np.stack([p[0] for p in parts]),
                        np.stack([p[1] for p in parts]), np.vectorize(remap.get)(ids), w,
                        np.stack([p[0] for p in sh]), np.stack([p[1] for p in sh]))
    assert_close_rel(out, ref, TOL, f"deepseek shared T={T}")


@pytest.mark.parametrize("layer", [0, 1])
def test_mixed_olmoe_stack_artifact_plan(layer, device, tmp_path):
    """The mixed stack exactly as the bench times it: tiers from the quant-plan
    artifact (router-ranked: the router's most frequent 10 % of experts BF16, the
    next 20 % INT8, the rest INT4; exq_artifact.py:96-192) read back with
    load_exq_artifact, full OLMoE shape, T = 32.  The hot BF16 experts then hold
    more than 16 rows (several 16-row tiles); sort_order is bit-exact and the
    output within 0.5 % of the oracle."""
    import json
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed, load_exq_artifact
    from oracle import routing
    banner(f"mixed olmoe stack, artifact plan, layer {layer}, T=32")
    cfg = synth.CONFIGS["mixed_olmoe"]
    path = tmp_path / "plan.json"
    path.write_text(json.dumps(synth.plan_artifact(cfg, n_layers=2)), encoding="utf-8")
    plan = load_exq_artifact(str(path), device="cpu")
    tiers = plan.tiers[layer].tolist()
    assert tiers == synth.router_tiers(cfg, layer)
    w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                       synth.seed_for(cfg, layer), device)
    bank = MixedExpertBank.from_weights(w13, w2, tiers)
    del w13, w2
    T = 32
    ids, w = synth.routing(cfg, T, layer)
    counts = np.bincount(ids.reshape(-1), minlength=cfg.n_experts)
    bf16 = [e for e in range(cfg.n_experts) if tiers[e] == 0]
    assert max(counts[bf16]) > 16, "the hot BF16 experts should span several 16-row tiles"
    x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 99)).to(torch.bfloat16).to(device)
    so = torch.empty(T * cfg.top_k, dtype=torch.int64, device=device)
    ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=device)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device), sort_order_out=so,
                              expert_ends_out=ends)
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, cfg.n_experts)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    used = np.unique(ids)
    parts = {int(e): _dequant_bank(bank, int(e)) for e in used}
    remap = {int(e): i for i, e in enumerate(used)}
    ref = moe.moe_layer(x.float().cpu().numpy(), np.stack([parts[int(e)][0] for e in used]),
                        np.stack([parts[int(e)][1] for e in used]),
                        np.vectorize(remap.get)(ids), w)
    assert_close_rel(out, ref, TOL, f"mixed olmoe stack artifact plan layer {layer} T=32")

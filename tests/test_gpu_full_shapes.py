"""The two BASELINE workloads at their full shapes, checked against the
oracle: Mixtral-8x7B (H=4096, I=14336, E=8, top-2) at decode T = 1, 16, 64 and
the 4096-token prefill chunk, and DeepSeek-V2-Lite (64 INT4 routed experts
top-6 + 2 BF16 shared, I=1408) at the 2048-token prefill chunk.

The GPU runs the whole batch.  Routing arrays are compared bit-exact over the
whole batch.  Token rows are independent of each other, so the layer output
is compared on every row for decode batches and on 64 seeded rows of a
prefill chunk; the oracle dequantises one routed expert at a time (host
memory stays bounded).  Tolerance: relative L2 <= 0.5% over the checked rows,
2x that per row."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import moe, quant, routing
from tests._helpers import assert_close_rel, banner

pytestmark = pytest.mark.gpu

TOL = 5e-3
N_SAMPLE = 64


class _LazyInt4Bank:
    """[E, N, K] float32 view of a packed bank for oracle.moe.moe_layer:
    expert e is copied to the host and dequantised on first use."""

    def __init__(self, packed: torch.Tensor, scales: torch.Tensor):
        self.packed, self.scales = packed, scales
        E, N, K2 = packed.shape
        self.shape = (E, N, 2 * K2)
        self._cache = {}

    def __getitem__(self, e):
        e = int(e)
        if e not in self._cache:
            self._cache[e] = quant.dequant_int4(self.packed[e].cpu().numpy(),
                                                self.scales[e].cpu().numpy())
        return self._cache[e]


def _rows(T, seed):
    if T <= N_SAMPLE:
        return np.arange(T)
    return np.sort(np.random.default_rng(seed).choice(T, size=N_SAMPLE, replace=False))


@pytest.fixture(scope="module")
def mixtral(device):
    from exq_amd.kernels import pack_experts_int4
    cfg = synth.CONFIGS["mixtral"]
    banner("mixtral full shape: pack 8 experts H=4096 I=14336")
    w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                       synth.seed_for(cfg, 0), device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    del w13, w2
    torch.cuda.empty_cache()
    yield cfg, (p13, s13, p2, s2), _LazyInt4Bank(p13, s13), _LazyInt4Bank(p2, s2)


@pytest.mark.parametrize("T", [1, 16, 64, 4096])
def test_mixtral_full_shape(T, mixtral, device):
    from exq_amd.kernels import fused_experts
    cfg, (p13, s13, p2, s2), d13, d2 = mixtral
    banner(f"mixtral full shape T={T}")
    ids, w = synth.routing(cfg, T, 0)
    x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 11 + T)).to(torch.bfloat16).to(device)
    so = torch.empty(T * cfg.top_k, dtype=torch.int64, device=device)
    ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=device)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device), sort_order_out=so,
                        expert_ends_out=ends)
    torch.cuda.synchronize()
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, cfg.n_experts)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    rows = _rows(T, 400 + T)
    ref = moe.moe_layer(x.float().cpu().numpy()[rows], d13, d2, ids[rows], w[rows])
    assert_close_rel(out[torch.from_numpy(rows).to(device)], ref, TOL,
                     f"mixtral full shape T={T} ({rows.size} rows)")


def test_deepseek_prefill_2048_with_shared_experts(device):
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    cfg = synth.CONFIGS["deepseek_v2_lite"]
    T = 2048
    banner("deepseek-v2-lite prefill T=2048 (+2 BF16 shared)")
    w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                       synth.seed_for(cfg, 0), device)
    sh13, sh2 = synth.expert_weights_gpu(cfg.n_shared, cfg.inter, cfg.hidden,
                                         synth.seed_for(cfg, 0) + 500, device)
    bank = MixedExpertBank.from_weights(w13, w2, [2] * cfg.n_experts, shared_w13=sh13,
                                        shared_w2=sh2, shared_tier=0)
    del w13, w2
    ids, w = synth.routing(cfg, T, 0)
    x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 3)).to(torch.bfloat16).to(device)
    so = torch.empty(T * cfg.top_k, dtype=torch.int64, device=device)
    ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=device)
    out = fused_experts_mixed(x, bank, torch.from_numpy(w).to(device),
                              torch.from_numpy(ids).to(device), sort_order_out=so,
                              expert_ends_out=ends)
    torch.cuda.synchronize()
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, cfg.n_experts)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    rows = _rows(T, 77)
    d13 = _LazyInt4Bank(bank.int4_w13, bank.int4_w13_scales)
    d2 = _LazyInt4Bank(bank.int4_w2, bank.int4_w2_scales)
    ref = moe.moe_layer(x.float().cpu().numpy()[rows], d13, d2, ids[rows], w[rows],
                        bank.bf16_w13.float().cpu().numpy(), bank.bf16_w2.float().cpu().numpy())
    assert_close_rel(out[torch.from_numpy(rows).to(device)], ref, TOL,
                     f"deepseek prefill T=2048 ({rows.size} rows)")

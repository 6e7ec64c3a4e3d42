"""Seeded random layers against the oracle: the fused INT4 entry point and the
mixed-tier entry point over random expert counts (2-130), top-k (1-8),
hidden / intermediate sizes (standard and general shapes), batches on both
sides of the decode / prefill switch (1-200 tokens), shared experts, random
tiers, activation / id / weight dtypes and dropped (-1) ids.  Each case prints
its parameters before it runs.  Tolerance: relative L2 <= 0.5 % over the
output, 1 % per token row."""
import os

import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import moe, quant
from tests._helpers import assert_close_rel, banner
from tests.test_gpu_mixed import _oracle

pytestmark = pytest.mark.gpu

# 32 seeded cases by default; EXQ_RANDOM_LAYER_CASES=N runs the first N seeds
N_CASES = int(os.environ.get("EXQ_RANDOM_LAYER_CASES", "32"))
TOL = 5e-3


def _case(i):
    rng = np.random.default_rng(5000 + i)
    general = i % 4 == 3  # pure INT4 with a group size of 32 and sizes off the 128 grid
    E = int(rng.choice([2, 5, 8, 16, 33, 64, 130]))
    k = int(rng.integers(1, min(8, E) + 1))
    if general:
        H, I, g = int(rng.choice([96, 160, 224])), int(rng.choice([64, 96, 160])), 32
    else:
        H, I, g = int(rng.choice([128, 256, 384, 512])), int(rng.choice([128, 256, 384])), 128
    T = int(rng.choice([1, 2, 5, 16, 17, 33, 64, 65, 80, 200]))
    mixed = (not general) and bool(rng.random() < 0.6)
    n_shared = int(rng.choice([0, 0, 1, 2])) if mixed else 0
    return dict(E=E, k=k, H=H, I=I, g=g, T=T, mixed=mixed, n_shared=n_shared,
                act=[torch.bfloat16, torch.float16][int(rng.integers(2))],
                ids_dt=[torch.int32, torch.int64][int(rng.integers(2))],
                w_dt=[torch.float32, torch.bfloat16][int(rng.integers(2))],
                drop=float(rng.choice([0.0, 0.0, 0.15])), seed=5000 + i)


def _routing(rng, T, E, k, drop):
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    if drop > 0:
        ids[rng.random(ids.shape) < drop] = -1
    logits = rng.standard_normal((T, k)).astype(np.float32)
    w = np.exp(logits) / np.exp(logits).sum(axis=1, keepdims=True)
    return ids, w.astype(np.float32)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_layer(i, device):
    from exq_amd.kernels import (MixedExpertBank, fused_experts, fused_experts_mixed,
                                 pack_experts_int4)
    c = _case(i)
    banner(f"random layer {i}: {c}")
    rng = np.random.default_rng(c["seed"])
    E, k, H, I, T = c["E"], c["k"], c["H"], c["I"], c["T"]
    w13, w2 = synth.expert_weights_gpu(E, I, H, c["seed"], device)
    ids, w = _routing(rng, T, E, k, c["drop"])
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(c["act"]).to(device)
    tid = torch.from_numpy(ids).to(c["ids_dt"]).to(device)
    tw = torch.from_numpy(w).to(c["w_dt"]).to(device)
    w_used = tw.float().cpu().numpy()  # the weights as the kernel reads them
    if c["mixed"]:
        tiers = rng.integers(0, 3, size=E).tolist()
        sh13 = sh2 = None
        if c["n_shared"]:
            sh13, sh2 = synth.expert_weights_gpu(c["n_shared"], I, H, c["seed"] + 77, device)
        bank = MixedExpertBank.from_weights(w13, w2, tiers, act_dtype=c["act"], shared_w13=sh13,
                                            shared_w2=sh2, shared_tier=int(rng.integers(0, 3)))
        out = fused_experts_mixed(x, bank, tw, tid)
        ref = _oracle(bank, x, ids, w_used)
    else:
        p13, s13 = pack_experts_int4(w13, group_size=c["g"])
        p2, s2 = pack_experts_int4(w2, group_size=c["g"])
        out = fused_experts(x, p13, s13, p2, s2, tw, tid)
        d13 = np.stack([quant.dequant_int4(p13[e].cpu().numpy(), s13[e].cpu().numpy()) for e in range(E)])
        d2 = np.stack([quant.dequant_int4(p2[e].cpu().numpy(), s2[e].cpu().numpy()) for e in range(E)])
        ref = moe.moe_layer(x.float().cpu().numpy(), d13, d2, ids, w_used)
    assert out.shape == (T, H) and out.dtype == c["act"]
    if np.abs(ref).max() == 0:  # every slot dropped: the layer is zero
        assert torch.count_nonzero(out) == 0
        return
    assert_close_rel(out, ref, TOL, f"random layer {i}")

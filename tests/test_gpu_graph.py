"""The layer entry points under HIP graph capture: router + fused layer
(decode and prefill sizes, INT4 and mixed banks) captured once, replayed
three times with unrelated eager calls and synchronisations in between; every
replay equals the eager result bitwise (the layer is deterministic)."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from tests._helpers import banner

pytestmark = pytest.mark.gpu


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up (workspace, lazily loaded state) outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


@pytest.mark.parametrize("T", [16, 64, 300])
def test_graph_replays_int4_layer(T, device):
    from exq_amd.kernels import fused_experts, fused_topk, pack_experts_int4
    from exq_amd.kernels.fused_moe import moe_workspace_bytes
    banner(f"graph int4 T={T}")
    cfg = synth.MoeConfig("graph", 61, 512, 256, 16, 4, True)
    w13, w2 = synth.expert_weights_gpu(16, 256, 512, 61, device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    x = torch.from_numpy(synth.hidden_np(T, 512, 3)).to(torch.bfloat16).to(device)
    logits = torch.from_numpy(synth.router_logits(cfg, T, 4)).to(device)
    ws = torch.zeros(moe_workspace_bytes(T, 512, 256, 16, 4), dtype=torch.uint8, device=device)
    out = torch.empty(T, 512, dtype=torch.bfloat16, device=device)

    def step():
        tw, tid = fused_topk(logits, 4, True)
        return fused_experts(x, p13, s13, p2, s2, tw, tid, out=out, workspace=ws)

    eager = step().clone()
    g, _ = _capture(step)
    x2 = torch.from_numpy(synth.hidden_np(T, 512, 8)).to(torch.bfloat16).to(device)
    for r in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        # unrelated eager work on the same workspace between replays
        tw2, tid2 = fused_topk(logits.flip(0), 4, True)
        fused_experts(x2, p13, s13, p2, s2, tw2, tid2, workspace=ws)
        torch.cuda.synchronize()


def test_graph_replays_mixed_layer(device):
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    banner("graph mixed T=32")
    T = 32
    cfg = synth.MoeConfig("graph_mix", 62, 512, 256, 16, 4, False)
    w13, w2 = synth.expert_weights_gpu(16, 256, 512, 62, device)
    bank = MixedExpertBank.from_weights(w13, w2, synth.mixed_tiers(16, 62))
    ids, w = synth.routing(cfg, T)
    tid = torch.from_numpy(ids).to(device)
    tw = torch.from_numpy(w).to(device)
    x = torch.from_numpy(synth.hidden_np(T, 512, 6)).to(torch.bfloat16).to(device)
    eager = fused_experts_mixed(x, bank, tw, tid).clone()
    g, out = _capture(lambda: fused_experts_mixed(x, bank, tw, tid))
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        fused_experts_mixed(x.flip(0), bank, tw, tid)
        torch.cuda.synchronize()

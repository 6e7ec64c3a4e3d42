"""bench_events times a layer call with HIP events (eager and as a graph
replay) and returns the reference harness's keys."""
import pytest
import torch

from exq_amd import synth
from tests._helpers import banner

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("graph", [False, True])
def test_bench_events_layer(graph, device):
    from exq_amd.eval import bench_events
    from exq_amd.kernels import fused_experts, pack_experts_int4
    banner(f"bench_events graph={graph}")
    cfg = synth.MoeConfig("evb", 71, 512, 256, 16, 4, True)
    w13, w2 = synth.expert_weights_gpu(16, 256, 512, 71, device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    ids, w = synth.routing(cfg, 16)
    tid = torch.from_numpy(ids).to(device)
    tw = torch.from_numpy(w).to(device)
    x = torch.from_numpy(synth.hidden_np(16, 512, 2)).to(torch.bfloat16).to(device)
    out = torch.empty(16, 512, dtype=torch.bfloat16, device=device)
    st = bench_events(lambda: fused_experts(x, p13, s13, p2, s2, tw, tid, out=out),
                      n_warmup=3, n_runs=25, graph=graph)
    assert st["n"] == 25
    assert 0.0 < st["p50"] <= st["p95"] <= st["p99"] < 50.0  # ms

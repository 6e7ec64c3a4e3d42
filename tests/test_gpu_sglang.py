"""The SGLang hook end to end on the GPU with stand-in SGLang classes: the
patched forward_cuda packs the layer once (through the on-disk cache when
given a directory), routes with the GPU router, runs the fused layer and
matches the oracle (relative L2 <= 0.5%); a second backend on the same
directory loads the packed bank instead of repacking."""
import json
import types

import numpy as np
import pytest
import torch

from exq_amd import synth
from tests._helpers import assert_close_rel, banner, oracle_int4_layer
from tests.test_host import _install_fake_sglang

pytestmark = pytest.mark.gpu


def test_sglang_forward_with_disk_cache(tmp_path, monkeypatch, device):
    from exq_amd.kernels import fused_topk
    from exq_amd.runtime import sglang_backend as sb
    banner("sglang hook + disk cache")
    cls = _install_fake_sglang(monkeypatch)
    art = tmp_path / "a.json"
    art.write_text(json.dumps({"quant_assignments": {"3:0": "INT4"}}))
    cfg = synth.MoeConfig("hook", 51, 512, 256, 8, 2, True)
    w13, w2 = synth.expert_weights_gpu(8, 256, 512, 51, device)
    layer = types.SimpleNamespace(layer_id=3, w13_weight=w13, w2_weight=w2)
    T = 12
    x = torch.from_numpy(synth.hidden_np(T, 512, 5)).to(torch.bfloat16).to(device)
    logits = torch.from_numpy(synth.router_logits(cfg, T, 9)).to(device)
    tw, tid = fused_topk(logits, 2, True)
    disp = types.SimpleNamespace(hidden_states=x,
                                 topk_output=types.SimpleNamespace(topk_weights=tw, topk_ids=tid))
    cache_dir = tmp_path / "packed"
    backend = sb.patch_sglang(str(art), pack_cache_dir=str(cache_dir))
    try:
        out = cls().forward_cuda(layer, disp).hidden_states
        st = backend.cache_stats()
        assert st["disk_misses"] == 1 and st["disk_hits"] == 0
        c = sb._exq_packed_cache[id(layer)]
        ref = oracle_int4_layer(x, c["w1_packed"], c["w1_scales"], c["w2_packed"],
                                c["w2_scales"], tid.cpu().numpy().astype(np.int64),
                                tw.cpu().numpy())
        assert_close_rel(out, ref, 5e-3, "sglang hook")
        backend2 = sb.patch_sglang(str(art), pack_cache_dir=str(cache_dir))  # a later run
        out2 = cls().forward_cuda(layer, disp).hidden_states
        st2 = backend2.cache_stats()
        assert st2["disk_hits"] == 1 and st2["disk_misses"] == 0
        assert torch.equal(out, out2)
    finally:
        sb.unpatch_sglang()


def test_sglang_mixed_plan_fp16_graph_capture(tmp_path, monkeypatch, device):
    """A BF16/INT8/INT4 plan (tiers from the router's own Zipf frequencies,
    written as an artifact and read back by the reader) through
    patch_sglang(honor_plan=True): fp16 activations into a layer whose BF16
    tier is stored bf16 come back fp16 (the caller's dtype, as the reference
    returns its activation dtype, sglang_backend.py:155), match the oracle,
    and the patched forward_cuda replays bitwise from a HIP graph."""
    from exq_amd.kernels import load_exq_artifact
    from exq_amd.runtime import sglang_backend as sb
    from tests.test_gpu_mixed import _oracle
    banner("sglang mixed plan fp16 + graph")
    cls = _install_fake_sglang(monkeypatch)
    cfg = synth.MoeConfig("hook_mix", 52, 512, 256, 16, 4, False, n_layers=2)
    art = tmp_path / "plan.json"
    art.write_text(json.dumps(synth.plan_artifact(cfg)))
    prof = load_exq_artifact(str(art), device="cpu")
    assert sorted(set(prof.tiers[1].tolist())) == [0, 1, 2]
    w13, w2 = synth.expert_weights_gpu(16, 256, 512, 52, device)
    layer = types.SimpleNamespace(layer_id=1, w13_weight=w13.to(torch.bfloat16),
                                  w2_weight=w2.to(torch.bfloat16))
    T = 24
    ids, w = synth.routing(cfg, T, 1)
    x = torch.from_numpy(synth.hidden_np(T, 512, 6)).to(torch.float16).to(device)
    disp = types.SimpleNamespace(hidden_states=x, topk_output=types.SimpleNamespace(
        topk_weights=torch.from_numpy(w).to(device), topk_ids=torch.from_numpy(ids).to(device)))
    backend = sb.patch_sglang(str(art), honor_plan=True)
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            eager = cls().forward_cuda(layer, disp).hidden_states  # packs the layer
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        assert eager.dtype == torch.float16 and eager.shape == (T, 512)
        bank = sb._exq_packed_cache[id(layer)]["bank"]
        assert bank is not None and bank.tier.tolist() == prof.tiers[1].tolist()
        assert bank.bf16_w13.dtype == torch.bfloat16
        # the oracle sees the activations the kernels saw (cast to the bank dtype)
        ref = _oracle(bank, x.to(torch.bfloat16), ids, w)
        assert_close_rel(eager, ref, 5e-3, "sglang mixed plan fp16")
        eager = eager.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = cls().forward_cuda(layer, disp).hidden_states
        for r in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {r}"
            cls().forward_cuda(layer, types.SimpleNamespace(  # unrelated eager call
                hidden_states=x.flip(0), topk_output=disp.topk_output))
            torch.cuda.synchronize()
    finally:
        sb.unpatch_sglang()

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

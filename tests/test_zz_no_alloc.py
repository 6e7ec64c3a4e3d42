"""The no-alloc INT4 layer entry point (exq_moe_int4_fused_forward_noalloc)
through the C ABI: two calls in a row, the second with a smaller batch, each
equal bitwise to exq_moe_int4_fused_forward with a caller workspace (the
same kernels; the layer is deterministic), plus routing copies; a problem
beyond the scratch maximum is rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from exq_amd import _lib, synth
from oracle import routing
from tests._helpers import banner

pytestmark = pytest.mark.gpu


def _call(noalloc, cfg, T, banks, x, tid, tw, device):
    p13, s13, p2, s2 = banks
    L = _lib.lib()
    p = _lib.MoeProblem(n_tokens=T, hidden_size=cfg.hidden, inter_size=cfg.inter,
                        n_experts=cfg.n_experts, top_k=cfg.top_k, n_shared=0, group_size=128,
                        act_dtype=_lib.BF16, ids_dtype=_lib.dtype_code(tid.dtype),
                        weights_dtype=_lib.F32)
    out = torch.full((T, cfg.hidden), float("nan"), dtype=torch.bfloat16, device=device)
    so = torch.full((T * cfg.top_k,), -1, dtype=torch.int64, device=device)
    ends = torch.full((cfg.n_experts + 1,), -1, dtype=torch.int32, device=device)
    args = [ctypes.byref(p), x.data_ptr(), tid.data_ptr(), tw.data_ptr(), p13.data_ptr(),
            s13.data_ptr(), p2.data_ptr(), s2.data_ptr(), out.data_ptr(), so.data_ptr(),
            ends.data_ptr()]
    stream = _lib.stream_handle(device)
    if noalloc:
        _lib.check(L.exq_moe_int4_fused_forward_noalloc(*args, stream), "noalloc")
    else:
        need = L.exq_moe_workspace_size(ctypes.byref(p))
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        _lib.check(L.exq_moe_int4_fused_forward(*args, ws.data_ptr(), ws.numel(), stream),
                   "workspace")
    torch.cuda.synchronize()
    return out, so, ends


@pytest.mark.parametrize("cfg,sizes", [
    (synth.MoeConfig("na_small", 31, 512, 256, 16, 4, True), (48, 5)),
    (synth.CONFIGS["qwen3"], (64, 16)),
    (synth.CONFIGS["olmoe"], (300, 1)),   # a prefill-sized batch, then a decode one
])
def test_noalloc_matches_workspace_entry_point(cfg, sizes, device):
    from exq_amd.kernels import pack_experts_int4
    w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 90, device)
    banks = pack_experts_int4(w13) + pack_experts_int4(w2)
    del w13, w2
    for T in sizes:
        banner(f"noalloc {cfg.name} T={T}")
        ids, w = synth.routing(cfg, T, 0)
        tid = torch.from_numpy(ids.astype(np.int32)).to(device)
        tw = torch.from_numpy(w).to(device)
        x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 40 + T)).to(torch.bfloat16).to(device)
        a = _call(True, cfg, T, banks, x, tid, tw, device)
        b = _call(False, cfg, T, banks, x, tid, tw, device)
        assert torch.equal(a[0], b[0]), f"{cfg.name} T={T}: outputs differ"
        assert not torch.isnan(a[0].float()).any()
        r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, cfg.n_experts)
        assert np.array_equal(a[1].cpu().numpy(), r_so)
        assert np.array_equal(a[2].cpu().numpy(), r_ends)


def test_noalloc_rejects_problem_beyond_scratch(device):
    L = _lib.lib()
    cfg = synth.CONFIGS["mixtral"]
    p = _lib.MoeProblem(n_tokens=16384, hidden_size=cfg.hidden, inter_size=cfg.inter,
                        n_experts=cfg.n_experts, top_k=cfg.top_k, n_shared=0, group_size=128,
                        act_dtype=_lib.BF16, ids_dtype=_lib.I32, weights_dtype=_lib.F32)
    assert L.exq_moe_workspace_size(ctypes.byref(p)) > (64 << 20)
    st = L.exq_moe_int4_fused_forward_noalloc(ctypes.byref(p), *([None] * 10), None,
                                              _lib.stream_handle(device))
    assert st == 3 and b"no-alloc" in L.exq_last_error()

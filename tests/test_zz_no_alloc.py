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
    # problem, the ten data pointers (hidden ... expert_ends_out), the stream
    st = L.exq_moe_int4_fused_forward_noalloc(ctypes.byref(p), *([None] * 10),
                                              _lib.stream_handle(device))
    assert st == 3 and b"no-alloc" in L.exq_last_error()


def _problem(cfg, T, ids_dtype):
    return _lib.MoeProblem(n_tokens=T, hidden_size=cfg.hidden, inter_size=cfg.inter,
                           n_experts=cfg.n_experts, top_k=cfg.top_k, n_shared=0,
                           group_size=128, act_dtype=_lib.BF16,
                           ids_dtype=_lib.dtype_code(ids_dtype), weights_dtype=_lib.F32)


def test_noalloc_captured_and_replayed(device):
    """Captured into a graph after a warm call on the device: each of three
    replays equals the workspace entry point bitwise, with an eager no-alloc
    call of another batch (which rewrites the shared scratch) between replays."""
    from exq_amd.kernels import pack_experts_int4
    banner("noalloc graph capture")
    cfg = synth.MoeConfig("na_graph", 33, 512, 256, 16, 4, True)
    w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 91, device)
    banks = pack_experts_int4(w13) + pack_experts_int4(w2)
    L = _lib.lib()

    def inputs(T, seed):
        ids, w = synth.routing(cfg, T, seed)
        x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, seed + 5)).to(torch.bfloat16)
        return (x.to(device), torch.from_numpy(ids.astype(np.int32)).to(device),
                torch.from_numpy(w).to(device))

    T = 16
    x, tid, tw = inputs(T, 1)
    want = _call(False, cfg, T, banks, x, tid, tw, device)
    p = _problem(cfg, T, tid.dtype)
    out = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device=device)
    so = torch.empty(T * cfg.top_k, dtype=torch.int64, device=device)
    ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=device)
    p13, s13, p2, s2 = banks

    def launch():
        _lib.check(L.exq_moe_int4_fused_forward_noalloc(
            ctypes.byref(p), x.data_ptr(), tid.data_ptr(), tw.data_ptr(), p13.data_ptr(),
            s13.data_ptr(), p2.data_ptr(), s2.data_ptr(), out.data_ptr(), so.data_ptr(),
            ends.data_ptr(), _lib.stream_handle(device)), "noalloc")

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch()  # warm call on the device, outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    x5, tid5, tw5 = inputs(5, 2)
    for r in range(3):
        out.fill_(float("nan"))
        so.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want[0]), f"replay {r}"
        assert torch.equal(so, want[1]) and torch.equal(ends, want[2])
        other = _call(True, cfg, 5, banks, x5, tid5, tw5, device)  # same scratch, eager
        assert not torch.isnan(other[0].float()).any()


_FRESH = r"""
import ctypes, sys
import numpy as np, torch
sys.path.insert(0, sys.argv[1])
from exq_amd import _lib, synth
from exq_amd.kernels import pack_experts_int4
dev = torch.device("cuda:0")
cfg = synth.MoeConfig("na_fresh", 35, 512, 256, 16, 4, True)
w13, w2 = synth.expert_weights_gpu(16, 256, 512, 92, dev)
p13, s13 = pack_experts_int4(w13)
p2, s2 = pack_experts_int4(w2)
T = 8
ids, w = synth.routing(cfg, T, 3)
x = torch.from_numpy(synth.hidden_np(T, 512, 4)).to(torch.bfloat16).to(dev)
tid = torch.from_numpy(ids.astype(np.int32)).to(dev)
tw = torch.from_numpy(w).to(dev)
L = _lib.lib()
def prob(n):
    return _lib.MoeProblem(n_tokens=n, hidden_size=512, inter_size=256, n_experts=16, top_k=4,
                           n_shared=0, group_size=128, act_dtype=_lib.BF16, ids_dtype=_lib.I32,
                           weights_dtype=_lib.F32)
p = prob(T)
out = torch.empty(T, 512, dtype=torch.bfloat16, device=dev)
so = torch.empty(T * 4, dtype=torch.int64, device=dev)
ends = torch.empty(17, dtype=torch.int32, device=dev)
args = [x.data_ptr(), tid.data_ptr(), tw.data_ptr(), p13.data_ptr(), s13.data_ptr(),
        p2.data_ptr(), s2.data_ptr(), out.data_ptr(), so.data_ptr(), ends.data_ptr()]
ws = torch.zeros(L.exq_moe_workspace_size(ctypes.byref(p)), dtype=torch.uint8, device=dev)
want = torch.empty_like(out)
_lib.check(L.exq_moe_int4_fused_forward(ctypes.byref(p), *args[:7], want.data_ptr(), *args[8:],
                                        ws.data_ptr(), ws.numel(), _lib.stream_handle(dev)), "ws")
torch.cuda.synchronize()
# the first no-alloc call of this process, under capture: refused, nothing launched
g0 = torch.cuda.CUDAGraph()
with torch.cuda.graph(g0):
    out.zero_()
    st = L.exq_moe_int4_fused_forward_noalloc(ctypes.byref(p), *args, _lib.stream_handle(dev))
    msg = L.exq_last_error()
assert st == 2 and b"outside capture" in msg, (st, msg)
# an empty call outside capture prepares the device; then capture and replay
e = prob(0)
assert L.exq_moe_int4_fused_forward_noalloc(ctypes.byref(e), *([None] * 10),
                                            _lib.stream_handle(dev)) == 0
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    _lib.check(L.exq_moe_int4_fused_forward_noalloc(ctypes.byref(p), *args,
                                                    _lib.stream_handle(dev)), "captured")
for r in range(3):
    out.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), r
print("FRESH_OK", flush=True)
"""


def test_noalloc_first_call_under_capture_in_fresh_process(device, tmp_path):
    """In a process that has not called it yet, a first call made under graph
    capture is refused with a clear error and launches nothing; one empty call
    outside capture prepares the device, and the captured call then replays
    bitwise equal to the workspace entry point."""
    import os
    import subprocess
    import sys
    banner("noalloc first call under capture (fresh process)")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FRESH, root], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0 and "FRESH_OK" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]

"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU tests: the oracle still reproduces the frozen fixtures bit-for-bit.
GPU tests: the HIP path against the same fixtures -- routing, packing and
INT8 quantisation bit-exact; the layer within 0.5 % relative L2 error.
"""
import os

import numpy as np
import pytest

from oracle import moe, quant, routing

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 5e-3


def _load(name):
    with np.load(os.path.join(GOLD, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_tiny_layer_fixture():
    g = _load("tiny_layer.npz")
    p, s = quant.pack_experts_int4(g["w13_src"])
    assert np.array_equal(p, g["w13_packed"][:, :16]) and np.array_equal(s, g["w13_scales"][:, :16])
    E = g["w13_packed"].shape[0]
    so, ends, max_tok = routing.sort_tokens_by_expert(g["topk_ids"], E)
    assert np.array_equal(so, g["sort_order"]) and np.array_equal(ends, g["expert_ends"])
    assert max_tok == int(g["max_tok"][0])
    a = routing.moe_align_block_size(g["topk_ids"], E + 1, 16)
    for got, key in zip(a, ("align_sorted_ids", "align_expert_ids", "align_ntpp", "align_cumsum")):
        assert np.array_equal(got, g[key]), key
    T, k = g["topk_ids"].shape
    e2, so2 = routing.build_ends_from_slots(g["align_sorted_ids"], g["topk_ids"].reshape(-1), T * k, E)
    assert np.array_equal(e2, g["slots_expert_ends"]) and np.array_equal(so2, g["slots_sort_order"])
    y = moe.moe_layer(g["hidden"], quant.dequant_int4(g["w13_packed"], g["w13_scales"]),
                      quant.dequant_int4(g["w2_packed"], g["w2_scales"]), g["topk_ids"],
                      g["topk_weights"], accum=np.float64)
    assert np.array_equal(y, g["out"])


def test_oracle_reproduces_pack_fixture():
    g = _load("pack_cases.npz")
    p, s = quant.pack_int4_weights(g["w"])
    assert np.array_equal(p, g["packed"]) and np.array_equal(s, g["scales"])
    q, s8 = quant.quantize_int8(g["w_int8"])
    assert np.array_equal(q, g["q_int8"]) and np.array_equal(s8, g["s_int8"])
    # the zero row packs to nibble 8 with the fp32-eps scale stored as fp16
    assert np.all(g["packed"][2] == 0x88)
    assert np.all(g["scales"][2] == np.float16(np.finfo(np.float32).eps))


@pytest.mark.gpu
def test_gpu_tiny_layer_against_fixture(device):
    import torch
    from exq_amd.kernels import exq_dispatch, fused_experts, pack_experts_int4
    from tests._helpers import assert_close_rel, banner
    g = _load("tiny_layer.npz")
    banner("golden tiny layer")
    dev = device
    T, k = g["topk_ids"].shape
    E = g["w13_packed"].shape[0]
    H = g["hidden"].shape[1]
    p, s = pack_experts_int4(torch.from_numpy(g["w13_src"]).to(dev))
    assert np.array_equal(p.cpu().numpy(), g["w13_packed"][:, :16])
    assert np.array_equal(s.cpu().numpy(), g["w13_scales"][:, :16])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    x = t(g["hidden"]).to(torch.bfloat16)
    ids, wts = t(g["topk_ids"]), t(g["topk_weights"])
    so = torch.empty(T * k, dtype=torch.int64, device=dev)
    ends = torch.empty(E + 1, dtype=torch.int32, device=dev)
    out = fused_experts(x, t(g["w13_packed"]), t(g["w13_scales"]), t(g["w2_packed"]),
                        t(g["w2_scales"]), wts, ids, sort_order_out=so, expert_ends_out=ends)
    torch.cuda.synchronize()
    assert np.array_equal(so.cpu().numpy(), g["sort_order"])
    assert np.array_equal(ends.cpu().numpy(), g["expert_ends"])
    assert_close_rel(out, g["out"], TOL, "golden tiny layer")
    # the block-padded layout + boundaries against the fixture
    cap = T * k + (E + 1) * 15
    sid = torch.empty(cap, dtype=torch.int32, device=dev)
    eblk = torch.empty(-(-cap // 16), dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    cs = torch.empty(E + 2, dtype=torch.int32, device=dev)
    exq_dispatch.moe_align_block_size(ids, E + 1, 16, sid, eblk, ntpp, cs, True)
    e2 = torch.empty(E + 1, dtype=torch.int32, device=dev)
    so2 = torch.empty(T * k, dtype=torch.int64, device=dev)
    exq_dispatch.build_ends_from_slots(sid, ids.reshape(-1).to(torch.int32), e2, so2, T * k, E)
    torch.cuda.synchronize()
    assert np.array_equal(sid.cpu().numpy(), g["align_sorted_ids"])
    assert np.array_equal(eblk.cpu().numpy(), g["align_expert_ids"])
    assert np.array_equal(ntpp.cpu().numpy(), g["align_ntpp"])
    assert np.array_equal(cs.cpu().numpy()[:E + 2], g["align_cumsum"])
    assert np.array_equal(e2.cpu().numpy(), g["slots_expert_ends"])
    assert np.array_equal(so2.cpu().numpy(), g["slots_sort_order"])
    del H


@pytest.mark.gpu
def test_gpu_pack_fixture(device):
    import torch
    from exq_amd.kernels import pack_int4_weights, quantize_int8_rows
    from tests._helpers import banner
    g = _load("pack_cases.npz")
    banner("golden pack cases")
    p, s = pack_int4_weights(torch.from_numpy(g["w"]).to(device))
    assert np.array_equal(p.cpu().numpy(), g["packed"]) and np.array_equal(s.cpu().numpy(), g["scales"])
    q, s8 = quantize_int8_rows(torch.from_numpy(g["w_int8"]).to(device))
    assert np.array_equal(q.cpu().numpy(), g["q_int8"]) and np.array_equal(s8.cpu().numpy(), g["s_int8"])

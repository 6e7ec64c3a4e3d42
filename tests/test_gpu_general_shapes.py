"""INT4 shapes outside the 128-multiples: group sizes 32 and 64, a group of
192, contraction lengths below 128 (one group = K, the reference's collapse at
moe_int4_kernel.py:61-64), and weight-row counts that are not multiples of 32
(the reference masks the N tail, moe_int4_kernel.py:206-207, 238-240).  Each
runs the general HIP kernels and is checked against the fp32
dequantise-then-matmul oracle; routing arrays bit-exact."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import moe, quant, routing
from tests._helpers import assert_close_rel, banner, oracle_int4_layer

pytestmark = pytest.mark.gpu

TOL = 5e-3


def _bank(E, N, K, g, seed, device):
    from exq_amd.kernels import pack_experts_int4
    gen = torch.Generator(device="cpu").manual_seed(seed)
    w = (torch.randn(E, N, K, generator=gen) * 0.02).to(torch.float16).to(device)
    return pack_experts_int4(w, g)


@pytest.mark.parametrize("K,N,g", [(256, 96, 32), (256, 100, 64), (96, 40, 128), (384, 72, 192),
                                   (64, 17, 32)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_moe_int4_forward_general_shapes(K, N, g, dtype, device):
    from exq_amd.kernels import moe_int4_forward
    banner(f"moe_int4_forward K={K} N={N} g={g} {dtype}")
    E, T, k = 6, 37, 2
    p, s = _bank(E, N, K, g, K + N, device)
    g_eff = min(g, K)
    assert s.shape == (E, N, K // g_eff)
    rng = np.random.default_rng(K * 7 + N)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int64)
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(dtype).to(device)
    out = moe_int4_forward(x, p, s, torch.from_numpy(ids).to(device), E)
    assert out.shape == (T * k, N) and out.dtype == dtype
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, E)
    a = moe.gather_hidden(x.float().cpu().numpy(), r_so, k)
    ref = moe.grouped_gemm_sorted(a, quant.dequant_int4(p.cpu().numpy(), s.cpu().numpy()), r_ends)
    assert_close_rel(out, ref, TOL, f"moe_int4_forward K={K} N={N} g={g_eff} {dtype}")


@pytest.mark.parametrize("H,I,g", [(256, 192, 64), (96, 64, 32), (384, 192, 192), (160, 96, 32)])
@pytest.mark.parametrize("T", [1, 5, 80])
def test_fused_general_shapes(H, I, g, T, device):
    from exq_amd.kernels import fused_experts
    banner(f"fused H={H} I={I} g={g} T={T}")
    E, k = 8, 2
    p13, s13 = _bank(E, 2 * I, H, g, H + I, device)
    p2, s2 = _bank(E, H, I, g, H + I + 1, device)
    cfg = synth.MoeConfig("gen", 41, H, I, E, k, True)
    ids, w = synth.routing(cfg, T, 0)
    tid = torch.from_numpy(ids).to(device)
    tw = torch.from_numpy(w).to(device)
    x = torch.from_numpy(synth.hidden_np(T, H, 3)).to(torch.bfloat16).to(device)
    so = torch.empty(T * k, dtype=torch.int64, device=device)
    ends = torch.empty(E + 1, dtype=torch.int32, device=device)
    out = fused_experts(x, p13, s13, p2, s2, tw, tid, sort_order_out=so, expert_ends_out=ends)
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, E)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"fused general H={H} I={I} g={g} T={T}")
    # repeatable bit for bit, and fp16 activations
    assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid), out)
    out16 = fused_experts(x.to(torch.float16), p13, s13, p2, s2, tw, tid)
    assert out16.dtype == torch.float16
    assert_close_rel(out16, ref, TOL, f"fused general fp16 H={H} I={I} g={g} T={T}")


def test_general_shape_rejections(device):
    from exq_amd import _lib
    from exq_amd.kernels import MixedExpertBank, fused_experts, fused_experts_mixed, \
        moe_int4_forward
    E, T, k = 4, 3, 2
    ids = torch.tensor([[0, 1], [2, 3], [1, 0]], device=device)
    # group size 16 is below the reference's minimum of 32 (moe_int4_kernel.py:286-290)
    p, s = _bank(E, 64, 64, 16, 1, device)
    x = torch.randn(T, 64, device=device).to(torch.bfloat16)
    with pytest.raises(ValueError, match="group_size"):
        moe_int4_forward(x, p, s, ids, E)
    p13, s13 = _bank(E, 128, 64, 16, 2, device)
    p2, s2 = _bank(E, 64, 64, 16, 3, device)
    with pytest.raises(ValueError, match="group_size"):
        fused_experts(x, p13, s13, p2, s2, torch.ones(T, k, device=device), ids)
    # mixed-precision banks keep the 128-multiple shapes
    w13 = torch.randn(E, 2 * 96, 96, device=device) * 0.02
    w2 = torch.randn(E, 96, 96, device=device) * 0.02
    bank = MixedExpertBank.from_weights(w13, w2, [2, 1, 0, 2], group_size=32)
    xb = torch.randn(T, 96, device=device).to(torch.bfloat16)
    with pytest.raises(_lib.ExqError, match="mixed-precision banks need"):
        fused_experts_mixed(xb, bank, torch.ones(T, k, device=device), ids)

"""The GPU router (fp32 softmax -> top-k -> optional renormalisation) vs the
oracle restatement: expert ids bit-exact (descending rounded fp32 softmax,
equal probabilities to the lower id, also where the logits differ), weights
within 2e-6 relative in fp32 (the kernel's exp and sum order differ from
numpy's in the last bits) and within bf16 / fp16 rounding otherwise.  Covers every config's expert count, E up to 1024, k up to 16,
all logit / id / weight dtypes, exact ties, masked (-inf) experts, T = 0 and
a large T."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import routing
from tests._helpers import banner

pytestmark = pytest.mark.gpu


def _check(logits_t, k, renorm, ids_dtype=torch.int32, w_dtype=torch.float32, rtol=2e-6):
    from exq_amd.kernels import fused_topk
    w, ids = fused_topk(logits_t.cuda(), k, renorm, ids_dtype=ids_dtype, weights_dtype=w_dtype)
    torch.cuda.synchronize()
    r_ids, r_w = routing.route_softmax_topk(logits_t.float().numpy(), k, renorm)
    assert ids.dtype == ids_dtype and w.dtype == w_dtype
    assert np.array_equal(ids.cpu().numpy().astype(np.int64), r_ids)
    got = w.float().cpu().numpy()
    ref = r_w if w_dtype == torch.float32 else torch.from_numpy(r_w).to(w_dtype).float().numpy()
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=1e-30)


@pytest.mark.parametrize("name", ["olmoe", "qwen3", "deepseek_v2_lite", "mixtral"])
@pytest.mark.parametrize("T", [1, 16, 64, 333])
def test_router_configs(name, T, device):
    cfg = synth.CONFIGS[name]
    banner(f"router {name} T={T}")
    logits = synth.router_logits(cfg, T, synth.seed_for(cfg) + 7)
    _check(torch.from_numpy(logits), cfg.top_k, cfg.renormalize)
    # the synthetic routing of the tests is exactly this router
    ids, w = synth.routing(cfg, T)
    from exq_amd.kernels import fused_topk
    gw, gids = fused_topk(torch.from_numpy(logits).cuda(), cfg.top_k, cfg.renormalize,
                          ids_dtype=torch.int64)
    assert np.array_equal(gids.cpu().numpy(), ids)


@pytest.mark.parametrize("E,k", [(8, 1), (60, 6), (256, 16), (257, 8), (1000, 16), (1024, 64)])
@pytest.mark.parametrize("renorm", [True, False])
def test_router_shapes(E, k, renorm, device):
    banner(f"router E={E} k={k} renorm={renorm}")
    rng = np.random.default_rng(E * 100 + k)
    logits = (rng.standard_normal((37, E)) * 2.0).astype(np.float32)
    _check(torch.from_numpy(logits), k, renorm, ids_dtype=torch.int64)


@pytest.mark.parametrize("ldt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16, torch.float16])
def test_router_dtypes_and_ties(ldt, wdt, device):
    """Half-precision logits have many exact ties: the lower id must win."""
    banner(f"router logits {ldt} weights {wdt}")
    rng = np.random.default_rng(7)
    logits = torch.from_numpy(rng.standard_normal((50, 64)).astype(np.float32)).to(ldt)
    logits[3] = 0.0                       # every expert tied: ids 0..k-1
    logits[4, 10:20] = 5.0                # a tied block at the top
    logits[5] = -1.0                      # +0 and -0 compare equal: a tie, lower ids first
    logits[5, 20:30:2] = 0.0
    logits[5, 21:31:2] = -0.0
    rtol = 2e-6 if wdt == torch.float32 else 1e-2
    _check(logits, 8, True, w_dtype=wdt, rtol=rtol)
    _check(logits, 8, False, w_dtype=wdt, rtol=rtol)
    from exq_amd.kernels import fused_topk
    _, ids = fused_topk(logits.cuda(), 8, False)
    assert ids[3].tolist() == list(range(8))
    assert ids[4].tolist() == list(range(10, 18))
    assert ids[5].tolist() == list(range(20, 28))


def test_router_masked_experts_and_edges(device):
    """-inf logits (masked experts) get weight 0 and are chosen only after
    every finite one; an empty batch launches nothing; 20k tokens cover a
    large grid."""
    from exq_amd.kernels import fused_topk
    banner("router masked / edges")
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((9, 16)).astype(np.float32)
    logits[:, 5:] = -np.inf               # only 5 finite experts, k = 8
    w, ids = fused_topk(torch.from_numpy(logits).cuda(), 8, False, ids_dtype=torch.int64)
    r_ids, r_w = routing.route_softmax_topk(logits, 8, False)
    assert np.array_equal(ids.cpu().numpy(), r_ids)
    assert np.all(w.cpu().numpy()[:, 5:] == 0)
    np.testing.assert_allclose(w.cpu().numpy(), r_w, rtol=2e-6, atol=1e-30)
    w0, ids0 = fused_topk(torch.zeros(0, 16, device="cuda"), 4, True)
    assert w0.shape == (0, 4) and ids0.shape == (0, 4)
    big = rng.standard_normal((20000, 128)).astype(np.float32)
    _check(torch.from_numpy(big), 8, True)


def test_router_rounded_softmax_ties(device):
    """The ranking is on the rounded fp32 softmax (torch.topk over F.softmax,
    triton_emitter.py:273-277): two different logits whose probabilities are
    bit-equal are a tie, and the lower id goes first, inside the top k and at
    its last place.  Ranking on the logits would give [0, 2, 1] and [0, 2]."""
    from exq_amd.kernels import fused_topk
    from tests.test_oracle_routing import _rounded_softmax_tie_rows
    banner("router rounded-softmax ties")
    a_row, b_row, wide = _rounded_softmax_tie_rows()
    small = torch.from_numpy(np.stack([a_row, b_row]))
    for k, want in ((3, [[0, 1, 2], [0, 1, 2]]), (2, [[0, 1], [0, 1]])):
        _, ids = fused_topk(small.cuda(), k, False, ids_dtype=torch.int64)
        assert ids.cpu().tolist() == want
        _check(small, k, False)
        _check(small, k, True)
    big = torch.from_numpy(np.stack([wide] * 5))
    _, ids = fused_topk(big.cuda(), 8, False, ids_dtype=torch.int64)
    assert ids.cpu().tolist() == [[63, 50, 51, 52, 53, 54, 55, 9]] * 5
    _check(big, 8, False)
    _check(big, 8, True)

"""The fused INT4 MoE layer on the GPU vs the fp32 dequantise-then-matmul
oracle.  Tolerance: relative L2 error <= 0.5% (the path's stated bound);
routing outputs bit-exact."""
import numpy as np
import pytest
import torch

from exq_amd import synth
from oracle import quant, routing
from tests._helpers import assert_close_rel, banner, oracle_int4_layer

pytestmark = pytest.mark.gpu

TOL = 5e-3


def _pack_gpu(E, I, H, seed, device):
    from exq_amd.kernels import pack_experts_int4
    w13, w2 = synth.expert_weights_gpu(E, I, H, seed, device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    del w13, w2
    return p13, s13, p2, s2


def _routing(cfg, T, device, ids_dtype=torch.int64, w_dtype=torch.float32, layer=0):
    ids, w = synth.routing(cfg, T, layer)
    return ids, w, torch.from_numpy(ids).to(ids_dtype).to(device), \
        torch.from_numpy(w).to(w_dtype).to(device)


def _hidden(T, H, seed, device, dtype=torch.bfloat16):
    return torch.from_numpy(synth.hidden_np(T, H, seed)).to(dtype).to(device)


def test_pack_on_gpu_bit_exact(device):
    from exq_amd.kernels import pack_experts_int4
    banner("pack_experts_int4 on GPU")
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((4, 256, 1024)) * 0.02).astype(np.float16)
    w[0, 3] = 0
    w[1, 7, :128] = 0
    p, s = pack_experts_int4(torch.from_numpy(w).to(device))
    rp, rs = quant.pack_experts_int4(w)
    assert np.array_equal(p.cpu().numpy(), rp)
    assert np.array_equal(s.cpu().numpy(), rs)
    # K < g collapses to g = K = 96 (serial kernel); bf16 and f32 inputs
    for arr, tdt in [(w[:, :8, :96], torch.float16), (w[:, :8, :512], torch.bfloat16),
                     (w[:, :8, :256], torch.float32)]:
        t = torch.from_numpy(arr.astype(np.float32)).to(tdt)
        p, s = pack_experts_int4(t.to(device))
        rp, rs = quant.pack_experts_int4(t.float().numpy())
        assert np.array_equal(p.cpu().numpy(), rp) and np.array_equal(s.cpu().numpy(), rs)


def test_quantize_int8_on_gpu_bit_exact(device):
    from exq_amd.kernels import quantize_int8_rows
    banner("quantize_int8_rows on GPU")
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((3, 64, 1000)) * 0.02).astype(np.float16)
    w[2, 5] = 0
    q, s = quantize_int8_rows(torch.from_numpy(w).to(device))
    rq, rs = quant.quantize_int8(w)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)


SMALL = synth.MoeConfig("small", 9, 256, 128, 4, 2, False)
MID = synth.MoeConfig("mid", 8, 512, 256, 16, 4, True)


@pytest.mark.parametrize("cfg,T", [(SMALL, 1), (SMALL, 3), (SMALL, 40), (MID, 16),
                                   (MID, 100), (MID, 257)])
def test_fused_small_shapes(cfg, T, device):
    from exq_amd.kernels import fused_experts
    banner(f"fused {cfg.name} T={T}")
    p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 5 + T, device)
    ids, w, tid, tw = _routing(cfg, T, device)
    x = _hidden(T, cfg.hidden, 17 + T, device)
    so = torch.empty(T * cfg.top_k, dtype=torch.int64, device=device)
    ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=device)
    out = fused_experts(x, p13, s13, p2, s2, tw, tid, sort_order_out=so, expert_ends_out=ends)
    torch.cuda.synchronize()
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, cfg.n_experts)
    assert np.array_equal(so.cpu().numpy(), r_so)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"{cfg.name} T={T}")


@pytest.mark.parametrize("T", [1, 4, 16, 64])
def test_fused_qwen3_shape(T, device):
    from exq_amd.kernels import fused_experts
    cfg = synth.CONFIGS["qwen3"]
    banner(f"fused qwen3 T={T}")
    p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, synth.seed_for(cfg), device)
    ids, w, tid, tw = _routing(cfg, T, device)
    x = _hidden(T, cfg.hidden, 100 + T, device)
    out = fused_experts(x, p13, s13, p2, s2, tw, tid)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"qwen3 T={T}")


def test_fused_olmoe_shape_determinism_and_dtypes(device):
    from exq_amd.kernels import fused_experts
    cfg = synth.CONFIGS["olmoe"]
    T = 16
    banner("fused olmoe T=16")
    p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, synth.seed_for(cfg), device)
    ids, w, tid, tw = _routing(cfg, T, device)
    x = _hidden(T, cfg.hidden, 1, device)
    out = fused_experts(x, p13, s13, p2, s2, tw, tid)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, "olmoe T=16 bf16")
    # bitwise repeatable (no atomics in any accumulation order)
    for _ in range(3):
        assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid), out)
    # int32 ids and bf16 routing weights give the same result
    out2 = fused_experts(x, p13, s13, p2, s2, tw.to(torch.bfloat16), tid.to(torch.int32))
    ref2 = oracle_int4_layer(x, p13, s13, p2, s2, ids, tw.to(torch.bfloat16).float().cpu().numpy())
    assert_close_rel(out2, ref2, TOL, "olmoe T=16 i32 ids, bf16 weights")
    # fp16 activations use the f16 MFMA path
    xh = x.to(torch.float16)
    out3 = fused_experts(xh, p13, s13, p2, s2, tw, tid)
    assert out3.dtype == torch.float16
    ref3 = oracle_int4_layer(xh, p13, s13, p2, s2, ids, w)
    assert_close_rel(out3, ref3, TOL, "olmoe T=16 fp16")


def test_workspace_contents_do_not_matter(device):
    """A caller workspace needs no zero fill: every call's first kernel clears
    the combine counters, so 0xFF bytes or random bytes (counters at -1 or at
    values that would trigger an early combine) give the same bits."""
    from exq_amd.kernels import fused_experts
    from exq_amd.kernels.fused_moe import moe_workspace_bytes
    gen = torch.Generator(device="cpu").manual_seed(3)
    # Qwen3 at 1 / 16 / 64 tokens (the rows kernels at one token, the tiled
    # kernels with the in-kernel combine at 16 and the combine launch at 64), and
    # a top-2 layer at one token (k < 4: the tiled gate/up and tiled down kernels,
    # the down kernel's in-kernel combine)
    top2 = synth.MoeConfig("top2", 34, 1024, 512, 8, 2, True, zipf=False)
    for cfg, Ts in ((synth.CONFIGS["qwen3"], (1, 16, 64)), (top2, (1,))):
        p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, synth.seed_for(cfg),
                                     device)
        for T in Ts:
            banner(f"dirty workspace {cfg.name} T={T}")
            ids, w, tid, tw = _routing(cfg, T, device)
            x = _hidden(T, cfg.hidden, 2, device)
            nbytes = moe_workspace_bytes(T, cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k)
            clean = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            want = fused_experts(x, p13, s13, p2, s2, tw, tid, workspace=clean)
            if cfg is top2:
                assert_close_rel(want, oracle_int4_layer(x, p13, s13, p2, s2, ids, w), TOL,
                                 f"top-2 T={T}")
            ones = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=device)
            rnd = torch.randint(0, 256, (nbytes,), generator=gen, dtype=torch.uint8).to(device)
            for ws in (ones, rnd):
                assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid, workspace=ws), want)
                assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid, workspace=ws), want)


def test_fused_dropped_ids_and_edges(device):
    from exq_amd.kernels import fused_experts
    cfg = MID
    banner("fused dropped ids / empty")
    p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 77, device)
    ids, w, tid, tw = _routing(cfg, 9, device)
    ids = ids.copy()
    ids[0, 1] = -1
    ids[3, :] = -1
    ids[5, 2] = cfg.n_experts + 3  # out of range is dropped too
    tid = torch.from_numpy(ids).to(device)
    x = _hidden(9, cfg.hidden, 3, device)
    out = fused_experts(x, p13, s13, p2, s2, tw, tid)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, "dropped ids")
    assert torch.count_nonzero(out[3]) == 0
    # every id dropped -> zeros; empty batch -> empty output
    allbad = torch.full_like(tid, -1)
    z = fused_experts(x, p13, s13, p2, s2, tw, allbad)
    torch.cuda.synchronize()
    assert torch.count_nonzero(z) == 0
    e = fused_experts(x[:0], p13, s13, p2, s2, tw[:0], tid[:0])
    assert e.shape == (0, cfg.hidden)


def test_fused_long_contraction_multi_round(device):
    """Intermediate 14336 (112 k-blocks) exercises several staging rounds."""
    from exq_amd.kernels import fused_experts
    cfg = synth.MoeConfig("mixtral_narrow", 4, 1024, 14336, 4, 2, True, zipf=False)
    banner("fused long K")
    p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 4000, device)
    for T in (3, 40):
        ids, w, tid, tw = _routing(cfg, T, device)
        x = _hidden(T, cfg.hidden, T, device)
        out = fused_experts(x, p13, s13, p2, s2, tw, tid)
        ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
        assert_close_rel(out, ref, TOL, f"long K T={T}")


@pytest.mark.parametrize("name,H,I,E,k,T", [("olmoe_t1", 2048, 1024, 64, 8, 1),
                                             ("uneven_split", 256, 1664, 4, 1, 1),
                                             ("uneven_split_t2", 256, 1664, 4, 1, 2)])
def test_fused_down_split_contraction(name, H, I, E, k, T, device):
    """Few active experts leave the down projection short of work-groups, so
    each contraction is split over several (2 for OLMoE at T=1; 3 uneven
    splits of 13 k-blocks here) and the splits are summed in a fixed order:
    the result matches the oracle and repeats bitwise."""
    from exq_amd.kernels import fused_experts
    cfg = synth.MoeConfig(name, 31, H, I, E, k, True, zipf=False)
    banner(f"fused split {name} T={T}")
    p13, s13, p2, s2 = _pack_gpu(E, I, H, 600 + I, device)
    ids, w, tid, tw = _routing(cfg, T, device)
    for dtype in (torch.bfloat16, torch.float16):
        x = _hidden(T, H, 7 + T, device).to(dtype)
        out = fused_experts(x, p13, s13, p2, s2, tw, tid)
        ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
        assert_close_rel(out, ref, TOL, f"split {name} {dtype}")
        for _ in range(2):
            assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid), out)


@pytest.mark.parametrize("H,I,gs", [(4096, 256, 128), (2560, 256, 128), (4096, 256, 256)])
@pytest.mark.parametrize("T", [1, 5, 40])
def test_fused_chunked_gateup(H, I, gs, T, device):
    """Hidden sizes past 2048 give each wave more k-blocks than its LDS region
    holds: the gate/up unit copies its slice in chunks (4096: two full
    chunks; 2560: 4 + 1 k-blocks; group size 256 shares a scale between
    k-blocks)."""
    from exq_amd.kernels import fused_experts, pack_experts_int4
    cfg = synth.MoeConfig(f"chunk_{H}", 33, H, I, 4, 2, True, zipf=False)
    banner(f"fused chunked H={H} gs={gs} T={T}")
    w13, w2 = synth.expert_weights_gpu(4, I, H, 700 + H, device)
    p13, s13 = pack_experts_int4(w13, group_size=gs)
    p2, s2 = pack_experts_int4(w2, group_size=gs)
    ids, w, tid, tw = _routing(cfg, T, device)
    x = _hidden(T, H, 9 + T, device)
    out = fused_experts(x, p13, s13, p2, s2, tw, tid)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"chunked H={H} gs={gs} T={T}")


@pytest.mark.parametrize("T", [33, 64])
def test_fused_chunked_gateup_multi_tile(T, device):
    """Hidden size 4096 (chunked gate/up) with two experts that every token
    routes to: each expert has T rows, so its later 16-row tiles are units of
    their own in the later tile segments of both kernels."""
    from exq_amd.kernels import fused_experts, pack_experts_int4
    H, I = 4096, 256
    cfg = synth.MoeConfig("chunk_multi", 38, H, I, 2, 2, True, zipf=False)
    banner(f"fused chunked multi-tile T={T}")
    w13, w2 = synth.expert_weights_gpu(2, I, H, 720 + T, device)
    p13, s13 = pack_experts_int4(w13)
    p2, s2 = pack_experts_int4(w2)
    ids, w, tid, tw = _routing(cfg, T, device)
    assert (np.sort(ids, axis=1) == np.array([0, 1])).all()
    x = _hidden(T, H, 10 + T, device)
    out = fused_experts(x, p13, s13, p2, s2, tw, tid)
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"chunked multi-tile T={T}")
    assert torch.equal(fused_experts(x, p13, s13, p2, s2, tw, tid), out)


def test_moe_int4_forward_sorted_output(device):
    from exq_amd.kernels import moe_int4_forward, sort_tokens_by_expert
    from oracle import moe
    banner("moe_int4_forward")
    cfg = MID
    p13, s13, _, _ = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 9, device)
    ids, w, tid, tw = _routing(cfg, 33, device)
    x = _hidden(33, cfg.hidden, 2, device)
    out = moe_int4_forward(x, p13, s13, tid, cfg.n_experts)
    so, sh, ends, max_tok = sort_tokens_by_expert(tid, x, cfg.n_experts)
    r_so, r_ends, r_max = routing.sort_tokens_by_expert(ids, cfg.n_experts)
    assert np.array_equal(so.cpu().numpy(), r_so) and max_tok == r_max
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    a = moe.gather_hidden(x.float().cpu().numpy(), r_so, cfg.top_k)
    # the gathered rows are copies: bit-exact
    assert np.array_equal(sh.float().cpu().numpy(), a)
    wdq = quant.dequant_int4(p13.cpu().numpy(), s13.cpu().numpy())
    ref = moe.grouped_gemm_sorted(a, wdq, r_ends)
    assert_close_rel(out, ref, TOL, "moe_int4_forward")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_moe_grouped_gemm_unquantised(dtype, device):
    from exq_amd.kernels import moe_grouped_gemm
    from oracle import moe
    banner(f"moe_grouped_gemm {dtype}")
    rng = np.random.default_rng(3)
    E, N, K, T, k = 8, 96, 384, 21, 2
    W = torch.from_numpy((rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)).to(dtype)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(dtype)
    mask = torch.ones(E, dtype=torch.int32)
    mask[2] = 0
    out = moe_grouped_gemm(x.to(device), W.to(device), torch.from_numpy(ids).to(device), E,
                           expert_mask=mask.to(device))
    r_so, r_ends, _ = routing.sort_tokens_by_expert(ids, E)
    a = moe.gather_hidden(x.float().numpy(), r_so, k)
    Wm = W.float().numpy().copy()
    Wm[2] = 0
    ref = moe.grouped_gemm_sorted(a, Wm, r_ends)
    assert_close_rel(out, ref, TOL, f"grouped gemm {dtype}")


@pytest.mark.parametrize("T", [4, 40, 100])
def test_fused_duplicate_ids_randint_routing(T, device):
    """torch.randint routing (the reference benches' convention) can repeat an
    expert inside one token's top-k; every (token, k) slot still counts."""
    from exq_amd.kernels import fused_experts
    banner(f"fused duplicate ids T={T}")
    cfg = SMALL
    p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 31, device)
    rng = np.random.default_rng(T)
    ids = rng.integers(0, cfg.n_experts, size=(T, 8))
    w = rng.random((T, 8)).astype(np.float32)
    x = _hidden(T, cfg.hidden, 8, device)
    out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device))
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, f"duplicate ids T={T}")


def _counts_routing(counts, T, k, seed):
    """[T, k] ids in which expert j takes counts[j] slots (sum = T * k) and no
    token repeats an expert: the sorted labels fill the columns one after
    another, so an expert's run covers distinct tokens."""
    labels = np.repeat(np.arange(len(counts)), counts)
    assert labels.size == T * k and max(counts) <= T
    ids = labels.reshape(k, T).T.copy()
    rng = np.random.default_rng(seed)
    for t in range(T):
        rng.shuffle(ids[t])
    return ids


@pytest.mark.parametrize("T,k,counts", [
    (64, 4, [64, 49, 33, 17, 48, 32, 12, 1]),      # 4, 4, 3, 2, 3, 2, 1, 1 tiles
    (48, 4, [48, 47, 31, 17, 16, 15, 10, 8]),      # 3, 3, 2, 2, 1, 1, 1, 1
    (40, 2, [40, 24, 16]),                          # 3, 2, 1
])
def test_fused_multi_tile_experts(T, k, counts, device):
    """Experts with 17-64 rows: a gate/up unit of the LDS path then covers two
    to four 16-row tiles over one copy of its weight slice (pairs of waves or
    single waves per tile instead of the four-way k-split).  Shape H=2048,
    I=768 (Qwen3's), 16 experts."""
    from exq_amd.kernels import fused_experts
    banner(f"fused multi-tile experts T={T} counts={counts}")
    E, I, H = 16, 768, 2048
    p13, s13, p2, s2 = _pack_gpu(E, I, H, 41, device)
    ids = _counts_routing(counts, T, k, T)
    w = np.random.default_rng(T + 1).random((T, k)).astype(np.float32)
    x = _hidden(T, H, 9, device)
    for ids_dt in (torch.int64, torch.int32):
        out = fused_experts(x, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                            torch.from_numpy(ids).to(ids_dt).to(device))
        ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
        assert_close_rel(out, ref, TOL, f"multi-tile T={T} {ids_dt}")
    # fp16 activations
    xh = x.to(torch.float16)
    out = fused_experts(xh, p13, s13, p2, s2, torch.from_numpy(w).to(device),
                        torch.from_numpy(ids).to(device))
    assert_close_rel(out, oracle_int4_layer(xh, p13, s13, p2, s2, ids, w), TOL,
                     f"multi-tile T={T} fp16")


def test_unsort_output_inverts_grouped_gemm(device):
    """unsort_output(moe_grouped_gemm(...)) is the reference's
    pytorch_moe_reference composition (moe_grouped_gemm.py:234-290): the
    inverse of the stable sort plus the router-weighted sum over top-k."""
    from exq_amd.kernels import moe_grouped_gemm, unsort_output
    from oracle import moe
    banner("unsort_output")
    rng = np.random.default_rng(4)
    E, N, K, T, k = 6, 64, 256, 13, 3
    W = torch.from_numpy((rng.standard_normal((E, N, K)) * 0.05).astype(np.float32))
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    wts = rng.random((T, k)).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(torch.bfloat16)
    tid = torch.from_numpy(ids).to(device)
    sorted_out = moe_grouped_gemm(x.to(device), W.to(torch.bfloat16).to(device), tid, E)
    # independent of any sort: out[t] = sum_j w[t, j] * (x[t] @ W[ids[t, j]]^T)
    xf, Wf = x.float().numpy().astype(np.float64), W.to(torch.bfloat16).float().numpy()
    ref = np.zeros((T, N))
    for t in range(T):
        for j in range(k):
            ref[t] += wts[t, j] * (Wf[ids[t, j]] @ xf[t])
    for n_exp in (None, E):
        out = unsort_output(sorted_out, tid, torch.from_numpy(wts).to(device), n_exp)
        assert_close_rel(out, ref, TOL, f"unsort_output n_experts={n_exp}")


def test_moe_int4_full_forward_delegate(device):
    from exq_amd.kernels import moe_int4_full_forward
    banner("moe_int4_full_forward")
    cfg = MID
    p13, s13, p2, s2 = _pack_gpu(cfg.n_experts, cfg.inter, cfg.hidden, 12, device)
    ids, w, tid, tw = _routing(cfg, 9, device)
    x = _hidden(9, cfg.hidden, 3, device)
    out = moe_int4_full_forward(x, p13, s13, p2, s2, tid, tw, cfg.n_experts)
    assert out.shape == (9, cfg.hidden) and out.dtype == x.dtype
    ref = oracle_int4_layer(x, p13, s13, p2, s2, ids, w)
    assert_close_rel(out, ref, TOL, "moe_int4_full_forward")

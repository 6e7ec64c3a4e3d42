"""Token -> expert routing preparation restated on the CPU (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Ordering convention.  The reference's GPU path orders slots inside an expert
non-deterministically (atomic cursors, exq_dispatch.cu:160-178; sgl_kernel's
atomics).  The canonical, pinnable order is the stable argsort of
``sort_tokens_by_expert`` (moe_grouped_gemm.py:156-157): inside an expert,
slots ascend.  Every function below produces that order.
"""
from __future__ import annotations

import numpy as np


def sort_tokens_by_expert(router_indices: np.ndarray, n_experts: int):
    """Restates moe_grouped_gemm.py:139-166 (minus the hidden-state gather).

    Returns ``(sort_order int64 [T*k], expert_ends int32 [E+1], max_tok int)``.

    pinned by: brute force ``sorted(range(n), key=lambda s: (id[s], s))`` and
    bincount-by-loop on tiny inputs, plus invariants (ends monotone,
    ends[E] = T*k, ascending inside each segment) in
    tests/test_oracle_routing.py.
    """
    flat = np.asarray(router_indices).reshape(-1).astype(np.int64)
    sort_order = np.argsort(flat, kind="stable").astype(np.int64)
    counts = np.bincount(flat, minlength=n_experts)[:n_experts]
    ends = np.zeros(n_experts + 1, dtype=np.int32)
    ends[1:] = np.cumsum(counts).astype(np.int32)
    max_tok = int(counts.max()) if flat.size > 0 else 1
    return sort_order, ends, max_tok


def dispatch(router_indices: np.ndarray, n_experts: int):
    """Restates ``exq_dispatch`` (exq_dispatch.cu:99-149).

    Stable radix sort of the flat expert ids with iota values, then
    ``expert_ends[0] = 0`` and ``expert_ends[e+1]`` = inclusive count.

    Returns ``(sort_order int64, sorted_expert_ids int64, expert_ends int32)``.

    pinned by: the same brute force as sort_tokens_by_expert.
    """
    flat = np.asarray(router_indices).reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable").astype(np.int64)
    _, ends, _ = sort_tokens_by_expert(flat.reshape(-1, 1), n_experts)
    return order, flat[order], ends


def moe_align_block_size(topk_ids: np.ndarray, num_experts: int, block_size: int,
                         pad_sorted_token_ids: bool = True):
    """Block-padded expert layout (the sgl_kernel.moe_align_block_size contract).

    Call site: sglang_backend.py:102-109, which passes ``num_experts = E + 1``
    and buffers of ``T*k + (E+1)*(B-1)`` ids, ``cdiv(.., B)`` block ids and
    ``E + 2`` cumsum entries.  sgl_kernel is not vendored by the reference, so
    the layout is restated from that contract:

    * bucket b = id + 1 (bucket 0 holds ids == -1, i.e. tokens filtered out by
      expert parallelism), for b in [0, num_experts);
    * cumsum[0] = 0, cumsum[b+1] = cumsum[b] + ceil(count_b / B) * B;
    * num_tokens_post_pad = cumsum[num_experts];
    * sorted_token_ids[cumsum[b] + r] = r-th slot of bucket b (ascending);
      padding entries hold ``numel`` (only if pad_sorted_token_ids);
    * expert_ids[blk] = b - 1 for each block of bucket b, -1 past the end.

    Returns ``(sorted_token_ids, expert_ids, num_tokens_post_pad, cumsum)``
    as int32 arrays sized like the reference call site.

    pinned by: closed form above checked against brute-force block layouts on
    tiny inputs (tests/test_oracle_routing.py).  The sgl_kernel-specific
    conventions (the +1 bucket shift and the fill values) are parity
    unpinned: the package is absent and the reference pins none of them.
    """
    flat = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    numel = flat.size
    B = int(block_size)
    max_padded = numel + num_experts * (B - 1)
    sorted_ids = np.full(max_padded, numel if pad_sorted_token_ids else -1, dtype=np.int32)
    n_blocks = -(-max_padded // B)
    expert_ids = np.full(n_blocks, -1, dtype=np.int32)
    bucket = flat + 1
    counts = np.array([(bucket == b).sum() for b in range(num_experts)], dtype=np.int64)
    padded = -(-counts // B) * B
    cumsum = np.zeros(num_experts + 1, dtype=np.int32)
    cumsum[1:] = np.cumsum(padded).astype(np.int32)
    for b in range(num_experts):
        slots = np.nonzero(bucket == b)[0]
        sorted_ids[cumsum[b]:cumsum[b] + slots.size] = slots.astype(np.int32)
        for blk in range(cumsum[b] // B, cumsum[b + 1] // B):
            expert_ids[blk] = b - 1
    ntpp = np.array([cumsum[num_experts]], dtype=np.int32)
    return sorted_ids, expert_ids, ntpp, cumsum


def build_ends_from_slots(sorted_slot_ids: np.ndarray, flat_router: np.ndarray,
                          n_active: int, n_experts: int):
    """Restates ``exq_build_ends_from_slots`` (exq_dispatch.cu:83-96, 160-229).

    * valid entries are ``slot < n_active`` (padding holds n_active);
    * expert_ends[0] = 0, expert_ends[e+1] = inclusive count of valid slots
      routed to e (histogram at 83-96, CUB scan at 202-214);
    * sort_order[expert_ends[e] + r] = r-th valid slot of expert e.  The
      reference claims positions with atomic cursors (160-178), so its order
      inside an expert is arbitrary; the oracle takes order of appearance in
      ``sorted_slot_ids`` (stable), the deterministic refinement.

    pinned by: composition with moe_align_block_size reproducing
    sort_tokens_by_expert exactly, and brute force on tiny inputs.
    """
    sid = np.asarray(sorted_slot_ids).reshape(-1).astype(np.int64)
    fr = np.asarray(flat_router).reshape(-1).astype(np.int64)
    valid = sid[(sid >= 0) & (sid < n_active)]
    experts = fr[valid]
    keep = (experts >= 0) & (experts < n_experts)
    valid, experts = valid[keep], experts[keep]
    counts = np.bincount(experts, minlength=n_experts)[:n_experts]
    ends = np.zeros(n_experts + 1, dtype=np.int32)
    ends[1:] = np.cumsum(counts).astype(np.int32)
    order = np.argsort(experts, kind="stable")
    sort_order = np.zeros(n_active, dtype=np.int64)
    sort_order[:valid.size] = valid[order]
    return ends, sort_order


def route_softmax_topk(logits: np.ndarray, top_k: int, renormalize: bool):
    """Router: fp32 softmax, top-k with ties to the lower expert index.

    This is the input convention of the synthetic workloads (the reference
    benches draw ids with ``torch.randint``; SGLang's router is a softmax +
    top-k, README.md:117-128 of the reference).

    pinned by: brute-force per-row sorting with key (-p, e) on tiny inputs.
    """
    lg = np.asarray(logits, dtype=np.float32)
    m = lg.max(axis=-1, keepdims=True)
    ex = np.exp(lg - m, dtype=np.float32)
    p = (ex / ex.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :top_k]
    w = np.take_along_axis(p, order, axis=-1)
    if renormalize:
        w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return order.astype(np.int64), w.astype(np.float32)

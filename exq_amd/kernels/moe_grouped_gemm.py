"""Unquantised grouped GEMM and the canonical sort, on the HIP library.

Mirrors exq/kernels/moe_grouped_gemm.py of the reference:
``sort_tokens_by_expert`` (139-166), ``moe_grouped_gemm`` (173-227) and
``unsort_output`` (234-260), same names and positional signatures.
"""
from __future__ import annotations

import torch

from .. import _lib
from .exq_dispatch import combine, dispatch, gather_hidden


def sort_tokens_by_expert(router_indices: torch.Tensor, hidden_states: torch.Tensor,
                          n_experts: int):
    """Stable sort of rows by expert + boundary array.

    Returns ``(sort_order int64 [n_active], sorted_hidden [n_active, K],
    expert_ends int32 [E+1], max_tok int)``.  ``max_tok`` needs one
    device->host read, as in the reference (moe_grouped_gemm.py:164); the
    fused layer path never reads it.
    """
    dev = _lib.require_gpu(hidden_states)
    top_k = router_indices.shape[1]
    n_active = router_indices.shape[0] * top_k
    ids = router_indices.reshape(-1).contiguous()
    sort_order = torch.empty(n_active, dtype=torch.int64, device=dev)
    sorted_ids = torch.empty(n_active, dtype=torch.int64, device=dev)
    ends = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    dispatch(ids, sort_order, sorted_ids, ends, n_experts)
    sorted_hidden = torch.empty(n_active, hidden_states.shape[1], dtype=hidden_states.dtype,
                                device=dev)
    gather_hidden(hidden_states.contiguous(), sort_order, sorted_hidden, top_k)
    max_tok = int((ends[1:] - ends[:-1]).max().item()) if n_active > 0 else 1
    return sort_order, sorted_hidden, ends, max_tok


def moe_grouped_gemm(hidden_states: torch.Tensor, expert_weights: torch.Tensor,
                     router_indices: torch.Tensor, n_experts: int, block_m: int = 64,
                     block_n: int = 64, block_k: int = 32,
                     expert_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Sorted-token grouped GEMM with unquantised [E, N, K] weights.

    Returns ``[n_tokens * top_k, N]`` in expert-sorted order, activation
    dtype.  ``expert_mask`` (int32 [E], optional) skips experts whose entry
    is 0, the reference kernel's USE_EXPERT_MASK (moe_grouped_gemm.py:67-85);
    skipped rows are zero.
    """
    dev = _lib.require_gpu(hidden_states, expert_weights, expert_mask)
    n_tok, K = hidden_states.shape
    E, N, K2 = expert_weights.shape
    if K != K2:
        raise ValueError(f"K mismatch: hidden_states K={K}, expert_weights K={K2}")
    if expert_weights.dtype != hidden_states.dtype:
        raise ValueError("expert_weights must have the activation dtype")
    top_k = router_indices.shape[1]
    n_active = n_tok * top_k
    ids = router_indices.reshape(-1).contiguous()
    sort_order = torch.empty(n_active, dtype=torch.int64, device=dev)
    sorted_ids = torch.empty(n_active, dtype=torch.int64, device=dev)
    ends = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    dispatch(ids, sort_order, sorted_ids, ends, n_experts)
    a = torch.empty(n_active, K, dtype=hidden_states.dtype, device=dev)
    gather_hidden(hidden_states.contiguous(), sort_order, a, top_k)
    out = torch.zeros(n_active, N, dtype=hidden_states.dtype, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(dev, L.exq_moe_gemm_workspace_size(n_active, n_experts, K))
    mask = None
    if expert_mask is not None:
        mask = expert_mask.to(torch.int32).contiguous()
    _lib.check(L.exq_moe_grouped_gemm(
        a.data_ptr(), _lib.dtype_code(a.dtype), n_active, K, expert_weights.data_ptr(),
        n_experts, N, ends.data_ptr(), _lib.ptr(mask), out.data_ptr(), ws.data_ptr(),
        ws.numel(), _lib.stream_handle(dev)), "moe_grouped_gemm")
    return out


def unsort_output(sorted_output: torch.Tensor, router_indices: torch.Tensor,
                  router_weights: torch.Tensor, n_experts: int | None = None) -> torch.Tensor:
    """Undo the stable sort and take the router-weighted sum over top-k
    (the reference's unsort_output, moe_grouped_gemm.py:234-260).

    Returns ``[n_tokens, N]`` in ``sorted_output``'s dtype.  The inverse
    permutation comes from the same stable dispatch sort as
    ``moe_grouped_gemm`` (so the two compose), with no device->host read:
    ``n_experts`` bounds the ids (default 1023, the largest expert count the
    one-work-group sort takes; up to 4095 with the multi-block sort); ids in
    ``[0, n_experts)`` give exactly the reference's
    ``torch.argsort(ids, stable=True)`` order.
    """
    dev = _lib.require_gpu(sorted_output, router_indices, router_weights)
    T, k = router_indices.shape
    n = T * k
    if sorted_output.dim() != 2 or sorted_output.shape[0] != n:
        raise ValueError(f"sorted_output must be [{n}, N]")
    E = 1023 if n_experts is None else int(n_experts)
    ids = router_indices.reshape(-1).contiguous()
    sort_order = torch.empty(n, dtype=torch.int64, device=dev)
    sorted_ids = torch.empty(n, dtype=torch.int64, device=dev)
    ends = torch.empty(E + 1, dtype=torch.int32, device=dev)
    dispatch(ids, sort_order, sorted_ids, ends, E)
    result = torch.empty(T, sorted_output.shape[1], dtype=sorted_output.dtype, device=dev)
    combine(sorted_output.contiguous(), sort_order, router_weights.contiguous(), result)
    return result

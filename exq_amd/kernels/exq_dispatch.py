"""Dispatch primitives on the HIP library.

Mirrors the pybind module ``exq_dispatch_cuda`` of the reference
(exq/kernels/cuda_src/exq_dispatch.cu:312-318: ``dispatch``,
``build_ends_from_slots``, ``gather_hidden``, ``combine``; all write into
caller-allocated outputs and return ``None``) plus the two sgl_kernel entry
points the reference pipeline calls (``moe_align_block_size`` and
``silu_and_mul``, exq/runtime/sglang_backend.py:79, 108-109, 140).
"""
from __future__ import annotations

import torch

from .. import _lib


def dispatch(router_indices: torch.Tensor, sort_order: torch.Tensor,
             sorted_expert_ids: torch.Tensor, expert_ends: torch.Tensor,
             n_experts: int) -> None:
    """Stable sort of the flat expert ids (exq_dispatch.cu:99-149).

    sort_order/sorted_expert_ids: int64 [n]; expert_ends: int32 [E+1].
    """
    ids = router_indices.reshape(-1)
    if not ids.is_contiguous():
        ids = ids.contiguous()
    dev = _lib.require_gpu(ids, sort_order, sorted_expert_ids, expert_ends)
    n = ids.numel()
    if sort_order.numel() != n or sorted_expert_ids.numel() != n:
        raise ValueError("sort_order / sorted_expert_ids must have n = T*k entries")
    if expert_ends.numel() != n_experts + 1 or expert_ends.dtype != torch.int32:
        raise ValueError("expert_ends must be int32 [n_experts + 1]")
    if sort_order.dtype != torch.int64 or sorted_expert_ids.dtype != torch.int64:
        raise ValueError("sort_order and sorted_expert_ids must be int64")
    L = _lib.lib()
    _lib.check(L.exq_dispatch(ids.data_ptr(), _lib.dtype_code(ids.dtype), n, n_experts,
                              sort_order.data_ptr(), sorted_expert_ids.data_ptr(),
                              expert_ends.data_ptr(), _lib.stream_handle(dev)), "dispatch")


def build_ends_from_slots(sorted_slot_ids: torch.Tensor, flat_router: torch.Tensor,
                          expert_ends: torch.Tensor, sort_order: torch.Tensor,
                          n_active: int, n_experts: int) -> None:
    """Expert boundaries + compacted slot order (exq_dispatch.cu:181-229).

    sorted_slot_ids: int32 [EM] (from moe_align_block_size); flat_router:
    int32 [n_active]; expert_ends: int32 [E+1] (need not be zeroed);
    sort_order: int64 [n_active].
    """
    dev = _lib.require_gpu(sorted_slot_ids, flat_router, expert_ends, sort_order)
    if sorted_slot_ids.dtype != torch.int32 or flat_router.dtype != torch.int32:
        raise ValueError("sorted_slot_ids and flat_router must be int32")
    if expert_ends.dtype != torch.int32 or expert_ends.numel() != n_experts + 1:
        raise ValueError("expert_ends must be int32 [n_experts + 1]")
    if sort_order.dtype != torch.int64 or sort_order.numel() < n_active:
        raise ValueError("sort_order must be int64 with n_active entries")
    L = _lib.lib()
    _lib.check(L.exq_build_ends_from_slots(
        sorted_slot_ids.data_ptr(), sorted_slot_ids.numel(), flat_router.data_ptr(), n_active,
        n_experts, expert_ends.data_ptr(), sort_order.data_ptr(), _lib.stream_handle(dev)),
        "build_ends_from_slots")


def gather_hidden(hidden: torch.Tensor, sort_order: torch.Tensor, out: torch.Tensor,
                  top_k: int) -> None:
    """out[i] = hidden[sort_order[i] // top_k] (exq_dispatch.cu:234-260).

    Unlike the reference (fp16 only, exq_dispatch.cu:256-258) this accepts
    f32, f16 and bf16.
    """
    dev = _lib.require_gpu(hidden, sort_order, out)
    if sort_order.dtype != torch.int64:
        raise ValueError("sort_order must be int64")
    if out.dtype != hidden.dtype or out.shape != (sort_order.numel(), hidden.shape[1]):
        raise ValueError("out must be [n_active, H] with hidden's dtype")
    L = _lib.lib()
    _lib.check(L.exq_gather_hidden(hidden.data_ptr(), _lib.dtype_code(hidden.dtype),
                                   hidden.shape[0], hidden.shape[1], sort_order.data_ptr(),
                                   sort_order.numel(), top_k, out.data_ptr(),
                                   _lib.stream_handle(dev)), "gather_hidden")


def combine(down_out: torch.Tensor, sort_order: torch.Tensor, router_weights: torch.Tensor,
            result: torch.Tensor) -> None:
    """result[t] = sum_j w[t, j] * down_out[pos(t*k+j)] (exq_dispatch.cu:262-310).

    fp32 accumulation in fixed slot order (deterministic); ``result`` has
    ``down_out``'s dtype.
    """
    dev = _lib.require_gpu(down_out, sort_order, router_weights, result)
    T, k = router_weights.shape
    H = down_out.shape[1]
    if result.shape != (T, H) or result.dtype != down_out.dtype:
        raise ValueError("result must be [T, H] with down_out's dtype")
    n_active = sort_order.numel()
    L = _lib.lib()
    ws = _lib.workspace(dev, L.exq_combine_workspace_size(n_active))
    _lib.check(L.exq_combine(down_out.data_ptr(), _lib.dtype_code(down_out.dtype),
                             sort_order.data_ptr(), n_active, router_weights.data_ptr(),
                             _lib.dtype_code(router_weights.dtype), T, k, H, result.data_ptr(),
                             ws.data_ptr(), ws.numel(), _lib.stream_handle(dev)), "combine")


def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int, block_size: int,
                         sorted_token_ids: torch.Tensor, experts_ids: torch.Tensor,
                         num_tokens_post_pad: torch.Tensor, cumsum_buffer: torch.Tensor,
                         pad_sorted_token_ids: bool = True) -> None:
    """Block-padded expert layout, with sgl_kernel's positional signature.

    Called by the reference as ``(topk_ids, E + 1, 16, sorted_ids, expert_blk,
    ntpp, cumsum, True)`` (sglang_backend.py:102-109).
    """
    ids = topk_ids.reshape(-1)
    if not ids.is_contiguous():
        ids = ids.contiguous()
    dev = _lib.require_gpu(ids, sorted_token_ids, experts_ids, num_tokens_post_pad,
                           cumsum_buffer)
    for t in (sorted_token_ids, experts_ids, num_tokens_post_pad, cumsum_buffer):
        if t.dtype != torch.int32:
            raise ValueError("moe_align_block_size outputs must be int32")
    if cumsum_buffer.numel() < num_experts + 1:
        raise ValueError("cumsum_buffer needs num_experts + 1 entries")
    L = _lib.lib()
    _lib.check(L.exq_moe_align_block_size(
        ids.data_ptr(), _lib.dtype_code(ids.dtype), ids.numel(), num_experts, block_size,
        sorted_token_ids.data_ptr(), sorted_token_ids.numel(), experts_ids.data_ptr(),
        experts_ids.numel(), num_tokens_post_pad.data_ptr(), cumsum_buffer.data_ptr(),
        1 if pad_sorted_token_ids else 0, _lib.stream_handle(dev)), "moe_align_block_size")


def silu_and_mul(input: torch.Tensor, out: torch.Tensor) -> None:
    """out = silu(input[:, :I]) * input[:, I:] (gate first), fp32 math."""
    dev = _lib.require_gpu(input, out)
    rows, two_i = input.reshape(-1, input.shape[-1]).shape
    if two_i % 2 or out.numel() != rows * (two_i // 2) or out.dtype != input.dtype:
        raise ValueError("silu_and_mul: out must be [..., I] with input's dtype")
    L = _lib.lib()
    _lib.check(L.exq_silu_and_mul(input.data_ptr(), _lib.dtype_code(input.dtype), rows,
                                  two_i // 2, out.data_ptr(), _lib.stream_handle(dev)),
               "silu_and_mul")


def fused_topk(gating_output: torch.Tensor, topk: int, renormalize: bool,
               ids_dtype: torch.dtype = torch.int32,
               weights_dtype: torch.dtype = torch.float32):
    """Router on the GPU: fp32 softmax over ``gating_output`` [T, E], the top-k
    experts per token (descending, equal logits to the lower id) and their
    softmax weights, divided by their sum when ``renormalize``.

    Returns ``(topk_weights [T, k], topk_ids [T, k])`` like SGLang's
    ``fused_topk``; the reference computes the same routing with
    ``F.softmax`` + ``torch.topk`` + a division by the sum
    (exq/codegen/triton_emitter.py:273-277) and its SGLang hook consumes it as
    ``dispatch_output.topk_output`` (exq/runtime/sglang_backend.py:88-90).
    """
    if gating_output.dim() != 2:
        raise ValueError("gating_output must be [T, E]")
    g = gating_output if gating_output.is_contiguous() else gating_output.contiguous()
    dev = _lib.require_gpu(g)
    T, E = g.shape
    if not 1 <= topk <= min(E, 64):
        raise ValueError(f"topk={topk} must be in [1, min(E, 64)]")
    if E > 1024:
        raise ValueError(f"E={E} > 1024 experts is not supported")
    ids = torch.empty(T, topk, dtype=ids_dtype, device=dev)
    wts = torch.empty(T, topk, dtype=weights_dtype, device=dev)
    L = _lib.lib()
    _lib.check(L.exq_topk_softmax(g.data_ptr(), _lib.dtype_code(g.dtype), T, E, topk,
                                  1 if renormalize else 0, ids.data_ptr(),
                                  _lib.dtype_code(ids.dtype), wts.data_ptr(),
                                  _lib.dtype_code(wts.dtype), _lib.stream_handle(dev)),
               "fused_topk")
    return wts, ids

"""INT4 MoE expert GEMMs on the HIP library.

Mirrors exq/kernels/moe_int4_kernel.py of the reference: the packing
utilities (``pack_int4_weights`` 37-93, ``pack_experts_int4`` 96-119) and the
wrappers ``moe_int4_forward`` (245-327) and ``moe_int4_full_forward``
(330-426), with the same names and positional signatures.  ``block_*``
arguments are accepted for signature compatibility; tiling is chosen by the
HIP kernels.

Weight storage format (identical to the reference, so packed banks are
interchangeable):
  packed [E, N, K//2] uint8 -- low nibble = even k, high nibble = odd k,
                               each stored as q + 8 with q in [-8, 7]
  scales [E, N, K//g] fp16  -- per-(row, group) absmax / 7
"""
from __future__ import annotations

import torch

from .. import _lib
from .exq_dispatch import dispatch, gather_hidden

_EPS = torch.finfo(torch.float32).eps


def _group_rule(K: int, group_size: int) -> int:
    # K must be even; K < g collapses to one group; otherwise g must divide K.
    if K % 2 != 0:
        raise ValueError(f"K={K} must be divisible by 2 for INT4 packing")
    if K < group_size:
        group_size = K
    if K % group_size != 0:
        raise ValueError(
            f"K={K} must be divisible by group_size={group_size}. "
            f"Choose a group_size that divides K, or use group_size=K for a single group.")
    return group_size


def _pack_rows(w: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    rows, K = w.shape
    g = w.to(torch.float32).view(rows, K // group_size, group_size)
    scale = torch.clamp_min(g.abs().amax(dim=-1) / 7.0, _EPS)
    q = torch.round(g / scale.unsqueeze(-1)).clamp_(-8, 7).to(torch.int16).view(rows, K)
    q += 8
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).to(torch.uint8)
    return packed, scale.to(torch.float16)


def _pack_gpu(flat: torch.Tensor, K: int, g: int) -> tuple[torch.Tensor, torch.Tensor]:
    rows = flat.shape[0]
    dev = _lib.require_gpu(flat)
    packed = torch.empty(rows, K // 2, dtype=torch.uint8, device=dev)
    scales = torch.empty(rows, K // g, dtype=torch.float16, device=dev)
    L = _lib.lib()
    _lib.check(L.exq_pack_int4(flat.data_ptr(), _lib.dtype_code(flat.dtype), rows, K, g,
                               packed.data_ptr(), scales.data_ptr(), _lib.stream_handle(dev)),
               "pack_int4")
    return packed, scales


def pack_int4_weights(weights: torch.Tensor, group_size: int = 128
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack [N, K] weights to INT4 with per-group fp16 scales (RTN, symmetric).

    Returns ``(packed uint8 [N, K//2], scales fp16 [N, K//g])``.  Raises
    ValueError if K is odd or not divisible by the group size.  Device
    tensors are packed by the HIP kernel; host tensors with torch CPU ops
    (same arithmetic, for offline packing).
    """
    N, K = weights.shape
    g = _group_rule(K, group_size)
    if weights.is_cuda:
        return _pack_gpu(weights.contiguous(), K, g)
    packed, scales = _pack_rows(weights, g)
    return packed.contiguous(), scales.contiguous()


def pack_experts_int4(expert_weights: torch.Tensor, group_size: int = 128,
                      rows_per_chunk: int = 1 << 16) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack an [E, N, K] bank: ``(packed [E, N, K//2], scales [E, N, K//g])``.

    Device banks go through the HIP kernel in one launch; host banks are
    packed with torch CPU ops in row chunks (bounded fp32 temporaries).
    """
    E, N, K = expert_weights.shape
    g = _group_rule(K, group_size)
    flat = expert_weights.reshape(E * N, K)
    if flat.is_cuda:
        p, s = _pack_gpu(flat.contiguous(), K, g)
        return p.view(E, N, K // 2), s.view(E, N, K // g)
    packed = torch.empty(E * N, K // 2, dtype=torch.uint8, device=expert_weights.device)
    scales = torch.empty(E * N, K // g, dtype=torch.float16, device=expert_weights.device)
    for r0 in range(0, E * N, rows_per_chunk):
        r1 = min(E * N, r0 + rows_per_chunk)
        p, s = _pack_rows(flat[r0:r1], g)
        packed[r0:r1] = p
        scales[r0:r1] = s
    return packed.view(E, N, K // 2), scales.view(E, N, K // g)


def _effective_group(K: int, scales: torch.Tensor) -> int:
    """Group size implied by the scales' shape (moe_int4_kernel.py:274-277);
    below 32 is rejected as the reference does (:286-290)."""
    n_groups = scales.shape[-1]
    if n_groups <= 0 or K % n_groups:
        raise ValueError(f"scales last dim {n_groups} does not divide K={K}")
    g = K // n_groups
    if g < 32:
        raise ValueError(f"group_size={g} is too small (minimum 32): K={K} has {n_groups} "
                         "scale groups")
    return g


def moe_int4_forward(hidden_states: torch.Tensor, expert_packed: torch.Tensor,
                     expert_scales: torch.Tensor, router_indices: torch.Tensor,
                     n_experts: int, group_size: int = 128, block_m: int = 64,
                     block_n: int = 128, block_k: int = 32) -> torch.Tensor:
    """Single INT4 projection: sort rows by expert, run the grouped GEMM.

    Returns ``[n_tokens * top_k, N]`` in expert-sorted order (stable), in the
    activation dtype.  The group size is taken from the scales' shape, as in
    the reference (moe_int4_kernel.py:274-277).
    """
    dev = _lib.require_gpu(hidden_states, expert_packed, expert_scales)
    n_tok, K = hidden_states.shape
    E, N, K2 = expert_packed.shape
    if K2 * 2 != K:
        raise ValueError(f"packed K={K2} != K//2={K // 2}")
    gs = _effective_group(K, expert_scales)
    top_k = router_indices.shape[1]
    n_active = n_tok * top_k
    ids = router_indices.reshape(-1).contiguous()
    sort_order = torch.empty(n_active, dtype=torch.int64, device=dev)
    sorted_ids = torch.empty(n_active, dtype=torch.int64, device=dev)
    ends = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    dispatch(ids, sort_order, sorted_ids, ends, n_experts)
    a = torch.empty(n_active, K, dtype=hidden_states.dtype, device=dev)
    gather_hidden(hidden_states, sort_order, a, top_k)
    out = torch.empty(n_active, N, dtype=hidden_states.dtype, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(dev, L.exq_moe_gemm_workspace_size(n_active, n_experts, K))
    _lib.check(L.exq_moe_int4_gemm(
        a.data_ptr(), _lib.dtype_code(a.dtype), n_active, K, expert_packed.data_ptr(),
        expert_scales.data_ptr(), n_experts, N, gs, ends.data_ptr(), out.data_ptr(),
        ws.data_ptr(), ws.numel(), _lib.stream_handle(dev)), "moe_int4_forward")
    return out


def moe_int4_full_forward(hidden_states: torch.Tensor, w13_packed: torch.Tensor,
                          w13_scales: torch.Tensor, w2_packed: torch.Tensor,
                          w2_scales: torch.Tensor, router_indices: torch.Tensor,
                          router_weights: torch.Tensor, n_experts: int,
                          group_size: int = 128, block_m: int = 64, block_n: int = 128,
                          block_k: int = 32) -> torch.Tensor:
    """Full INT4 MoE layer: gate/up -> SiLU*up -> down -> top-k weighted sum.

    Returns ``[n_tokens, H]`` in the activation dtype.  (The reference's
    version raises NameError at moe_int4_kernel.py:424; this one runs the
    fused HIP pipeline.)
    """
    from .fused_moe import fused_experts
    return fused_experts(hidden_states, w13_packed, w13_scales, w2_packed, w2_scales,
                         router_weights, router_indices)

"""Fused MoE layer entry points on the HIP library.

``fused_experts`` is the SGLang ``fused_experts_impl(..., use_int4_w4a16=True,
block_shape=[0, 128])``-style call the reference benchmarks against
(README.md:121; scripts/bench_sglang_integration.py:138-149) over ExQ's
packed INT4 layout.  ``MixedExpertBank`` + ``fused_experts_mixed`` dispatch
BF16, INT8 and INT4 experts of one layer by the compiled quant plan in one
launch sequence (exq/kernels/exq_artifact.py:25-26 tier codes).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .. import _lib
from .moe_int4_kernel import _effective_group, pack_experts_int4

_EPS = torch.finfo(torch.float32).eps


def _problem(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
             n_experts: int, inter: int, group_size: int, n_shared: int = 0) -> _lib.MoeProblem:
    T, H = hidden.shape
    p = _lib.MoeProblem()
    p.n_tokens = T
    p.hidden_size = H
    p.inter_size = inter
    p.n_experts = n_experts
    p.top_k = topk_ids.shape[1]
    p.n_shared = n_shared
    p.group_size = group_size
    p.act_dtype = _lib.dtype_code(hidden.dtype)
    p.ids_dtype = _lib.dtype_code(topk_ids.dtype)
    p.weights_dtype = _lib.dtype_code(topk_weights.dtype)
    return p


def _check_routing(hidden, topk_weights, topk_ids):
    if hidden.dim() != 2:
        raise ValueError("hidden_states must be [T, H]")
    if (topk_ids.dim() != 2 or topk_ids.shape != topk_weights.shape
            or topk_ids.shape[0] != hidden.shape[0]):
        raise ValueError("topk_ids / topk_weights must both be [T, k]")
    if hidden.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("hidden_states must be float16 or bfloat16")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("topk_ids must be int32 or int64")
    if topk_weights.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("topk_weights must be float32, float16 or bfloat16")


def _check_outputs(hidden, topk_ids, n_experts, out, sort_order_out, expert_ends_out):
    """Caller-supplied output buffers are written through raw pointers by the
    kernels, so their sizes and dtypes are checked here, before any launch."""
    T, H = hidden.shape
    if out is not None and (tuple(out.shape) != (T, H) or out.dtype != hidden.dtype):
        raise ValueError(f"out must be [{T}, {H}] with dtype {hidden.dtype}")
    if sort_order_out is not None and (sort_order_out.dtype != torch.int64
                                       or sort_order_out.numel() != topk_ids.numel()):
        raise ValueError(f"sort_order_out must be int64 with {topk_ids.numel()} elements")
    if expert_ends_out is not None and (expert_ends_out.dtype != torch.int32
                                        or expert_ends_out.numel() != n_experts + 1):
        raise ValueError(f"expert_ends_out must be int32 with {n_experts + 1} elements")
    for t in (out, sort_order_out, expert_ends_out):
        if t is not None and not t.is_contiguous():
            raise ValueError("output buffers must be contiguous")


def fused_experts(hidden_states: torch.Tensor, w13_packed: torch.Tensor,
                  w13_scales: torch.Tensor, w2_packed: torch.Tensor,
                  w2_scales: torch.Tensor, topk_weights: torch.Tensor,
                  topk_ids: torch.Tensor, *, activation: str = "silu",
                  out: torch.Tensor | None = None,
                  sort_order_out: torch.Tensor | None = None,
                  expert_ends_out: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """INT4 MoE layer: ``out[t] = sum_j w[t,j] * down_e(silu(gate_e x) * up_e x)``.

    hidden_states [T, H] f16/bf16; w13_packed [E, 2I, H/2] u8, w13_scales
    [E, 2I, H/g] f16; w2_packed [E, H, I/2], w2_scales [E, H, I/g];
    topk_weights [T, k] f32/f16/bf16; topk_ids [T, k] i32/i64 (ids outside
    [0, E) are dropped).  Returns [T, H] in the activation dtype.  The call is
    stream-ordered and never synchronises with the host.  ``workspace`` (uint8,
    at least ``moe_workspace_bytes(...)``) replaces the per-stream cached one,
    e.g. for HIP-graph capture; any contents will do (``torch.empty``), since
    each call's first kernel clears the counters its first bytes hold, but it
    must not be shared by calls that may run concurrently.
    """
    if activation != "silu":
        raise ValueError(f"unsupported activation {activation!r} (only 'silu')")
    _check_routing(hidden_states, topk_weights, topk_ids)
    T, H = hidden_states.shape
    if w13_packed.dim() != 3 or w2_packed.dim() != 3:
        raise ValueError("packed weights must be [E, N, K/2]")
    E, two_i, h2 = w13_packed.shape
    I = two_i // 2
    if h2 * 2 != H or tuple(w2_packed.shape) != (E, H, I // 2):
        raise ValueError("packed weight shapes do not match hidden / intermediate sizes")
    if w13_packed.dtype != torch.uint8 or w2_packed.dtype != torch.uint8:
        raise ValueError("packed weights must be uint8")
    if w13_scales.dtype != torch.float16 or w2_scales.dtype != torch.float16:
        raise ValueError("INT4 scales must be float16")
    _check_outputs(hidden_states, topk_ids, E, out, sort_order_out, expert_ends_out)
    gs = _effective_group(H, w13_scales)
    if _effective_group(I, w2_scales) != gs:
        raise ValueError("w13 and w2 must use the same group size")
    if (tuple(w13_scales.shape) != (E, two_i, H // gs)
            or tuple(w2_scales.shape) != (E, H, I // gs)):
        raise ValueError("scale shapes do not match the packed weights")
    dev = _lib.require_gpu(hidden_states, w13_packed, w13_scales, w2_packed, w2_scales,
                           topk_weights, topk_ids, out, sort_order_out, expert_ends_out)
    if out is None:
        out = torch.empty(T, H, dtype=hidden_states.dtype, device=dev)
    p = _problem(hidden_states, topk_ids, topk_weights, E, I, gs)
    L = _lib.lib()
    need = L.exq_moe_workspace_size(p)
    ws = workspace if workspace is not None else _lib.workspace(dev, need, "fused")
    _lib.check(L.exq_moe_int4_fused_forward(
        p, hidden_states.data_ptr(), topk_ids.data_ptr(), topk_weights.data_ptr(),
        w13_packed.data_ptr(), w13_scales.data_ptr(), w2_packed.data_ptr(),
        w2_scales.data_ptr(), out.data_ptr(), _lib.ptr(sort_order_out),
        _lib.ptr(expert_ends_out), ws.data_ptr(), ws.numel(), _lib.stream_handle(dev)),
        "fused_experts")
    return out


def moe_workspace_bytes(n_tokens: int, hidden: int, inter: int, n_experts: int, top_k: int,
                        n_shared: int = 0, group_size: int = 128) -> int:
    """Workspace bytes the fused entry points need for this problem size."""
    p = _lib.MoeProblem(n_tokens=n_tokens, hidden_size=hidden, inter_size=inter,
                        n_experts=n_experts, top_k=top_k, n_shared=n_shared,
                        group_size=group_size, act_dtype=_lib.BF16, ids_dtype=_lib.I32,
                        weights_dtype=_lib.F32)
    return int(_lib.lib().exq_moe_workspace_size(p))


def quantize_int8_rows(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-row INT8 RTN (exq/eval/quant_shim.py:84-96 rule).

    ``w [..., N, K]`` -> ``(q int8 [..., N, K], scales fp16 [..., N])``; the
    scale is max|w|/127 in fp32 (floored at fp32 eps), stored as fp16.
    Device tensors are quantised by the HIP kernel.
    """
    if w.is_cuda:
        flat = w.reshape(-1, w.shape[-1]).contiguous()
        dev = _lib.require_gpu(flat)
        q = torch.empty(flat.shape, dtype=torch.int8, device=dev)
        s = torch.empty(flat.shape[0], dtype=torch.float16, device=dev)
        _lib.check(_lib.lib().exq_quantize_int8(
            flat.data_ptr(), _lib.dtype_code(flat.dtype), flat.shape[0], flat.shape[1],
            q.data_ptr(), s.data_ptr(), _lib.stream_handle(dev)), "quantize_int8")
        return q.view(w.shape), s.view(w.shape[:-1])
    w32 = w.to(torch.float32)
    scale = torch.clamp_min(w32.abs().amax(dim=-1, keepdim=True) / 127.0, _EPS)
    q = torch.round(w32 / scale).clamp_(-128, 127).to(torch.int8)
    return q.contiguous(), scale.squeeze(-1).to(torch.float16).contiguous()


@dataclass
class MixedExpertBank:
    """Weights of one mixed-precision MoE layer, grouped per tier.

    ``tier[e]`` (0 BF16, 1 INT8, 2 INT4) and ``index[e]`` select the bank and
    the row in it for routed expert ``e`` and, after the routed experts, for
    each always-on shared expert.
    """
    n_experts: int
    n_shared: int
    hidden_size: int
    inter_size: int
    group_size: int
    tier: torch.Tensor              # int8 [E + S]
    index: torch.Tensor             # int32 [E + S]
    bf16_w13: torch.Tensor | None = None
    bf16_w2: torch.Tensor | None = None
    int8_w13: torch.Tensor | None = None
    int8_w13_scales: torch.Tensor | None = None
    int8_w2: torch.Tensor | None = None
    int8_w2_scales: torch.Tensor | None = None
    int4_w13: torch.Tensor | None = None
    int4_w13_scales: torch.Tensor | None = None
    int4_w2: torch.Tensor | None = None
    int4_w2_scales: torch.Tensor | None = None
    _keep: list = field(default_factory=list, repr=False)

    def __post_init__(self):
        # The kernels read tier / index on the device unchecked (tier in the top
        # two bits of a 32-bit entry, the row in the other 30), so the values
        # are checked once here, when the bank is built.
        n = self.n_experts + self.n_shared
        if self.tier.numel() != n or self.index.numel() != n:
            raise ValueError(f"tier and index need {n} entries (routed + shared experts)")
        if self.tier.dtype != torch.int8 or self.index.dtype != torch.int32:
            raise ValueError("tier must be int8 and index int32")
        t = self.tier.cpu()
        i = self.index.cpu()
        if n and not bool(((t >= 0) & (t <= 2)).all()):
            raise ValueError("tier values must be 0 (BF16), 1 (INT8) or 2 (INT4)")
        if n and not bool(((i >= 0) & (i < (1 << 30))).all()):
            raise ValueError("index values must be bank rows in [0, 2^30)")

    @classmethod
    def from_weights(cls, w13: torch.Tensor, w2: torch.Tensor, tiers, *,
                     act_dtype: torch.dtype = torch.bfloat16, group_size: int = 128,
                     shared_w13: torch.Tensor | None = None,
                     shared_w2: torch.Tensor | None = None,
                     shared_tier: int = 0) -> "MixedExpertBank":
        """Quantise full-precision weights ``w13 [E, 2I, H]``, ``w2 [E, H, I]``
        per the plan ``tiers`` (sequence or tensor of 0/1/2); shared experts
        ``[S, 2I, H]`` / ``[S, H, I]`` get ``shared_tier``.
        """
        dev = w13.device
        E = w13.shape[0]
        tiers = [int(t) for t in (tiers.tolist() if torch.is_tensor(tiers) else tiers)]
        if len(tiers) != E:
            raise ValueError(f"need {E} tiers, got {len(tiers)}")
        all13, all2 = [w13], [w2]
        S = 0
        if shared_w13 is not None:
            S = shared_w13.shape[0]
            all13.append(shared_w13)
            all2.append(shared_w2)
            tiers = tiers + [int(shared_tier)] * S
        W13 = torch.cat(all13) if len(all13) > 1 else w13
        W2 = torch.cat(all2) if len(all2) > 1 else w2
        index = [0] * (E + S)
        members = {0: [], 1: [], 2: []}
        for e, t in enumerate(tiers):
            if t not in members:
                raise ValueError(f"tier {t} of expert {e} not in (0, 1, 2)")
            index[e] = len(members[t])
            members[t].append(e)
        H = w13.shape[2]
        I = w13.shape[1] // 2
        bank = cls(n_experts=E, n_shared=S, hidden_size=H, inter_size=I,
                   group_size=group_size,
                   tier=torch.tensor(tiers, dtype=torch.int8, device=dev),
                   index=torch.tensor(index, dtype=torch.int32, device=dev))
        if members[0]:
            sel = torch.tensor(members[0], device=dev)
            bank.bf16_w13 = W13[sel].to(act_dtype).contiguous()
            bank.bf16_w2 = W2[sel].to(act_dtype).contiguous()
        if members[1]:
            sel = torch.tensor(members[1], device=dev)
            bank.int8_w13, bank.int8_w13_scales = quantize_int8_rows(W13[sel])
            bank.int8_w2, bank.int8_w2_scales = quantize_int8_rows(W2[sel])
        if members[2]:
            sel = torch.tensor(members[2], device=dev)
            bank.int4_w13, bank.int4_w13_scales = pack_experts_int4(
                W13[sel].to(torch.float16), group_size)
            bank.int4_w2, bank.int4_w2_scales = pack_experts_int4(
                W2[sel].to(torch.float16), group_size)
        return bank

    def c_bank(self) -> _lib.ExpertBank:
        b = _lib.ExpertBank()
        for name in ("tier", "index", "bf16_w13", "bf16_w2", "int8_w13", "int8_w13_scales",
                     "int8_w2", "int8_w2_scales", "int4_w13", "int4_w13_scales", "int4_w2",
                     "int4_w2_scales"):
            t = getattr(self, name)
            setattr(b, name, None if t is None else t.data_ptr())
        return b

    def tensors(self) -> list[torch.Tensor]:
        return [t for t in (self.tier, self.index, self.bf16_w13, self.bf16_w2, self.int8_w13,
                            self.int8_w13_scales, self.int8_w2, self.int8_w2_scales,
                            self.int4_w13, self.int4_w13_scales, self.int4_w2,
                            self.int4_w2_scales) if t is not None]

    def stored_bytes(self, expert: int) -> int:
        """Bytes of weights + scales streamed for one expert of this bank."""
        H, I = self.hidden_size, self.inter_size
        t = int(self.tier[expert].item())
        if t == 0:
            return 3 * H * I * 2
        if t == 1:
            return 3 * H * I + (2 * I + H) * 2
        return 3 * H * I // 2 + 2 * (2 * I * H // self.group_size + H * I // self.group_size)


def fused_experts_mixed(hidden_states: torch.Tensor, bank: MixedExpertBank,
                        topk_weights: torch.Tensor, topk_ids: torch.Tensor, *,
                        out: torch.Tensor | None = None,
                        sort_order_out: torch.Tensor | None = None,
                        expert_ends_out: torch.Tensor | None = None,
                        workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Mixed BF16/INT8/INT4 MoE layer (plus shared experts) in one launch sequence."""
    _check_routing(hidden_states, topk_weights, topk_ids)
    T, H = hidden_states.shape
    if H != bank.hidden_size:
        raise ValueError("hidden size does not match the bank")
    if bank.bf16_w13 is not None and bank.bf16_w13.dtype != hidden_states.dtype:
        raise ValueError("BF16-tier weights must have the activation dtype")
    _check_outputs(hidden_states, topk_ids, bank.n_experts, out, sort_order_out,
                   expert_ends_out)
    dev = _lib.require_gpu(hidden_states, topk_weights, topk_ids, out, sort_order_out,
                           expert_ends_out, *bank.tensors())
    if out is None:
        out = torch.empty(T, H, dtype=hidden_states.dtype, device=dev)
    p = _problem(hidden_states, topk_ids, topk_weights, bank.n_experts, bank.inter_size,
                 bank.group_size, bank.n_shared)
    L = _lib.lib()
    ws = workspace if workspace is not None else _lib.workspace(
        dev, L.exq_moe_workspace_size(p), "fused")
    cb = bank.c_bank()
    _lib.check(L.exq_moe_mixed_forward(
        p, hidden_states.data_ptr(), topk_ids.data_ptr(), topk_weights.data_ptr(), cb,
        out.data_ptr(), _lib.ptr(sort_order_out), _lib.ptr(expert_ends_out), ws.data_ptr(),
        ws.numel(), _lib.stream_handle(dev)), "fused_experts_mixed")
    return out

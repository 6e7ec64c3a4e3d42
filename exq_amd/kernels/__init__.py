"""ExQ MoE expert-dispatch kernels on MI355X (hand-written HIP for gfx950).

Same public names as the reference's ``exq.kernels``
(exq/kernels/__init__.py:3-21), plus the fused and mixed-precision layer
entry points and the dispatch primitives.
"""
from .exq_artifact import ExpertProfile, load_exq_artifact
from .fused_moe import MixedExpertBank, fused_experts, fused_experts_mixed, quantize_int8_rows
from .moe_grouped_gemm import moe_grouped_gemm, sort_tokens_by_expert, unsort_output
from .moe_int4_kernel import (moe_int4_forward, moe_int4_full_forward, pack_experts_int4,
                              pack_int4_weights)
from . import exq_dispatch
from .exq_dispatch import fused_topk
from .quant_shim import quantize_tensor_int4, quantize_tensor_int8

__all__ = [
    "moe_grouped_gemm",
    "sort_tokens_by_expert",
    "unsort_output",
    "moe_int4_forward",
    "moe_int4_full_forward",
    "pack_experts_int4",
    "pack_int4_weights",
    "load_exq_artifact",
    "ExpertProfile",
    "fused_experts",
    "fused_experts_mixed",
    "MixedExpertBank",
    "quantize_int8_rows",
    "exq_dispatch",
    "fused_topk",
    "quantize_tensor_int4",
    "quantize_tensor_int8",
]

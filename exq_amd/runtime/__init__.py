"""Runtime integration of the ExQ MoE kernels (SGLang drop-in, caches)."""
from .expert_cache import ExpertWeightCache
from .pack_cache import PackedWeightCache
from .sglang_backend import ExQSGLangBackend, patch_sglang, unpatch_sglang

__all__ = ["ExQSGLangBackend", "ExpertWeightCache", "PackedWeightCache", "patch_sglang",
           "unpatch_sglang"]

"""Runtime integration of the ExQ MoE kernels (SGLang drop-in)."""
from .pack_cache import PackedWeightCache
from .sglang_backend import ExQSGLangBackend, patch_sglang, unpatch_sglang

__all__ = ["ExQSGLangBackend", "PackedWeightCache", "patch_sglang", "unpatch_sglang"]

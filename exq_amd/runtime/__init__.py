"""Runtime integration of the ExQ MoE kernels (SGLang drop-in)."""
from .sglang_backend import ExQSGLangBackend, patch_sglang, unpatch_sglang

__all__ = ["ExQSGLangBackend", "patch_sglang", "unpatch_sglang"]

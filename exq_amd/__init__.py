"""exq_amd: the ExQ MoE expert-dispatch hot path, MI355X-native.

Hand-written HIP kernels for gfx950 behind a C ABI (include/exq_hip.h,
``libexq_hip.so``), bound with ctypes.  ``exq_amd.kernels`` mirrors the
reference's ``exq.kernels`` API and ``exq_amd.runtime`` its SGLang backend.
"""
from . import _lib
from ._lib import ExqError, library_path

__version__ = "0.1.0"

__all__ = ["ExqError", "library_path", "__version__"]

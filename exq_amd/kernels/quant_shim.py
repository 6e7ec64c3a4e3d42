"""Fake quantisation on the GPU: the accuracy-simulation helpers of the
reference's exq/eval/quant_shim.py:84-125 (``quantize_tensor_int8``,
``quantize_tensor_int4``), same names and results, run by the HIP kernels of
exq_fake_quant (quantise, then dequantise back to the weights' dtype).
"""
from __future__ import annotations

import torch

from .. import _lib


def _fake(weight: torch.Tensor, bits: int, group_size: int) -> torch.Tensor:
    w = weight.contiguous()
    dev = _lib.require_gpu(w)
    if w.dim() == 0:
        # quant_shim.py:90-96 reduces a 0-dim tensor over dim -1 as one element;
        # quant_shim.py:108 indexes shape[-1], which raises for 0-dim input
        if bits == 4:
            raise IndexError("quantize_tensor_int4: a 0-dim tensor has no last dimension")
        return _fake(w.reshape(1), bits, group_size).reshape(())
    if w.numel() == 0:
        return w.clone()
    K = w.shape[-1]
    rows = w.numel() // K
    out = torch.empty_like(w)
    L = _lib.lib()
    _lib.check(L.exq_fake_quant(w.data_ptr(), _lib.dtype_code(w.dtype), rows, K, bits, group_size,
                                out.data_ptr(), _lib.stream_handle(dev)), "fake quant")
    return out


def quantize_tensor_int8(weight: torch.Tensor) -> torch.Tensor:
    """Per-output-channel (last-dim row) RTN to int8 and back, in the weight's
    dtype: scale = max|w| / 127 in fp32 floored at fp32 eps
    (exq/eval/quant_shim.py:84-96)."""
    return _fake(weight, 8, 0)


def quantize_tensor_int4(weight: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Per-group (128 along the last dim) RTN to [-8, 7] and back, in the
    weight's dtype: scale = max|w| / 7 in fp32 floored at fp32 eps; a short
    last group behaves as padded with zeros (exq/eval/quant_shim.py:99-125)."""
    return _fake(weight, 4, group_size)

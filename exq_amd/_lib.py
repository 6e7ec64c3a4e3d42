"""ctypes binding of libexq_hip.so (the C ABI declared in include/exq_hip.h).

The library is loaded lazily and must exist: there is no fallback path.  Every
call checks the returned status and raises ``ExqError`` with the library's
message on failure.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch

_LIB_PATH = Path(__file__).resolve().parent / "libexq_hip.so"
_lock = threading.Lock()
_lib = None

# exq_dtype codes
F32, F16, BF16, I32, I64, U8, I8 = range(7)
_TORCH_TO_CODE = {
    torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
    torch.int32: I32, torch.int64: I64, torch.uint8: U8, torch.int8: I8,
}

TIER_BF16, TIER_INT8, TIER_INT4 = 0, 1, 2


class ExqError(RuntimeError):
    """A libexq_hip entry point returned a non-success status."""


class MoeProblem(C.Structure):
    _fields_ = [
        ("n_tokens", C.c_int64), ("hidden_size", C.c_int64), ("inter_size", C.c_int64),
        ("n_experts", C.c_int64), ("top_k", C.c_int64), ("n_shared", C.c_int64),
        ("group_size", C.c_int64), ("act_dtype", C.c_int), ("ids_dtype", C.c_int),
        ("weights_dtype", C.c_int),
    ]


class ExpertBank(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "tier", "index", "bf16_w13", "bf16_w2", "int8_w13", "int8_w13_scales", "int8_w2",
        "int8_w2_scales", "int4_w13", "int4_w13_scales", "int4_w2", "int4_w2_scales")]


_P, _I64, _INT, _SZ = C.c_void_p, C.c_int64, C.c_int, C.c_size_t

_SIGNATURES = {
    "exq_abi_version": ([], _INT),
    "exq_last_error": ([], C.c_char_p),
    "exq_status_name": ([_INT], C.c_char_p),
    "exq_moe_align_block_size": ([_P, _INT, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P, _INT, _P], _INT),
    "exq_topk_softmax": ([_P, _INT, _I64, _I64, _I64, _INT, _P, _INT, _P, _INT, _P], _INT),
    "exq_build_ends_from_slots": ([_P, _I64, _P, _I64, _I64, _P, _P, _P], _INT),
    "exq_dispatch": ([_P, _INT, _I64, _I64, _P, _P, _P, _P], _INT),
    "exq_gather_hidden": ([_P, _INT, _I64, _I64, _P, _I64, _I64, _P, _P], _INT),
    "exq_combine_workspace_size": ([_I64], _SZ),
    "exq_combine": ([_P, _INT, _P, _I64, _P, _INT, _I64, _I64, _I64, _P, _P, _SZ, _P], _INT),
    "exq_silu_and_mul": ([_P, _INT, _I64, _I64, _P, _P], _INT),
    "exq_moe_gemm_workspace_size": ([_I64, _I64, _I64], _SZ),
    "exq_moe_int4_gemm": ([_P, _INT, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _P, _P, _SZ, _P], _INT),
    "exq_moe_grouped_gemm": ([_P, _INT, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _SZ, _P], _INT),
    "exq_moe_workspace_size": ([C.POINTER(MoeProblem)], _SZ),
    "exq_moe_int4_fused_forward": ([C.POINTER(MoeProblem), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P], _INT),
    "exq_moe_mixed_forward": ([C.POINTER(MoeProblem), _P, _P, _P, C.POINTER(ExpertBank), _P, _P, _P, _P, _SZ, _P], _INT),
    "exq_moe_int4_fused_forward_noalloc": ([C.POINTER(MoeProblem), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P], _INT),
    "exq_set_stage_events": ([C.POINTER(C.c_void_p), _INT], _INT),
    "exq_pack_int4": ([_P, _INT, _I64, _I64, _I64, _P, _P, _P], _INT),
    "exq_quantize_int8": ([_P, _INT, _I64, _I64, _P, _P, _P], _INT),
    "exq_fake_quant": ([_P, _INT, _I64, _I64, _INT, _I64, _P, _P], _INT),
    "exq_stream_read": ([_P, _I64, _P, _I64, _P], _INT),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def library_path() -> Path:
    return _LIB_PATH


def lib():
    """Load (once) and return the ctypes handle; raise if the library is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not _LIB_PATH.exists():
                raise ExqError(
                    f"{_LIB_PATH} is missing: build it with `python -m exq_amd.build` "
                    "(or __graft_entry__.build()); exq_amd has no fallback path")
            h = C.CDLL(str(_LIB_PATH))
            for name, (args, res) in _SIGNATURES.items():
                fn = getattr(h, name)
                fn.argtypes = args
                fn.restype = res
            _lib = h
    return _lib


def check(status: int, what: str = "") -> None:
    if status != 0:
        L = lib()
        msg = L.exq_last_error().decode(errors="replace")
        name = L.exq_status_name(status).decode()
        raise ExqError(f"{what}: {name}: {msg}" if what else f"{name}: {msg}")


def dtype_code(t: torch.dtype) -> int:
    try:
        return _TORCH_TO_CODE[t]
    except KeyError:
        raise ExqError(f"unsupported dtype {t}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device and be contiguous."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ExqError("exq_amd kernels need tensors on a HIP device (got CPU tensor)")
        if not t.is_contiguous():
            raise ExqError("exq_amd kernels need contiguous tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ExqError(f"tensors on different devices: {dev} and {t.device}")
    return dev


# Per-(device, stream, kind) workspace cache: reused across calls on one
# stream, which is safe because launches on one stream are ordered.  The
# fused-layer workspace ("fused") is kept apart from the scratch of the other
# entry points (its first bytes hold the decode kernels' combine counters,
# which each fused call clears itself).
_ws_cache: dict[tuple[int, int, str], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int, kind: str = "scratch") -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           stream_handle(device), kind)
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 1 << 20)
        if buf is not None:
            size = max(size, buf.numel() * 3 // 2)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _ws_cache[key] = buf
    return buf


def clear_workspace_cache() -> None:
    _ws_cache.clear()

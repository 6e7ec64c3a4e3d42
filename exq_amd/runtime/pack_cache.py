"""Packed INT4 expert banks kept on disk between runs.

The reference packs every MoE layer on its first forward call and keeps the
result only in process memory (``_get_or_pack``, exq/runtime/sglang_backend.py:
32-60, calling ``pack_experts_int4``, exq/kernels/moe_int4_kernel.py:96-119).
Here a layer's packed bank (w13/w2 packed nibbles + fp16 scales, the layout of
``pack_experts_int4``) is written once to ``<directory>/<key>.safetensors`` and
read back on later runs, so a restart skips the quantisation.

A file is used only when its metadata matches the layer: format version,
group size, the shapes and dtype of the fp weights, and a fingerprint of their
contents (SHA-256 over the raw bytes of a strided row sample of each tensor
plus its exact element sum).  Anything else is treated as a miss and the file is
rewritten.  Files are written to a temporary name and renamed, so a reader
never sees a partial file.  Loading uses safetensors only (no pickle).
"""
from __future__ import annotations

import hashlib
import json
import os
import tempfile
from pathlib import Path
from typing import Callable

import torch

FORMAT_VERSION = 2
_TENSORS = ("w13_packed", "w13_scales", "w2_packed", "w2_scales")


def fingerprint(*weights: torch.Tensor, sample_rows: int = 64) -> str:
    """Content fingerprint of fp weight tensors [E, N, K].

    SHA-256 over shape, dtype, the raw bytes of `sample_rows` evenly spaced
    rows of every expert, and the float64 sum of all elements (computed on the
    tensor's device, so a full pass costs one reduction, not a host copy).
    """
    h = hashlib.sha256()
    for w in weights:
        h.update(json.dumps([list(w.shape), str(w.dtype)]).encode())
        E, N = w.shape[0], w.shape[1]
        rows = torch.linspace(0, N - 1, min(sample_rows, N)).round().long().to(w.device)
        sample = w.index_select(1, rows).contiguous()
        h.update(sample.view(torch.uint8).cpu().numpy().tobytes())
        h.update(repr(float(w.sum(dtype=torch.float64).item())).encode())
    return h.hexdigest()


def _default_packer(w13: torch.Tensor, w2: torch.Tensor, group_size: int):
    from exq_amd.kernels import pack_experts_int4
    p13, s13 = pack_experts_int4(w13.to(torch.float16), group_size)
    p2, s2 = pack_experts_int4(w2.to(torch.float16), group_size)
    return p13, s13, p2, s2


class PackedWeightCache:
    """On-disk cache of packed INT4 expert banks, one safetensors file per key."""

    def __init__(self, directory: str | os.PathLike,
                 packer: Callable | None = None):
        self.directory = Path(directory)
        self.directory.mkdir(parents=True, exist_ok=True)
        self._packer = packer or _default_packer
        self.hits = 0
        self.misses = 0

    def path(self, key: str) -> Path:
        safe = "".join(c if c.isalnum() or c in "-_." else "_" for c in key)
        return self.directory / f"{safe}.safetensors"

    def _meta(self, w13: torch.Tensor, w2: torch.Tensor, group_size: int) -> dict:
        return {"format": str(FORMAT_VERSION), "group_size": str(group_size),
                "fingerprint": fingerprint(w13, w2)}

    def load(self, key: str, meta: dict, device: torch.device):
        """The cached bank for `key` if its metadata equals `meta`, else None."""
        from safetensors import safe_open
        p = self.path(key)
        if not p.exists():
            return None
        try:
            with safe_open(str(p), framework="pt", device="cpu") as f:
                if f.metadata() != meta or set(f.keys()) != set(_TENSORS):
                    return None
                return tuple(f.get_tensor(n).to(device) for n in _TENSORS)
        except Exception:  # unreadable or truncated: repack
            return None

    def store(self, key: str, meta: dict, bank) -> None:
        from safetensors.torch import save_file
        tensors = {n: t.detach().contiguous().cpu() for n, t in zip(_TENSORS, bank)}
        fd, tmp = tempfile.mkstemp(dir=self.directory, suffix=".tmp")
        os.close(fd)
        try:
            save_file(tensors, tmp, metadata=meta)
            os.replace(tmp, self.path(key))
        finally:
            if os.path.exists(tmp):
                os.unlink(tmp)

    def get_or_pack(self, key: str, w13: torch.Tensor, w2: torch.Tensor,
                    group_size: int = 128):
        """(w13_packed, w13_scales, w2_packed, w2_scales) for w13 [E, 2I, H],
        w2 [E, H, I]: read from disk when the file matches these weights,
        otherwise packed (on the GPU) and written."""
        meta = self._meta(w13, w2, group_size)
        bank = self.load(key, meta, w13.device)
        if bank is not None:
            self.hits += 1
            return bank
        self.misses += 1
        bank = self._packer(w13, w2, group_size)
        self.store(key, meta, bank)
        return bank

"""Shared helpers of the GPU parity tests (CPU-side reference assembly)."""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import moe, quant


def banner(msg: str) -> None:
    """Name the case before a GPU step, so a fault report says which one."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def used_experts(ids: np.ndarray, E: int) -> np.ndarray:
    flat = np.asarray(ids).reshape(-1)
    return np.unique(flat[(flat >= 0) & (flat < E)])


def oracle_int4_layer(hidden: torch.Tensor, w13p: torch.Tensor, w13s: torch.Tensor,
                      w2p: torch.Tensor, w2s: torch.Tensor, ids: np.ndarray, wts: np.ndarray,
                      accum=np.float32) -> np.ndarray:
    """fp32 dequantise-then-matmul reference, dequantising only routed experts."""
    E = w13p.shape[0]
    used = used_experts(ids, E)
    remap = np.full(E, -1, dtype=np.int64)
    remap[used] = np.arange(used.size)
    ids = np.asarray(ids).astype(np.int64)
    ids_c = np.where((ids >= 0) & (ids < E), remap[np.clip(ids, 0, E - 1)], -1)
    sel = torch.from_numpy(used).to(w13p.device)
    w13 = quant.dequant_int4(w13p[sel].cpu().numpy(), w13s[sel].cpu().numpy())
    w2 = quant.dequant_int4(w2p[sel].cpu().numpy(), w2s[sel].cpu().numpy())
    x = hidden.float().cpu().numpy()
    return moe.moe_layer(x, w13, w2, ids_c, np.asarray(wts, dtype=np.float32), accum=accum)


def assert_close_rel(y: torch.Tensor, ref: np.ndarray, tol: float, what: str) -> float:
    """Relative L2 error gate (tolerance stated by the caller)."""
    yy = y.float().cpu().numpy()
    assert np.all(np.isfinite(yy)), f"{what}: non-finite output"
    err = moe.rel_l2(yy, ref)
    mx = float(np.abs(yy - ref).max()) if yy.size else 0.0
    print(f"[parity] {what}: rel_l2={err:.3e} max_abs={mx:.3e} "
          f"max/rms={moe.max_over_rms(yy, ref) if yy.size else 0:.3e}", flush=True)
    assert err <= tol, f"{what}: rel_l2 {err:.3e} > {tol}"
    return err

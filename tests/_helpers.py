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


# (what, rel_l2, worst per-token rel_l2, max_abs, max/rms) of every parity check
# in this session; tests/conftest.py prints them in the terminal summary.
PARITY_LOG: list[tuple[str, float, float, float, float]] = []


def row_rel_l2(y: np.ndarray, ref: np.ndarray) -> float:
    """Worst per-token relative L2 error.  Each row's error is divided by the
    larger of its own norm and a tenth of the mean row norm, so a row whose
    reference is nearly zero (no routed slot, tiny weights) does not dominate."""
    y2 = y.reshape(y.shape[0], -1).astype(np.float64)
    r2 = ref.reshape(ref.shape[0], -1).astype(np.float64)
    if y2.size == 0:
        return 0.0
    en = np.linalg.norm(y2 - r2, axis=1)
    rn = np.linalg.norm(r2, axis=1)
    floor = 0.1 * float(rn.mean()) if rn.size else 0.0
    return float((en / np.maximum(rn, max(floor, 1e-30))).max())


def assert_close_rel(y: torch.Tensor, ref: np.ndarray, tol: float, what: str,
                     row_tol: float | None = None) -> float:
    """Relative L2 error gate over the whole output (``tol``) and per token row
    (``row_tol``, default 2 * tol: a single row has fewer elements to average
    the bf16 output rounding over)."""
    yy = y.float().cpu().numpy()
    assert np.all(np.isfinite(yy)), f"{what}: non-finite output"
    err = moe.rel_l2(yy, ref)
    rerr = row_rel_l2(yy, ref)
    mx = float(np.abs(yy - ref).max()) if yy.size else 0.0
    mor = moe.max_over_rms(yy, ref) if yy.size else 0.0
    PARITY_LOG.append((what, err, rerr, mx, mor))
    print(f"[parity] {what}: rel_l2={err:.3e} row_rel_l2={rerr:.3e} max_abs={mx:.3e} "
          f"max/rms={mor:.3e}", flush=True)
    assert err <= tol, f"{what}: rel_l2 {err:.3e} > {tol}"
    rt = 2 * tol if row_tol is None else row_tol
    assert rerr <= rt, f"{what}: worst token row rel_l2 {rerr:.3e} > {rt}"
    return err

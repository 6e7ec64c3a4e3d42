"""MoE layer arithmetic restated on the CPU (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The layer is the reference's fp32 dequantise-then-matmul path:

    for each token t, for each of its k routed experts e (weight w):
        gate_up = W13[e] @ x[t]                       (W13 rows: gate first, then up;
                                                       exq_dispatch.cu:36-37)
        mid     = silu(gate_up[:I]) * gate_up[I:]     (sgl_kernel.silu_and_mul,
                                                       sglang_backend.py:137-140)
        out[t] += w * (W2[e] @ mid)                   (moe_grouped_gemm.py:284-289,
                                                       exq_dispatch.cu:263-278)

with W13/W2 dequantised in float32 from the stored weights and fp16 scales
(scripts/bench_int4.py:62-78).  ``accum`` selects float32 (the reference's
accumulation type) or float64 (used for golden fixtures).
"""
from __future__ import annotations

import numpy as np


def silu(x: np.ndarray) -> np.ndarray:
    """x * sigmoid(x) = x / (1 + exp(-x)).

    pinned by: scipy.special.expit and torch.nn.functional.silu (library
    routines) and the closed values silu(0) = 0, silu(x) -> x (x >> 0),
    silu(x) -> 0 (x << 0) in tests/test_oracle_moe.py.
    """
    x = np.asarray(x)
    with np.errstate(over="ignore"):
        return x / (1.0 + np.exp(-x))


def silu_and_mul(gate_up: np.ndarray) -> np.ndarray:
    """out[:, j] = silu(x[:, j]) * x[:, I + j]  (gate first; exq_dispatch.cu:36-37).

    pinned by: library silu composed with an explicit per-element loop on a
    tiny input (tests/test_oracle_moe.py).
    """
    x = np.asarray(gate_up)
    I = x.shape[-1] // 2
    return silu(x[..., :I]) * x[..., I:]


def gather_hidden(hidden: np.ndarray, sort_order: np.ndarray, top_k: int) -> np.ndarray:
    """out[i] = hidden[sort_order[i] // top_k]  (exq_dispatch.cu:234-246)."""
    return np.asarray(hidden)[np.asarray(sort_order).astype(np.int64) // top_k]


def combine(down_out: np.ndarray, sort_order: np.ndarray, router_weights: np.ndarray,
            accum=np.float64) -> np.ndarray:
    """result[tok] += w[s] * down[i], s = sort_order[i], tok = s // k.

    Restates exq_dispatch.cu:263-310 (fp32 atomics there; here an ordered sum
    in ``accum`` precision).  Returns ``accum`` [T, H].

    pinned by: an explicit Python double loop on a tiny input and the
    linearity identity combine(a*d1 + b*d2) = a*combine(d1) + b*combine(d2).
    """
    w = np.asarray(router_weights)
    T, k = w.shape
    d = np.asarray(down_out).astype(accum)
    so = np.asarray(sort_order).astype(np.int64)
    out = np.zeros((T, d.shape[1]), dtype=accum)
    wf = w.reshape(-1).astype(accum)
    np.add.at(out, so // k, wf[so][:, None] * d)
    return out


def grouped_gemm_sorted(a_sorted: np.ndarray, weights: np.ndarray, expert_ends: np.ndarray,
                        accum=np.float32) -> np.ndarray:
    """C[rows of e] = A[rows of e] @ W[e]^T for each expert segment.

    Restates the per-program contraction of ``_moe_gemm_kernel`` /
    ``_moe_gemm_int4_kernel`` (moe_grouped_gemm.py:87-132,
    moe_int4_kernel.py:165-240) with W already dequantised to float.

    pinned by: the per-(row) matvec definition on tiny inputs and the special
    case of a single expert, which is a plain matmul (numpy BLAS).
    """
    a = np.asarray(a_sorted).astype(accum)
    w = np.asarray(weights).astype(accum)
    ends = np.asarray(expert_ends).astype(np.int64)
    out = np.zeros((a.shape[0], w.shape[1]), dtype=accum)
    for e in range(w.shape[0]):
        lo, hi = ends[e], ends[e + 1]
        if hi > lo:
            out[lo:hi] = a[lo:hi] @ w[e].T
    return out


def moe_layer(hidden: np.ndarray, w13: np.ndarray, w2: np.ndarray,
              topk_ids: np.ndarray, topk_weights: np.ndarray,
              shared_w13: np.ndarray | None = None, shared_w2: np.ndarray | None = None,
              accum=np.float32) -> np.ndarray:
    """Full MoE layer, float weights (already dequantised), grouped by expert.

    ``hidden [T,H]``, ``w13 [E,2I,H]``, ``w2 [E,H,I]``, ``topk_ids [T,k]``
    (ids outside [0, E) are dropped, the expert-parallel ``-1`` convention),
    ``topk_weights [T,k]``.  ``shared_w13 [S,2I,H]`` / ``shared_w2 [S,H,I]``
    are always-on experts added with weight 1.  Returns ``accum`` [T, H].

    The contraction for each (token, expert) pair is exactly the reference's
    per-(token, k) matvec (moe_grouped_gemm.py:284-289); grouping the tokens
    of one expert into one matmul changes only the BLAS blocking.

    pinned by: moe_layer_loop (the literal per-(token,k) loop) on small
    inputs, the single-expert/single-token closed form against torch, and
    linearity in the router weights (tests/test_oracle_moe.py).
    """
    x = np.asarray(hidden).astype(accum)
    ids = np.asarray(topk_ids).astype(np.int64)
    wts = np.asarray(topk_weights).astype(accum)
    T, k = ids.shape
    E = w13.shape[0]
    I = w13.shape[1] // 2
    out = np.zeros((T, x.shape[1]), dtype=accum)
    for e in range(E):
        tok, j = np.nonzero(ids == e)
        if tok.size == 0:
            continue
        we13 = np.asarray(w13[e]).astype(accum)
        we2 = np.asarray(w2[e]).astype(accum)
        gu = x[tok] @ we13.T
        mid = silu(gu[:, :I]) * gu[:, I:]
        d = mid @ we2.T
        np.add.at(out, tok, wts[tok, j][:, None] * d)
    if shared_w13 is not None:
        for s in range(shared_w13.shape[0]):
            ws13 = np.asarray(shared_w13[s]).astype(accum)
            ws2 = np.asarray(shared_w2[s]).astype(accum)
            Is = ws13.shape[0] // 2
            gu = x @ ws13.T
            out += (silu(gu[:, :Is]) * gu[:, Is:]) @ ws2.T
    return out


def moe_layer_loop(hidden, w13, w2, topk_ids, topk_weights, accum=np.float64):
    """The literal per-(token, k) loop of pytorch_moe_reference
    (moe_grouped_gemm.py:280-290) extended with SiLU-and-mul and the down
    projection.  Small inputs only.
    """
    x = np.asarray(hidden).astype(accum)
    ids = np.asarray(topk_ids)
    wts = np.asarray(topk_weights).astype(accum)
    T, k = ids.shape
    I = w13.shape[1] // 2
    out = np.zeros((T, x.shape[1]), dtype=accum)
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if e < 0 or e >= w13.shape[0]:
                continue
            gu = np.asarray(w13[e]).astype(accum) @ x[t]
            mid = silu(gu[:I]) * gu[I:]
            out[t] += wts[t, j] * (np.asarray(w2[e]).astype(accum) @ mid)
    return out


def rel_l2(y: np.ndarray, ref: np.ndarray) -> float:
    """||y - ref||_2 / ||ref||_2 (the primary error metric)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(r)
    return float(np.linalg.norm(y - r) / den) if den > 0 else float(np.linalg.norm(y - r))


def max_over_rms(y: np.ndarray, ref: np.ndarray) -> float:
    """max|y - ref| / rms(ref): the reference bench's metric (bench_int4.py:88-91)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(r * r)))
    return float(np.abs(y - r).max() / max(rms, 1e-6))

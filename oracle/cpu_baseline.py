"""The reference's PyTorch CPU path, restated for the timed CPU baseline.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): imported by
``bench.py``'s cpu_baseline leg and by tests, never by the product.

Steps (the reference's CPU path, composed into a full layer):
  1. fp32 nibble dequant with the stored fp16 scales (scripts/bench_int4.py:62-78);
  2. the per-(token, k) matvec loop of pytorch_moe_reference
     (exq/kernels/moe_grouped_gemm.py:280-290) for gate/up;
  3. SiLU(gate) * up (gate rows first);
  4. the down projection;
  5. the top-k weighted sum.
Variant ``"dequant_per_call"`` dequantises the routed experts inside every
call (reference-faithful); ``"predequantized"`` keeps fp32 weights and times
the matmuls only; ``"grouped"`` (context only, not the reference) keeps fp32
weights and multiplies each expert's token rows at once.  Mixed-precision banks dequantise each expert by its tier
(INT4 as above, INT8 per-row fp16 scale, BF16 widened); always-on shared
experts are added with weight 1, as the GPU path does.

pinned by: tests/test_oracle_cpu_baseline.py -- ``dequant_int4_torch`` and
``dequant_int8_torch`` equal ``oracle.quant.dequant_int4`` / ``dequant_int8``
bit for bit, and ``moe_layer_loop`` (with and without shared experts) equals
``oracle.moe.moe_layer`` (float64) to 1e-5 relative L2, while a dropped top-k
term or a dropped shared expert misses it by more than 1e-2; ``moe_layer_grouped``
equals ``moe_layer_loop`` to 1e-5 relative L2.
"""
from __future__ import annotations

import os
import statistics
import time

import torch


def dequant_int4_torch(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """[..., N, K/2] u8 + [..., N, K/g] f16 -> fp32 [..., N, K] (bench_int4.py:62-78)."""
    p = packed.to(torch.uint8)
    lo = (p & 0x0F).float() - 8.0
    hi = ((p >> 4) & 0x0F).float() - 8.0
    K = p.shape[-1] * 2
    g = K // scales.shape[-1]
    s = scales.float().repeat_interleave(g // 2, dim=-1)
    w = torch.empty(p.shape[:-1] + (K,), dtype=torch.float32)
    w[..., 0::2] = lo * s
    w[..., 1::2] = hi * s
    return w


def dequant_int8_torch(q: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """[..., N, K] i8 + [..., N] f16 per-row scales -> fp32 [..., N, K]."""
    return q.float() * scales.float().unsqueeze(-1)


def moe_layer_loop(x: torch.Tensor, w13: dict, w2: dict, ids: torch.Tensor,
                   wts: torch.Tensor, shared: tuple = ()) -> torch.Tensor:
    """pytorch_moe_reference's per-(token, k) loop, extended to the full layer;
    ``shared`` holds (w13, w2) of always-on experts, added with weight 1."""
    T, k = ids.shape
    out = torch.zeros(T, x.shape[1], dtype=torch.float32)
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if e < 0 or e not in w13:  # dropped slot
                continue
            gu = w13[e] @ x[t]
            I = gu.shape[0] // 2
            mid = torch.nn.functional.silu(gu[:I]) * gu[I:]
            out[t] += float(wts[t, j]) * (w2[e] @ mid)
        for s13, s2 in shared:
            gu = s13 @ x[t]
            I = gu.shape[0] // 2
            out[t] += s2 @ (torch.nn.functional.silu(gu[:I]) * gu[I:])
    return out


def moe_layer_grouped(x: torch.Tensor, w13: dict, w2: dict, ids: torch.Tensor,
                      wts: torch.Tensor, shared: tuple = ()) -> torch.Tensor:
    """Vectorised per-expert grouping of the same layer, for context only (NOT
    the reference's path): each routed expert multiplies all of its token rows
    at once (one [n_e, H] x [H, 2I] and one [n_e, I] x [I, H] product), and the
    weighted rows are scattered back with index_add_."""
    T, k = ids.shape
    out = torch.zeros(T, x.shape[1], dtype=torch.float32)
    flat = ids.reshape(-1)
    for e in sorted(w13):
        slots = torch.nonzero(flat == e, as_tuple=True)[0]
        if slots.numel() == 0:
            continue
        tok = torch.div(slots, k, rounding_mode="floor")
        gu = x[tok] @ w13[e].T
        I = gu.shape[1] // 2
        y = (torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]) @ w2[e].T
        out.index_add_(0, tok, y * wts.reshape(-1)[slots].unsqueeze(1))
    for s13, s2 in shared:
        gu = x @ s13.T
        I = gu.shape[1] // 2
        out += (torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]) @ s2.T
    return out


def time_cpu_experts(x, deq: dict, ids, wts, shared_deq=(), variant: str = "dequant_per_call",
                     reps: int = 20, warmup: int = 1, threads: int | None = None,
                     budget_s: float | None = None) -> dict:
    """Time one MoE layer whose routed expert e dequantises with ``deq[e]()``
    (returning fp32 (w13, w2) from host copies of the stored tensors) and whose
    shared experts with ``shared_deq``; P5/P50/P95 in microseconds.

    With ``budget_s`` the first warm-up call sizes the run: 20 reps (``reps``)
    when a call takes under a second, otherwise as many as fit the budget, at
    least 3."""
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    x = x.float().cpu()
    ids = ids.cpu()
    wts = wts.float().cpu()
    used = sorted(set(int(v) for v in ids.reshape(-1).tolist()) & set(deq))

    def dequant_all():
        w13, w2 = {}, {}
        for e in used:
            w13[e], w2[e] = deq[e]()
        return w13, w2, tuple(f() for f in shared_deq)

    pre = dequant_all() if variant in ("predequantized", "grouped") else None
    layer = moe_layer_grouped if variant == "grouped" else moe_layer_loop

    def run():
        a, b, sh = pre if pre is not None else dequant_all()
        return layer(x, a, b, ids, wts, sh)

    with torch.no_grad():
        first = None
        for _ in range(max(warmup, 1 if budget_s else 0)):
            t0 = time.perf_counter()
            run()
            first = time.perf_counter() - t0
        if budget_s and first is not None and first >= 1.0:
            reps = max(3, min(reps, int(budget_s / first)))
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            run()
            times.append((time.perf_counter() - t0) * 1e6)
    times.sort()
    n = len(times)
    return {"variant": variant, "threads": threads, "reps": n,
            "p50_us": times[n // 2], "p5_us": times[int(0.05 * (n - 1))],
            "p95_us": times[int(0.95 * (n - 1))], "mean_us": statistics.mean(times)}


def int4_deq(p13, s13, p2, s2) -> dict:
    """Per-expert INT4 dequantisers over host copies of a packed bank."""
    p13, s13, p2, s2 = (t.cpu() for t in (p13, s13, p2, s2))
    return {e: (lambda e=e: (dequant_int4_torch(p13[e], s13[e]),
                             dequant_int4_torch(p2[e], s2[e])))
            for e in range(p13.shape[0])}


def bank_deq(tier, index, tensors: dict, used) -> tuple[dict, list]:
    """Per-expert dequantisers of a mixed-precision bank (tier 0 BF16, 1 INT8,
    2 INT4; ``index`` the row in the tier's tensors), for the routed experts in
    ``used`` and every shared expert (ids from len(used bank) on).  Only the
    rows that are needed are copied to the host."""
    tier = [int(v) for v in tier]
    index = [int(v) for v in index]

    def host(name, i):
        return tensors[name][i].cpu()

    def make(e):
        t, i = tier[e], index[e]
        if t == 0:
            a, b = host("bf16_w13", i), host("bf16_w2", i)
            return lambda: (a.float(), b.float())
        if t == 1:
            a, sa = host("int8_w13", i), host("int8_w13_scales", i)
            b, sb = host("int8_w2", i), host("int8_w2_scales", i)
            return lambda: (dequant_int8_torch(a, sa), dequant_int8_torch(b, sb))
        a, sa = host("int4_w13", i), host("int4_w13_scales", i)
        b, sb = host("int4_w2", i), host("int4_w2_scales", i)
        return lambda: (dequant_int4_torch(a, sa), dequant_int4_torch(b, sb))

    n_routed = tensors["n_experts"]
    routed = {e: make(e) for e in sorted(set(int(u) for u in used)) if 0 <= e < n_routed}
    shared = [make(e) for e in range(n_routed, len(tier))]
    return routed, shared


def time_cpu_layer(x, p13, s13, p2, s2, ids, wts, variant: str = "dequant_per_call",
                   reps: int = 20, warmup: int = 2, threads: int | None = None) -> dict:
    """Time one all-INT4 MoE layer on the host CPU; P5/P50/P95 in microseconds."""
    return time_cpu_experts(x, int4_deq(p13, s13, p2, s2), ids, wts, (), variant, reps,
                            warmup, threads)

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
the matmuls only.

pinned by: tests/test_oracle_cpu_baseline.py -- ``dequant_int4_torch`` equals
``oracle.quant.dequant_int4`` bit for bit, and ``moe_layer_loop`` equals
``oracle.moe.moe_layer`` (float64) to 1e-5 relative L2, while a dropped top-k
term misses it by more than 1e-2.
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


def moe_layer_loop(x: torch.Tensor, w13: dict, w2: dict, ids: torch.Tensor,
                   wts: torch.Tensor) -> torch.Tensor:
    """pytorch_moe_reference's per-(token, k) loop, extended to the full layer."""
    T, k = ids.shape
    out = torch.zeros(T, x.shape[1], dtype=torch.float32)
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            gu = w13[e] @ x[t]
            I = gu.shape[0] // 2
            mid = torch.nn.functional.silu(gu[:I]) * gu[I:]
            out[t] += float(wts[t, j]) * (w2[e] @ mid)
    return out


def time_cpu_layer(x, p13, s13, p2, s2, ids, wts, variant: str = "dequant_per_call",
                   reps: int = 20, warmup: int = 2, threads: int | None = None) -> dict:
    """Time one MoE layer on the host CPU; returns P5/P50/P95 in microseconds."""
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    x = x.float().cpu()
    ids = ids.cpu()
    wts = wts.float().cpu()
    used = sorted(set(int(v) for v in ids.reshape(-1).tolist()))
    p13, s13, p2, s2 = (t.cpu() for t in (p13, s13, p2, s2))

    def deq():
        return ({e: dequant_int4_torch(p13[e], s13[e]) for e in used},
                {e: dequant_int4_torch(p2[e], s2[e]) for e in used})

    pre = deq() if variant == "predequantized" else None

    def run():
        a, b = pre if pre is not None else deq()
        return moe_layer_loop(x, a, b, ids, wts)

    with torch.no_grad():
        for _ in range(warmup):
            run()
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

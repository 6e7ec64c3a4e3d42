#!/usr/bin/env python3
"""Benchmark of the INT4 MoE expert-dispatch hot path on one MI355X.

Workload: Qwen3-30B-A3B-shaped INT4 MoE layer
(H=2048, I=768, 128 experts, top-8, g=128), all 48 layers with distinct
seeded weights streamed so no layer is cache-resident (14.3 GiB of packed
banks).  One step = one decode step through the 48 layers at batch T (16 by
default), replayed from a HIP graph (how a serving loop issues decode
steps); inputs are resident in HBM before the timed region.

Printed: one JSON line with µs per MoE layer (value: the P50 over the timed
steps of each step's µs/layer, with P5 / P95 and the mean beside it),
tokens/s, the achieved HBM bandwidth on activated-expert weight bytes, the
roofline of the dominant kernel (the gate/up INT4 GEMM + SiLU decode kernel,
timed with HIP events recorded on its stream around it, over >= 300 layer
calls), the OLMoE T=16 line (`north_star`: BASELINE.json configs[0], the
target configuration, with its own kernel roofline), the decode-batch sweep
(1, 4, 16, 64), the other configurations (P50 / P5 / P95 over >= 300 layer
calls each), the streaming-read ceiling of this box (exq_stream_read over
2 GiB), a plain streaming read of exactly the dominant kernel's bytes per
launch (48 distinct buffers replayed from a graph: the floor at that
transfer size) and the reference's CPU path timed on this host at every
configuration, both variants (`cpu_baseline.configs`).

    python bench.py [--gpus 1] [--steps 50] [--warmup 100] [--batch 16]
                    [--sweep 1,4,16,64] [--layers 48] [--no-cpu] [--no-configs]

Counter runs (HBM traffic of the dominant kernel, rocprofv3 --pmc), one per
counter and configuration:

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d DIR -o fetch -- \
        python3 bench.py --pmc-run [--config olmoe --layers 3] [--batch T]
    python3 bench.py --pmc-summary DIR/.../fetch_counter_collection.csv

--pmc-run first copies a 256 MiB buffer (the calibration: a plain copy of
known size) and then runs the layers once at the bench batch, eagerly.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer µs/decode step + achieved HBM GB/s (% of peak) at batch 1–64"
HBM_PEAK_GBPS = 8000.0


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # 100 steps of 48 Qwen3 layers at T=16 are about 150 ms: the clocks have
    # settled before the timed steps, also after the long idle spell of
    # building the stack (25 steps left the P95 step 10 % above the P50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--sweep", type=str, default="1,4,16,64")
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead")
    ap.add_argument("--cpu-reps", type=int, default=20,
                    help="CPU baseline reps per variant and configuration (calls under 1 s)")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds per variant and configuration for calls over 1 s (>= 3 reps)")
    ap.add_argument("--config", type=str, default="qwen3",
                    help="with --pmc-run: the configuration of the eager pass (qwen3, olmoe)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other BASELINE.json configurations")
    ap.add_argument("--pmc-run", action="store_true",
                    help="calibration copy + eager passes over the layers, for rocprofv3")
    ap.add_argument("--passes", type=int, default=1,
                    help="with --pmc-run: eager passes over the layers (default 1)")
    ap.add_argument("--pmc-summary", type=str, default="",
                    help="per-kernel mean of a rocprofv3 counter CSV")
    ap.add_argument("--north-star-only", action="store_true",
                    help="measure only the OLMoE T=16 line (BASELINE configs[0]) and exit")
    ap.add_argument("--routing-only", action="store_true",
                    help="time only the standalone stable sort (exq_dispatch) and exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill configurations (DeepSeek-V2-Lite 2048, Mixtral 4096)")
    ap.add_argument("--eager", action="store_true",
                    help="with --prefill-only: one eager call per configuration (counter runs)")
    return ap.parse_args()


CALIB_BYTES = 256 << 20
PMC_SUMMARY = os.path.join(ROOT, "profiles", "decode_gateup_traffic_pmc.md")


def pmc_summary(path):
    """Mean counter value per (kernel, counter) of a rocprofv3 counter CSV."""
    import csv
    from collections import defaultdict
    acc = defaultdict(list)
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = row.get("Kernel_Name") or row.get("Kernel-Name") or ""
            ctr = row.get("Counter_Name") or row.get("Counter-Name") or ""
            val = row.get("Counter_Value") or row.get("Counter-Value") or "nan"
            acc[(name, ctr)].append(float(val))
    for (name, ctr), v in sorted(acc.items(), key=lambda kv: -sum(kv[1])):
        print(f"{len(v):6d}  {ctr:12s} mean {sum(v) / len(v):14.1f}  {name[:110]}")


def traffic_from_profile(config="qwen3", T=16):
    """HBM bytes per launch of the gate/up decode kernel at (config, T) from
    the committed counter summary (lines `traffic_bytes_per_launch[qwen3,T=16]:
    N`), or None when no counter run covers that configuration."""
    key = f"traffic_bytes_per_launch[{config},T={T}]:"
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                if line.strip().startswith(key):
                    return int(float(line.split(":", 1)[1]))
    except (OSError, ValueError):
        return None
    return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Stack:
    """48 distinct seeded Qwen3-shaped INT4 layers resident in HBM."""

    def __init__(self, cfg, n_layers, device):
        import torch
        from exq_amd import synth
        from exq_amd.kernels import pack_experts_int4
        self.cfg = cfg
        self.layers = []
        for l in range(n_layers):
            w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                               synth.seed_for(cfg, l), device)
            p13, s13 = pack_experts_int4(w13)
            p2, s2 = pack_experts_int4(w2)
            del w13, w2
            self.layers.append((p13, s13, p2, s2))
        torch.cuda.synchronize()
        self.expert_bytes = synth.int4_expert_bytes(cfg.hidden, cfg.inter, cfg.group_size)
        g = cfg.group_size
        self.w13_bytes = 2 * cfg.inter * cfg.hidden // 2 + 2 * cfg.inter * (cfg.hidden // g) * 2
        self.w2_bytes = cfg.hidden * cfg.inter // 2 + cfg.hidden * (cfg.inter // g) * 2


class Batch:
    """Routing + activations of one decode batch for every layer."""

    def __init__(self, stack, T, device):
        import numpy as np
        import torch
        from exq_amd import synth
        from exq_amd.kernels.fused_moe import moe_workspace_bytes
        cfg = stack.cfg
        self.T = T
        self.x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 12345 + T)).to(
            torch.bfloat16).to(device)
        self.ids, self.wts, self.active = [], [], []
        for l in range(len(stack.layers)):
            ids, w = synth.routing(cfg, T, l)
            self.active.append(int(np.unique(ids).size))
            self.ids.append(torch.from_numpy(ids.astype(np.int32)).to(device))
            self.wts.append(torch.from_numpy(w).to(device))
        self.out = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device=device)
        need = moe_workspace_bytes(T, cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k)
        self.ws = torch.zeros(need, dtype=torch.uint8, device=device)
        self.bytes = sum(a * stack.expert_bytes for a in self.active)


def run_step(stack, b):
    from exq_amd.kernels import fused_experts
    for l, (p13, s13, p2, s2) in enumerate(stack.layers):
        fused_experts(b.x, p13, s13, p2, s2, b.wts[l], b.ids[l], out=b.out, workspace=b.ws)


def pct(v, q):
    """q-th percentile (nearest rank) of the values v."""
    v = sorted(v)
    return v[min(len(v) - 1, max(0, int(round(q / 100.0 * (len(v) - 1)))))]


def time_steps(stack, b, steps, warmup, use_graph, warmup_ms=0.0):
    """Returns (ms per step over the bracketed K steps, host wall ms per step,
    list of per-step ms from events recorded between the steps), after
    `warmup` untimed steps (or at least warmup_ms of them)."""
    import torch
    if use_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            run_step(stack, b)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run_step(stack, b)
        fn = g.replay
    else:
        fn = lambda: run_step(stack, b)  # noqa: E731
    for _ in range(_warmup_count(fn, warmup, warmup_ms)):
        fn()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(steps):
        fn()
        evs[i + 1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    return evs[0].elapsed_time(evs[-1]) / steps, wall, per


def stage_times(layers, b, reps=7):
    """Per-kernel durations (µs) of every layer call (eager launches, `reps`
    passes over the layers): the decode kernels are launched with
    hipExtLaunchKernelGGL start / stop events on the call's stream, so events
    0 -> 1 time the gate/up kernel and 2 -> 3 the down kernel exactly.  Mean
    and P5 / P50 / P95 over all calls."""
    import torch
    from exq_amd import _lib
    from exq_amd.kernels import fused_experts
    L = _lib.lib()
    n = len(layers)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n * reps)]
    for row in evs:  # torch creates the HIP event on first record
        for e in row:
            e.record()
    for l, (p13, s13, p2, s2) in enumerate(layers):
        fused_experts(b.x, p13, s13, p2, s2, b.wts[l], b.ids[l], out=b.out, workspace=b.ws)
    torch.cuda.synchronize()
    i = 0
    try:
        for _ in range(reps):
            for l, (p13, s13, p2, s2) in enumerate(layers):
                arr = (ctypes.c_void_p * 4)(*[e.cuda_event for e in evs[i]])
                _lib.check(L.exq_set_stage_events(arr, 4), "exq_set_stage_events")
                fused_experts(b.x, p13, s13, p2, s2, b.wts[l], b.ids[l], out=b.out,
                              workspace=b.ws)
                i += 1
    finally:
        _lib.check(L.exq_set_stage_events(None, 0), "exq_set_stage_events")
    torch.cuda.synchronize()
    out = {"calls": len(evs)}
    for name, (a, z) in (("gateup", (0, 1)), ("down", (2, 3)), ("layer", (0, 3))):
        v = [e[a].elapsed_time(e[z]) * 1e3 for e in evs]
        out[f"{name}_us"] = sum(v) / len(v)
        out[f"{name}_p5_us"], out[f"{name}_p50_us"], out[f"{name}_p95_us"] = (
            pct(v, 5), pct(v, 50), pct(v, 95))
    return out


MFMA_PEAK_BF16_TFLOPS = 2500.0


# Untimed work before a timed series of a configuration: after an idle spell
# the first ~10-15 ms of back-to-back work run slower while the clocks settle
# (measured from a cold start: Qwen3 T=1 15.2 -> 13.4 us per layer over the
# first 15 steps of 48 layers, T=16 35.8 -> 33.2 over 11; DeepSeek-V2-Lite
# prefill 519 -> 450 us over the first 20 replays).
WARMUP_MS = 40.0


def _warmup_count(replay, minimum, warmup_ms):
    """Replays of `replay` (already warm once) that make up warmup_ms."""
    import torch
    if warmup_ms <= 0:
        return minimum
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    replay()
    e1.record()
    torch.cuda.synchronize()
    return max(minimum, int(warmup_ms / max(e0.elapsed_time(e1), 1e-3)) + 1)


def _graph_times(fn, reps, warmup=3, warmup_ms=0.0):
    """Per-replay ms of `fn` captured once in a HIP graph and replayed `reps`
    times (events recorded between the replays), after `warmup` replays or
    at least warmup_ms of them."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(_warmup_count(g.replay, warmup, warmup_ms)):
        g.replay()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    evs[0].record()
    for i in range(reps):
        g.replay()
        evs[i + 1].record()
    torch.cuda.synchronize()
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(reps)]


def _graph_time(fn, reps, warmup=3):
    """Mean ms per call of `fn` replayed from a HIP graph."""
    v = _graph_times(fn, reps, warmup)
    return sum(v) / len(v)


def _deepseek_bank(cfg, layer, dev):
    """DeepSeek-V2-Lite layer: 64 INT4 routed experts + 2 BF16 shared experts."""
    from exq_amd import synth
    from exq_amd.kernels import MixedExpertBank
    w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                       synth.seed_for(cfg, layer), dev)
    s13, s2 = synth.expert_weights_gpu(cfg.n_shared, cfg.inter, cfg.hidden,
                                       synth.seed_for(cfg, layer) + 500, dev)
    return MixedExpertBank.from_weights(w13, w2, [2] * cfg.n_experts, shared_w13=s13,
                                        shared_w2=s2, shared_tier=0)


def _int4_layer(cfg, layer, dev):
    from exq_amd import synth
    from exq_amd.kernels import pack_experts_int4
    w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                       synth.seed_for(cfg, layer), dev)
    return pack_experts_int4(w13) + pack_experts_int4(w2)


def _prefill_call(dev, name, weights=None):
    """(name, T, fn, flops) of one prefill configuration: DeepSeek-V2-Lite (2048
    tokens, top-6 + 2 shared, `weights` a MixedExpertBank) or Mixtral (4096
    tokens, top-2, `weights` the packed (w13, s13, w2, s2)); built if None."""
    import numpy as np
    import torch
    from exq_amd import synth
    from exq_amd.kernels import fused_experts, fused_experts_mixed
    from exq_amd.kernels.fused_moe import moe_workspace_bytes
    T, seed = {"deepseek_v2_lite": (2048, 3), "mixtral": (4096, 4)}[name]
    cfg = synth.CONFIGS[name]
    x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, seed)).to(torch.bfloat16).to(dev)
    ids, w = synth.routing(cfg, T, 0)
    tid = torch.from_numpy(ids.astype(np.int32)).to(dev)
    tw = torch.from_numpy(w).to(dev)
    ws = torch.zeros(moe_workspace_bytes(T, cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k,
                                         cfg.n_shared), dtype=torch.uint8, device=dev)
    flops = 2.0 * T * (cfg.top_k + cfg.n_shared) * 3 * cfg.hidden * cfg.inter
    if name == "deepseek_v2_lite":
        bank = weights if weights is not None else _deepseek_bank(cfg, 0, dev)
        return name, T, lambda: fused_experts_mixed(x, bank, tw, tid, workspace=ws), flops
    p13, s13, p2, s2 = weights if weights is not None else _int4_layer(cfg, 0, dev)
    return name, T, lambda: fused_experts(x, p13, s13, p2, s2, tw, tid, workspace=ws), flops


def prefill_rows(calls, reps):
    """µs per layer (P50 over `reps` graph replays, P5 / P95 beside it) of each
    prefill call, after WARMUP_MS of untimed replays."""
    rows = []
    for name, T, fn, flops in calls:
        per = [ms * 1e3 for ms in _graph_times(fn, reps, warmup_ms=WARMUP_MS)]
        us = pct(per, 50)
        tf = flops / (us * 1e-6) / 1e12
        rows.append({"config": name, "batch": T, "us_per_layer": round(us, 1),
                     "p5_us": round(pct(per, 5), 1), "p95_us": round(pct(per, 95), 1),
                     "replays_timed": reps, "warmup_ms": WARMUP_MS,
                     "tokens_per_s": round(T / (us * 1e-6)), "TFLOPs": round(tf, 1),
                     "frac_of_mfma_peak": round(tf / MFMA_PEAK_BF16_TFLOPS, 4)})
        log(f"config {name} prefill T={T}: {us:.1f} us/layer P50, {tf:.1f} TFLOP/s")
    return rows


class _Calls:
    """Inputs of one decode batch over a rotation of layers (stage_times'
    batch interface)."""

    def __init__(self, x, ids, wts, out, ws):
        self.x, self.ids, self.wts, self.out, self.ws = x, ids, wts, out, ws


def measure_configs(dev, reps, cpu=None, north_star_only=False):
    """The other BASELINE.json configurations: decode µs/layer and achieved GB/s
    on activated-expert bytes (weights + scales; shared experts included) over
    distinct seeded layers replayed from a HIP graph, and prefill TFLOP/s.

    Returns (rows, north_star, cpu_rows): north_star is the OLMoE T=16 line
    (the target configuration) with its own stage
    events and roofline; cpu_rows (when ``cpu`` holds the CPU settings) the
    reference CPU path timed on layer 0 of each configuration, same inputs.
    ``north_star_only`` measures the OLMoE T=16 line alone (for profiling)."""
    import json as _json
    import tempfile
    import numpy as np
    import torch
    from exq_amd import synth
    from exq_amd.kernels import (MixedExpertBank, fused_experts, fused_experts_mixed,
                                 load_exq_artifact, pack_experts_int4)
    from exq_amd.kernels.fused_moe import moe_workspace_bytes
    rows, cpu_rows = [], []
    north_star = None

    def ws_for(cfg, T):  # explicit workspace: nothing allocates inside graph capture
        return torch.empty(moe_workspace_bytes(T, cfg.hidden, cfg.inter, cfg.n_experts,
                                               cfg.top_k, cfg.n_shared), dtype=torch.uint8,
                           device=dev)

    def decode_row(name, cfg, T, calls, bytes_per_call, n_layers):
        # One graph holds at least 48 layer calls (the rotation repeated), as a
        # model's decode step does, so one graph launch is not charged to a few
        # layers; µs/layer of each replay, P50 (P5 / P95 beside it) over `reps`
        # replays (>= 300 layer calls).
        seq = calls * max(1, -(-48 // len(calls)))
        n_rep = max(reps, -(-300 // len(seq)))
        per = [ms * 1e3 / len(seq)
               for ms in _graph_times(lambda: [c() for c in seq], n_rep, warmup_ms=WARMUP_MS)]
        us = pct(per, 50)
        gbps = bytes_per_call / (us * 1e-6) / 1e9
        rows.append({"config": name, "batch": T, "layers_rotated": n_layers,
                     "calls_per_graph": len(seq), "layer_calls_timed": len(seq) * n_rep,
                     "us_per_layer": round(us, 2), "p5_us": round(pct(per, 5), 2),
                     "p95_us": round(pct(per, 95), 2),
                     "mean_us": round(sum(per) / len(per), 2),
                     "tokens_per_s": round(T / (us * 1e-6)),
                     "achieved_GBps": round(gbps, 1), "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4)})
        log(f"config {name} T={T}: {us:.2f} us/layer P50, {gbps:.0f} GB/s")
        return rows[-1]

    def routing_for(cfg, T, layer):
        ids, w = synth.routing(cfg, T, layer)
        return (torch.from_numpy(ids.astype(np.int32)).to(dev), torch.from_numpy(w).to(dev),
                ids)

    def int4_layers(cfg, n_layers):
        out = []
        for l in range(n_layers):
            w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                               synth.seed_for(cfg, l), dev)
            out.append(pack_experts_int4(w13) + pack_experts_int4(w2))
            del w13, w2
        return out

    def cpu_int4(name, T, x, layer, tid, tw):
        if cpu is not None:
            from oracle.cpu_baseline import int4_deq
            cpu_rows.append(cpu_config_row(name, T, x, int4_deq(*layer), (), tid, tw, cpu))

    def cpu_bank(name, T, x, bank, tid, tw):
        if cpu is not None:
            from oracle.cpu_baseline import bank_deq
            tensors = {n: getattr(bank, n) for n in (
                "bf16_w13", "bf16_w2", "int8_w13", "int8_w13_scales", "int8_w2",
                "int8_w2_scales", "int4_w13", "int4_w13_scales", "int4_w2", "int4_w2_scales")}
            tensors["n_experts"] = bank.n_experts
            routed, shared = bank_deq(bank.tier.tolist(), bank.index.tolist(), tensors,
                                      tid.reshape(-1).tolist())
            cpu_rows.append(cpu_config_row(name, T, x, routed, shared, tid, tw, cpu))

    # OLMoE single INT4 layer; 48 distinct seeded layers (9.3 GiB)
    # rotated, so no bank sits in the 256 MB Infinity Cache between its calls
    # (the same layers as the counter runs of profiles/)
    cfg = synth.CONFIGS["olmoe"]
    layers = int4_layers(cfg, 48)
    eb = synth.int4_expert_bytes(cfg.hidden, cfg.inter, cfg.group_size)
    w13_bytes = 2 * cfg.inter * cfg.hidden // 2 + 2 * cfg.inter * (cfg.hidden // cfg.group_size) * 2
    for T in ((16,) if north_star_only else (1, 16, 64)):
        x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 77 + T)).to(torch.bfloat16).to(dev)
        ws = ws_for(cfg, T)
        calls, nbytes, active, rts = [], 0, [], []
        for l, (p13, s13, p2, s2) in enumerate(layers):
            tid, tw, ids = routing_for(cfg, T, l)
            rts.append((tid, tw))
            active.append(np.unique(ids).size)
            nbytes += active[-1] * eb
            calls.append(lambda p13=p13, s13=s13, p2=p2, s2=s2, tw=tw, tid=tid, x=x, ws=ws:
                         fused_experts(x, p13, s13, p2, s2, tw, tid, workspace=ws))
        row = decode_row("olmoe", cfg, T, calls, nbytes / len(layers), len(layers))
        if T == 16:
            out = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device=dev)
            b = _Calls(x, [r[0] for r in rts], [r[1] for r in rts], out, ws)
            st = stage_times(layers, b, reps=max(3, -(-300 // len(layers))))
            kb = w13_bytes * sum(active) / len(active)
            kg = kb / (st["gateup_us"] * 1e-6) / 1e9
            north_star = dict(row)
            north_star.update({
                "active_experts_mean": round(sum(active) / len(active), 2),
                "roofline": {"bound": "hbm",
                             "kernel": "moe_decode_kernel<bf16, gate/up, NT=1, INT4 LDS path>",
                             "achieved": round(kg, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                             "frac": round(kg / HBM_PEAK_GBPS, 4),
                             "traffic": traffic_from_profile("olmoe", T),
                             "bytes_per_launch": round(kb), "launch_us": round(st["gateup_us"], 3)},
                "stages_us": {k: round(v, 3) for k, v in st.items()}})
            log(f"north star olmoe T=16: {row['us_per_layer']} us/layer, gate/up {kg:.0f} GB/s")
        cpu_int4("olmoe", T, x, layers[0], rts[0][0], rts[0][1])
    del layers
    torch.cuda.empty_cache()
    if north_star_only:
        return rows, north_star, cpu_rows

    # Mixed-precision OLMoE stack: 16 layers, BF16/INT8/INT4 per
    # expert from the quant-plan artifact (tiers ranked by the router's own
    # Zipf frequencies), read back with the artifact reader as a deployment would
    cfg = synth.CONFIGS["mixed_olmoe"]
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "mixed_olmoe_plan.json")
        with open(path, "w", encoding="utf-8") as f:
            _json.dump(synth.plan_artifact(cfg), f)
        plan = load_exq_artifact(path, device="cpu")
    banks = []
    for l in range(cfg.n_layers):
        w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                           synth.seed_for(cfg, l), dev)
        banks.append(MixedExpertBank.from_weights(w13, w2, plan.tiers[l].tolist()))
        del w13, w2
    T = 32
    x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 99)).to(torch.bfloat16).to(dev)
    ws = ws_for(cfg, T)
    calls, nbytes, share, rts = [], 0, [], []
    for l, bank in enumerate(banks):
        tid, tw, ids = routing_for(cfg, T, l)
        rts.append((tid, tw))
        used = np.unique(ids)
        b = [bank.stored_bytes(int(e)) for e in used]
        nbytes += sum(b)
        share.append(sum(v for e, v in zip(used, b) if int(bank.tier[int(e)]) == 0) / sum(b))
        calls.append(lambda bank=bank, tw=tw, tid=tid: fused_experts_mixed(x, bank, tw, tid,
                                                                         workspace=ws))
    row = decode_row("mixed_olmoe", cfg, T, calls, nbytes / len(banks), len(banks))
    row["plan"] = "artifact (router-ranked: top 10% BF16, next 20% INT8, rest INT4)"
    row["bf16_byte_share"] = round(sum(share) / len(share), 4)
    cpu_bank("mixed_olmoe", T, x, banks[0], rts[0][0], rts[0][1])
    del banks
    torch.cuda.empty_cache()

    # DeepSeek-V2-Lite: 64 INT4 routed experts + 2 BF16 shared
    cfg = synth.CONFIGS["deepseek_v2_lite"]
    banks = []
    for l in range(3):
        w13, w2 = synth.expert_weights_gpu(cfg.n_experts, cfg.inter, cfg.hidden,
                                           synth.seed_for(cfg, l), dev)
        s13, s2 = synth.expert_weights_gpu(cfg.n_shared, cfg.inter, cfg.hidden,
                                           synth.seed_for(cfg, l) + 500, dev)
        banks.append(MixedExpertBank.from_weights(w13, w2, [2] * cfg.n_experts, shared_w13=s13,
                                                  shared_w2=s2, shared_tier=0))
        del w13, w2, s13, s2
    shared_bytes = cfg.n_shared * synth.bf16_expert_bytes(cfg.hidden, cfg.inter)
    eb = synth.int4_expert_bytes(cfg.hidden, cfg.inter, cfg.group_size)
    for T in (1, 16, 64):
        x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 55 + T)).to(torch.bfloat16).to(dev)
        ws = ws_for(cfg, T)
        calls, nbytes, rts = [], 0, []
        for l, bank in enumerate(banks):
            tid, tw, ids = routing_for(cfg, T, l)
            rts.append((tid, tw))
            nbytes += np.unique(ids).size * eb + shared_bytes
            calls.append(lambda bank=bank, tw=tw, tid=tid, x=x, ws=ws:
                         fused_experts_mixed(x, bank, tw, tid, workspace=ws))
        decode_row("deepseek_v2_lite", cfg, T, calls, nbytes / len(banks), len(banks))
        if T != 16:
            cpu_bank("deepseek_v2_lite", T, x, banks[0], rts[0][0], rts[0][1])
    rows += prefill_rows([_prefill_call(dev, "deepseek_v2_lite", banks[0])], max(20, reps))
    del banks
    torch.cuda.empty_cache()

    # Mixtral-8x7B: 8 huge INT4 experts, top-2; 2 layers (1.45 GB)
    cfg = synth.CONFIGS["mixtral"]
    layers = int4_layers(cfg, 2)
    eb = synth.int4_expert_bytes(cfg.hidden, cfg.inter, cfg.group_size)
    for T in (1, 16, 64):
        x = torch.from_numpy(synth.hidden_np(T, cfg.hidden, 11 + T)).to(torch.bfloat16).to(dev)
        ws = ws_for(cfg, T)
        calls, nbytes, rts = [], 0, []
        for l, (p13, s13, p2, s2) in enumerate(layers):
            tid, tw, ids = routing_for(cfg, T, l)
            rts.append((tid, tw))
            nbytes += np.unique(ids).size * eb
            calls.append(lambda p13=p13, s13=s13, p2=p2, s2=s2, tw=tw, tid=tid, x=x, ws=ws:
                         fused_experts(x, p13, s13, p2, s2, tw, tid, workspace=ws))
        decode_row("mixtral", cfg, T, calls, nbytes / len(layers), len(layers))
        cpu_int4("mixtral", T, x, layers[0], rts[0][0], rts[0][1])
    rows += prefill_rows([_prefill_call(dev, "mixtral", layers[0])], max(20, reps))
    del layers
    torch.cuda.empty_cache()

    # Router (fp32 softmax -> top-k -> renormalise) on the seeded logits of
    # Qwen3 (128 experts, top-8) at decode and prefill batch sizes.
    from exq_amd.kernels import fused_topk
    cfg = synth.CONFIGS["qwen3"]
    for T in (16, 2048):
        lg = torch.from_numpy(synth.router_logits(cfg, T, synth.seed_for(cfg) + 7)).to(dev)
        n = 32  # calls per graph, so one graph launch is not charged to one call
        ms = _graph_time(lambda lg=lg: [fused_topk(lg, cfg.top_k, cfg.renormalize)
                                        for _ in range(n)], reps) / n
        rows.append({"config": "router_qwen3", "batch": T, "experts": cfg.n_experts,
                     "top_k": cfg.top_k, "calls_per_graph": n, "us_per_call": round(ms * 1e3, 2)})
        log(f"config router qwen3 T={T}: {ms * 1e3:.2f} us")
    rows += routing_rows(dev, reps)
    return rows, north_star, cpu_rows


def routing_rows(dev, reps):
    """The standalone stable sort (exq_dispatch, under sort_tokens_by_expert
    and moe_grouped_gemm) on seeded DeepSeek-V2-Lite ids: a decode batch (one
    work-group) and a 2048-token prefill chunk at top-6 and top-8 (12,288 and
    16,384 slots: the multi-block sort, one launch over 12 / 16 work-groups)."""
    import torch
    from exq_amd import synth
    from exq_amd.kernels.exq_dispatch import dispatch
    cfg = synth.CONFIGS["deepseek_v2_lite"]
    rows = []
    for T, k in ((16, 6), (2048, 6), (2048, 8)):
        c = synth.MoeConfig("routing", cfg.config_id, cfg.hidden, cfg.inter, cfg.n_experts, k,
                            False)
        ids, _ = synth.routing(c, T)
        t = torch.from_numpy(ids.reshape(-1)).to(dev)
        n_slots = ids.size
        so = torch.empty(n_slots, dtype=torch.int64, device=dev)
        si = torch.empty(n_slots, dtype=torch.int64, device=dev)
        ends = torch.empty(cfg.n_experts + 1, dtype=torch.int32, device=dev)
        n = 32  # calls per graph
        ms = _graph_time(lambda: [dispatch(t, so, si, ends, cfg.n_experts) for _ in range(n)],
                         reps) / n
        rows.append({"config": "dispatch_sort", "batch": T, "top_k": k, "slots": n_slots,
                     "experts": cfg.n_experts, "work_groups": 1 if n_slots <= 2048 else
                     min(128, -(-n_slots // 1024)), "calls_per_graph": n,
                     "us_per_call": round(ms * 1e3, 2)})
        log(f"config dispatch sort {n_slots} slots: {ms * 1e3:.2f} us")
    return rows


def stream_read_ceiling(dev, nbytes=2 << 30, reps=10):
    """HBM streaming-read rate (GB/s) of exq_stream_read over a buffer far
    larger than the 256 MB Infinity Cache: the read rate a kernel on this box
    can reach, beside the 8 TB/s data-sheet peak."""
    import torch
    from exq_amd import _lib
    L = _lib.lib()
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(8192, dtype=torch.int32, device=dev)
    stream = _lib.stream_handle(dev)

    def run():
        _lib.check(L.exq_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(), sink.numel(),
                                     stream), "exq_stream_read")
    for _ in range(2):
        run()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    cross = stream_cross_check(buf, reps)
    del buf, sink
    return {"GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes, "reps": reps,
            "kernel": "exq_stream_read (16-byte nontemporal loads, 8 in flight per thread)",
            "cross_check": cross}


def stream_cross_check(buf, reps):
    """Two other readers of the same buffer, timed the same way: torch's own
    reduction kernel (a float32 sum over the bytes, which reads every byte once
    and writes one value) and a device-to-device copy (torch's copy kernel; its
    rate counts the bytes read, with as many written beside them)."""
    import torch
    out = {}
    v = buf.view(torch.float32)
    v.sum()
    dst = torch.empty_like(buf)
    dst.copy_(buf)
    torch.cuda.synchronize()
    for name, fn in (("torch_sum_read_GBps", lambda: v.sum()),
                     ("d2d_copy_read_GBps", lambda: dst.copy_(buf))):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(buf.numel() / (e0.elapsed_time(e1) / reps * 1e-3) / 1e9, 1)
    del dst
    return out


def stream_read_at_size(dev, nbytes, n_bufs=48, reps=5, grid=2048):
    """Plain streaming read of `nbytes` (a kernel's bytes per launch) with
    exq_stream_read: n_bufs distinct buffers (together beyond the 256 MB
    Infinity Cache) read back to back in one HIP graph, as the decode layers
    are.  The time per read is the floor a kernel moving those bytes meets at
    this transfer size (launch and ramp included)."""
    import torch
    from exq_amd import _lib
    L = _lib.lib()
    nbytes = nbytes // 16 * 16
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(n_bufs)]
    sink = torch.zeros(grid, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()

    def run():
        h = s.cuda_stream
        for bb in bufs:
            _lib.check(L.exq_stream_read(bb.data_ptr(), nbytes, sink.data_ptr(), grid, h),
                       "exq_stream_read")
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * n_bufs)
    del g, bufs, sink
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "reads_timed": reps * n_bufs, "grid": grid}


def cpu_model():
    """The host CPU's model name as `lscpu` prints it (/proc/cpuinfo otherwise)."""
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10,
                           env={**os.environ, "LC_ALL": "C"})
        for line in r.stdout.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_threads():
    # the box's CPU share (OMP_NUM_THREADS), not every core the host reports
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def cpu_counts():
    """What the host reports beside the threads the baseline uses."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"os_cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_config_row(name, T, x, routed, shared, tid, tw, cpu):
    """Both variants of the reference CPU path on one configuration's layer:
    dequantise per call (reference-faithful) and pre-dequantised; plus, for
    context only, a vectorised per-expert grouping that is not the reference."""
    from oracle.cpu_baseline import time_cpu_experts
    row = {"config": name, "batch": T}
    for variant in ("dequant_per_call", "predequantized", "grouped"):
        r = time_cpu_experts(x, routed, tid, tw, shared, variant, reps=cpu["reps"], warmup=1,
                             threads=cpu["threads"], budget_s=cpu["budget_s"])
        row[variant] = {"p50_us": round(r["p50_us"], 1), "p5_us": round(r["p5_us"], 1),
                        "p95_us": round(r["p95_us"], 1), "reps": r["reps"],
                        "tokens_per_s": round(T / (r["p50_us"] * 1e-6), 1)}
    row["grouped"]["label"] = "context only: per-expert grouped matmuls, not the reference"
    log(f"cpu {name} T={T}: {row['dequant_per_call']['p50_us'] / 1e3:.1f} ms "
        f"(predequantized {row['predequantized']['p50_us'] / 1e3:.1f} ms, "
        f"grouped {row['grouped']['p50_us'] / 1e3:.1f} ms)")
    return row


def cpu_int4_bank(stack):
    from oracle.cpu_baseline import int4_deq
    return int4_deq(*stack.layers[0])


def cpu_baseline(deq, b, cpu):
    """The reference's PyTorch CPU path (oracle/cpu_baseline.py) on this host:
    the headline sample, Qwen3 layer 0 (dequantisers ``deq``) at the bench
    batch."""
    import torch
    row = cpu_config_row("qwen3", b.T, b.x, deq, (), b.ids[0], b.wts[0], cpu)
    d, p = row["dequant_per_call"], row["predequantized"]
    return {"value": d["p50_us"], "unit": "us/layer", "cores": cpu["threads"],
            "kind": "port",
            "sample": f"qwen3 layer 0, T={b.T}, {d['reps']} reps P50, dequant per call "
                      f"(pytorch_moe_reference loop, torch {torch.__version__} CPU fp32, "
                      f"{cpu['threads']} threads, {cpu_model()})",
            "p5_us": d["p5_us"], "p95_us": d["p95_us"],
            "predequantized_p50_us": p["p50_us"],
            "grouped_p50_us_not_reference": row["grouped"]["p50_us"],
            "cpu_model": cpu_model(), **cpu_counts()}


def main():
    from exq_amd.eval import latency_stats
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); sharding the experts over GPUs (an all-to-all of "
              "token rows before and after the expert kernels) is not built", file=sys.stderr)
        sys.exit(2)
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    import torch
    from exq_amd import synth
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    cfg = synth.CONFIGS["qwen3" if not args.pmc_run else args.config]
    if args.north_star_only:  # the OLMoE T=16 line alone (profiles)
        _, ns, _ = measure_configs(dev, max(20, args.steps), None, north_star_only=True)
        print(json.dumps({"north_star": ns}), flush=True)
        return
    if args.routing_only:  # the standalone sort alone (profiles)
        print(json.dumps({"routing": routing_rows(dev, max(5, args.steps // 5))}), flush=True)
        return
    if args.prefill_only:  # the MFMA-path configurations alone (profiles, counter runs)
        rows = []
        for name in ("deepseek_v2_lite", "mixtral"):
            call = _prefill_call(dev, name)
            if args.eager:
                call[2]()
                torch.cuda.synchronize()
                log(f"{name} prefill: one eager call")
            else:
                rows += prefill_rows([call], max(20, args.steps))
            del call
            torch.cuda.empty_cache()
        if rows:
            print(json.dumps({"prefill": rows}), flush=True)
        return
    if args.pmc_run:
        src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {CALIB_BYTES} bytes read, {CALIB_BYTES} written")
        del src, dst
    t0 = time.time()
    stack = Stack(cfg, args.layers, dev)
    log(f"packed {args.layers} layers in {time.time() - t0:.1f}s "
        f"({args.layers * cfg.n_experts * stack.expert_bytes / 2**30:.2f} GiB)")
    use_graph = not args.no_graph

    b = Batch(stack, args.batch, dev)
    if args.pmc_run:
        for _ in range(max(1, args.passes)):
            run_step(stack, b)
        torch.cuda.synchronize()
        log(f"{max(1, args.passes)} eager pass(es) of {args.layers} layers at T={args.batch}; "
            f"activated experts per layer {sum(b.active) / len(b.active):.2f}")
        return
    ms, wall, per = time_steps(stack, b, args.steps, args.warmup, use_graph)
    per_layer = [m * 1e3 / args.layers for m in per]  # µs/layer of each step
    us_layer = pct(per_layer, 50)
    gbps = b.bytes / (us_layer * args.layers * 1e-6) / 1e9
    log(f"T={args.batch}: {ms:.3f} ms/step mean, {us_layer:.2f} us/layer P50 "
        f"(P5 {pct(per_layer, 5):.2f}, P95 {pct(per_layer, 95):.2f}), {gbps:.0f} GB/s "
        f"(host wall {wall:.3f} ms/step)")
    st = stage_times(stack.layers, b, reps=max(1, -(-300 // args.layers)))
    log(f"stage events: {st}")
    # Dominant kernel: the gate/up decode kernel (events 0 -> 1 time it on the
    # call's stream); its algorithmic bytes are the activated experts'
    # gate/up weights + fp16 scales (2I*H/2 + 2I*(H/128)*2 bytes per expert).
    kern_us = st["gateup_us"]
    kern_bytes = stack.w13_bytes * sum(b.active) / len(b.active)
    kern_gbps = kern_bytes / (kern_us * 1e-6) / 1e9
    traffic = traffic_from_profile("qwen3", args.batch)
    ceiling = stream_read_ceiling(dev)
    log(f"streaming-read ceiling: {ceiling['GBps']:.0f} GB/s")
    floor = stream_read_at_size(dev, int(kern_bytes))
    log(f"streaming read of the kernel's {floor['bytes']} bytes: {floor['us']:.2f} us "
        f"({floor['GBps']:.0f} GB/s)")

    sweep = []
    for T in [int(v) for v in args.sweep.split(",") if v.strip()]:
        bb = b if T == args.batch else Batch(stack, T, dev)
        _, _, pr = time_steps(stack, bb, max(10, args.steps // 2), args.warmup, use_graph,
                              warmup_ms=WARMUP_MS)
        pl = [m * 1e3 / args.layers for m in pr]
        ul = pct(pl, 50)
        g = bb.bytes / (ul * args.layers * 1e-6) / 1e9
        sweep.append({"batch": T, "us_per_layer": round(ul, 2), "p5_us": round(pct(pl, 5), 2),
                      "p95_us": round(pct(pl, 95), 2), "layer_calls_timed": len(pl) * args.layers,
                      "tokens_per_s": round(T / (ul * 1e-6)),
                      "active_experts_mean": round(sum(bb.active) / len(bb.active), 2),
                      "achieved_GBps": round(g, 1), "frac_of_peak": round(g / HBM_PEAK_GBPS, 4)})
        log(f"sweep T={T}: {ul:.2f} us/layer P50, {g:.0f} GB/s")
        if bb is not b:
            del bb
    cpu_set = None if args.no_cpu else {"threads": cpu_threads(), "reps": args.cpu_reps,
                                        "budget_s": args.cpu_budget}
    cpu, cpu_rows = None, []
    if cpu_set is not None:
        t1 = time.time()
        deq = cpu_int4_bank(stack)
        cpu = cpu_baseline(deq, b, cpu_set)
        for T in [int(v) for v in args.sweep.split(",") if v.strip()]:
            if T == args.batch:
                continue
            bb = Batch(stack, T, dev)
            cpu_rows.append(cpu_config_row("qwen3", T, bb.x, deq, (), bb.ids[0], bb.wts[0],
                                           cpu_set))
            del bb
        del deq
        log(f"cpu baseline {cpu['value']} us/layer in {time.time() - t1:.1f}s")
    configs, north_star = None, None
    if not args.no_configs:
        t1 = time.time()
        configs, north_star, more = measure_configs(dev, max(20, args.steps), cpu_set)
        cpu_rows += more
        log(f"configs measured in {time.time() - t1:.1f}s")
    if cpu is not None:
        cpu["configs"] = cpu_rows

    out = {
        "metric": METRIC,
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "weights": "int4 (g=128, fp16 scales)",
        "data": "synthetic (seeded fp16 N(0,0.02) weights RTN-packed to INT4; bf16 N(0,1) "
                "activations; Zipf(1.1)-biased softmax top-8 routing)",
        "config": {"workload": f"Qwen3-30B-A3B-shaped INT4 MoE layer x{args.layers} distinct "
                               f"layers streamed, decode batch {args.batch}",
                   "batch": args.batch, "layers": args.layers, "hidden": cfg.hidden,
                   "inter": cfg.inter, "experts": cfg.n_experts, "top_k": cfg.top_k,
                   "launch": "hip-graph replay" if use_graph else "eager"},
        "statistic": f"P50 of per-step µs/layer over {args.steps} steps "
                     f"({args.steps * args.layers} layer calls)",
        "p5_us": round(pct(per_layer, 5), 3),
        "p95_us": round(pct(per_layer, 95), 3),
        # the reference harness's statistics (exq/eval/bench.py) of the same series
        "latency_stats_us": {k: (round(v, 3) if isinstance(v, float) else v)
                             for k, v in latency_stats(per_layer).items()},
        "mean_us": round(ms * 1e3 / args.layers, 3),
        "tokens_per_s": round(args.batch / (us_layer * 1e-6)),
        "achieved_GBps": round(gbps, 1),
        "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm",
                     "kernel": "moe_decode_kernel<bf16, gate/up, NT=1, INT4 LDS path>",
                     "achieved": round(kern_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(kern_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "bytes_per_launch": round(kern_bytes), "launch_us": round(kern_us, 3),
                     "frac_of_stream_ceiling": round(kern_gbps / ceiling["GBps"], 4),
                     "stream_read_same_bytes_us": floor["us"],
                     "frac_of_stream_same_bytes": round(floor["us"] / kern_us, 4)},
        "stream_read_ceiling": ceiling,
        "stream_read_same_bytes": floor,
        "stages_us": {k: round(v, 3) for k, v in st.items()},
        "north_star": north_star,
        "sweep": sweep,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

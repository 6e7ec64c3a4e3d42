"""Seeded synthetic MoE workloads (the configurations benchmarked for this path).

* weights: fp16 N(0, 0.02), gate/up bank [E, 2I, H] and down bank [E, H, I];
* activations: bf16 N(0, 1) [T, H];
* router logits: N(0, 1) + ln p_pi(e) with p_r proportional to r^-1.1 (Zipf
  s = 1.1) over a seeded expert permutation pi (plain N(0, 1) for the
  near-uniform Mixtral case); fp32 softmax, top-k with ties to the lower
  expert id, renormalised where the model does so (Qwen3, Mixtral);
* seeds: ``1000 * config_id + layer``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class MoeConfig:
    name: str
    config_id: int
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    renormalize: bool
    zipf: bool = True
    n_shared: int = 0
    n_layers: int = 1
    group_size: int = 128


CONFIGS = {
    "olmoe": MoeConfig("olmoe", 0, 2048, 1024, 64, 8, False),
    "qwen3": MoeConfig("qwen3", 1, 2048, 768, 128, 8, True, n_layers=48),
    "mixed_olmoe": MoeConfig("mixed_olmoe", 2, 2048, 1024, 64, 8, False, n_layers=16),
    "deepseek_v2_lite": MoeConfig("deepseek_v2_lite", 3, 2048, 1408, 64, 6, False, n_shared=2),
    "mixtral": MoeConfig("mixtral", 4, 4096, 14336, 8, 2, True, zipf=False),
}


def seed_for(cfg: MoeConfig, layer: int = 0) -> int:
    return 1000 * cfg.config_id + layer


def zipf_bias(n_experts: int, rng: np.random.Generator, s: float = 1.1) -> np.ndarray:
    perm = rng.permutation(n_experts)
    p = (perm + 1.0) ** (-s)
    p /= p.sum()
    return np.log(p).astype(np.float32)


def router_logits(cfg: MoeConfig, T: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    bias = zipf_bias(cfg.n_experts, rng) if cfg.zipf else np.zeros(cfg.n_experts, np.float32)
    return (rng.standard_normal((T, cfg.n_experts)).astype(np.float32) + bias).astype(np.float32)


def softmax_topk(logits: np.ndarray, top_k: int, renormalize: bool):
    """fp32 softmax, top-k (stable: ties to the lower id), optional renorm."""
    lg = np.asarray(logits, dtype=np.float32)
    ex = np.exp(lg - lg.max(axis=-1, keepdims=True), dtype=np.float32)
    p = (ex / ex.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    ids = np.argsort(-p, axis=-1, kind="stable")[:, :top_k]
    w = np.take_along_axis(p, ids, axis=-1)
    if renormalize:
        w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return ids.astype(np.int64), w.astype(np.float32)


def routing(cfg: MoeConfig, T: int, layer: int = 0):
    """(topk_ids int64 [T, k], topk_weights f32 [T, k]) for a seeded batch."""
    return softmax_topk(router_logits(cfg, T, seed_for(cfg, layer) + 7), cfg.top_k,
                        cfg.renormalize)


def hidden_np(T: int, H: int, seed: int) -> np.ndarray:
    """bf16-representable N(0, 1) activations as float32."""
    x = np.random.default_rng(seed + 3).standard_normal((T, H)).astype(np.float32)
    return torch.from_numpy(x).to(torch.bfloat16).float().numpy()


def expert_weights_np(E: int, I: int, H: int, seed: int):
    """fp16 N(0, 0.02) banks w13 [E, 2I, H], w2 [E, H, I] (CPU, small shapes)."""
    rng = np.random.default_rng(seed)
    w13 = (rng.standard_normal((E, 2 * I, H), dtype=np.float32) * 0.02).astype(np.float16)
    w2 = (rng.standard_normal((E, H, I), dtype=np.float32) * 0.02).astype(np.float16)
    return w13, w2


def expert_weights_gpu(E: int, I: int, H: int, seed: int, device="cuda"):
    """fp16 N(0, 0.02) banks generated on the device (large shapes)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    w13 = torch.randn(E, 2 * I, H, generator=g, device=device, dtype=torch.float16)
    w13.mul_(0.02)
    w2 = torch.randn(E, H, I, generator=g, device=device, dtype=torch.float16)
    w2.mul_(0.02)
    return w13, w2


def mixed_tiers(n_experts: int, seed: int, bf16_frac: float = 0.1,
                int8_frac: float = 0.2) -> list[int]:
    """Per-expert tiers from seeded Zipf activation frequencies: the most
    frequent 10% BF16 (0), the next 20% INT8 (1), the rest INT4 (2)."""
    rng = np.random.default_rng(seed + 11)
    freq = np.exp(zipf_bias(n_experts, rng))
    order = np.argsort(-freq, kind="stable")
    n_bf = int(round(bf16_frac * n_experts))
    n_i8 = int(round(int8_frac * n_experts))
    tiers = [2] * n_experts
    for r, e in enumerate(order):
        tiers[int(e)] = 0 if r < n_bf else (1 if r < n_bf + n_i8 else 2)
    return tiers


def router_tiers(cfg: MoeConfig, layer: int = 0, bf16_frac: float = 0.1,
                 int8_frac: float = 0.2) -> list[int]:
    """Per-expert tiers of a layer ranked by the router's own Zipf activation
    frequencies (the permutation ``router_logits`` draws first for this layer):
    the most frequently routed 10% BF16 (0), the next 20% INT8 (1), the rest
    INT4 (2), so the hot tier is the set of experts the router favours."""
    rng = np.random.default_rng(seed_for(cfg, layer) + 7)
    freq = np.exp(zipf_bias(cfg.n_experts, rng))
    order = np.argsort(-freq, kind="stable")
    n_bf = int(round(bf16_frac * cfg.n_experts))
    n_i8 = int(round(int8_frac * cfg.n_experts))
    tiers = [2] * cfg.n_experts
    for r, e in enumerate(order):
        tiers[int(e)] = 0 if r < n_bf else (1 if r < n_bf + n_i8 else 2)
    return tiers


def plan_artifact(cfg: MoeConfig, n_layers: int | None = None) -> dict:
    """Quant-plan artifact of the mixed stack in the reference's format
    (``quant_assignments`` {"L:E": "BF16" | "INT8" | "INT4"}), tiers from
    ``router_tiers`` of each layer."""
    names = {0: "BF16", 1: "INT8", 2: "INT4"}
    qa = {}
    for l in range(cfg.n_layers if n_layers is None else n_layers):
        for e, t in enumerate(router_tiers(cfg, l)):
            qa[f"{l}:{e}"] = names[t]
    return {"model": f"synthetic-{cfg.name}", "quant_assignments": qa}


def int4_expert_bytes(H: int, I: int, g: int = 128) -> int:
    return 3 * H * I // 2 + 2 * (2 * I * (H // g) + H * (I // g))


def int8_expert_bytes(H: int, I: int) -> int:
    return 3 * H * I + 2 * (2 * I + H)


def bf16_expert_bytes(H: int, I: int) -> int:
    return 3 * H * I * 2

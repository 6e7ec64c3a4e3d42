"""ExQ artifact (compiled quant plan) reader.

Mirrors exq/kernels/exq_artifact.py of the reference: the tier codes
(25-26), the BLOCK_M schedule (32-45), ``ExpertProfile`` (48-93) and
``load_exq_artifact`` (96-192), plus the legacy ``quant_plan`` key accepted
by the reference's second reader (exq/model_utils.py:138-144).

Artifact JSON (written by scripts/compile_model.py:91-101 of the reference):
``{"model_id": ..., "quant_assignments": {"<layer>:<expert>": "BF16"|"INT8"|"INT4"}, ...}``
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

PRECISION_TO_INT = {"BF16": 0, "INT8": 1, "INT4": 2}
INT_TO_PRECISION = {0: "BF16", 1: "INT8", 2: "INT4"}

# BLOCK_M by tier: BF16 128, INT8 64, INT4 32 (the reference's decode tiling
# hint; the HIP kernels tile by tokens-per-expert themselves).
_TIER_TO_BLOCK_M = {0: 128, 1: 64, 2: 32}
# Frequencies assumed per tier when no routing profile is found.
_TIER_TO_FREQ = {0: 0.15, 1: 0.05, 2: 0.01}


def freq_to_block_m(freq: float, tier: int) -> int:
    """Recommended BLOCK_M for an expert: INT8 experts split at freq 0.03."""
    if tier == 1:
        return 64 if freq >= 0.03 else 32
    return _TIER_TO_BLOCK_M[tier]


@dataclass
class ExpertProfile:
    """Per-layer expert metadata as [n_layers, n_experts] tensors."""

    n_layers: int
    n_experts_per_layer: int
    tiers: torch.Tensor      # int8: 0=BF16, 1=INT8, 2=INT4
    freqs: torch.Tensor      # float32 activation frequency
    block_m: torch.Tensor    # int32
    hot_mask: torch.Tensor   # bool: BF16 tier

    @property
    def n_experts_total(self) -> int:
        return self.n_layers * self.n_experts_per_layer

    def layer_profile(self, layer_idx: int) -> dict:
        return {"tiers": self.tiers[layer_idx], "freqs": self.freqs[layer_idx],
                "block_m": self.block_m[layer_idx], "hot_mask": self.hot_mask[layer_idx]}

    def hot_expert_count(self, layer_idx: int) -> int:
        return int(self.hot_mask[layer_idx].sum().item())

    def expected_memory_ratio(self) -> float:
        """Mean weight footprint relative to all-BF16 (1, 1/2, 1/4 per tier)."""
        ratios = torch.tensor([1.0, 0.5, 0.25], device=self.tiers.device)
        return float(ratios[self.tiers.long()].mean().item())

    def precision_counts(self) -> dict[str, int]:
        return {name: int((self.tiers == t).sum().item()) for t, name in INT_TO_PRECISION.items()}

    def block_m_distribution(self) -> dict[int, int]:
        vals, counts = torch.unique(self.block_m.flatten().cpu(), return_counts=True)
        return {int(v): int(c) for v, c in zip(vals.tolist(), counts.tolist())}


def _parse_key(key: str) -> tuple[int, int]:
    l_str, e_str = key.split(":")
    return int(l_str), int(e_str)


def _assignments(artifact: dict) -> dict:
    return artifact.get("quant_assignments") or artifact.get("quant_plan") or {}


def load_exq_artifact(artifact_path: str, profile_path: str | None = None,
                      device: str = "cuda") -> ExpertProfile:
    """Read an artifact (and optionally a routing profile) into an ExpertProfile.

    Rules: the layer/expert grid spans the largest ids seen; experts missing
    from the plan, and unknown precision strings, default to INT4; an
    artifact without assignments raises ValueError.  Frequencies come from
    ``profile_path`` (or ``profiles/<artifact stem>.json``, then
    ``profiles/olmoe-1b-7b-0924-256.json``, relative to the working
    directory); without a profile each tier gets a fixed frequency.
    """
    with open(artifact_path, encoding="utf-8") as f:
        artifact = json.load(f)
    assignments = _assignments(artifact)
    if not assignments:
        raise ValueError(f"Artifact at {artifact_path} has no quant_assignments")

    keys = [_parse_key(k) for k in assignments]
    n_layers = max(l for l, _ in keys) + 1
    n_experts = max(e for _, e in keys) + 1
    tiers = np.full((n_layers, n_experts), PRECISION_TO_INT["INT4"], dtype=np.int8)
    for (l, e), prec in zip(keys, assignments.values()):
        tiers[l, e] = PRECISION_TO_INT.get(prec, PRECISION_TO_INT["INT4"])

    freqs = np.zeros((n_layers, n_experts), dtype=np.float32)
    candidates = [profile_path]
    if profile_path is None:
        stem = Path(artifact_path).stem
        candidates += [str(Path("profiles") / f"{stem}.json"),
                       str(Path("profiles") / "olmoe-1b-7b-0924-256.json")]
    loaded = False
    for cand in candidates:
        if cand and Path(cand).exists():
            with open(cand, encoding="utf-8") as f:
                prof = json.load(f)
            for l_str, layer in prof.get("layers", {}).items():
                l = int(l_str)
                if l >= n_layers:
                    continue
                for st in layer.get("expert_stats", []):
                    e = st.get("expert_id", 0)
                    if e < n_experts:
                        freqs[l, e] = float(st.get("activation_freq", 0.0))
            loaded = True
            break
    if not loaded:
        for t, fq in _TIER_TO_FREQ.items():
            freqs[tiers == t] = fq

    block_m = np.empty((n_layers, n_experts), dtype=np.int32)
    for l in range(n_layers):
        for e in range(n_experts):
            block_m[l, e] = freq_to_block_m(float(freqs[l, e]), int(tiers[l, e]))

    return ExpertProfile(
        n_layers=n_layers,
        n_experts_per_layer=n_experts,
        tiers=torch.from_numpy(tiers).to(device),
        freqs=torch.from_numpy(freqs).to(device),
        block_m=torch.from_numpy(block_m).to(device),
        hot_mask=torch.from_numpy(tiers == PRECISION_TO_INT["BF16"]).to(device),
    )


def layer_tiers(artifact_path: str, layer_id: int, n_experts: int) -> list[int] | None:
    """Tier list of one layer from an artifact, or None if the layer is absent.

    Experts of a covered layer that the plan omits are INT4.
    """
    with open(artifact_path, encoding="utf-8") as f:
        assignments = _assignments(json.load(f))
    tiers = [PRECISION_TO_INT["INT4"]] * n_experts
    seen = False
    for key, prec in assignments.items():
        l, e = _parse_key(key)
        if l == layer_id and e < n_experts:
            tiers[e] = PRECISION_TO_INT.get(prec, PRECISION_TO_INT["INT4"])
            seen = True
    return tiers if seen else None


def print_profile_summary(profile: ExpertProfile) -> None:
    print(f"Expert profile: {profile.n_layers} layers x {profile.n_experts_per_layer} experts "
          f"({profile.n_experts_total} total)")
    c = profile.precision_counts()
    print(f"Precision: {c.get('BF16', 0)} BF16  {c.get('INT8', 0)} INT8  {c.get('INT4', 0)} INT4")
    print(f"Memory vs all-BF16: {profile.expected_memory_ratio():.1%}")
    print(f"BLOCK_M distribution: {profile.block_m_distribution()}")

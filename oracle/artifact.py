"""Quant-plan artifact rules restated on the CPU.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import numpy as np

PRECISION_TO_INT = {"BF16": 0, "INT8": 1, "INT4": 2}


def freq_to_block_m(freq: float, tier: int) -> int:
    """exq_artifact.py:32-45: BF16 128, INT8 64 (freq >= 0.03) else 32, INT4 32.

    pinned by: the reference's table restated as known answers.
    """
    if tier == 0:
        return 128
    if tier == 1:
        return 64 if freq >= 0.03 else 32
    return 32


def tiers_from_assignments(assignments: dict) -> np.ndarray:
    """exq_artifact.py:124-138: grid from max ids, default INT4, unknown -> INT4."""
    if not assignments:
        raise ValueError("artifact has no quant_assignments")
    ls, es = set(), set()
    for key in assignments:
        l, e = key.split(":")
        ls.add(int(l))
        es.add(int(e))
    tiers = np.full((max(ls) + 1, max(es) + 1), 2, dtype=np.int8)
    for key, prec in assignments.items():
        l, e = map(int, key.split(":"))
        tiers[l, e] = PRECISION_TO_INT.get(prec, 2)
    return tiers


def tier_fallback_freqs(tiers: np.ndarray) -> np.ndarray:
    """exq_artifact.py:168-173: BF16 0.15, INT8 0.05, INT4 0.01."""
    lut = np.array([0.15, 0.05, 0.01], dtype=np.float32)
    return lut[tiers.astype(np.int64)]

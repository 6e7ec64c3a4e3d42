"""Writes the small golden fixtures of the MoE dispatch path (tests/golden/*.npz).

The reference holds no golden vectors for this path, so the fixtures come from
this repository's CPU oracle (``oracle/``), itself pinned by known answers and
brute force in tests/test_oracle_*.py.  They freeze the oracle's outputs so that
any later change to it, or to the HIP path, is caught against fixed data.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import moe, quant, routing  # noqa: E402


def tiny_layer(seed=2024, E=4, H=256, I=128, T=3, k=2):
    rng = np.random.default_rng(seed)
    w13 = (rng.standard_normal((E, 2 * I, H), dtype=np.float32) * 0.02).astype(np.float16)
    w2 = (rng.standard_normal((E, H, I), dtype=np.float32) * 0.02).astype(np.float16)
    w13[1, 5] = 0  # an all-zero row: scale floor, nibbles 8
    p13, s13 = quant.pack_experts_int4(w13)
    p2, s2 = quant.pack_experts_int4(w2)
    # bf16-representable activations (round-to-nearest-even of N(0,1) draws)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xb = x.view(np.uint32)
    xb = ((xb + 0x7FFF + ((xb >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    x = xb.view(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids, wts = routing.route_softmax_topk(logits, k, renormalize=False)
    so, ends, max_tok = routing.sort_tokens_by_expert(ids, E)
    s_ids, e_blk, ntpp, cumsum = routing.moe_align_block_size(ids, E + 1, 16)
    ends2, so2 = routing.build_ends_from_slots(s_ids, ids.reshape(-1), T * k, E)
    y = moe.moe_layer(x, quant.dequant_int4(p13, s13), quant.dequant_int4(p2, s2), ids, wts,
                      accum=np.float64)
    return dict(w13_src=w13[:, :16], w13_packed=p13, w13_scales=s13, w2_packed=p2,
                w2_scales=s2, hidden=x, topk_ids=ids, topk_weights=wts, sort_order=so,
                expert_ends=ends, max_tok=np.array([max_tok]), align_sorted_ids=s_ids,
                align_expert_ids=e_blk, align_ntpp=ntpp, align_cumsum=cumsum,
                slots_expert_ends=ends2, slots_sort_order=so2, out=y.astype(np.float64))


def pack_cases(seed=7):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((6, 384)) * 0.02).astype(np.float16)
    w[2] = 0
    w[3, :128] = np.float16(1e-3)
    w[4, 7] = np.float16(0.5)  # a lone large weight: every other nibble near 8
    p, s = quant.pack_int4_weights(w)
    wi = (rng.standard_normal((5, 200)) * 0.02).astype(np.float16)
    wi[1] = 0
    q8, s8 = quant.quantize_int8(wi)
    return dict(w=w, packed=p, scales=s, w_int8=wi, q_int8=q8, s_int8=s8)


def main():
    np.savez_compressed(os.path.join(HERE, "tiny_layer.npz"), **tiny_layer())
    np.savez_compressed(os.path.join(HERE, "pack_cases.npz"), **pack_cases())
    for f in ("tiny_layer.npz", "pack_cases.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()

"""Weight quantisation restated on the CPU (numpy, IEEE float32).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import numpy as np

# torch.finfo(torch.float32).eps, used as the scale floor by the reference.
FP32_EPS = np.float32(np.finfo(np.float32).eps)


def effective_group_size(K: int, group_size: int = 128) -> int:
    """Group-size rule of moe_int4_kernel.py:58-69.

    K must be even; K < group_size collapses to a single group of K; otherwise
    K must be divisible by group_size.

    pinned by: tests/test_oracle_quant.py::test_group_rule_* (hand-derived
    cases incl. the K<g collapse and both ValueError paths).
    """
    if K % 2 != 0:
        raise ValueError(f"K={K} must be divisible by 2 for INT4 packing")
    if K < group_size:
        group_size = K
    if K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    return group_size


def pack_int4_weights(weights: np.ndarray, group_size: int = 128):
    """INT4 RTN packing, restating moe_int4_kernel.py:37-93.

    * per (row, group): scale = max|w| / 7 in float32, floored at fp32 eps
      (lines 77-78);
    * q = round_half_even(w / scale) clamped to [-8, 7] (lines 80-82);
    * nibble = q + 8; low nibble = even k, high nibble = odd k (lines 87-89);
    * scales are stored as float16 (line 91).

    Returns ``(packed uint8 [N, K//2], scales float16 [N, K//g])``.

    pinned by: hand-derived known answers (byte 0x1F for w=[1,-1], half-even
    ties 2.5->2 and 3.5->4, the zero-row scale fp16(2^-23)), the invariants
    nibble in [1,15] and |w - deq| <= scale/2, and an element-by-element
    Python brute force on tiny inputs, g = 128, the K < g collapse and g = 32
    (tests/test_oracle_quant.py::test_pack_matches_elementwise_brute_force).
    """
    w = np.asarray(weights)
    N, K = w.shape
    g = effective_group_size(K, group_size)
    ng = K // g
    w32 = w.astype(np.float32).reshape(N, ng, g)
    scales32 = (np.abs(w32).max(axis=-1) / np.float32(7.0)).astype(np.float32)
    scales32 = np.maximum(scales32, FP32_EPS)
    q = np.rint(w32 / scales32[..., None])
    q = np.clip(q, -8, 7).astype(np.int8).reshape(N, K)
    lo = (q[:, 0::2] + 8).astype(np.uint8)
    hi = (q[:, 1::2] + 8).astype(np.uint8)
    packed = (lo | (hi << np.uint8(4))).astype(np.uint8)
    return np.ascontiguousarray(packed), scales32.astype(np.float16)


def pack_experts_int4(expert_weights: np.ndarray, group_size: int = 128):
    """Per-expert loop + stack, restating moe_int4_kernel.py:96-119.

    pinned by: equality with per-expert pack_int4_weights (the stack is the
    whole algorithm) and the reference's INT4 byte counts 3*H*I/2 per expert
    (tests/test_stress.py:770, 796 of the reference).
    """
    E = expert_weights.shape[0]
    outs = [pack_int4_weights(expert_weights[e], group_size) for e in range(E)]
    return (np.stack([o[0] for o in outs]), np.stack([o[1] for o in outs]))


def dequant_int4(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """fp32 nibble dequant with the stored fp16 scales (scripts/bench_int4.py:62-78).

    ``packed [..., N, K//2] uint8``, ``scales [..., N, K//g] float16`` ->
    ``float32 [..., N, K]`` with w[k] = (nibble_k - 8) * float(scale[k // g]).
    Every product is exact in float32 (4-bit integer times an fp16 value).

    pinned by: round trip against pack_int4_weights known answers and the
    bound |w - deq| <= scale/2 (tests/test_oracle_quant.py).
    """
    p = np.asarray(packed).astype(np.uint8, copy=False)
    s = np.asarray(scales).astype(np.float32)
    K = p.shape[-1] * 2
    ng = s.shape[-1]
    g = K // ng
    # byte -> (low nibble - 8, high nibble - 8): one table lookup per byte puts
    # the even-k and odd-k values side by side in k order
    w = _NIBBLE_PAIRS[p].reshape(p.shape[:-1] + (ng, g))
    w *= s[..., None]
    return w.reshape(p.shape[:-1] + (K,))


_NIBBLE_PAIRS = np.stack([(np.arange(256) & 0x0F) - 8.0, (np.arange(256) >> 4) - 8.0],
                         axis=-1).astype(np.float32)


def quantize_int8(weights: np.ndarray):
    """INT8 per-output-channel RTN, restating quant_shim.py:84-96.

    scale = max_k |w| / 127 (float32, floored at fp32 eps); q = round(w/scale)
    clamped to [-128, 127].  The build stores ``q`` as int8 and the scale as
    float16 (the same storage rule the reference applies to INT4 scales,
    moe_int4_kernel.py:91); the dequantised weight is q * float(fp16 scale).

    Returns ``(q int8 [..., N, K], scales float16 [..., N])``.

    pinned by: the reference's own zero-row test (tests/test_eval.py:158-163 of
    the reference: zero rows stay finite and exact), hand-derived known
    answers (max element -> +-127, half-even ties) and |w - deq| <= scale/2.
    """
    w32 = np.asarray(weights).astype(np.float32)
    scale = (np.abs(w32).max(axis=-1, keepdims=True) / np.float32(127.0)).astype(np.float32)
    scale = np.maximum(scale, FP32_EPS)
    q = np.clip(np.rint(w32 / scale), -128, 127).astype(np.int8)
    return q, scale[..., 0].astype(np.float16)


def dequant_int8(q: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """q * float(fp16 per-row scale) in float32 (exact products).

    pinned by: known answers with distinct per-row scales, 2-D and batched
    (tests/test_oracle_quant.py::test_dequant_int8_per_row_scales_known_answer).
    """
    return (np.asarray(q).astype(np.float32)
            * np.asarray(scales).astype(np.float32)[..., None]).astype(np.float32)


def fake_quant_int8(weights: np.ndarray) -> np.ndarray:
    """quant_shim.py:84-96 verbatim semantics (fp32 scale, output in input dtype).

    pinned by: the reference's zero-row known answer (test_eval.py:158-163) and
    hand-derived answers with four distinct per-row scales (one exact in fp32
    but not in fp16, one set by the fp32-eps clamp) and half-way ties
    (tests/test_oracle_quant.py::test_fake_quant_int8_known_answers_per_row_scales).
    """
    w = np.asarray(weights)
    if w.ndim == 0:  # torch reduces a 0-dim tensor over dim -1 as one element
        return fake_quant_int8(w.reshape(1)).reshape(())
    w32 = w.astype(np.float32)
    scale = np.maximum(np.abs(w32).max(axis=-1, keepdims=True) / np.float32(127.0), FP32_EPS)
    q = np.clip(np.rint(w32 / scale), -128, 127)
    return (q * scale).astype(w.dtype)


def fake_quant_int4(weights: np.ndarray, group_size: int = 128) -> np.ndarray:
    """quant_shim.py:99-125 semantics: pad K to a multiple of g, per-group RTN.

    pinned by: the reference's zero-row known answer (test_eval.py:151-155) and
    agreement with pack->dequant up to the fp16 rounding of the scale.
    """
    w = np.asarray(weights)
    shape = w.shape
    if w.ndim == 0:  # quant_shim.py:108 reads shape[-1]
        raise IndexError("fake_quant_int4: a 0-dim array has no last dimension")
    w32 = w.astype(np.float32)
    pad = (-shape[-1]) % group_size
    if pad:
        w32 = np.pad(w32, [(0, 0)] * (w32.ndim - 1) + [(0, pad)])
    gw = w32.reshape(-1, group_size)
    scale = np.maximum(np.abs(gw).max(axis=-1, keepdims=True) / np.float32(7.0), FP32_EPS)
    q = np.clip(np.rint(gw / scale), -8, 7)
    deq = (q * scale).reshape(w32.shape)[..., :shape[-1]]
    return deq.astype(w.dtype)


def int4_expert_bytes(H: int, I: int, group_size: int = 128) -> int:
    """Stored bytes of one INT4 expert (w13 + w2, packed weights + fp16 scales)."""
    g1 = effective_group_size(H, group_size)
    g2 = effective_group_size(I, group_size)
    return 2 * I * H // 2 + 2 * I * (H // g1) * 2 + H * I // 2 + H * (I // g2) * 2

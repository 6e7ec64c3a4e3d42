"""Pins of the quantisation oracle: hand-derived known answers, the
reference's own expectations (zero rows, byte counts) and error bounds."""
import numpy as np
import pytest

from oracle import quant


def _row(vals, K=128):
    w = np.zeros((1, K), dtype=np.float16)
    w[0, :len(vals)] = np.asarray(vals, dtype=np.float16)
    return w


def test_pack_known_bytes_plus_minus_one():
    # max|w| = 1 -> q = +-7 -> nibbles 15 (k=0, low) and 1 (k=1, high) -> 0x1F.
    packed, scales = quant.pack_int4_weights(_row([1.0, -1.0]))
    assert packed.shape == (1, 64) and scales.shape == (1, 1)
    assert packed[0, 0] == 0x1F
    assert np.all(packed[0, 1:] == 0x88)  # zeros -> nibble 8 in both halves
    assert scales[0, 0] == np.float16(1.0 / 7.0)


def test_pack_round_half_even_known_answers():
    # absmax 7 -> scale exactly 1.0, so q = round_half_even(w).
    vals = [7.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -7.0]
    packed, scales = quant.pack_int4_weights(_row(vals))
    assert scales[0, 0] == np.float16(1.0)
    # q = 7, 2, 4, -2, 0, 0, 2, -7 -> nibbles 15, 10, 12, 6, 8, 8, 10, 1
    assert list(packed[0, :4]) == [0xAF, 0x6C, 0x88, 0x1A]


def test_pack_zero_row_scale_is_fp32_eps():
    packed, scales = quant.pack_int4_weights(np.zeros((2, 256), np.float16))
    assert np.all(packed == 0x88)
    # fp32 eps = 2^-23 rounds to the fp16 subnormal 2 * 2^-24 (bits 0x0002).
    assert np.all(scales.view(np.uint16) == 0x0002)


def test_group_rule_collapse_and_errors():
    p, s = quant.pack_int4_weights(np.ones((3, 64), np.float16), group_size=128)
    assert p.shape == (3, 32) and s.shape == (3, 1)
    with pytest.raises(ValueError):
        quant.pack_int4_weights(np.ones((1, 127), np.float16))
    with pytest.raises(ValueError):
        quant.pack_int4_weights(np.ones((1, 192), np.float16), group_size=128)
    assert quant.effective_group_size(256, 128) == 128


def test_pack_invariants_random():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float16)
    packed, scales = quant.pack_int4_weights(w)
    lo, hi = packed & 0xF, packed >> 4
    # |q| <= 7 by construction of the scale, so stored nibbles are 1..15.
    assert lo.min() >= 1 and hi.min() >= 1 and lo.max() <= 15 and hi.max() <= 15
    deq = quant.dequant_int4(packed, scales)
    s32 = np.abs(w.astype(np.float32).reshape(64, 4, 128)).max(-1) / np.float32(7)
    s16 = scales.astype(np.float32)
    bound = s32 / 2 + 7 * np.abs(s32 - s16) + 1e-7
    err = np.abs(w.astype(np.float32) - deq).reshape(64, 4, 128).max(-1)
    assert np.all(err <= bound)
    # each group's extreme element is reproduced as +-7 * scale
    g = w.astype(np.float32).reshape(64, 4, 128)
    idx = np.abs(g).argmax(-1)
    q_ext = np.take_along_axis(deq.reshape(64, 4, 128), idx[..., None], -1)[..., 0] / s16
    assert np.all(np.abs(np.abs(q_ext) - 7) < 1e-6)


def test_dequant_layout_low_nibble_is_even_k():
    packed = np.array([[0x9F, 0x18]], dtype=np.uint8)  # k0=15, k1=9, k2=8, k3=1
    scales = np.array([[2.0]], dtype=np.float16)
    deq = quant.dequant_int4(packed, scales)
    assert deq.tolist() == [[14.0, 2.0, 0.0, -14.0]]


def test_expert_byte_counts_match_reference():
    # Reference: INT4 bytes per expert = 3*H*I/2 (tests/test_stress.py:770, 796),
    # plus fp16 scales = 3,244,032 (OLMoE) / 2,433,024 (Qwen3).
    for H, I, wbytes, total in [(2048, 1024, 3145728, 3244032), (2048, 768, 2359296, 2433024)]:
        w13 = np.zeros((1, 2 * I, H), np.float16)
        w2 = np.zeros((1, H, I), np.float16)
        p13, s13 = quant.pack_experts_int4(w13)
        p2, s2 = quant.pack_experts_int4(w2)
        assert p13.nbytes + p2.nbytes == wbytes
        assert p13.nbytes + p2.nbytes + s13.nbytes + s2.nbytes == total
        assert quant.int4_expert_bytes(H, I) == total


def test_int8_known_answers_and_zero_rows():
    w = np.zeros((2, 8), np.float32)
    w[0, :4] = [127.0, -63.5, 0.5, 1.5]
    q, s = quant.quantize_int8(w)
    assert s[0] == np.float16(1.0)
    assert q[0, :4].tolist() == [127, -64, 0, 2]
    assert np.all(q[1] == 0)
    # reference test_eval.py:158-163: zero rows stay finite and exact
    z = np.zeros((4, 128), np.float16)
    fz = quant.fake_quant_int8(z)
    assert np.all(np.isfinite(fz)) and np.array_equal(fz, z)
    assert np.array_equal(quant.dequant_int8(*quant.quantize_int8(z)), z.astype(np.float32))


def test_fake_quant_int4_zero_rows_and_agreement():
    z = np.zeros((4, 128), np.float16)
    fz = quant.fake_quant_int4(z)  # reference test_eval.py:151-155
    assert np.all(np.isfinite(fz)) and np.array_equal(fz, z)
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((8, 256)) * 0.02).astype(np.float16)
    fq = quant.fake_quant_int4(w).astype(np.float32)
    p, s = quant.pack_int4_weights(w)
    deq = quant.dequant_int4(p, s)
    # same integers; only the fp16 rounding of the scale differs (<= 2^-11 rel)
    assert np.allclose(fq, deq, rtol=2e-3, atol=1e-6)


def _brute_pack_row(row, g):
    """Element-by-element restatement of pack_int4_weights for one row: scale per
    group from a Python max over |w|, q by Python's round-half-even, nibbles
    placed one byte at a time (low nibble = even k)."""
    K = len(row)
    eps = float(np.finfo(np.float32).eps)
    out, scales = [], []
    for g0 in range(0, K, g):
        grp = [np.float32(v) for v in row[g0:g0 + g]]
        amax = np.float32(0.0)
        for v in grp:
            amax = max(amax, np.float32(abs(v)))
        s = np.float32(max(np.float32(amax / np.float32(7.0)), np.float32(eps)))
        scales.append(np.float16(s))
        qs = []
        for v in grp:
            q = round(float(np.float32(v / s)))  # Python round() is half-even
            qs.append(min(7, max(-8, q)))
        for i in range(0, len(qs), 2):
            out.append((qs[i] + 8) | ((qs[i + 1] + 8) << 4))
    return out, scales


@pytest.mark.parametrize("N,K,g,seed", [(3, 256, 128, 11), (2, 64, 128, 12), (4, 96, 32, 13)])
def test_pack_matches_elementwise_brute_force(N, K, g, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    w[0, :8] = np.float16(0.0)  # a partly zero group
    packed, scales = quant.pack_int4_weights(w, group_size=g)
    geff = quant.effective_group_size(K, g)
    for r in range(N):
        bp, bs = _brute_pack_row(w[r], geff)
        assert packed[r].tolist() == bp
        assert scales[r].view(np.uint16).tolist() == np.array(bs, np.float16).view(np.uint16).tolist()


def test_dequant_int8_per_row_scales_known_answer():
    # rows carry different fp16 scales: a per-row broadcast mix-up changes the answer
    q = np.array([[1, -2, 127], [-128, 3, 0]], dtype=np.int8)
    s = np.array([0.5, 0.25], dtype=np.float16)
    deq = quant.dequant_int8(q, s)
    assert deq.tolist() == [[0.5, -1.0, 63.5], [-32.0, 0.75, 0.0]]
    # batched [E, N, K] with [E, N] scales
    qq = np.stack([q, q[::-1]])
    ss = np.stack([s, np.array([2.0, 4.0], np.float16)])
    d2 = quant.dequant_int8(qq, ss)
    assert d2[1].tolist() == [[-256.0, 6.0, 0.0], [4.0, -8.0, 508.0]]


def test_fake_quant_int8_known_answers_per_row_scales():
    """quant_shim.py:84-96 on non-zero data, answers derived by hand.

    Every row has its own scale = max|w| / 127 (fp32), and every expected value
    is q * scale with q an integer, exact in fp32:
      row 0: scale 1; half-way ties round to even (63.5 -> 64, 2.5 -> 2,
             -0.5 -> -0, -126.5 -> -126);
      row 1: scale 1 + 2^-12, exact in fp32 but not in fp16 (fp16 rounds it to
             1.0, which would give q instead of q * scale);
      row 2: max|w| = 127 * 2^-24, so max|w| / 127 = 2^-24 is below fp32 eps and
             the clamp makes the scale 2^-23 (127 * 2^-24 / 2^-23 = 63.5 -> 64);
      row 3: scale 2^-7.
    Column 0 holds the largest value of every row and row 0's 127 dominates each
    column, so a per-column scale fails rows 1-3; a scale kept in fp16 fails row 1;
    a missing eps clamp or rounding half away from zero fails rows 0 and 2."""
    s1 = 1.0 + 2.0 ** -12
    s2 = 2.0 ** -23
    s3 = 2.0 ** -7
    w = np.array([
        [127.0, 63.5, -0.5, 1.5, 2.5, -126.5, 0.0, 5.0],
        [127 * s1, -3 * s1, 2.5 * s1, 3.5 * s1, -6.5 * s1, 100 * s1, 0.25 * s1, -127 * s1],
        [127 * 2.0 ** -24, -1 * 2.0 ** -24, 3 * 2.0 ** -24, 0.0, 0.0, 0.0, 0.0, 0.0],
        [127 * s3, 0.5 * s3, -1.5 * s3, 126.5 * s3, -2 * s3, 7 * s3, -127 * s3, 64 * s3],
    ], dtype=np.float64)
    w32 = w.astype(np.float32)
    assert np.array_equal(w32.astype(np.float64), w)          # inputs exact in fp32
    want = np.array([
        [127.0, 64.0, -0.0, 2.0, 2.0, -126.0, 0.0, 5.0],
        [127 * s1, -3 * s1, 2 * s1, 4 * s1, -6 * s1, 100 * s1, 0.0, -127 * s1],
        [64 * s2, -0.0, 2 * s2, 0.0, 0.0, 0.0, 0.0, 0.0],
        [127 * s3, 0.0, -2 * s3, 126 * s3, -2 * s3, 7 * s3, -127 * s3, 64 * s3],
    ], dtype=np.float64)
    got = quant.fake_quant_int8(w32)
    assert got.dtype == np.float32
    assert np.array_equal(got.astype(np.float64), want)
    assert np.signbit(got[0, 2]) and np.signbit(got[2, 1])    # rint(-0.5) is -0
    # the storage form keeps the same integers (scales then rounded to fp16)
    q, s = quant.quantize_int8(w32)
    assert q[0].tolist() == [127, 64, 0, 2, 2, -126, 0, 5]
    assert q[1].tolist() == [127, -3, 2, 4, -6, 100, 0, -127]
    assert q[2, :3].tolist() == [64, 0, 2]
    assert s[1] == np.float16(1.0) and s[2] == np.float16(2.0 ** -23)
    # fp16 and bf16 weights: the result is cast back to the input dtype
    h = np.array([[127.0, 1.5, -0.5, 2.5, 0.0, 0.0, 0.0, 0.0],
                  [0.5 * 127 / 128, 0.5 * 2.5 / 128, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]],
                 dtype=np.float16)
    assert quant.fake_quant_int8(h).tolist() == [[127.0, 2.0, -0.0, 2.0, 0.0, 0.0, 0.0, 0.0],
                                                 [0.5 * 127 / 128, 0.5 * 2 / 128, 0.0, 0.0,
                                                  0.0, 0.0, 0.0, 0.0]]
    assert quant.fake_quant_int8(h).dtype == np.float16


def test_fake_quant_nan_and_0dim_follow_torch():
    """torch's amax and clamp keep NaN, so a NaN or infinite weight makes its
    row (INT8) or group (INT4) NaN; a 0-dim tensor is one INT8 element and
    makes the INT4 form raise (quant_shim.py:90-96, 108)."""
    w = np.zeros((3, 256), np.float32)
    w[:, ::3] = 0.25
    w[0, 4] = np.nan
    w[1, 130] = np.inf
    i8 = quant.fake_quant_int8(w)
    assert np.isnan(i8[0]).all() and np.isnan(i8[1]).all() and not np.isnan(i8[2]).any()
    i4 = quant.fake_quant_int4(w)
    assert np.isnan(i4[0, :128]).all() and not np.isnan(i4[0, 128:]).any()
    assert np.isnan(i4[1, 128:]).all() and not np.isnan(i4[1, :128]).any()
    # 0.3 / (0.3 / 127) rounds to 127, and 127 * (0.3 / 127) is 0.3 again in fp32
    assert quant.fake_quant_int8(np.float32(0.3)) == np.float32(0.3)
    assert quant.fake_quant_int8(np.float32(0.3)).shape == ()
    with pytest.raises(IndexError):
        quant.fake_quant_int4(np.float32(0.3))

"""Pins of the MoE-layer oracle: library routines (scipy/torch), the literal
per-(token, k) loop, closed forms and linearity."""
import numpy as np
import pytest
import scipy.special
import torch
import torch.nn.functional as F

from oracle import moe, quant


def test_silu_against_libraries_and_limits():
    x = np.linspace(-30, 30, 1001)
    ref = x * scipy.special.expit(x)
    assert np.allclose(moe.silu(x), ref, rtol=1e-12, atol=1e-300)
    assert np.allclose(moe.silu(x), F.silu(torch.from_numpy(x)).numpy(), rtol=1e-12)
    assert moe.silu(np.array([0.0]))[0] == 0.0
    assert abs(moe.silu(np.array([40.0]))[0] - 40.0) < 1e-12
    assert abs(moe.silu(np.array([-40.0]))[0]) < 1e-15


def test_silu_and_mul_gate_first():
    x = np.array([[1.0, -2.0, 3.0, 5.0]])
    out = moe.silu_and_mul(x)
    assert np.allclose(out, [[moe.silu(1.0) * 3.0, moe.silu(-2.0) * 5.0]])


def test_gather_and_combine_against_loops():
    rng = np.random.default_rng(0)
    T, k, H = 5, 3, 8
    hidden = rng.standard_normal((T, H))
    order = rng.permutation(T * k)
    g = moe.gather_hidden(hidden, order, k)
    for i in range(T * k):
        assert np.array_equal(g[i], hidden[order[i] // k])
    down = rng.standard_normal((T * k, H))
    w = rng.standard_normal((T, k))
    out = moe.combine(down, order, w)
    ref = np.zeros((T, H))
    for i in range(T * k):
        s = order[i]
        ref[s // k] += w[s // k, s % k] * down[i]
    assert np.allclose(out, ref, rtol=1e-12)
    d2 = rng.standard_normal((T * k, H))
    lin = moe.combine(2.0 * down - 3.0 * d2, order, w)
    assert np.allclose(lin, 2.0 * out - 3.0 * moe.combine(d2, order, w), rtol=1e-10)


def _setup(T=6, k=2, E=4, H=256, I=128, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32)
    w2 = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    wts = rng.random((T, k)).astype(np.float32)
    return x, w13, w2, ids, wts


def test_layer_grouped_equals_literal_loop():
    x, w13, w2, ids, wts = _setup()
    grouped = moe.moe_layer(x, w13, w2, ids, wts, accum=np.float64)
    loop = moe.moe_layer_loop(x, w13, w2, ids, wts)
    assert np.allclose(grouped, loop, rtol=1e-12, atol=1e-12)
    grouped32 = moe.moe_layer(x, w13, w2, ids, wts, accum=np.float32)
    assert moe.rel_l2(grouped32, loop) < 1e-5


def test_layer_single_pair_matches_torch_functional():
    x, w13, w2, ids, wts = _setup(T=1, k=1, E=1)
    xt = torch.from_numpy(x).double()
    gu = F.linear(xt, torch.from_numpy(w13[0]).double())
    I = w13.shape[1] // 2
    ref = float(wts[0, 0]) * F.linear(F.silu(gu[:, :I]) * gu[:, I:], torch.from_numpy(w2[0]).double())
    out = moe.moe_layer(x, w13, w2, ids, wts, accum=np.float64)
    assert np.allclose(out, ref.numpy(), rtol=1e-12)


def test_layer_linear_in_router_weights_and_drops_invalid_ids():
    x, w13, w2, ids, wts = _setup(seed=3)
    wts = wts.astype(np.float64)
    w_b = np.random.default_rng(9).random(wts.shape)
    a = moe.moe_layer(x, w13, w2, ids, wts, accum=np.float64)
    b = moe.moe_layer(x, w13, w2, ids, w_b, accum=np.float64)
    ab = moe.moe_layer(x, w13, w2, ids, 0.5 * wts + 2.0 * w_b, accum=np.float64)
    assert np.allclose(ab, 0.5 * a + 2.0 * b, rtol=1e-10, atol=1e-12)
    ids2 = ids.copy()
    ids2[0, 0] = -1
    dropped = moe.moe_layer(x, w13, w2, ids2, wts, accum=np.float64)
    wz = wts.copy()
    wz[0, 0] = 0.0
    assert np.allclose(dropped, moe.moe_layer(x, w13, w2, ids, wz, accum=np.float64))


def test_shared_experts_equal_routed_with_unit_weight():
    x, w13, w2, ids, wts = _setup(E=5, seed=4)
    shared13, shared2 = w13[4:], w2[4:]
    out = moe.moe_layer(x, w13[:4], w2[:4], ids % 4, wts, shared13, shared2, accum=np.float64)
    ids_ext = np.concatenate([ids % 4, np.full((ids.shape[0], 1), 4)], axis=1)
    w_ext = np.concatenate([wts, np.ones((ids.shape[0], 1), np.float32)], axis=1)
    ref = moe.moe_layer_loop(x, w13, w2, ids_ext, w_ext)
    assert np.allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_grouped_gemm_sorted_single_expert_is_matmul():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((7, 64)).astype(np.float32)
    w = rng.standard_normal((1, 32, 64)).astype(np.float32)
    out = moe.grouped_gemm_sorted(a, w, np.array([0, 7]))
    assert np.allclose(out, a @ w[0].T, rtol=1e-6)


def test_error_metrics():
    ref = np.array([3.0, 4.0])
    assert moe.rel_l2(ref * 1.01, ref) == pytest.approx(0.01)
    assert moe.max_over_rms(ref + [0.0, 0.1], ref) == pytest.approx(0.1 / np.sqrt(12.5))

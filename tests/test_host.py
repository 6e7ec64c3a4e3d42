"""Host-side checks that need no GPU: the C-ABI library loads and exports every
symbol the header declares, argument validation, the artifact reader, the
synthetic workloads and the SGLang patch plumbing."""
import ctypes
import json
import re
import sys
import types
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "exq_hip.h").read_text()
    return sorted(set(re.findall(r"^(?:int|size_t|const char\*)\s+(exq_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from exq_amd import _lib
    L = _lib.lib()
    declared = _declared_symbols()
    assert len(declared) >= 16
    for name in declared:
        assert hasattr(L, name), f"{name} missing from libexq_hip.so"
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    assert L.exq_abi_version() == 1


def test_argument_validation_without_gpu():
    from exq_amd import _lib
    L = _lib.lib()
    # Bad dtypes / sizes are rejected on the host before any HIP call.
    st = L.exq_dispatch(None, _lib.F32, 4, 8, None, None, None, None)
    assert st == 1 and b"ids dtype" in L.exq_last_error()
    st = L.exq_moe_align_block_size(None, _lib.I32, 10, 5, 16, None, 3, None, 100, None,
                                    None, 1, None)
    assert st == 1 and b"capacity" in L.exq_last_error()
    p = _lib.MoeProblem(n_tokens=4, hidden_size=2048, inter_size=1000, n_experts=64, top_k=8,
                        n_shared=0, group_size=128, act_dtype=_lib.BF16, ids_dtype=_lib.I64,
                        weights_dtype=_lib.F32)
    st = L.exq_moe_int4_fused_forward(p, None, None, None, None, None, None, None, None, None,
                                      None, None, 0, None)
    assert st == 2 and b"inter_size" in L.exq_last_error()
    p.inter_size = 1024
    st = L.exq_moe_int4_fused_forward(p, None, None, None, None, None, None, None, None, None,
                                      None, None, 0, None)
    assert st == 1 and b"null weights" in L.exq_last_error()
    need = L.exq_moe_workspace_size(p)
    assert need > 4 * 8 * 2048 * 4  # partial rows dominate
    st = L.exq_moe_int4_fused_forward(p, None, None, None, 1, 1, 1, 1, None, None, None, None,
                                      need - 1, None)
    assert st == 3
    assert L.exq_status_name(3) == b"EXQ_ERROR_WORKSPACE_TOO_SMALL"


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from exq_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "_LIB_PATH", tmp_path / "libexq_hip.so")
    with pytest.raises(_lib.ExqError, match="no fallback"):
        _lib.lib()


def test_kernels_reject_cpu_tensors():
    from exq_amd import kernels
    from exq_amd._lib import ExqError
    x = torch.zeros(2, 256, dtype=torch.bfloat16)
    with pytest.raises(ExqError, match="HIP device"):
        kernels.fused_experts(x, torch.zeros(1, 256, 128, dtype=torch.uint8),
                              torch.zeros(1, 256, 2, dtype=torch.float16),
                              torch.zeros(1, 256, 64, dtype=torch.uint8),
                              torch.zeros(1, 256, 1, dtype=torch.float16),
                              torch.ones(2, 1), torch.zeros(2, 1, dtype=torch.int64))


def test_pack_host_api_matches_oracle_bit_exact():
    from exq_amd.kernels import pack_experts_int4, pack_int4_weights
    from oracle import quant
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((3, 64, 384)) * 0.02).astype(np.float16)
    w[1, 5] = 0  # zero row
    p, s = pack_experts_int4(torch.from_numpy(w))
    rp, rs = quant.pack_experts_int4(w)
    assert np.array_equal(p.numpy(), rp) and np.array_equal(s.numpy(), rs)
    p1, s1 = pack_int4_weights(torch.from_numpy(w[0, :, :64]))
    rp1, rs1 = quant.pack_int4_weights(w[0, :, :64])
    assert s1.shape == (64, 1) and np.array_equal(p1.numpy(), rp1) and np.array_equal(s1.numpy(), rs1)
    with pytest.raises(ValueError):
        pack_int4_weights(torch.zeros(4, 7, dtype=torch.float16))


def test_int8_host_quant_matches_oracle():
    from exq_amd.kernels import quantize_int8_rows
    from oracle import quant
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((2, 32, 256)) * 0.02).astype(np.float16)
    q, s = quantize_int8_rows(torch.from_numpy(w))
    rq, rs = quant.quantize_int8(w)
    assert np.array_equal(q.numpy(), rq) and np.array_equal(s.numpy(), rs)


def _write(tmp_path, obj, name="a.json"):
    p = tmp_path / name
    p.write_text(json.dumps(obj))
    return str(p)


def test_artifact_reader_rules(tmp_path, monkeypatch):
    from exq_amd.kernels import load_exq_artifact
    from exq_amd.kernels.exq_artifact import freq_to_block_m, layer_tiers
    from oracle import artifact as ora
    monkeypatch.chdir(tmp_path)
    qa = {"0:0": "BF16", "0:1": "INT8", "0:3": "INT4", "1:2": "FP8", "2:0": "INT8"}
    path = _write(tmp_path, {"model_id": "m", "quant_assignments": qa})
    prof = load_exq_artifact(path, device="cpu")
    assert (prof.n_layers, prof.n_experts_per_layer) == (3, 4)
    assert np.array_equal(prof.tiers.numpy(), ora.tiers_from_assignments(qa))
    assert prof.tiers[1, 2] == 2 and prof.tiers[0, 2] == 2  # unknown / missing -> INT4
    assert np.allclose(prof.freqs.numpy(), ora.tier_fallback_freqs(prof.tiers.numpy()))
    for t in range(3):
        for f in (0.0, 0.029, 0.03, 0.2):
            assert freq_to_block_m(f, t) == ora.freq_to_block_m(f, t)
    assert prof.precision_counts() == {"BF16": 1, "INT8": 2, "INT4": 9}
    assert prof.hot_expert_count(0) == 1
    assert layer_tiers(path, 0, 4) == [0, 1, 2, 2]
    assert layer_tiers(path, 7, 4) is None
    # explicit profile frequencies
    prof_path = _write(tmp_path, {"layers": {"0": {"expert_stats": [
        {"expert_id": 1, "activation_freq": 0.04}]}}}, "p.json")
    prof2 = load_exq_artifact(path, prof_path, device="cpu")
    assert prof2.freqs[0, 1] == pytest.approx(0.04) and prof2.block_m[0, 1] == 64
    # legacy key and the empty-plan error
    assert load_exq_artifact(_write(tmp_path, {"quant_plan": qa}, "l.json"), device="cpu").n_layers == 3
    with pytest.raises(ValueError, match="no quant_assignments"):
        load_exq_artifact(_write(tmp_path, {"model_id": "m"}, "e.json"), device="cpu")


def test_synthetic_workloads_are_seeded():
    from exq_amd import synth
    cfg = synth.CONFIGS["olmoe"]
    a = synth.routing(cfg, 16)
    b = synth.routing(cfg, 16)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    ids, w = a
    assert ids.shape == (16, 8) and all(len(set(r)) == 8 for r in ids.tolist())
    assert np.all(w > 0) and np.all(w.sum(1) < 1.0)  # OLMoE: no renormalisation
    ids_q, w_q = synth.routing(synth.CONFIGS["qwen3"], 4)
    assert np.allclose(w_q.sum(1), 1.0, atol=1e-6)
    t = synth.mixed_tiers(64, 2000)
    assert (t.count(0), t.count(1), t.count(2)) == (6, 13, 45)
    assert synth.int4_expert_bytes(2048, 1024) == 3244032


def _install_fake_sglang(monkeypatch):
    class UnquantizedFusedMoEMethod:
        def forward_cuda(self, layer, dispatch_output):
            return ("original", layer.layer_id)

    class StandardCombineInput:
        def __init__(self, hidden_states):
            self.hidden_states = hidden_states

    mods = {
        "sglang": types.ModuleType("sglang"),
        "sglang.srt": types.ModuleType("sglang.srt"),
        "sglang.srt.layers": types.ModuleType("sglang.srt.layers"),
        "sglang.srt.layers.quantization": types.ModuleType("sglang.srt.layers.quantization"),
        "sglang.srt.layers.quantization.unquant": types.ModuleType("u"),
        "sglang.srt.layers.moe": types.ModuleType("sglang.srt.layers.moe"),
        "sglang.srt.layers.moe.token_dispatcher": types.ModuleType("td"),
        "sglang.srt.layers.moe.token_dispatcher.standard": types.ModuleType("std"),
    }
    mods["sglang.srt.layers.quantization.unquant"].UnquantizedFusedMoEMethod = UnquantizedFusedMoEMethod
    mods["sglang.srt.layers.moe.token_dispatcher.standard"].StandardCombineInput = StandardCombineInput
    for k, v in mods.items():
        monkeypatch.setitem(sys.modules, k, v)
    return UnquantizedFusedMoEMethod


def test_sglang_patch_unpatch_and_fallback(tmp_path, monkeypatch):
    from exq_amd.runtime import sglang_backend as sb
    cls = _install_fake_sglang(monkeypatch)
    orig = cls.forward_cuda
    path = _write(tmp_path, {"quant_assignments": {"0:0": "INT4", "1:5": "BF16"}})
    backend = sb.patch_sglang(path)
    assert backend.n_layers == 2 and cls._exq_patched
    assert backend.cache_stats() == {"n_layers_cached": 0, "n_layers_in_artifact": 2}
    layer = types.SimpleNamespace(layer_id=7)  # beyond the artifact -> original forward
    assert cls().forward_cuda(layer, None) == ("original", 7)
    layer = types.SimpleNamespace(layer_id=None)
    assert cls().forward_cuda(layer, None) == ("original", None)
    sb.patch_sglang(path)  # re-patch keeps the true original
    sb.unpatch_sglang()
    assert cls.forward_cuda is orig and not cls._exq_patched


def _cpu_layer(T=4, H=256, I=128, E=4, k=2):
    x = torch.zeros(T, H, dtype=torch.bfloat16)
    p13 = torch.zeros(E, 2 * I, H // 2, dtype=torch.uint8)
    s13 = torch.zeros(E, 2 * I, H // 128, dtype=torch.float16)
    p2 = torch.zeros(E, H, I // 2, dtype=torch.uint8)
    s2 = torch.zeros(E, H, I // 128, dtype=torch.float16)
    ids = torch.zeros(T, k, dtype=torch.int64)
    w = torch.zeros(T, k, dtype=torch.float32)
    return x, p13, s13, p2, s2, w, ids


@pytest.mark.parametrize("bad", ["out_shape", "out_dtype", "so_dtype", "so_size", "ends_dtype",
                                 "ends_size", "ids_dtype", "scale_shape"])
def test_fused_wrappers_reject_bad_buffers_before_launch(bad):
    """Output buffers the kernels write through raw pointers are checked on the
    host (ValueError) before the device check or any launch."""
    from exq_amd.kernels import fused_experts
    x, p13, s13, p2, s2, w, ids = _cpu_layer()
    kw = {}
    if bad == "out_shape":
        kw["out"] = torch.empty(3, 256, dtype=torch.bfloat16)
    elif bad == "out_dtype":
        kw["out"] = torch.empty(4, 256, dtype=torch.float16)
    elif bad == "so_dtype":
        kw["sort_order_out"] = torch.empty(8, dtype=torch.int32)
    elif bad == "so_size":
        kw["sort_order_out"] = torch.empty(7, dtype=torch.int64)
    elif bad == "ends_dtype":
        kw["expert_ends_out"] = torch.empty(5, dtype=torch.int64)
    elif bad == "ends_size":
        kw["expert_ends_out"] = torch.empty(4, dtype=torch.int32)
    elif bad == "ids_dtype":
        ids = ids.to(torch.int16)
    elif bad == "scale_shape":
        s13 = s13[:, :, :1].contiguous().repeat(1, 1, 3)
    with pytest.raises(ValueError):
        fused_experts(x, p13, s13, p2, s2, w, ids, **kw)


def test_fused_wrappers_accept_good_buffers_up_to_the_device_check():
    from exq_amd import ExqError
    from exq_amd.kernels import fused_experts
    x, p13, s13, p2, s2, w, ids = _cpu_layer()
    with pytest.raises(ExqError, match="HIP device"):
        fused_experts(x, p13, s13, p2, s2, w, ids, out=torch.empty(4, 256, dtype=torch.bfloat16),
                      sort_order_out=torch.empty(8, dtype=torch.int64),
                      expert_ends_out=torch.empty(5, dtype=torch.int32))


def test_mixed_wrapper_rejects_bad_out():
    from exq_amd.kernels import MixedExpertBank, fused_experts_mixed
    x, *_, w, ids = _cpu_layer()
    bank = MixedExpertBank(n_experts=4, n_shared=0, hidden_size=256, inter_size=128,
                           group_size=128, tier=torch.full((4,), 2, dtype=torch.int8),
                           index=torch.arange(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="out must be"):
        fused_experts_mixed(x, bank, w, ids, out=torch.empty(4, 256, dtype=torch.float16))
    with pytest.raises(ValueError, match="sort_order_out"):
        fused_experts_mixed(x, bank, w, ids, sort_order_out=torch.empty(8, dtype=torch.int32))
    with pytest.raises(ValueError, match="expert_ends_out"):
        fused_experts_mixed(x, bank, w, ids, expert_ends_out=torch.empty(6, dtype=torch.int32))


def test_pack_cache_fingerprint_uses_no_float64_copy():
    """The fingerprint's exact sum reduces in float64 without materialising a
    float64 copy of the bank (w.sum(dtype=float64)); a changed element changes it."""
    from exq_amd.runtime.pack_cache import fingerprint
    w = torch.randn(2, 16, 256, dtype=torch.float32).to(torch.bfloat16)
    f0 = fingerprint(w)
    assert f0 == fingerprint(w.clone())
    w2 = w.clone()
    w2[1, 7, 3] += 1
    assert fingerprint(w2) != f0
    src = (ROOT / "exq_amd" / "runtime" / "pack_cache.py").read_text()
    assert "sum(dtype=torch.float64)" in src and ".double()" not in src


def test_mixed_plan_hot_tier_is_the_routers_favoured_experts(tmp_path):
    """The mixed stack's BF16 tier is the experts the router sends most slots
    to, and the plan round-trips through the artifact reader."""
    from exq_amd import synth
    from exq_amd.kernels import load_exq_artifact
    cfg = synth.CONFIGS["mixed_olmoe"]
    art = synth.plan_artifact(cfg, 2)
    path = tmp_path / "plan.json"
    path.write_text(json.dumps(art))
    prof = load_exq_artifact(str(path), device="cpu")
    for l in range(2):
        tiers = synth.router_tiers(cfg, l)
        assert prof.tiers[l].tolist() == tiers
        assert tiers.count(0) == 6 and tiers.count(1) == 13 and tiers.count(2) == 45
        ids, _ = synth.routing(cfg, 4096, l)
        counts = np.bincount(ids.reshape(-1), minlength=64)
        bf = [e for e in range(64) if tiers[e] == 0]
        i4 = [e for e in range(64) if tiers[e] == 2]
        # hot experts take far more slots than the INT4 tail on average
        assert counts[bf].mean() > 4 * counts[i4].mean()


def test_mixed_bank_checks_tier_and_index_values():
    """The kernels read tier / index unchecked on the device (the row in 30
    bits of the expert map), so MixedExpertBank rejects other values when built."""
    from exq_amd.kernels import MixedExpertBank
    kw = dict(n_experts=4, n_shared=0, hidden_size=256, inter_size=128, group_size=128)
    ok = MixedExpertBank(tier=torch.tensor([0, 1, 2, 2], dtype=torch.int8),
                         index=torch.tensor([0, 0, 0, (1 << 30) - 1], dtype=torch.int32), **kw)
    assert ok.n_experts == 4
    for tier, index, msg in (([0, 1, 3, 2], [0, 0, 0, 1], "tier values"),
                             ([0, 1, -1, 2], [0, 0, 0, 1], "tier values"),
                             ([0, 1, 2, 2], [0, 0, 0, 1 << 30], "index values"),
                             ([0, 1, 2, 2], [0, 0, -1, 1], "index values"),
                             ([0, 1, 2], [0, 0, 0], "entries")):
        with pytest.raises(ValueError, match=msg):
            MixedExpertBank(tier=torch.tensor(tier, dtype=torch.int8),
                            index=torch.tensor(index, dtype=torch.int32), **kw)

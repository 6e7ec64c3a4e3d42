"""SGLang integration: route UnquantizedFusedMoEMethod.forward_cuda through the
HIP MoE pipeline.

Mirrors exq/runtime/sglang_backend.py of the reference: ``patch_sglang``
(183-210), ``unpatch_sglang`` (213-225), ``ExQSGLangBackend`` (163-180), the
per-layer packed-weight cache ``_get_or_pack`` (32-60) and the replacement
forward ``_exq_forward_cuda`` (65-158).  Differences, all deliberate:

* the whole layer is one ``fused_experts`` call (routing preparation,
  gate/up+SiLU, down, combine) with no device->host synchronisation, so the
  patched forward can be captured in a HIP graph;
* ``honor_plan=True`` (the default) applies the artifact's per-expert
  precision (BF16 / INT8 / INT4) instead of packing every expert INT4;
* activations stay in the model dtype (bf16 or fp16), routing weights may be
  fp32/fp16/bf16, and the result is returned in the activation dtype.
"""
from __future__ import annotations

import json
import logging
import threading
import time

import torch

from ..kernels.exq_artifact import PRECISION_TO_INT
from ..kernels.fused_moe import MixedExpertBank, fused_experts, fused_experts_mixed
from ..kernels.moe_int4_kernel import pack_experts_int4
from .pack_cache import PackedWeightCache

logger = logging.getLogger(__name__)

# Per-layer packed weights, keyed by id(layer).  Guarded by a lock: SGLang may
# call forward_cuda from more than one thread.
_exq_packed_cache: dict[int, dict] = {}
_cache_lock = threading.Lock()
_original_forward = None


def _layer_tiers(backend: "ExQSGLangBackend", layer_id: int, n_experts: int) -> list[int]:
    tiers = [PRECISION_TO_INT["INT4"]] * n_experts
    for e, prec in backend.assignments.get(layer_id, {}).items():
        if e < n_experts:
            tiers[e] = PRECISION_TO_INT.get(prec, PRECISION_TO_INT["INT4"])
    return tiers


def _get_or_pack(layer, backend: "ExQSGLangBackend | None" = None) -> dict:
    """Quantise the layer's w13_weight [E, 2I, H] / w2_weight [E, H, I] once."""
    key = id(layer)
    with _cache_lock:
        hit = _exq_packed_cache.get(key)
    if hit is not None:
        return hit
    t0 = time.perf_counter()
    w13 = layer.w13_weight
    w2 = layer.w2_weight
    E = w13.shape[0]
    layer_id = getattr(layer, "layer_id", None)
    tiers = None
    if backend is not None and backend.honor_plan and layer_id is not None:
        tiers = _layer_tiers(backend, layer_id, E)
        if all(t == PRECISION_TO_INT["INT4"] for t in tiers):
            tiers = None
    cache = {"n_experts": E, "inter2": w13.shape[1], "hidden": w13.shape[2]}
    if tiers is None:
        if backend is not None and backend.disk_cache is not None and layer_id is not None:
            (cache["w1_packed"], cache["w1_scales"], cache["w2_packed"],
             cache["w2_scales"]) = backend.disk_cache.get_or_pack(f"layer{layer_id}", w13, w2)
        else:
            cache["w1_packed"], cache["w1_scales"] = pack_experts_int4(w13.to(torch.float16), 128)
            cache["w2_packed"], cache["w2_scales"] = pack_experts_int4(w2.to(torch.float16), 128)
        cache["bank"] = None
    else:
        act = w13.dtype if w13.dtype in (torch.float16, torch.bfloat16) else torch.bfloat16
        cache["bank"] = MixedExpertBank.from_weights(w13, w2, tiers, act_dtype=act)
    with _cache_lock:
        _exq_packed_cache[key] = cache
    logger.info("ExQ: packed layer %s in %.1f ms", layer_id, (time.perf_counter() - t0) * 1e3)
    return cache


def _exq_forward_cuda(self_method, layer, dispatch_output, _original_forward_cuda,
                      backend: "ExQSGLangBackend"):
    """Replacement for UnquantizedFusedMoEMethod.forward_cuda."""
    from sglang.srt.layers.moe.token_dispatcher.standard import StandardCombineInput

    layer_id = getattr(layer, "layer_id", None)
    if layer_id is None or layer_id >= backend.n_layers:
        return _original_forward_cuda(self_method, layer, dispatch_output)

    hidden = dispatch_output.hidden_states
    in_dtype = hidden.dtype
    topk = dispatch_output.topk_output
    cache = _get_or_pack(layer, backend)
    if hidden.dtype not in (torch.float16, torch.bfloat16):
        hidden = hidden.to(torch.bfloat16)
    hidden = hidden.contiguous()
    ids = topk.topk_ids.contiguous()
    wts = topk.topk_weights.contiguous()
    if cache["bank"] is None:
        out = fused_experts(hidden, cache["w1_packed"], cache["w1_scales"],
                            cache["w2_packed"], cache["w2_scales"], wts, ids)
    else:
        bank = cache["bank"]
        if bank.bf16_w13 is not None and bank.bf16_w13.dtype != hidden.dtype:
            hidden = hidden.to(bank.bf16_w13.dtype)
        out = fused_experts_mixed(hidden, bank, wts, ids)
    if out.dtype != in_dtype:  # the caller's activation dtype, whatever the bank stores
        out = out.to(in_dtype)
    return StandardCombineInput(hidden_states=out)


class ExQSGLangBackend:
    """Holds the artifact's plan and the per-layer weight cache."""

    def __init__(self, artifact_path: str, honor_plan: bool = True,
                 pack_cache_dir: str | None = None):
        with open(artifact_path, encoding="utf-8") as f:
            artifact = json.load(f)
        qa = artifact.get("quant_assignments") or artifact.get("quant_plan") or {}
        self.assignments: dict[int, dict[int, str]] = {}
        for key, prec in qa.items():
            l, e = (int(v) for v in key.split(":"))
            self.assignments.setdefault(l, {})[e] = prec
        self.n_layers = max(self.assignments) + 1 if self.assignments else 0
        self.artifact_path = artifact_path
        self.honor_plan = honor_plan
        # INT4 layers packed once and kept on disk across runs (None: in memory only)
        self.disk_cache = PackedWeightCache(pack_cache_dir) if pack_cache_dir else None
        logger.info("ExQ SGLang backend: %d layers (%d assignments)", self.n_layers, len(qa))

    def clear_cache(self) -> None:
        with _cache_lock:
            _exq_packed_cache.clear()

    def cache_stats(self) -> dict:
        with _cache_lock:
            n = len(_exq_packed_cache)
        st = {"n_layers_cached": n, "n_layers_in_artifact": self.n_layers}
        if self.disk_cache is not None:
            st.update(disk_hits=self.disk_cache.hits, disk_misses=self.disk_cache.misses)
        return st


def patch_sglang(artifact_path: str, honor_plan: bool = True,
                 pack_cache_dir: str | None = None) -> ExQSGLangBackend:
    """Replace UnquantizedFusedMoEMethod.forward_cuda for the artifact's layers.

    ``pack_cache_dir``: keep the packed INT4 banks on disk there (one
    safetensors file per layer), so later runs load instead of repacking."""
    global _original_forward
    try:
        from sglang.srt.layers.quantization.unquant import UnquantizedFusedMoEMethod
    except ImportError as exc:
        raise ImportError("SGLang not installed: pip install sglang") from exc

    backend = ExQSGLangBackend(artifact_path, honor_plan=honor_plan,
                               pack_cache_dir=pack_cache_dir)
    if getattr(UnquantizedFusedMoEMethod, "_exq_patched", False):
        logger.warning("ExQ: re-patching SGLang (cache cleared)")
        backend.clear_cache()
    else:
        _original_forward = UnquantizedFusedMoEMethod.forward_cuda
    original = _original_forward

    def patched(self, layer, dispatch_output):
        return _exq_forward_cuda(self, layer, dispatch_output, original, backend)

    UnquantizedFusedMoEMethod.forward_cuda = patched
    UnquantizedFusedMoEMethod._exq_patched = True
    logger.info("ExQ: patched SGLang (%d layers covered)", backend.n_layers)
    return backend


def unpatch_sglang() -> None:
    """Restore SGLang's original forward_cuda and drop the weight cache."""
    global _original_forward
    try:
        from sglang.srt.layers.quantization.unquant import UnquantizedFusedMoEMethod
    except ImportError:
        return
    if not getattr(UnquantizedFusedMoEMethod, "_exq_patched", False):
        return
    if _original_forward is not None:
        UnquantizedFusedMoEMethod.forward_cuda = _original_forward
    UnquantizedFusedMoEMethod._exq_patched = False
    _original_forward = None
    with _cache_lock:
        _exq_packed_cache.clear()
    logger.info("ExQ: SGLang patch removed")

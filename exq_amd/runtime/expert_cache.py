"""Two-tier expert weight cache: device-resident hot experts, pinned-host cold ones.

Mirrors ``ExpertWeightCache`` (exq/runtime/__init__.py:35-106) and the static
prefetch loop of ``CompiledMoEForward._issue_prefetches`` (same file, 146-166):

* ``register_expert(layer, expert, weight)``: experts the plan marks BF16 or
  INT8 are copied to the device and stay there; everything else (INT4, the
  default) is kept on the host.
* ``prefetch(layer, expert, stream)`` copies a host-resident expert to the
  device on ``stream``; ``get(layer, expert)`` returns the device copy (counting
  a hit) or ``None`` (a miss); ``sync_prefetches(stream)`` waits for the stream.

What differs from the reference, for HIP streams on MI355X:

* Host copies live in pinned memory allocated for them (``pin_memory=True``),
  so a prefetch is an asynchronous DMA over PCIe rather than a staged copy.
* The reference inserts a prefetched tensor into its device map before the
  copy has finished, so a consumer on another stream can read it early.  Here
  every prefetch records an event on its stream, and ``get`` makes the calling
  stream wait for that event (a stream-ordered wait, no host synchronisation)
  and records the tensor as used by that stream for the allocator.
* An optional ``capacity_bytes`` bounds the device bytes of prefetched cold
  experts; beyond it the least recently used prefetched experts are dropped
  (their host copies remain, so a later prefetch brings them back).  Hot
  experts are never dropped.  The reference has no bound.

A registered weight may be a tensor or a tuple of tensors (for example the
packed INT4 weights and scales of one expert); a prefetch copies all of them.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Iterable, Union

import torch

Weight = Union[torch.Tensor, tuple]

_HOT = ("BF16", "INT8")


def _as_tuple(w: Weight) -> tuple:
    return tuple(w) if isinstance(w, (tuple, list)) else (w,)


def _unwrap(ts: tuple, like: Weight) -> Weight:
    return ts if isinstance(like, (tuple, list)) else ts[0]


def _nbytes(ts: Iterable[torch.Tensor]) -> int:
    return sum(t.numel() * t.element_size() for t in ts)


class ExpertWeightCache:
    """Device (hot) + pinned host (cold) expert weights with stream-ordered prefetch."""

    def __init__(self, quant_assignments: dict[str, str], device: str | torch.device = "cuda",
                 capacity_bytes: int | None = None):
        self.device = torch.device(device)
        self.assignments = quant_assignments
        self.capacity_bytes = capacity_bytes
        self._hot: dict[tuple[int, int], tuple] = {}
        self._host: dict[tuple[int, int], tuple] = {}
        self._like: dict[tuple[int, int], Weight] = {}
        # prefetched cold experts in least-recently-used order: key -> (tensors, event)
        self._dev: OrderedDict[tuple[int, int], tuple] = OrderedDict()
        self._in_flight: set[tuple[int, int]] = set()
        self.hits = 0
        self.misses = 0
        self.evictions = 0

    # -- registration -------------------------------------------------------
    def register_expert(self, layer: int, expert: int, weight: Weight) -> None:
        """Hot experts (BF16 / INT8 in the plan) go to the device; the rest to pinned host memory."""
        key = (layer, expert)
        ts = _as_tuple(weight)
        self._like[key] = weight
        prec = self.assignments.get(f"{layer}:{expert}", "INT4")
        if prec in _HOT:
            self._hot[key] = tuple(t.detach().to(self.device) for t in ts)
            self._host.pop(key, None)
            self._drop(key)
        else:
            pin = self.device.type == "cuda"
            host = []
            for t in ts:
                h = torch.empty(t.shape, dtype=t.dtype, device="cpu", pin_memory=pin)
                h.copy_(t.detach())
                host.append(h)
            self._host[key] = tuple(host)
            self._hot.pop(key, None)
            self._drop(key)

    # -- queries ------------------------------------------------------------
    def is_gpu_resident(self, layer: int, expert: int) -> bool:
        key = (layer, expert)
        return key in self._hot or key in self._dev

    def get(self, layer: int, expert: int) -> Weight | None:
        """The device copy of the expert (a hit) or None (a miss).

        For a prefetched expert the current stream waits for its copy."""
        key = (layer, expert)
        if key in self._hot:
            self.hits += 1
            return _unwrap(self._hot[key], self._like[key])
        if key in self._dev:
            self.hits += 1
            ts, ev = self._dev[key]
            self._dev.move_to_end(key)
            if ev is not None:
                cur = torch.cuda.current_stream(self.device)
                cur.wait_event(ev)
                for t in ts:
                    t.record_stream(cur)
            return _unwrap(ts, self._like[key])
        self.misses += 1
        return None

    # -- prefetch -----------------------------------------------------------
    def prefetch(self, layer: int, expert: int, stream: torch.cuda.Stream | None) -> None:
        """Copy a host-resident expert to the device on `stream` (asynchronous)."""
        key = (layer, expert)
        if key in self._dev:
            self._dev.move_to_end(key)
            return
        if key in self._hot:
            return
        if key not in self._host:
            return  # not registered
        host = self._host[key]
        self._make_room(_nbytes(host))
        if self.device.type == "cuda":
            stream = stream or torch.cuda.current_stream(self.device)
            with torch.cuda.stream(stream):
                dev = tuple(h.to(self.device, non_blocking=True) for h in host)
                ev = torch.cuda.Event()
                ev.record(stream)
        else:
            dev, ev = tuple(h.to(self.device) for h in host), None
        self._dev[key] = (dev, ev)
        self._in_flight.add(key)

    def sync_prefetches(self, stream: torch.cuda.Stream | None) -> None:
        """Wait for every prefetch issued on `stream`."""
        if stream is not None:
            stream.synchronize()
        self._in_flight.clear()

    def issue_prefetches(self, prefetch_table: dict, stream: torch.cuda.Stream | None,
                         max_priority: int = 1) -> int:
        """The static prefetch schedule of one layer: for every source expert's
        targets (dst_layer, dst_expert, priority) with priority <= max_priority
        (HIGH 0 or MEDIUM 1), prefetch the target.  Returns the number issued
        (exq/runtime/__init__.py:146-166)."""
        if not self.has_offloaded_weights:
            return 0
        n = 0
        for targets in prefetch_table.values():
            for dst_layer, dst_expert, priority in targets:
                if priority <= max_priority:
                    self.prefetch(dst_layer, dst_expert, stream)
                    n += 1
        return n

    # -- capacity -----------------------------------------------------------
    def _drop(self, key) -> None:
        self._dev.pop(key, None)
        self._in_flight.discard(key)

    def _make_room(self, need: int) -> None:
        if self.capacity_bytes is None:
            return
        if need > self.capacity_bytes:
            raise ValueError(f"expert of {need} bytes exceeds capacity_bytes={self.capacity_bytes}")
        used = sum(_nbytes(ts) for ts, _ in self._dev.values())
        while used + need > self.capacity_bytes and self._dev:
            key, (ts, _) = self._dev.popitem(last=False)
            self._in_flight.discard(key)
            used -= _nbytes(ts)
            self.evictions += 1

    @property
    def device_bytes(self) -> int:
        return (sum(_nbytes(ts) for ts in self._hot.values())
                + sum(_nbytes(ts) for ts, _ in self._dev.values()))

    @property
    def stats(self) -> dict:
        return {
            "gpu_resident": len(self._hot) + len(self._dev),
            "cpu_stored": len(self._host),
            "hits": self.hits,
            "misses": self.misses,
            "hit_rate": self.hits / max(self.hits + self.misses, 1),
            "evictions": self.evictions,
            "device_bytes": self.device_bytes,
        }

    @property
    def has_offloaded_weights(self) -> bool:
        """Whether any expert is held on the host only (something to prefetch)."""
        return bool(self._host)

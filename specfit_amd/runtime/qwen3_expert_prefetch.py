"""Predicted expert prefetch for exactly one target forward.

Drop-in for src/specfit/runtime/qwen3_expert_prefetch.py:34-418
(``Qwen3ExpertPrefetch``): the executor every measured decode of the
reference runs under (with ``predictions={}`` it is the "ready_demand"
executor).  Policy, all host-side:

* every layer cache's copies go to one shared copy stream; at most
  ``max_inflight`` new transfers are incomplete at a time;
* the current layer's demand is served before future predictions; while a
  layer has no routes yet, speculation keeps at least one slot of it free
  for demand (``max_prefetch_per_layer`` can lower that limit further);
* predicted experts that are already resident are protected once per layer
  before any earlier-id miss could evict them;
* when a layer's router has run, wrong predictions are dropped and the
  actual experts are yielded ready-first (transfer complete), else the
  oldest in-flight, else a free queue credit is awaited or a demand copy is
  forced into a busy slot (the only case that queues a use-guard wait);
* streams, hooks and leases are restored on exit, including on exceptions.

GPU work is ordered with events; the only host waits are the queue-credit
``Event.synchronize`` of the reference.
"""
from __future__ import annotations

import math
from collections import deque
from contextlib import ExitStack
from dataclasses import asdict, dataclass
from numbers import Real
from typing import Mapping, Sequence

import torch

from .lease import ExpertLease
from .qwen3_offloaded_experts import Qwen3OffloadedExperts, ReductionMode
from .state import ExpertKey


@dataclass(slots=True)
class _LayerStats:
    layer_id: int
    predicted_experts: int
    actual_experts: int = 0
    ready_at_router: int = 0
    inflight_at_router: int = 0
    missing_at_router: int = 0
    prediction_copies: int = 0
    demand_copies: int = 0
    unused_prediction_copies: int = 0
    computed_experts: int = 0
    compute_waits: int = 0


def _is_int(value) -> bool:
    return type(value) is int


class Qwen3ExpertPrefetch:
    """Scheduling context for one complete eager forward of the target."""

    def __init__(self, loaded, predictions: Mapping[int, Sequence[int]], *,
                 lookahead_layers: int = 1, max_inflight: int = 2,
                 max_prefetch_per_layer: int | None = None, trace: bool = False,
                 prediction_probabilities: Mapping[int, Mapping[int, float]] | None = None,
                 eviction_policy: str = "lru") -> None:
        if not _is_int(lookahead_layers) or lookahead_layers < 0:
            raise ValueError("lookahead_layers must be an integer >= 0")
        if not _is_int(max_inflight) or max_inflight < 1:
            raise ValueError("max_inflight must be an integer >= 1")
        if max_prefetch_per_layer is not None and (
                not _is_int(max_prefetch_per_layer) or max_prefetch_per_layer < 0):
            raise ValueError("max_prefetch_per_layer must be a non-negative integer or None")
        if type(trace) is not bool:
            raise ValueError("trace must be a boolean")
        if not isinstance(predictions, Mapping):
            raise TypeError("predictions must map layer IDs to expert IDs")
        if eviction_policy not in ("lru", "probability"):
            raise ValueError("eviction_policy must be 'lru' or 'probability'")
        if prediction_probabilities is None and eviction_policy != "lru":
            raise ValueError("probability eviction requires prediction_probabilities")
        if prediction_probabilities is not None and not isinstance(prediction_probabilities, Mapping):
            raise TypeError("prediction_probabilities must map layers to expert probabilities")
        self._loaded = loaded
        self._layers = tuple(loaded.model.model.layers)
        self._caches = tuple(loaded.expert_caches)
        n_layers = len(self._layers)
        if not self._layers or n_layers != len(self._caches):
            raise ValueError("decoder layers and expert caches must match")
        for name, mapping in (("prediction", predictions),
                              ("probability", prediction_probabilities or {})):
            if any(not _is_int(layer) or not 0 <= layer < n_layers for layer in mapping):
                raise ValueError(f"{name} layer is outside the loaded model")
        # Speculation may hold at most slots-1 slots of a layer.
        self._limits = tuple(
            min(len(c._slots) - 1, len(c._slots) - 1 if max_prefetch_per_layer is None
                else max_prefetch_per_layer)
            for c in self._caches)
        self._probabilities: list[dict | None] = []
        self._requests: list[deque] = []
        normalized = []
        for layer, cache in enumerate(self._caches):
            ids = tuple(predictions.get(layer, ()))
            keys = {}
            if ids or prediction_probabilities is not None:
                keys = {k.expert_id: k for k in cache._sources
                        if type(k) is ExpertKey and k.layer_id == layer}
            if any(not _is_int(e) or e not in keys for e in ids):
                raise ValueError(f"invalid predicted expert in layer {layer}")
            probs = None
            if prediction_probabilities is not None:
                supplied = prediction_probabilities.get(layer, {})
                if not isinstance(supplied, Mapping):
                    raise TypeError("each probability layer must map expert IDs to probabilities")
                scores: dict[int, float] = {}
                probs = {}
                for expert, value in supplied.items():
                    if (not _is_int(expert) or expert not in keys or type(value) is bool
                            or not isinstance(value, Real) or not math.isfinite(value)
                            or not 0 <= value <= 1):
                        raise ValueError(f"invalid expert probability in layer {layer}")
                    scores[expert] = float(value)
                    probs[keys[expert]] = float(value)
                if any(e not in scores for e in ids):
                    raise ValueError("every predicted expert needs an explicit probability")
                ids = tuple(sorted((e for e in set(ids) if scores[e] > 0),
                                   key=lambda e: (-scores[e], e)))[: self._limits[layer]]
            else:
                ids = tuple(sorted(set(ids)))
            self._probabilities.append(probs)
            normalized.append(ids)
            self._requests.append(deque(keys[e] for e in ids))
        if len({c.device for c in self._caches}) != 1:
            raise ValueError("prefetch requires all layers on one GPU")
        self.predictions = tuple(normalized)
        self.lookahead_layers = lookahead_layers
        self.max_inflight = max_inflight
        self.eviction_policy = eviction_policy
        self._trace = trace
        self._events: list[dict] = []
        self._stack = ExitStack()
        self._leases: dict[ExpertKey, ExpertLease] = {}
        self._held_counts = [0] * n_layers
        self._speculative_leases = 0
        self._ranks: dict[ExpertKey, tuple[int, int]] = {}
        self._pending: list[torch.cuda.Event] = []
        # A transfer's event never becomes incomplete again, so once seen
        # complete it is remembered (bounds event queries).
        self._ready_events: set = set()
        self._prediction_copies: set[ExpertKey] = set()
        self._prediction_residents_checked: set[int] = set()
        self._actual: dict[int, set[int]] = {}
        self._layer_stats = [_LayerStats(i, len(ids)) for i, ids in enumerate(self.predictions)]
        self._copy_sequence = 0
        self._next_layer = 0
        self._open_layer: int | None = None
        self._current_layer = 0
        self._entered = self._used = self._complete = False
        self._peak_inflight = self._peak_speculative_leases = 0
        self._queue_capacity_waits = self._slot_wait_copies = 0

    # ------------------------------------------------------------ context --
    def __enter__(self) -> "Qwen3ExpertPrefetch":
        if self._used:
            raise RuntimeError("a prefetch context cannot be reused")
        modules = tuple(layer.mlp.experts for layer in self._layers)
        for layer, (module, cache) in enumerate(zip(modules, self._caches)):
            if (not isinstance(module, Qwen3OffloadedExperts) or module.cache is not cache
                    or module.layer_id != layer):
                raise RuntimeError("every decoder layer must contain its offloaded expert cache")
        if any(m.reduction_mode is not ReductionMode.CANONICAL for m in modules):
            raise ValueError("predicted prefetch requires canonical reduction")
        if any(m._prediction_scheduler is not None for m in modules):
            raise RuntimeError("another predicted prefetch context is active")
        if any(c.closed or c.active_lease_count for c in self._caches):
            raise RuntimeError("prefetch requires open caches without active leases")
        self._used = True
        try:
            self._copy_stream = torch.cuda.Stream(device=self._caches[0].device)
            for cache in self._caches:
                original = cache.copy_stream
                self._copy_stream.wait_stream(original)
                if cache._aux_copy_stream is not original:
                    self._copy_stream.wait_stream(cache._aux_copy_stream)
                # Earlier incomplete transfers keep consuming queue credits.
                self._pending.extend(t.ready_event for t in cache._outstanding_transfers
                                     if not t.ready_event.query())
                cache.copy_stream = self._copy_stream
                self._stack.callback(self._restore_stream, cache, original)
            for lid, (layer, module) in enumerate(zip(self._layers, modules)):
                module._prediction_scheduler = self
                self._stack.callback(setattr, module, "_prediction_scheduler", None)
                handle = layer.self_attn.register_forward_pre_hook(self._attention_hook(lid))
                self._stack.callback(handle.remove)
            self._entered = True
            self._record("prediction_available")
            self._pump()
            return self
        except BaseException:
            for key in tuple(self._leases):
                self._take_lease(key).release()
            self._entered = False
            self._stack.close()
            raise

    def _restore_stream(self, cache, original) -> None:
        original.wait_stream(self._copy_stream)
        cache.copy_stream = original

    def __exit__(self, exc_type, exc, tb) -> None:
        try:
            for key in tuple(self._leases):
                self._take_lease(key).release()
        finally:
            self._entered = False
            self._stack.close()
        self._complete = exc_type is None and self._next_layer == len(self._layers)
        if exc_type is None and not self._complete:
            raise RuntimeError("prefetch context requires exactly one complete target forward")

    # ------------------------------------------------------------ helpers --
    def _record(self, action, *, layer=None, expert=None, **values) -> None:
        if self._trace:
            self._events.append(dict(sequence=len(self._events), action=action,
                                     current_layer=self._current_layer, layer_id=layer,
                                     expert_id=expert, **values))

    def _attention_hook(self, layer: int):
        def hook(module, inputs):
            del module, inputs
            self._begin_layer(layer)
        return hook

    def _begin_layer(self, layer: int) -> None:
        if not self._entered or self._open_layer is not None or layer != self._next_layer:
            raise RuntimeError("predicted prefetch requires one ordered eager layer traversal")
        self._current_layer = self._open_layer = layer
        self._record("attention", layer=layer)
        self._pump()

    def _event_ready(self, event) -> bool:
        if event in self._ready_events:
            return True
        if event.query():
            self._ready_events.add(event)
            return True
        return False

    def _reap(self) -> None:
        self._pending = [e for e in self._pending if not self._event_ready(e)]

    def _take_lease(self, key: ExpertKey) -> ExpertLease:
        lease = self._leases.pop(key)
        self._ranks.pop(key, None)
        self._held_counts[key.layer_id] -= 1
        if key.layer_id not in self._actual:
            self._speculative_leases -= 1
        return lease

    def _hold(self, key: ExpertKey, *, resident_only: bool = False, force: bool = False,
              prediction: bool = False) -> bool:
        """Lease ``key``: resident/in-flight only, non-blocking, or (force) a
        demand acquisition that may queue a wait on a busy slot."""
        cache = self._caches[key.layer_id]
        if resident_only and key not in cache._resident and key not in cache._inflight:
            # The cache's resident-only probe returns None for such a key
            # (publishing completed transfers only moves keys from in-flight
            # to resident), so skip the call and its lock.
            return False
        before = cache._submission_sequence
        if force:
            lease = cache._prefetch(key)
        elif prediction and self.eviction_policy == "probability":
            lease = cache._prefetch_nonblocking(
                key, resident_only=resident_only,
                eviction_probabilities=self._probabilities[key.layer_id])
        else:
            lease = cache._prefetch_nonblocking(key, resident_only=resident_only)
        if lease is None:
            return False
        self._leases[key] = lease
        self._held_counts[key.layer_id] += 1
        if key.layer_id not in self._actual:
            self._speculative_leases += 1
        if key in cache._resident:  # published only after its transfer completed
            self._ready_events.add(lease.ready_event)
        if cache._submission_sequence != before:
            self._pending.append(lease.ready_event)
            self._ranks[key] = (0, self._copy_sequence)
            self._copy_sequence += 1
            stats = self._layer_stats[key.layer_id]
            if prediction:
                self._prediction_copies.add(key)
                stats.prediction_copies += 1
            else:
                stats.demand_copies += 1
            self._peak_inflight = max(self._peak_inflight, len(self._pending))
            self._record("copy", layer=key.layer_id, expert=key.expert_id,
                         prediction=prediction, slot_wait=force)
        else:
            transfer = cache._inflight.get(key)
            self._ranks[key] = (-1, transfer.submission_sequence if transfer else -1)
        self._peak_speculative_leases = max(self._peak_speculative_leases,
                                            self._speculative_leases)
        return True

    def _pump(self) -> None:
        """Place requests, nearest layer first, within the queue and slot
        limits."""
        self._reap()
        last = min(len(self._layers), self._current_layer + self.lookahead_layers + 1)
        for layer in range(self._current_layer, last):
            demand = layer in self._actual
            if not demand and layer not in self._prediction_residents_checked:
                cache = self._caches[layer]
                if cache._resident or cache._inflight:
                    for key in self._requests[layer]:
                        if self._held_counts[layer] >= self._limits[layer]:
                            break
                        if key not in self._leases:
                            self._hold(key, resident_only=True)
                self._prediction_residents_checked.add(layer)
            requests = self._requests[layer]
            while requests:
                key = requests[0]
                if key in self._leases:
                    requests.popleft()
                    continue
                if not demand and self._held_counts[layer] >= self._limits[layer]:
                    return
                if self._hold(key, resident_only=True):
                    requests.popleft()
                    continue
                if len(self._pending) >= self.max_inflight:
                    return
                if not self._hold(key, prediction=not demand):
                    return
                requests.popleft()

    # ---------------------------------------------------------- execution --
    def experts(self, layer: int, active_experts: tuple[int, ...]):
        """Yield each actual expert of ``layer`` once, completed transfers
        first; the yielded lease is released when the generator resumes."""
        if not self._entered or self._open_layer != layer or layer in self._actual:
            raise RuntimeError("expert scheduling must follow this layer's Attention exactly once")
        actual = set(active_experts)
        self._speculative_leases -= self._held_counts[layer]
        self._actual[layer] = actual
        remaining = dict.fromkeys(ExpertKey(layer, e) for e in sorted(actual))
        stats = self._layer_stats[layer]
        stats.actual_experts = len(actual)
        self._record("router", layer=layer, experts=list(active_experts))
        for key in tuple(self._leases):
            if key.layer_id == layer and key.expert_id not in actual:
                self._take_lease(key).release()
        stats.unused_prediction_copies = sum(k.layer_id == layer and k.expert_id not in actual
                                             for k in self._prediction_copies)
        for key in remaining:
            if key not in self._leases:
                self._hold(key, resident_only=True)
            lease = self._leases.get(key)
            if lease is None:
                stats.missing_at_router += 1
            elif self._event_ready(lease.ready_event):
                stats.ready_at_router += 1
            else:
                stats.inflight_at_router += 1
        self._requests[layer] = deque(k for k in remaining if k not in self._leases)
        while remaining:
            self._pump()
            ready = oldest = None
            for candidate in remaining:
                lease = self._leases.get(candidate)
                if lease is None:
                    continue
                if self._event_ready(lease.ready_event):
                    ready = candidate
                    break
                if oldest is None or self._ranks[candidate] < self._ranks[oldest]:
                    oldest = candidate
            if ready is not None:
                key, waited = ready, False
            elif oldest is not None:
                key, waited = oldest, True
                stats.compute_waits += 1
            else:
                self._reap()
                if len(self._pending) >= self.max_inflight:
                    # Only earlier or speculative transfers are in flight and
                    # nothing can run: free one queue credit.
                    self._queue_capacity_waits += 1
                    self._pending[0].synchronize()
                    continue
                # Every reusable slot may still be read by submitted kernels:
                # only this demand fallback queues a use-guard wait.
                key = next(iter(remaining))
                self._hold(key, force=True)
                self._slot_wait_copies += 1
                continue
            lease = self._take_lease(key)
            del remaining[key]
            self._record("compute", layer=layer, expert=key.expert_id, waited=waited)
            try:
                yield key.expert_id, lease
                stats.computed_experts += 1
            finally:
                lease.release()
        self._pump()
        self._open_layer = None
        self._next_layer = layer + 1
        self._record("layer_complete", layer=layer)

    def stats(self) -> dict:
        """Host-side statistics (no GPU synchronisation)."""
        return dict(complete=self._complete, lookahead_layers=self.lookahead_layers,
                    max_inflight=self.max_inflight, prefetch_slot_limits=list(self._limits),
                    peak_inflight=self._peak_inflight,
                    peak_speculative_leases=self._peak_speculative_leases,
                    queue_capacity_waits=self._queue_capacity_waits,
                    slot_wait_copies=self._slot_wait_copies,
                    layers=[asdict(row) for row in self._layer_stats])

    def events(self) -> tuple[dict, ...]:
        return tuple(dict(row) for row in self._events)

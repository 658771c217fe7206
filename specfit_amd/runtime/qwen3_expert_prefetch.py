"""Predicted expert prefetch for exactly one target forward.

Interface of src/specfit/runtime/qwen3_expert_prefetch.py:34-418
(``Qwen3ExpertPrefetch``: constructor arguments and their errors, context
protocol, ``experts(layer, active)``, ``stats()``, ``events()``), the
executor every measured decode of the reference runs under
(run_specfit_main_comparison.py:552-555; with ``predictions={}`` it is the
"ready_demand" executor).

Policy (the reference's):

* every layer cache's copies go to the scheduler's shared copy queue, and
  at most ``max_inflight`` transfers (including ones still running from
  before the context) are incomplete at a time;
* the current layer's demand is placed before future layers' predictions;
  a layer without routes yet may hold at most ``slot_count - 1`` experts
  (``max_prefetch_per_layer`` can lower that), so one slot stays free for
  demand; with ``lookahead_layers`` = n, predictions of the n layers after
  the current one are placed too;
* predicted experts that are already resident are protected (held) once
  per layer, before any earlier-id miss could evict them;
* once a layer's router has run, wrong predictions are dropped and actual
  experts are handed out completed-transfer first (ascending id), else the
  oldest held one in flight (the layer's kernel waits for it on the GPU),
  else one queue credit is awaited or a demand copy is forced into a busy
  slot (the only case that may queue a use-guard wait);
* with ``eviction_policy="probability"``, a speculative copy only replaces
  a writable victim of strictly lower predicted probability.

How it runs here (MI355X host path):

* The shared copy queue is a pair of SDMA streams that the caches
  alternate over (consecutive copies overlap one engine's setup with the
  other's transfer).  The scheduler tracks its own transfers as a FIFO of
  holds in submission order and learns which are complete by querying only
  the oldest incomplete one: no per-expert event polling, and a hold
  becomes "ready" exactly once.  A copy that completes before an older one
  is noticed when the older one completes (readiness is never early).
* Ready experts of the routed layer are collected in a set as their
  transfers complete; ``expert_batches`` hands the layer every ready expert
  at once (ascending id), which the layer computes with ONE grouped K3
  launch and releases together (one use-guard event for the batch).
  ``experts`` keeps the reference's one-expert-at-a-time protocol.
* Each layer's queue, holdings and counters live in a ``_LayerPlan``.
* While a layer's router counts are on their way to the host, the layer
  keeps calling ``_place_while_routing``, which places requests as queue
  credits free up (the attention hook's placement, repeated).  Otherwise
  the copy link idles from the previous layer's last copy until the routes
  arrive; the decisions are the same, only earlier.

Batches change when leases are released relative to the scheduler's own
decisions (a batch's leases are released together, after its launch), not
what is computed: outputs are bitwise those of the per-layer path.
"""
from __future__ import annotations

import math
from collections import deque
from contextlib import ExitStack, closing
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


# Ways the scheduler asks a cache for an expert.
_RESIDENT_ONLY = 0   # join an in-flight transfer or hit a resident slot, else nothing
_SPECULATE = 1       # non-blocking copy of a predicted expert
_DEMAND = 2          # non-blocking copy of a routed expert
_FORCE = 3           # routed expert into a busy slot (may queue a use-guard wait)


class _Hold:
    """A lease the scheduler holds for one expert."""

    __slots__ = ("key", "lease", "rank", "ready")

    def __init__(self, key: ExpertKey, lease: ExpertLease, rank: tuple, ready: bool) -> None:
        self.key = key
        self.lease = lease
        # Order of "oldest in flight": joined transfers (-1, cache sequence)
        # before the scheduler's own copies (0, copy number).
        self.rank = rank
        self.ready = ready


class _LayerPlan:
    """Requests, holdings and counters of one decoder layer."""

    __slots__ = ("layer", "cache", "limit", "keys", "requests", "held", "routed", "protected",
                 "scores", "stats", "prediction_copies")

    def __init__(self, layer: int, cache, limit: int, keys: dict, predicted: tuple,
                 scores: dict | None) -> None:
        self.layer = layer
        self.cache = cache
        self.limit = limit
        self.keys = keys                      # expert id -> the cache's key object
        self.requests = deque(keys[e] for e in predicted)
        self.held = 0                         # holds of this layer
        self.routed: set | None = None        # actual experts, once the router ran
        self.protected = False                # predicted residents held once
        self.scores = scores                  # key -> probability (probability eviction)
        self.stats = _LayerStats(layer, len(predicted))
        self.prediction_copies: set[int] = set()

    def key(self, expert: int) -> ExpertKey:
        k = self.keys.get(expert)
        return k if k is not None else ExpertKey(self.layer, expert)


def _natural(value, minimum: int) -> bool:
    return type(value) is int and value >= minimum


def _layer_keys(cache, layer: int) -> dict:
    return {k.expert_id: k for k in cache._sources
            if type(k) is ExpertKey and k.layer_id == layer}


def _checked_scores(supplied, keys: dict, layer: int) -> dict[int, float]:
    if not isinstance(supplied, Mapping):
        raise TypeError("each probability layer must map expert IDs to probabilities")
    scores = {}
    for expert, value in supplied.items():
        if (type(expert) is not int or expert not in keys or type(value) is bool
                or not isinstance(value, Real) or not math.isfinite(value)
                or not 0 <= value <= 1):
            raise ValueError(f"invalid expert probability in layer {layer}")
        scores[expert] = float(value)
    return scores


class Qwen3ExpertPrefetch:
    """Scheduling context for one complete eager forward of the target."""

    def __init__(self, loaded, predictions: Mapping[int, Sequence[int]], *,
                 lookahead_layers: int = 1, max_inflight: int = 2,
                 max_prefetch_per_layer: int | None = None, trace: bool = False,
                 prediction_probabilities: Mapping[int, Mapping[int, float]] | None = None,
                 eviction_policy: str = "lru") -> None:
        if not _natural(lookahead_layers, 0):
            raise ValueError("lookahead_layers must be an integer >= 0")
        if not _natural(max_inflight, 1):
            raise ValueError("max_inflight must be an integer >= 1")
        if max_prefetch_per_layer is not None and not _natural(max_prefetch_per_layer, 0):
            raise ValueError("max_prefetch_per_layer must be a non-negative integer or None")
        if type(trace) is not bool:
            raise ValueError("trace must be a boolean")
        if not isinstance(predictions, Mapping):
            raise TypeError("predictions must map layer IDs to expert IDs")
        if eviction_policy not in ("lru", "probability"):
            raise ValueError("eviction_policy must be 'lru' or 'probability'")
        scored = prediction_probabilities is not None
        if not scored and eviction_policy != "lru":
            raise ValueError("probability eviction requires prediction_probabilities")
        if scored and not isinstance(prediction_probabilities, Mapping):
            raise TypeError("prediction_probabilities must map layers to expert probabilities")
        self._layers = tuple(loaded.model.model.layers)
        caches = tuple(loaded.expert_caches)
        n = len(self._layers)
        if not n or n != len(caches):
            raise ValueError("decoder layers and expert caches must match")
        for what, mapping in (("prediction", predictions),
                              ("probability", prediction_probabilities or {})):
            if not all(type(lid) is int and 0 <= lid < n for lid in mapping):
                raise ValueError(f"{what} layer is outside the loaded model")
        plans, normalized = [], []
        for lid, cache in enumerate(caches):
            slots = len(cache._slots)
            limit = slots - 1 if max_prefetch_per_layer is None else min(
                slots - 1, max_prefetch_per_layer)
            wanted = tuple(predictions.get(lid, ()))
            keys = _layer_keys(cache, lid)
            if not all(type(e) is int and e in keys for e in wanted):
                raise ValueError(f"invalid predicted expert in layer {lid}")
            scores = None
            if scored:
                given = _checked_scores(prediction_probabilities.get(lid, {}), keys, lid)
                if not all(e in given for e in wanted):
                    raise ValueError("every predicted expert needs an explicit probability")
                # Highest probability first (ties: lower id), zero dropped,
                # at most the layer's speculation limit.
                ranked = sorted((e for e in set(wanted) if given[e] > 0),
                                key=lambda e: (-given[e], e))
                wanted = tuple(ranked[:limit])
                scores = {keys[e]: p for e, p in given.items()}
            else:
                wanted = tuple(sorted(set(wanted)))
            normalized.append(wanted)
            plans.append(_LayerPlan(lid, cache, limit, keys, wanted, scores))
        if len({c.device for c in caches}) != 1:
            raise ValueError("prefetch requires all layers on one GPU")
        self.predictions = tuple(normalized)
        self.lookahead_layers = lookahead_layers
        self.max_inflight = max_inflight
        self.eviction_policy = eviction_policy
        self._caches = caches
        self._plans = plans
        self._trace = trace
        self._log: list[dict] = []
        self._stack = ExitStack()
        self._owned_streams: tuple = ()
        self._holds: dict[ExpertKey, _Hold] = {}
        self._copies: deque[_Hold] = deque()   # own transfers not yet seen complete, in order
        self._prior: list[torch.cuda.Event] = []  # incomplete transfers from before entry
        self._joined: list[_Hold] = []          # holds that joined a transfer not ours
        self._copy_count = 0
        self._speculative = 0
        self._routed_layer: int | None = None   # layer whose experts are being handed out
        self._remaining: dict[int, ExpertKey] = {}
        self._ready_ids: set[int] = set()
        self._next_layer = 0
        self._open_layer: int | None = None
        self._current = 0
        self._entered = self._used = self._complete = False
        self._peak_inflight = self._peak_speculative = 0
        self._capacity_waits = self._slot_wait_copies = 0

    # -------------------------------------------------------------- context --
    def __enter__(self) -> "Qwen3ExpertPrefetch":
        if self._used:
            raise RuntimeError("a prefetch context cannot be reused")
        modules = tuple(layer.mlp.experts for layer in self._layers)
        if not all(isinstance(m, Qwen3OffloadedExperts) and m.cache is c and m.layer_id == lid
                   for lid, (m, c) in enumerate(zip(modules, self._caches))):
            raise RuntimeError("every decoder layer must contain its offloaded expert cache")
        if any(m.reduction_mode is not ReductionMode.CANONICAL for m in modules):
            raise ValueError("predicted prefetch requires canonical reduction")
        if any(m._prediction_scheduler is not None for m in modules):
            raise RuntimeError("another predicted prefetch context is active")
        if any(c.closed or c.active_lease_count for c in self._caches):
            raise RuntimeError("prefetch requires open caches without active leases")
        self._used = True
        try:
            dev = self._caches[0].device
            pair = (torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev))
            self._copy_stream, self._copy_pair = pair[0], pair
            # Copies of the context start after every copy the caches queued
            # before it (the layer caches of a model share one stream pair:
            # each distinct stream is waited for once).
            owned = {}
            for cache in self._caches:
                for s in (cache.copy_stream, cache._aux_copy_stream, cache._own_copy_stream):
                    owned.setdefault(int(s.cuda_stream), s)
            for earlier in owned.values():
                for s in pair:
                    s.wait_stream(earlier)
            self._owned_streams = tuple(owned.values())
            for cache in self._caches:
                own = (cache.copy_stream, cache._aux_copy_stream, cache._own_copy_stream)
                # Transfers still running keep their queue credits.
                self._prior += [t.ready_event for t in cache._outstanding_transfers
                                if not t.ready_event.query()]
                # The caches alternate their transfers over the scheduler's
                # two SDMA streams (one stream's copies run back to back at
                # ~54 GB/s, two alternating ones at ~57 GB/s on MI355X).
                cache.copy_stream, cache._aux_copy_stream = pair
                cache._own_copy_stream = pair[0]
                self._stack.callback(self._give_back_streams, cache, own)
            # Runs first at exit (callbacks run last-in first-out): the
            # caches' own streams wait for the context's copies, once each.
            self._stack.callback(self._order_owned_streams)
            for lid, (layer, module) in enumerate(zip(self._layers, modules)):
                module._prediction_scheduler = self
                self._stack.callback(setattr, module, "_prediction_scheduler", None)
                hook = layer.self_attn.register_forward_pre_hook(self._attention_hook(lid))
                self._stack.callback(hook.remove)
            self._entered = True
            self._note("prediction_available")
            self._pump()
            return self
        except BaseException:
            self._release_all()
            self._entered = False
            self._stack.close()
            raise

    def _order_owned_streams(self) -> None:
        for s in self._owned_streams:
            for mine in self._copy_pair:
                s.wait_stream(mine)

    @staticmethod
    def _give_back_streams(cache, own) -> None:
        cache.copy_stream, cache._aux_copy_stream, cache._own_copy_stream = own

    def __exit__(self, exc_type, exc, tb) -> None:
        try:
            self._release_all()
        finally:
            self._entered = False
            self._stack.close()
        self._complete = exc_type is None and self._next_layer == len(self._layers)
        if exc_type is None and not self._complete:
            raise RuntimeError("prefetch context requires exactly one complete target forward")

    def _release_all(self) -> None:
        for key in tuple(self._holds):
            self._drop(key).release()

    # ---------------------------------------------------------------- trace --
    def _note(self, action, *, layer=None, expert=None, **values) -> None:
        if self._trace:
            self._log.append(dict(sequence=len(self._log), action=action,
                                  current_layer=self._current, layer_id=layer,
                                  expert_id=expert, **values))

    def _attention_hook(self, layer: int):
        def hook(module, inputs):
            self._begin_layer(layer)
        return hook

    def _begin_layer(self, layer: int) -> None:
        if not self._entered or self._open_layer is not None or layer != self._next_layer:
            raise RuntimeError("predicted prefetch requires one ordered eager layer traversal")
        self._current = self._open_layer = layer
        self._note("attention", layer=layer)
        self._pump()

    # ------------------------------------------------------------- holdings --
    def _in_flight(self) -> int:
        return len(self._prior) + len(self._copies)

    def _mark_ready(self, hold: _Hold) -> None:
        hold.ready = True
        key = hold.key
        if key.layer_id == self._routed_layer and key.expert_id in self._remaining:
            self._ready_ids.add(key.expert_id)

    def _advance(self) -> None:
        """Learn which transfers completed: own copies in order (one query
        for the oldest incomplete one, then the next...), then the few
        transfers from before the context and joined ones."""
        copies = self._copies
        while copies and copies[0].lease.ready_event.query():
            self._mark_ready(copies.popleft())
        if self._prior:
            self._prior = [ev for ev in self._prior if not ev.query()]
        if self._joined:
            waiting = []
            for hold in self._joined:
                if self._holds.get(hold.key) is not hold:
                    continue
                if hold.lease.ready_event.query():
                    self._mark_ready(hold)
                else:
                    waiting.append(hold)
            self._joined = waiting

    def _hold(self, key: ExpertKey, mode: int) -> _Hold | None:
        plan = self._plans[key.layer_id]
        cache = plan.cache
        if (mode == _RESIDENT_ONLY and key not in cache._resident and key not in cache._inflight
                and key in cache._sources and not cache._closed):
            # The resident-only lookup of such a key returns None (reaping
            # moves keys from in flight to resident only); an unknown key or
            # a closed cache still goes to the cache, which raises.
            return None
        before = cache._submission_sequence
        if mode == _FORCE:
            lease = cache._prefetch(key)
        elif mode == _SPECULATE and self.eviction_policy == "probability":
            lease = cache._prefetch_nonblocking(key, eviction_probabilities=plan.scores)
        else:
            lease = cache._prefetch_nonblocking(key, resident_only=mode == _RESIDENT_ONLY)
        if lease is None:
            return None
        plan.held += 1
        if plan.routed is None:
            self._speculative += 1
            self._peak_speculative = max(self._peak_speculative, self._speculative)
        if cache._submission_sequence != before:  # this call copied the expert
            hold = _Hold(key, lease, (0, self._copy_count), False)
            self._copy_count += 1
            self._copies.append(hold)
            self._peak_inflight = max(self._peak_inflight, self._in_flight())
            if mode == _SPECULATE:
                plan.stats.prediction_copies += 1
                plan.prediction_copies.add(key.expert_id)
            else:
                plan.stats.demand_copies += 1
            self._note("copy", layer=key.layer_id, expert=key.expert_id,
                       prediction=mode == _SPECULATE, slot_wait=mode == _FORCE)
        elif key in cache._resident:  # residency is published after completion
            hold = _Hold(key, lease, (-1, -1), True)
        else:
            transfer = cache._inflight.get(key)
            hold = _Hold(key, lease, (-1, transfer.submission_sequence if transfer else -1), False)
            self._joined.append(hold)
        self._holds[key] = hold
        if hold.ready:
            self._mark_ready(hold)
        return hold

    def _drop(self, key: ExpertKey) -> ExpertLease:
        hold = self._holds.pop(key)
        plan = self._plans[key.layer_id]
        plan.held -= 1
        if plan.routed is None:
            self._speculative -= 1
        return hold.lease

    # ------------------------------------------------------------ placement --
    def _pump(self) -> None:
        """Place requests nearest layer first within the queue credits and
        the per-layer speculation limits; a layer that cannot place its
        next request stops placement for the layers after it."""
        self._advance()
        stop = min(len(self._plans), self._current + self.lookahead_layers + 1)
        for plan in self._plans[self._current:stop]:
            if not self._place(plan):
                return

    def _place_while_routing(self) -> bool:
        """Called by the open layer while its router's counts are on their
        way to the host: place what the queue credits allow, as the
        attention hook does.  True while a placement waits for a credit
        (the caller polls again), False when nothing more can be placed
        before the routes arrive (the caller then blocks)."""
        if self._open_layer is None:
            return False
        self._pump()
        if self._in_flight() < self.max_inflight:
            return False
        stop = min(len(self._plans), self._current + self.lookahead_layers + 1)
        return any(plan.requests and (plan.routed is not None or plan.held < plan.limit)
                   for plan in self._plans[self._current:stop])

    def _place(self, plan: _LayerPlan) -> bool:
        demand = plan.routed is not None
        holds = self._holds
        if not demand and not plan.protected:
            plan.protected = True
            cache = plan.cache
            if cache._resident or cache._inflight:
                for key in plan.requests:
                    if plan.held >= plan.limit:
                        break
                    if key not in holds:
                        self._hold(key, _RESIDENT_ONLY)
        queue = plan.requests
        mode = _DEMAND if demand else _SPECULATE
        while queue:
            key = queue[0]
            if key not in holds:
                if not demand and plan.held >= plan.limit:
                    return False
                if self._hold(key, _RESIDENT_ONLY) is None:
                    if self._in_flight() >= self.max_inflight or self._hold(key, mode) is None:
                        return False
            queue.popleft()
        return True

    # ------------------------------------------------------------ execution --
    def _route(self, layer: int, active_experts) -> _LayerPlan:
        """The router of ``layer`` ran: drop wrong predictions, hold the
        actual residents, count what is ready, queue the rest as demand."""
        if not self._entered or self._open_layer != layer or self._plans[layer].routed is not None:
            raise RuntimeError("expert scheduling must follow this layer's Attention exactly once")
        plan = self._plans[layer]
        actual = set(active_experts)
        self._speculative -= plan.held
        plan.routed = actual
        stats = plan.stats
        stats.actual_experts = len(actual)
        self._note("router", layer=layer, experts=list(active_experts))
        for key in [k for k in self._holds if k.layer_id == layer and k.expert_id not in actual]:
            self._drop(key).release()
        stats.unused_prediction_copies = len(plan.prediction_copies - actual)
        self._advance()
        self._routed_layer = layer
        keys = plan.keys
        get = keys.get
        self._remaining = remaining = {e: get(e) or ExpertKey(layer, e) for e in sorted(actual)}
        self._ready_ids = set()
        cache = plan.cache
        # Expert ids (int hashing) rather than keys from here on.
        held = {k.expert_id: h for k, h in self._holds.items() if k.layer_id == layer}
        if cache._closed:
            lookup = actual  # the cache raises for any of them
        else:
            # Only these experts can be held (or make the cache raise: ids
            # the layer's sources lack); the resident-only lookup of any
            # other returns nothing and touches nothing, so it is skipped.
            lookup = {k.expert_id for m in (cache._resident, cache._inflight) for k in m
                      if type(k) is ExpertKey and k.layer_id == layer}
            lookup.update(e for e in actual if e not in keys)
        for e, key in remaining.items():
            hold = held.get(e)
            if hold is None and e in lookup:
                hold = self._hold(key, _RESIDENT_ONLY)
            if hold is None:
                stats.missing_at_router += 1
            elif hold.ready:
                stats.ready_at_router += 1
                self._ready_ids.add(e)
            else:
                stats.inflight_at_router += 1
        held = {k.expert_id for k in self._holds if k.layer_id == layer}
        plan.requests = deque(k for e, k in remaining.items() if e not in held)
        return plan

    def _oldest_in_flight(self) -> _Hold | None:
        """The held, not yet ready routed expert with the smallest rank."""
        remaining, layer = self._remaining, self._routed_layer
        best = None
        for hold in self._joined:
            k = hold.key
            if (k.layer_id == layer and k.expert_id in remaining and not hold.ready
                    and self._holds.get(k) is hold and (best is None or hold.rank < best.rank)):
                best = hold
        if best is not None:
            return best
        for hold in self._copies:
            k = hold.key
            if k.layer_id == layer and k.expert_id in remaining and self._holds.get(k) is hold:
                return hold
        return None

    def _steps(self, layer: int, active_experts, batched: bool):
        """Core of ``experts`` / ``expert_batches``: yields lists of
        (expert id, lease); the leases are released when it resumes."""
        plan = self._route(layer, active_experts)
        stats = plan.stats
        remaining = self._remaining
        try:
            while remaining:
                self._pump()
                ready = self._ready_ids
                if ready:
                    ids = sorted(ready) if batched else [min(ready)]
                    ready.difference_update(ids)
                    waited = False
                else:
                    hold = self._oldest_in_flight()
                    if hold is None:
                        if self._in_flight() >= self.max_inflight:
                            # Only speculative or earlier transfers are in
                            # flight and nothing routed can run: free a credit.
                            self._capacity_waits += 1
                            first = self._prior[0] if self._prior else self._copies[0].lease.ready_event
                            first.synchronize()
                            continue
                        # Every writable slot is taken: the one demand copy
                        # allowed to queue a wait on a busy slot.
                        self._hold(next(iter(remaining.values())), _FORCE)
                        self._slot_wait_copies += 1
                        continue
                    ids = [hold.key.expert_id]
                    waited = True
                    stats.compute_waits += 1
                keys = [remaining.pop(e) for e in ids]
                leases = [self._drop(k) for k in keys]
                for e in ids:
                    self._note("compute", layer=layer, expert=e, waited=waited)
                try:
                    yield list(zip(ids, leases))
                    stats.computed_experts += len(ids)
                finally:
                    self._release_batch(plan.cache, leases)
        finally:
            self._routed_layer = None
            self._ready_ids = set()
        self._pump()
        self._open_layer = None
        self._next_layer = layer + 1
        self._note("layer_complete", layer=layer)

    @staticmethod
    def _release_batch(cache, leases: list) -> None:
        """Release a batch whose weights one launch read: per-lease release
        bookkeeping, then one use-guard event per reader stream."""
        if len(leases) == 1:
            leases[0].release()
            return
        for lease in leases:
            lease._release_keep_pinned()
        cache._unpin_many(leases)

    def expert_batches(self, layer: int, active_experts: tuple[int, ...]):
        """Yield the actual experts of ``layer`` in batches: every expert
        whose transfer has completed (ascending id), else the oldest in
        flight alone.  A batch's leases are released when the generator
        resumes, so the caller enqueues the batch's kernel before that."""
        return self._steps(layer, active_experts, True)

    def experts(self, layer: int, active_experts: tuple[int, ...]):
        """Yield each actual expert of ``layer`` once, completed transfers
        first; the yielded lease is released when the generator resumes."""
        steps = self._steps(layer, active_experts, False)
        with closing(steps):
            for batch in steps:
                yield batch[0]

    def stats(self) -> dict:
        """Host-side statistics (no GPU synchronisation)."""
        return dict(complete=self._complete, lookahead_layers=self.lookahead_layers,
                    max_inflight=self.max_inflight,
                    prefetch_slot_limits=[p.limit for p in self._plans],
                    peak_inflight=self._peak_inflight,
                    peak_speculative_leases=self._peak_speculative,
                    queue_capacity_waits=self._capacity_waits,
                    slot_wait_copies=self._slot_wait_copies,
                    layers=[asdict(p.stats) for p in self._plans])

    def events(self) -> tuple[dict, ...]:
        return tuple(dict(row) for row in self._log)

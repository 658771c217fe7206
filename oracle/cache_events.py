"""Independent replay of recorded cache transitions.

TEST INFRASTRUCTURE ONLY (see the package docstring): the independent side
of the cross-layer prefetch audit.  It restates the event audit of
src/specfit/cross_layer_prefetch.py:60-142 (``CompactTransitions`` and
``replay_events``): starting from a logical pre-state of every layer cache
(slots, LRU and submission sequences, counters, as read from snapshots), it
rebuilds assignments, generations, leases, LRU touches and counters from the
host decisions a cache observer recorded, validating each decision on the
way, and returns the post-state, which must equal the live caches'.

Touch rule per runtime variant (how the executor leases experts):
``demand`` acquires every expert with an immediate LRU touch; ``one_ahead``
touches its first acquisition of each layer at once and defers the others
(prefetches) to their consume wait; the scheduler variants defer every
lease.  For the predicted variants, a layer whose routed experts fit in all
but one slot is "accurate": its speculation must never evict a routed expert
that has not been consumed yet.
"""
from __future__ import annotations

from copy import deepcopy

VARIANTS = ("demand", "one_ahead", "ready_demand", "predicted_same_layer",
            "predicted_cross_layer", "wrong_cross_layer")

_COUNTER = {"h2d_submit": "h2d_submissions", "resident_hit": "resident_hits",
            "inflight_join": "inflight_joins", "evict": "evictions"}
_LEASING = ("h2d_submit", "resident_hit", "inflight_join")


class CompactTransitions:
    """Cache observer keeping (kind, layer, expert, slot, generation,
    submission sequence, victim expert) per transition; the same observer
    serves every variant."""

    def __init__(self) -> None:
        self.events: list[tuple] = []

    def record(self, *, kind, expert_id, slot_id, generation, submission_sequence=None,
               victim_expert_id=None, **_ignored) -> None:
        victim = None if victim_expert_id is None else victim_expert_id.expert_id
        self.events.append((kind.value, expert_id.layer_id, expert_id.expert_id, slot_id,
                            generation, submission_sequence, victim))


class _Replay:
    def __init__(self, pre: dict, actual: set, variant: str) -> None:
        if variant not in VARIANTS:
            raise ValueError("unknown runtime variant")
        self.state = deepcopy(pre)
        self.actual = actual
        self.variant = variant
        self.consumed: set = set()
        self.evicting: dict = {}   # (layer, slot) -> (incoming expert, its generation)
        self.deferred: dict = {}   # (layer, slot) -> touch still owed to the wait
        self.first_done: set = set()
        self.accurate = set()
        if variant in ("predicted_same_layer", "predicted_cross_layer"):
            for lid, layer in enumerate(self.state["layers"]):
                routed = sum(1 for key in actual if key[0] == lid)
                if routed <= len(layer["slots"]) - 1:
                    self.accurate.add(lid)

    @staticmethod
    def _touch(layer: dict, slot: dict) -> None:
        layer["lru_sequence"] += 1
        slot["last_used_sequence"] = layer["lru_sequence"]

    def apply(self, event) -> None:
        if len(event) != 7:
            raise ValueError("invalid cache event shape")
        kind, lid, expert, sid, gen, submission, victim = event
        if (any(type(v) is not int or v < 0 for v in (lid, expert, sid, gen))
                or lid >= len(self.state["layers"]) or expert >= 128):
            raise ValueError("invalid event identity")
        layer = self.state["layers"][lid]
        if sid >= len(layer["slots"]):
            raise ValueError("event slot outside cache")
        slot = layer["slots"][sid]
        where = (lid, sid)
        handler = getattr(self, "_on_" + kind, None)
        if handler is None:
            raise ValueError("unknown cache event")
        handler(layer, slot, where, lid, expert, gen, submission, victim)
        if kind != "evict" and (slot["expert_id"] != expert or slot["generation"] != gen):
            raise ValueError("event uses a stale slot generation")
        if kind in _LEASING:
            self._lease(layer, slot, where, lid)
        if kind in _COUNTER:
            layer["counters"][_COUNTER[kind]] += 1

    def _on_evict(self, layer, slot, where, lid, expert, gen, submission, victim):
        if (lid in self.accurate and (lid, victim) in self.actual
                and (lid, victim) not in self.consumed):
            raise ValueError("accurate prefetch evicted an unconsumed actual expert")
        if (slot["active_leases"] or victim is None or slot["expert_id"] != victim
                or gen != slot["generation"] + 1 or where in self.evicting):
            raise ValueError("invalid eviction or leased victim")
        self.evicting[where] = (expert, gen)

    def _on_h2d_submit(self, layer, slot, where, lid, expert, gen, submission, victim):
        if slot["active_leases"] or gen != slot["generation"] + 1:
            raise ValueError("invalid copy, generation, sequence or protected slot")
        if submission != layer["submission_sequence"]:
            raise ValueError("invalid copy, generation, sequence or protected slot")
        if any(s["expert_id"] == expert for s in layer["slots"]):
            raise ValueError("invalid copy, generation, sequence or protected slot")
        if slot["expert_id"] is not None and self.evicting.pop(where, None) != (expert, gen):
            raise ValueError("invalid copy, generation, sequence or protected slot")
        slot.update(expert_id=expert, generation=gen, ready=True, pending_use_guards=0)
        layer["submission_sequence"] += 1

    def _on_resident_hit(self, *args):
        pass

    def _on_inflight_join(self, *args):
        pass

    def _lease(self, layer, slot, where, lid):
        if slot["active_leases"]:
            raise ValueError("experiment acquired the same expert twice concurrently")
        slot["active_leases"] += 1
        if self.variant == "demand":
            later = False
        elif self.variant == "one_ahead":
            later = lid in self.first_done
        else:
            later = True
        self.first_done.add(lid)
        self.deferred[where] = later
        if not later:
            self._touch(layer, slot)

    def _on_consume_wait(self, layer, slot, where, lid, expert, gen, submission, victim):
        key = (lid, expert)
        if not slot["active_leases"] or key not in self.actual or key in self.consumed:
            raise ValueError("unleased, duplicate or non-router expert consumption")
        self.consumed.add(key)
        if self.deferred.pop(where, False):
            self._touch(layer, slot)

    def _on_release(self, layer, slot, where, lid, expert, gen, submission, victim):
        if slot["active_leases"] != 1:
            raise ValueError("release without a live lease")
        slot["active_leases"] -= 1
        self.deferred.pop(where, None)
        self._touch(layer, slot)

    def finish(self) -> dict:
        leased = any(s["active_leases"] for layer in self.state["layers"] for s in layer["slots"])
        if self.consumed != self.actual or self.evicting or leased:
            raise ValueError("incomplete actual computation, copy or lease release")
        return self.state


_SLOT_FIELDS = ("slot_id", "generation", "active_leases", "last_used_sequence", "ready",
                "pending_use_guards")


def logical_state(snapshots) -> dict:
    """The logical state the replay works on, read from one snapshot per
    layer cache (in layer order): per layer its capacity, LRU and submission
    sequences and counters, and per slot its expert id (the id within the
    layer), generation, leases, last use, readiness and pending use guards."""
    from dataclasses import fields

    layers = []
    for lid, snap in enumerate(snapshots):
        slots = []
        for s in snap.slots:
            row = {name: getattr(s, name) for name in _SLOT_FIELDS}
            row["expert_id"] = None if s.expert_id is None else s.expert_id.expert_id
            slots.append(row)
        counters = {f.name: getattr(snap.stats, f.name) for f in fields(snap.stats)}
        layers.append({"layer_id": lid, "capacity": snap.capacity,
                       "lru_sequence": snap.lru_sequence,
                       "submission_sequence": snap.submission_sequence,
                       "counters": counters, "slots": slots})
    return {"layers": layers}


def replay_events(pre: dict, events, actual: set, variant: str) -> dict:
    """Post-state of ``pre`` after ``events`` (CompactTransitions tuples)
    under ``variant``; ``actual`` is the set of (layer, expert) the routers
    chose.  Raises ValueError on the first inconsistent decision."""
    replay = _Replay(pre, actual, variant)
    for event in events:
        replay.apply(event)
    return replay.finish()

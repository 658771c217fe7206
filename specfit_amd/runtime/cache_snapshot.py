"""Immutable, validated cache snapshots.

Interface of src/specfit/runtime/cache_snapshot.py:21-144: the three frozen
records, their fields, and the error type and message of every invariant.
The invariants are kept as rule tables (``_checks.Rule``), evaluated in
table order by ``__post_init__``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Hashable

import torch

from ._checks import Rule, count_rules, enforce
from .lease import ExpertCacheStats


def _empty_slot_is_idle(s) -> bool:
    return s.expert_id is not None or not (s.ready or s.active_leases or s.pending_use_guards)


_SLOT_RULES = count_rules("slot_id", "generation", "active_leases", "last_used_sequence",
                          "pending_use_guards") + (
    Rule(lambda s: isinstance(s.ready, bool), TypeError, "ready must be a boolean"),
    Rule(_empty_slot_is_idle, ValueError, "an empty slot cannot be ready or in use"),
)


@dataclass(frozen=True, slots=True)
class CacheSlotSnapshot:
    slot_id: int
    expert_id: Hashable | None
    generation: int
    active_leases: int
    last_used_sequence: int
    ready: bool
    pending_use_guards: int

    def __post_init__(self) -> None:
        enforce(self, _SLOT_RULES)


_TRANSFER_RULES = count_rules("slot_id", "generation", "submission_sequence") + (
    Rule(lambda t: isinstance(t.ready_event_completed, bool), TypeError,
         "ready_event_completed must be a boolean"),
)


@dataclass(frozen=True, slots=True)
class PendingTransferSnapshot:
    expert_id: Hashable
    slot_id: int
    generation: int
    submission_sequence: int
    ready_event: torch.cuda.Event
    ready_event_completed: bool

    def __post_init__(self) -> None:
        enforce(self, _TRANSFER_RULES)


def _pending_sequences(snap) -> list[int]:
    return [t.submission_sequence for t in snap.pending_transfers]


def _assignments_unique(snap) -> bool:
    held = [s.expert_id for s in snap.slots if s.expert_id is not None]
    return len(held) == len(set(held))


def _transfer_slots(snap):
    """(transfer, its slot or None) for every pending transfer."""
    by_slot = {s.slot_id: s for s in snap.slots}
    return [(t, by_slot.get(t.slot_id)) for t in snap.pending_transfers]


_SNAPSHOT_RULES = (
    Rule(lambda g: bool(g.cache_id) and bool(g.queue_id), ValueError,
         "cache_id and queue_id must be non-empty"),
    *count_rules("capacity", "host_state_version", "lru_sequence", "submission_sequence"),
    Rule(lambda g: g.capacity != 0, ValueError, "cache capacity must be positive"),
    Rule(lambda g: isinstance(g.slots, tuple), TypeError, "slots must be an immutable tuple"),
    Rule(lambda g: isinstance(g.pending_transfers, tuple), TypeError,
         "pending_transfers must be an immutable tuple"),
    Rule(lambda g: len(g.slots) == g.capacity, ValueError,
         "snapshot must contain every cache slot"),
    Rule(lambda g: [s.slot_id for s in g.slots] == list(range(g.capacity)), ValueError,
         "slot IDs must cover range(capacity)"),
    Rule(_assignments_unique, ValueError, "current expert assignments must be unique"),
    Rule(lambda g: _pending_sequences(g) == sorted(_pending_sequences(g)), ValueError,
         "pending transfers must follow submission order"),
    Rule(lambda g: len(set(_pending_sequences(g))) == len(g.pending_transfers), ValueError,
         "pending submission sequences must be unique"),
    Rule(lambda g: all(q < g.submission_sequence for q in _pending_sequences(g)), ValueError,
         "pending sequence must precede the submission counter"),
    Rule(lambda g: all(slot is not None for _, slot in _transfer_slots(g)), ValueError,
         "pending transfer references an unknown slot"),
    Rule(lambda g: all(t.generation <= slot.generation for t, slot in _transfer_slots(g)),
         ValueError, "pending transfer generation exceeds its current slot"),
    Rule(lambda g: all(t.generation != slot.generation or t.expert_id == slot.expert_id
                       for t, slot in _transfer_slots(g)),
         ValueError, "current pending transfer does not match its slot"),
)


@dataclass(frozen=True, slots=True)
class GpuExpertCacheSnapshot:
    cache_id: str
    queue_id: str
    capacity: int
    host_state_version: int
    lru_sequence: int
    submission_sequence: int
    slots: tuple
    pending_transfers: tuple
    stats: ExpertCacheStats

    def __post_init__(self) -> None:
        enforce(self, _SNAPSHOT_RULES)

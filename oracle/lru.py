"""CPU restatement of the expert cache's LRU decisions -- TEST INFRASTRUCTURE.

Follows src/specfit/replay.py:217-279 (``_LayerState.access`` and
``_choose_lru_slot``), which restates GpuExpertCache._acquire /
_choose_lru_slot / _assign_and_submit / _release
(src/specfit/runtime/gpu_expert_cache.py:224-266, 495-518, 543-589, 684-718)
for sequential acquire -> consume -> release accesses.  The resident-first
execution order follows replay.py:339-363 and
qwen3_offloaded_experts.py:277-292.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class Slot:
    slot_id: int
    expert_id: object = None
    generation: int = 0
    active_leases: int = 0
    last_used_sequence: int = 0


@dataclass
class LayerLRU:
    slot_count: int
    lru_sequence: int = 0
    submission_sequence: int = 0
    h2d_submissions: int = 0
    resident_hits: int = 0
    evictions: int = 0
    slots: list = field(default_factory=list)
    events: list = field(default_factory=list)

    def __post_init__(self):
        if not self.slots:
            self.slots = [Slot(i) for i in range(self.slot_count)]

    def _touch(self, slot: Slot) -> None:
        self.lru_sequence += 1
        slot.last_used_sequence = self.lru_sequence

    def choose_lru_slot(self) -> Slot:
        available = [s for s in self.slots if s.active_leases == 0]
        if not available:
            raise RuntimeError("no replaceable expert slot")
        return min(available, key=lambda s: (s.expert_id is not None,
                                             s.last_used_sequence, s.slot_id))

    def access(self, expert_id) -> str:
        """One acquire + consume + release.  Returns 'hit' or 'miss'."""
        resident = next((s for s in self.slots if s.expert_id == expert_id), None)
        if resident is not None:
            slot = resident
            self.resident_hits += 1
            kind = "hit"
            self.events.append(("resident_hit", expert_id, slot.slot_id, slot.generation))
        else:
            slot = self.choose_lru_slot()
            victim = slot.expert_id
            slot.generation += 1
            slot.expert_id = expert_id
            if victim is not None:
                self.evictions += 1
                self.events.append(("evict", expert_id, slot.slot_id, slot.generation, victim))
            self.events.append(("h2d_submit", expert_id, slot.slot_id, slot.generation,
                                self.submission_sequence))
            self.submission_sequence += 1
            self.h2d_submissions += 1
            kind = "miss"
        slot.active_leases += 1
        self._touch(slot)
        slot.active_leases -= 1
        self._touch(slot)
        return kind

    def resident(self) -> set:
        return {s.expert_id for s in self.slots if s.expert_id is not None}

    def resident_first(self, active) -> tuple:
        res = self.resident()
        active = tuple(sorted(active))
        return tuple(e for e in active if e in res) + tuple(e for e in active if e not in res)

    def state(self) -> tuple:
        return tuple((s.slot_id, s.expert_id, s.generation, s.last_used_sequence)
                     for s in self.slots)

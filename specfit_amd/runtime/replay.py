"""Logical replay of the expert caches: what a given access sequence would
do to cache state, without a GPU.

Restates the counterfactual replay of src/specfit/replay.py:14-121
(result types) and :217-455 (``_LayerState.access``,
``replay_qwen3_accesses``, ``replay_qwen3_access_cycles``): starting from a
quiescent snapshot of every layer's cache, each accessed expert is a
resident hit or a miss that takes the LRU victim ``min(occupied,
last_used_sequence, slot_id)``, then an acquire touch, a consume wait and a
release touch; per access the same events and counters the runtime
records.  The closing checks of the reference hold on every result
(occupancy equation, event count, H2D = initially non-resident accesses +
reloads).

The BEFORE state is a sequence of per-layer ``GpuExpertCacheSnapshot``s
(``LoadedOffloadedQwen3.cache_snapshots()``), layer ``l`` at index ``l``;
slot expert ids may be ``ExpertKey``s or plain ints.  This is the input the
cost model's selector consumes; the trace-bundle chain replay of the
reference (``replay_qwen3_chain``) sits on its trace schemas and is not
restated.
"""
from __future__ import annotations

from dataclasses import dataclass

from .state import ExpertKey
from .trace import RuntimeEventKind


class LogicalReplayError(ValueError):
    """A replay input is malformed or a closing check failed."""


@dataclass(frozen=True, slots=True)
class ReplayCounters:
    h2d_submissions: int = 0
    resident_hits: int = 0
    inflight_joins: int = 0
    evictions: int = 0
    consume_waits: int = 0
    releases: int = 0

    @property
    def acquisitions(self) -> int:
        return self.h2d_submissions + self.resident_hits + self.inflight_joins

    @property
    def event_count(self) -> int:
        return self.acquisitions + self.evictions + self.consume_waits + self.releases

    def __add__(self, other: "ReplayCounters") -> "ReplayCounters":
        if not isinstance(other, ReplayCounters):
            return NotImplemented
        return ReplayCounters(*(a + b for a, b in zip(
            (self.h2d_submissions, self.resident_hits, self.inflight_joins, self.evictions,
             self.consume_waits, self.releases),
            (other.h2d_submissions, other.resident_hits, other.inflight_joins, other.evictions,
             other.consume_waits, other.releases))))


@dataclass(frozen=True, slots=True)
class LogicalReplayEvent:
    kind: RuntimeEventKind
    layer_id: int
    expert_id: int
    slot_id: int
    generation: int
    submission_sequence: int | None = None
    victim_expert_id: int | None = None


@dataclass(frozen=True, slots=True)
class ReplaySlotState:
    layer_id: int
    slot_id: int
    expert_id: int | None
    generation: int
    last_used_sequence: int


@dataclass(frozen=True, slots=True)
class ExpertAccessReplayResult:
    accessed_experts_by_layer: tuple[tuple[int, ...], ...]
    counters: ReplayCounters
    events: tuple[LogicalReplayEvent, ...]
    initial_occupancy: int
    final_occupancy: int
    final_slots: tuple[ReplaySlotState, ...]
    final_submission_sequences: tuple[int, ...]
    final_lru_sequences: tuple[int, ...]
    initial_resident_reload_h2d: int


def _expert_int(expert) -> int | None:
    if expert is None:
        return None
    return expert.expert_id if isinstance(expert, ExpertKey) else int(expert)


class _Layer:
    """Mutable replay state of one layer's cache."""

    __slots__ = ("layer_id", "submission_sequence", "lru_sequence", "stats", "slots")

    def __init__(self, layer_id: int, snapshot) -> None:
        where = f"counterfactual BEFORE layer {layer_id}"
        if snapshot.pending_transfers:
            raise LogicalReplayError(f"{where}: pending transfer remains at the cycle boundary")
        if snapshot.stats.pending_use_guards:
            raise LogicalReplayError(f"{where}: cycle boundary still has pending use guard")
        for s in snapshot.slots:
            if s.active_leases:
                raise LogicalReplayError(f"{where}: active lease remains at cycle boundary")
            if s.pending_use_guards:
                raise LogicalReplayError(f"{where}: slot still has a pending use guard")
            if s.expert_id is not None and not s.ready:
                raise LogicalReplayError(f"{where}: assigned slot not yet ready")
        self.layer_id = layer_id
        self.submission_sequence = snapshot.submission_sequence
        self.lru_sequence = snapshot.lru_sequence
        st = snapshot.stats
        self.stats = [st.h2d_submissions, st.resident_hits, st.inflight_joins, st.evictions]
        # slot: [slot_id, expert, generation, active_leases, last_used]
        self.slots = [[s.slot_id, _expert_int(s.expert_id), s.generation, 0, s.last_used_sequence]
                      for s in snapshot.slots]

    @property
    def occupancy(self) -> int:
        return sum(s[1] is not None for s in self.slots)

    def _touch(self, slot) -> None:
        self.lru_sequence += 1
        slot[4] = self.lru_sequence

    def _event(self, kind, expert, slot, **kw) -> LogicalReplayEvent:
        return LogicalReplayEvent(kind=kind, layer_id=self.layer_id, expert_id=expert,
                                  slot_id=slot[0], generation=slot[2], **kw)

    def access(self, expert: int) -> list[LogicalReplayEvent]:
        events = []
        slot = next((s for s in self.slots if s[1] == expert), None)
        if slot is not None:
            self.stats[1] += 1
            events.append(self._event(RuntimeEventKind.RESIDENT_HIT, expert, slot))
        else:
            free = [s for s in self.slots if s[3] == 0]
            if not free:
                raise LogicalReplayError(f"layer {self.layer_id}: no replaceable expert slot")
            slot = min(free, key=lambda s: (s[1] is not None, s[4], s[0]))
            victim = slot[1]
            slot[2] += 1
            slot[1] = expert
            if victim is not None:
                self.stats[3] += 1
                events.append(self._event(RuntimeEventKind.EVICT, expert, slot,
                                          victim_expert_id=victim))
            seq = self.submission_sequence
            self.submission_sequence += 1
            self.stats[0] += 1
            events.append(self._event(RuntimeEventKind.H2D_SUBMIT, expert, slot,
                                      submission_sequence=seq))
        slot[3] += 1
        self._touch(slot)
        events.append(self._event(RuntimeEventKind.CONSUME_WAIT, expert, slot))
        events.append(self._event(RuntimeEventKind.RELEASE, expert, slot))
        slot[3] -= 1
        self._touch(slot)
        return events


def replay_qwen3_accesses(before_layers, accessed_experts_by_layer) -> ExpertAccessReplayResult:
    """One cycle of accesses (each layer's experts unique, ascending)."""
    return replay_qwen3_access_cycles(before_layers, (tuple(accessed_experts_by_layer),))[0]


def replay_qwen3_access_cycles(before_layers, accessed_experts_by_cycle, *,
                               resident_first: bool = False
                               ) -> tuple[ExpertAccessReplayResult, ...]:
    """Consecutive cycles from one BEFORE state; with ``resident_first``
    each layer runs its currently resident experts first, then the rest,
    each group ascending (the RESIDENT_FIRST execution policy)."""
    if not isinstance(resident_first, bool):
        raise LogicalReplayError("resident_first must be bool")
    cycles = tuple(tuple(tuple(layer) for layer in cycle) for cycle in accessed_experts_by_cycle)
    if not cycles:
        raise LogicalReplayError("counterfactual cycle sequence must not be empty")
    before_layers = tuple(before_layers)
    for cycle in cycles:
        if len(cycle) != len(before_layers):
            raise LogicalReplayError("counterfactual access layer count does not match BEFORE")
        for lid, experts in enumerate(cycle):
            bad = any(isinstance(e, bool) or not isinstance(e, int) or e < 0 for e in experts)
            if bad or experts != tuple(sorted(set(experts))):
                raise LogicalReplayError(
                    f"counterfactual layer {lid} experts must be unique and in ascending order")
    layers = [_Layer(lid, snap) for lid, snap in enumerate(before_layers)]
    results = []
    for cycle in cycles:
        order = cycle
        if resident_first:
            order = tuple(
                tuple(e for e in experts if e in {s[1] for s in layer.slots})
                + tuple(e for e in experts if e not in {s[1] for s in layer.slots})
                for layer, experts in zip(layers, cycle))
        results.append(_replay_cycle(layers, cycle, order))
    return tuple(results)


def _replay_cycle(layers: list[_Layer], accessed, order) -> ExpertAccessReplayResult:
    initial_occupancy = sum(layer.occupancy for layer in layers)
    initial_resident = {(layer.layer_id, s[1]) for layer in layers for s in layer.slots
                        if s[1] is not None}
    stats_before = [list(layer.stats) for layer in layers]
    events: list[LogicalReplayEvent] = []
    for layer, experts in zip(layers, order):
        for expert in experts:
            events.extend(layer.access(expert))
    delta = [0, 0, 0, 0]
    for layer, before in zip(layers, stats_before):
        d = [a - b for a, b in zip(layer.stats, before)]
        if any(v < 0 for v in d):
            raise LogicalReplayError(f"counterfactual layer {layer.layer_id}: "
                                     "cumulative counter regressed")
        delta = [x + y for x, y in zip(delta, d)]
    counters = ReplayCounters(
        h2d_submissions=delta[0], resident_hits=delta[1], inflight_joins=delta[2],
        evictions=delta[3],
        consume_waits=sum(e.kind is RuntimeEventKind.CONSUME_WAIT for e in events),
        releases=sum(e.kind is RuntimeEventKind.RELEASE for e in events))
    final_slots = tuple(ReplaySlotState(layer.layer_id, s[0], s[1], s[2], s[4])
                        for layer in layers for s in layer.slots)
    final_occupancy = sum(s.expert_id is not None for s in final_slots)
    if final_occupancy - initial_occupancy != counters.h2d_submissions - counters.evictions:
        raise LogicalReplayError("counterfactual occupancy equation cannot close")
    if counters.event_count != len(events):
        raise LogicalReplayError("counterfactual event count cannot be reconciled")
    reloads = sum(e.kind is RuntimeEventKind.H2D_SUBMIT
                  and (e.layer_id, e.expert_id) in initial_resident for e in events)
    nonresident = sum((lid, e) not in initial_resident
                      for lid, experts in enumerate(accessed) for e in experts)
    if counters.h2d_submissions != nonresident + reloads:
        raise LogicalReplayError("counterfactual H2D dynamic classification cannot be closed")
    return ExpertAccessReplayResult(
        accessed_experts_by_layer=accessed, counters=counters, events=tuple(events),
        initial_occupancy=initial_occupancy, final_occupancy=final_occupancy,
        final_slots=final_slots,
        final_submission_sequences=tuple(layer.submission_sequence for layer in layers),
        final_lru_sequences=tuple(layer.lru_sequence for layer in layers),
        initial_resident_reload_h2d=reloads)

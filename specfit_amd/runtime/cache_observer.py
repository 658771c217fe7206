"""Cache transition observer protocol and recorder
(src/specfit/runtime/cache_observer.py:14-198)."""
from __future__ import annotations

from dataclasses import dataclass
from threading import Lock
from time import perf_counter_ns
from typing import Hashable, Protocol

import torch

from .trace import RuntimeEventKind


class CacheTransitionObserver(Protocol):
    def record(self, *, kind: RuntimeEventKind, cache_id: str, queue_id: str,
               expert_id: Hashable, slot_id: int, generation: int,
               submission_sequence: int | None = None,
               victim_expert_id: Hashable | None = None,
               ready_event: torch.cuda.Event | None = None,
               stream_ids: tuple[int, ...] = ()) -> None: ...


def _is_nonneg_int(value) -> bool:
    return not isinstance(value, bool) and isinstance(value, int) and value >= 0


@dataclass(frozen=True, slots=True)
class CacheTransition:
    run_id: str
    sequence: int
    host_time_ns: int
    kind: RuntimeEventKind
    cache_id: str
    queue_id: str
    expert_id: Hashable
    slot_id: int
    generation: int
    submission_sequence: int | None = None
    victim_expert_id: Hashable | None = None
    ready_event: torch.cuda.Event | None = None
    stream_ids: tuple[int, ...] = ()

    def __post_init__(self) -> None:
        if not self.run_id or not self.cache_id or not self.queue_id:
            raise ValueError("run_id, cache_id and queue_id must be non-empty")
        for name in ("sequence", "host_time_ns", "slot_id", "generation"):
            if not _is_nonneg_int(getattr(self, name)):
                raise ValueError(f"{name} must be a non-negative integer")
        if not isinstance(self.kind, RuntimeEventKind):
            object.__setattr__(self, "kind", RuntimeEventKind(self.kind))
        if self.submission_sequence is not None and not _is_nonneg_int(self.submission_sequence):
            raise ValueError("submission_sequence must be non-negative")
        if not isinstance(self.stream_ids, tuple):
            raise TypeError("stream_ids must be an immutable tuple")
        if (any(not _is_nonneg_int(s) for s in self.stream_ids)
                or len(self.stream_ids) != len(set(self.stream_ids))):
            raise ValueError("stream_ids must contain unique non-negative integers")
        if self.kind is RuntimeEventKind.H2D_SUBMIT and (
                self.submission_sequence is None or self.ready_event is None):
            raise ValueError("H2D submit requires a sequence and ready event")
        if self.kind is RuntimeEventKind.EVICT and self.victim_expert_id is None:
            raise ValueError("eviction requires a victim expert")


@dataclass(frozen=True, slots=True)
class CacheTransitionCounters:
    h2d_submissions: int = 0
    resident_hits: int = 0
    inflight_joins: int = 0
    evictions: int = 0


class RecordingCacheTransitionObserver:
    """Thread-safe in-memory recorder with a per-run sequence number."""

    def __init__(self, *, run_id: str) -> None:
        if not isinstance(run_id, str) or not run_id:
            raise ValueError("run_id must be a non-empty string")
        self.run_id = run_id
        self._events: list[CacheTransition] = []
        self._lock = Lock()

    def record(self, *, kind, cache_id, queue_id, expert_id, slot_id, generation,
               submission_sequence=None, victim_expert_id=None, ready_event=None,
               stream_ids=()) -> None:
        with self._lock:
            self._events.append(CacheTransition(
                run_id=self.run_id, sequence=len(self._events), host_time_ns=perf_counter_ns(),
                kind=kind, cache_id=cache_id, queue_id=queue_id, expert_id=expert_id,
                slot_id=slot_id, generation=generation, submission_sequence=submission_sequence,
                victim_expert_id=victim_expert_id, ready_event=ready_event,
                stream_ids=stream_ids))

    def events(self) -> tuple[CacheTransition, ...]:
        with self._lock:
            return tuple(self._events)

    def cursor(self) -> int:
        with self._lock:
            return len(self._events)

    def reset(self, *, run_id: str | None = None) -> None:
        if run_id is not None and (not isinstance(run_id, str) or not run_id):
            raise ValueError("run_id must be a non-empty string")
        with self._lock:
            if run_id is not None:
                self.run_id = run_id
            self._events.clear()


def aggregate_cache_transition_counters(events: tuple) -> CacheTransitionCounters:
    if not isinstance(events, tuple):
        raise TypeError("events must be an immutable tuple")
    count = {k: 0 for k in RuntimeEventKind}
    for event in events:
        count[event.kind] += 1
    return CacheTransitionCounters(h2d_submissions=count[RuntimeEventKind.H2D_SUBMIT],
                                   resident_hits=count[RuntimeEventKind.RESIDENT_HIT],
                                   inflight_joins=count[RuntimeEventKind.INFLIGHT_JOIN],
                                   evictions=count[RuntimeEventKind.EVICT])

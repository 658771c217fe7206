"""Cache transition observer protocol, transition record and recorder.

Interface of src/specfit/runtime/cache_observer.py:14-198: the observer
``record`` keyword protocol, the frozen ``CacheTransition`` record (fields,
error types and messages as rule rows, ``_checks.Rule``), the counters
record, the thread-safe in-memory recorder and the counter aggregation.
"""
from __future__ import annotations

from collections import Counter
from dataclasses import dataclass
from threading import Lock
from time import perf_counter_ns
from typing import Hashable, Protocol

import torch

from ._checks import Rule, enforce
from .trace import RuntimeEventKind


class CacheTransitionObserver(Protocol):
    def record(self, *, kind: RuntimeEventKind, cache_id: str, queue_id: str,
               expert_id: Hashable, slot_id: int, generation: int,
               submission_sequence: int | None = None,
               victim_expert_id: Hashable | None = None,
               ready_event: torch.cuda.Event | None = None,
               stream_ids: tuple[int, ...] = ()) -> None: ...


def _natural(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool) and value >= 0


def _natural_field(name: str) -> Rule:
    return Rule(lambda t: _natural(getattr(t, name)), ValueError,
                f"{name} must be a non-negative integer")


_TRANSITION_RULES = (
    Rule(lambda t: bool(t.run_id) and bool(t.cache_id) and bool(t.queue_id), ValueError,
         "run_id, cache_id and queue_id must be non-empty"),
    *(_natural_field(n) for n in ("sequence", "host_time_ns", "slot_id", "generation")),
)
# Checked after ``kind`` is coerced to RuntimeEventKind.
_KIND_RULES = (
    Rule(lambda t: t.submission_sequence is None or _natural(t.submission_sequence),
         ValueError, "submission_sequence must be non-negative"),
    Rule(lambda t: isinstance(t.stream_ids, tuple), TypeError,
         "stream_ids must be an immutable tuple"),
    Rule(lambda t: all(_natural(s) for s in t.stream_ids)
         and len(set(t.stream_ids)) == len(t.stream_ids),
         ValueError, "stream_ids must contain unique non-negative integers"),
    Rule(lambda t: t.kind is not RuntimeEventKind.H2D_SUBMIT
         or (t.submission_sequence is not None and t.ready_event is not None),
         ValueError, "H2D submit requires a sequence and ready event"),
    Rule(lambda t: t.kind is not RuntimeEventKind.EVICT or t.victim_expert_id is not None,
         ValueError, "eviction requires a victim expert"),
)


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
        enforce(self, _TRANSITION_RULES)
        object.__setattr__(self, "kind", RuntimeEventKind(self.kind))
        enforce(self, _KIND_RULES)


@dataclass(frozen=True, slots=True)
class CacheTransitionCounters:
    h2d_submissions: int = 0
    resident_hits: int = 0
    inflight_joins: int = 0
    evictions: int = 0


def _valid_run_id(run_id) -> str:
    if not isinstance(run_id, str) or not run_id:
        raise ValueError("run_id must be a non-empty string")
    return run_id


class RecordingCacheTransitionObserver:
    """Thread-safe in-memory log of transitions; an event's ``sequence`` is
    its position in the log since the last ``reset``."""

    def __init__(self, *, run_id: str) -> None:
        self.run_id = _valid_run_id(run_id)
        self._log: list[CacheTransition] = []
        self._guard = Lock()

    def record(self, *, kind, cache_id, queue_id, expert_id, slot_id, generation,
               submission_sequence=None, victim_expert_id=None, ready_event=None,
               stream_ids=()) -> None:
        fields = dict(kind=kind, cache_id=cache_id, queue_id=queue_id, expert_id=expert_id,
                      slot_id=slot_id, generation=generation,
                      submission_sequence=submission_sequence,
                      victim_expert_id=victim_expert_id, ready_event=ready_event,
                      stream_ids=stream_ids)
        with self._guard:
            log = self._log
            log.append(CacheTransition(run_id=self.run_id, sequence=len(log),
                                       host_time_ns=perf_counter_ns(), **fields))

    def events(self) -> tuple[CacheTransition, ...]:
        with self._guard:
            return tuple(self._log)

    def cursor(self) -> int:
        """Sequence number the next recorded event will get."""
        with self._guard:
            return len(self._log)

    def reset(self, *, run_id: str | None = None) -> None:
        if run_id is not None:
            _valid_run_id(run_id)
        with self._guard:
            if run_id is not None:
                self.run_id = run_id
            self._log = []


_COUNTER_OF_KIND = {
    RuntimeEventKind.H2D_SUBMIT: "h2d_submissions",
    RuntimeEventKind.RESIDENT_HIT: "resident_hits",
    RuntimeEventKind.INFLIGHT_JOIN: "inflight_joins",
    RuntimeEventKind.EVICT: "evictions",
}


def aggregate_cache_transition_counters(events: tuple) -> CacheTransitionCounters:
    if not isinstance(events, tuple):
        raise TypeError("events must be an immutable tuple")
    tally = Counter(_COUNTER_OF_KIND.get(e.kind) for e in events)
    return CacheTransitionCounters(**{name: tally[name] for name in _COUNTER_OF_KIND.values()})

"""Expert leases and cache counters.

Interface of src/specfit/runtime/lease.py:13-105: ``NoEvictableSlotError``,
the frozen ``ExpertCacheStats`` record and ``ExpertLease`` (context manager,
``wait(stream=None) -> Tensor``, idempotent ``release()``, ``slot_id``,
``ready_event``).

A lease is a handle on one *generation* of one cache slot.  Its life is a
three-state machine:

    OPEN --wait()--> OPEN (stream recorded as a reader)
    OPEN --release()--> CLOSED                 (guards recorded, pin dropped)
    OPEN --_release_keep_pinned()--> PINNED --_unpin()--> CLOSED

PINNED exists for the batched layer forward: the release bookkeeping (LRU
touch, observer event) happens at the reference's point in the lease
sequence, while the pin that keeps the slot from being chosen as a victim
stays until the kernel that reads the slot has been enqueued; ``_unpin``
then records that kernel's stream as the slot's use guard.  All policy
state (pins, touches, guards, observer events) lives in the cache; the
lease only carries its identity, its readers and its state.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING, Hashable

import torch

if TYPE_CHECKING:
    from .gpu_expert_cache import GpuExpertCache


class NoEvictableSlotError(RuntimeError):
    """Every slot of the cache holds an active lease."""


@dataclass(frozen=True, slots=True)
class ExpertCacheStats:
    h2d_submissions: int
    resident_hits: int
    inflight_joins: int
    evictions: int
    pending_use_guards: int


_OPEN, _PINNED, _CLOSED = 0, 1, 2


class ExpertLease:
    """One leased slot generation (see the module docstring)."""

    __slots__ = ("_cache", "_key", "_generation", "_state", "_readers", "_touch_pending",
                 "_ready_known", "_ready_stream", "_ready_seq", "ready_event", "slot_id")

    def __init__(self, cache: "GpuExpertCache", key: Hashable, slot_id: int, generation: int,
                 ready_event: torch.cuda.Event, *, touch_pending: bool = False,
                 ready_known: bool = False) -> None:
        self._cache = cache
        self._key = key
        self._generation = generation
        self._state = _OPEN
        # Streams that consumed the weights: {raw stream handle: Stream}.
        self._readers: dict[int, torch.cuda.Stream] = {}
        # A prefetch lease defers its LRU touch to its first wait.
        self._touch_pending = touch_pending
        # True when the ready event is known complete (a resident hit): the
        # wait then queues no stream dependency.
        self._ready_known = ready_known
        # Stream and cache submission sequence of the transfer that records
        # ready_event (set by the cache; None when unknown).
        self._ready_stream = None
        self._ready_seq = -1
        self.slot_id = slot_id
        self.ready_event = ready_event

    @property
    def expert_id(self) -> Hashable:
        return self._key

    @property
    def generation(self) -> int:
        return self._generation

    @property
    def released(self) -> bool:
        return self._state != _OPEN

    def wait(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """Make ``stream`` (default: the current stream) wait for the slot's
        H2D transfer and return the slot's packed weights."""
        if self._state != _OPEN:
            raise RuntimeError("cannot wait on a released expert lease")
        cache = self._cache
        if stream is None:
            stream = torch.cuda.current_stream(cache.device)
        if not self._ready_known:
            stream.wait_event(self.ready_event)
        self._readers[int(stream.cuda_stream)] = stream
        return cache._consume(self, stream)

    def _wait_pending(self, stream: torch.cuda.Stream, pending: dict) -> torch.Tensor:
        """``wait`` for a batched launch: instead of queueing the stream wait
        now, keep in ``pending`` (transfer stream -> (sequence, event)) the
        latest transfer event per copy stream; the launch that reads the
        batch waits on those only (transfers on one stream complete in
        order).  Everything else -- readers, touch, observer -- as ``wait``."""
        if self._state != _OPEN:
            raise RuntimeError("cannot wait on a released expert lease")
        if not self._ready_known:
            key = self._ready_stream
            if key is None:
                stream.wait_event(self.ready_event)
            else:
                held = pending.get(key)
                if held is None or held[0] < self._ready_seq:
                    pending[key] = (self._ready_seq, self.ready_event)
        self._readers[int(stream.cuda_stream)] = stream
        return self._cache._consume(self, stream)

    def release(self) -> None:
        """Record use guards on the consuming streams and drop the pin.
        Idempotent."""
        if self._state == _OPEN:
            self._cache._finish(self, keep_pin=False)
            self._state = _CLOSED

    def _release_keep_pinned(self) -> None:
        """Release bookkeeping now; the pin (and the guard) when ``_unpin``."""
        if self._state == _OPEN:
            self._cache._finish(self, keep_pin=True)
            self._state = _PINNED

    def _unpin(self) -> None:
        if self._state == _PINNED:
            self._cache._unpin_many((self,))

    # The pin protocol shared with the cache's run pins: the slots this pin
    # holds, as (slot id, key, generation) triples.
    def _pinned_slots(self):
        return ((self.slot_id, self._key, self._generation),)

    def __enter__(self) -> "ExpertLease":
        if self._state != _OPEN:
            raise RuntimeError("cannot re-enter a released expert lease")
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        self.release()

"""Expert leases and cache counters (src/specfit/runtime/lease.py:13-105).

A lease pins one *generation* of one cache slot: while any lease is active
the slot is never chosen as an eviction victim.  ``wait(stream)`` orders the
stream after the slot's H2D ready event and returns the packed weights;
``release()`` records a use event on every stream that consumed the weights,
so a later overwrite of the slot waits for those readers.
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


class ExpertLease:
    """Context manager over one leased slot generation."""

    __slots__ = ("_cache", "_expert_id", "_generation", "_released", "_streams",
                 "_touch_on_wait", "_ready_known", "_unpin_pending", "ready_event", "slot_id")

    def __init__(self, cache: "GpuExpertCache", expert_id: Hashable, slot_id: int,
                 generation: int, ready_event: torch.cuda.Event, *,
                 _defer_touch: bool = False) -> None:
        self._cache = cache
        self._expert_id = expert_id
        self._generation = generation
        self._released = False
        self._streams: dict[int, torch.cuda.Stream] = {}
        self._touch_on_wait = _defer_touch
        # Set only when the ready event is already known to be complete; the
        # lease still protects this generation.
        self._ready_known = False
        self._unpin_pending = False
        self.slot_id = slot_id
        self.ready_event = ready_event

    @property
    def expert_id(self) -> Hashable:
        return self._expert_id

    @property
    def generation(self) -> int:
        return self._generation

    @property
    def released(self) -> bool:
        return self._released

    def wait(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """Order ``stream`` (default: current) after the slot's H2D and return
        the slot's packed weights."""
        if self._released:
            raise RuntimeError("cannot wait on a released expert lease")
        if stream is None:
            stream = torch.cuda.current_stream(self._cache.device)
        if not self._ready_known:
            stream.wait_event(self.ready_event)
        self._streams[int(stream.cuda_stream)] = stream
        weights = self._cache._lease_tensor(self._expert_id, self.slot_id, self._generation,
                                            touch=self._touch_on_wait)
        self._touch_on_wait = False
        if self._cache._observer is not None:
            self._cache._record_consume_wait(expert_id=self._expert_id, slot_id=self.slot_id,
                                             generation=self._generation,
                                             ready_event=self.ready_event, stream=stream)
        return weights

    def release(self) -> None:
        """Idempotent: record use guards on the consuming streams and unpin."""
        if self._released:
            return
        self._cache._release(self._expert_id, self.slot_id, self._generation,
                             tuple(self._streams.values()))
        self._released = True

    def _release_keep_pinned(self) -> None:
        """Do the release bookkeeping now (LRU touch, observer event) but keep
        the slot pinned until ``_unpin`` -- used when the kernel that reads the
        weights is enqueued after this point in host order."""
        if self._released:
            return
        self._cache._release(self._expert_id, self.slot_id, self._generation,
                             tuple(self._streams.values()), keep_pinned=True)
        self._released = True
        self._unpin_pending = True

    def _unpin(self) -> None:
        """Record the use guards and drop the pin taken by _release_keep_pinned."""
        if not self._unpin_pending:
            return
        self._unpin_pending = False
        self._cache._unpin(self._expert_id, self.slot_id, self._generation,
                           tuple(self._streams.values()))

    def __enter__(self) -> "ExpertLease":
        if self._released:
            raise RuntimeError("cannot re-enter a released expert lease")
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        self.release()

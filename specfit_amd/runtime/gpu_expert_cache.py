"""Per-layer GPU expert cache: fixed HBM slots in front of pinned host experts.

Drop-in for src/specfit/runtime/gpu_expert_cache.py:75-745 (same
constructor, public methods, the private methods other modules call, error
types and messages).  Policy, all on the host:

* lookup order: in-flight transfer (join it) -> resident slot (hit) -> miss;
* a miss evicts the unleased slot with the smallest
  (occupied, last_used_sequence, slot_id) -- empty slots first, then LRU
  (gpu_expert_cache.py:495-518);
* every assignment bumps the slot generation; a lease pins one generation;
* the H2D copy of a miss runs on the cache's copy stream after the victim's
  use guards (events recorded by the streams that read the old weights), and
  records a ready event that consumers wait on (lease.wait);
* completed transfers are reaped in submission order and only then become
  "resident".

HBM layout: one contiguous ``[slot_count, expert_numel]`` bf16 tensor, so a
slot is a 9 MiB-aligned row that the grouped SwiGLU kernel reads directly.
The copy itself is ``sf_copy_h2d`` (hipMemcpyAsync from page-locked memory,
an SDMA transfer that leaves the compute units to the expert GEMMs).
"""
from __future__ import annotations

import itertools
from collections import deque
from dataclasses import dataclass, field, replace
from threading import RLock
from time import perf_counter_ns
from typing import Hashable, Mapping, Protocol, Sequence

import torch

from .. import ops
from .cache_observer import CacheTransitionObserver
from .cache_snapshot import CacheSlotSnapshot, GpuExpertCacheSnapshot, PendingTransferSnapshot
from .lease import ExpertCacheStats, ExpertLease, NoEvictableSlotError
from .trace import RuntimeEventKind


@dataclass(slots=True)
class _Counters:
    h2d_submissions: int = 0
    resident_hits: int = 0
    inflight_joins: int = 0
    evictions: int = 0


@dataclass(slots=True)
class _Slot:
    slot_id: int
    tensor: torch.Tensor
    expert_id: Hashable | None = None
    generation: int = 0
    active_leases: int = 0
    last_used_sequence: int = 0
    ready_event: torch.cuda.Event | None = None
    use_events: dict = field(default_factory=dict)
    write_stream: torch.cuda.Stream | None = None  # stream of the last H2D into the slot

    def lru_key(self) -> tuple:
        return (self.expert_id is not None, self.last_used_sequence, self.slot_id)


@dataclass(frozen=True, slots=True)
class _Transfer:
    expert_id: Hashable
    slot_id: int
    generation: int
    submission_sequence: int
    ready_event: torch.cuda.Event


class _SourceOwner(Protocol):
    def close(self) -> None: ...


@dataclass(frozen=True)
class _ExpertCacheCheckpoint:
    owner: object
    weights: torch.Tensor
    slots: tuple
    resident: dict
    inflight: dict
    transfers: tuple
    stats: _Counters
    sequence: int
    submission_sequence: int
    state_version: int


_shared_stream_cache_ids = itertools.count()
_READER_POLL_NS = 50_000_000  # host wait for a slot's reader before an H2D (see _await_reader)


class _PinRun:
    """What is left of the leases of a run of resident experts after their
    release bookkeeping (``_resident_run_unobserved``): each slot stays
    pinned (``active_leases``) until the kernels that read it are enqueued;
    the cache's ``_unpin_many`` (or ``_unpin``) then records the use guards
    and drops the pins of the whole run."""

    __slots__ = ("_cache", "keys", "slot_ids", "generations", "_streams", "_unpin_pending")

    def __init__(self, cache: "GpuExpertCache", keys: Sequence[Hashable], slot_ids: list[int],
                 generations: list[int], streams: dict) -> None:
        self._cache = cache
        self.keys = keys
        self.slot_ids = slot_ids
        self.generations = generations
        self._streams = streams
        self._unpin_pending = True

    def _unpin(self) -> None:
        if not self._unpin_pending:
            return
        self._unpin_pending = False
        self._cache._unpin_run(self, tuple(self._streams.values()))


class GpuExpertCache:
    """LRU cache of packed expert weights in HBM slots (one per layer)."""

    def __init__(self, cpu_sources: Mapping[Hashable, torch.Tensor], *, slot_count: int,
                 device: torch.device | str, adopt_pinned_sources: bool = False,
                 cache_id: str | None = None, queue_id: str | None = None,
                 observer: CacheTransitionObserver | None = None,
                 source_owner: _SourceOwner | None = None,
                 copy_streams: tuple[torch.cuda.Stream, torch.cuda.Stream] | None = None) -> None:
        """``copy_streams``: the two SDMA streams the cache's transfers
        alternate between, instead of a pair of its own.  The layer caches
        of one model share a pair: layers copy one after another, and one
        pair keeps the transfers on the same two engine queues (per-cache
        pairs of 48 layers ran at ~89% of the link rate that one pair
        reaches)."""
        if not cpu_sources:
            raise ValueError("cpu_sources must contain at least one expert")
        if slot_count <= 0:
            raise ValueError("slot_count must be positive")
        if source_owner is not None and not adopt_pinned_sources:
            raise ValueError("source_owner requires adopt_pinned_sources=True")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("GpuExpertCache requires a CUDA device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        for name, value in (("cache_id", cache_id), ("queue_id", queue_id)):
            if value is not None and (not isinstance(value, str) or not value):
                raise ValueError(f"{name} must be a non-empty string")

        items = tuple(cpu_sources.items())
        shape, dtype = items[0][1].shape, items[0][1].dtype
        self._sources: dict[Hashable, torch.Tensor] = {}
        # Each source key maps to itself: slots, the resident and in-flight
        # maps store these objects, so lookups with them match by identity.
        self._canonical_keys: dict[Hashable, Hashable] = {}
        self._table_version = 0  # bumped on every slot assignment, reset and restore
        # (keys, table version, table) of the last _slot_table without
        # transfers in flight; callers only read the table.
        self._slot_table_cache: tuple | None = None
        self._source_order: dict[Hashable, int] = {}
        for order, (expert_id, src) in enumerate(items):
            if src.device.type != "cpu":
                raise ValueError(f"expert {expert_id!r} source must be on CPU")
            if src.shape != shape:
                raise ValueError("all expert sources must have the same shape")
            if src.dtype != dtype:
                raise ValueError("all expert sources must have the same dtype")
            if adopt_pinned_sources and src.is_pinned() and src.is_contiguous():
                pinned = src.detach()
            else:
                if source_owner is not None:
                    raise ValueError("owned expert sources must be contiguous pinned CPU tensors")
                pinned = torch.empty(shape, dtype=dtype, device="cpu", pin_memory=True)
                pinned.copy_(src.detach())
            self._sources[expert_id] = pinned
            self._source_order[expert_id] = order
            self._canonical_keys[expert_id] = expert_id

        if copy_streams is not None:
            if (len(copy_streams) != 2 or copy_streams[0] is copy_streams[1]
                    or any(not isinstance(st, torch.cuda.Stream) or st.device != self.device
                           for st in copy_streams)):
                raise ValueError("copy_streams must be two distinct streams of the cache device")
        with torch.cuda.device(self.device):
            # A second SDMA stream: consecutive transfers alternate between the
            # two so one engine's per-transfer setup overlaps the other's data
            # movement (9 MiB copies reach ~98% of the host-link peak instead
            # of ~92% on one stream).  Used only while copy_stream is the
            # cache's first stream.
            if copy_streams is None:
                self.copy_stream = torch.cuda.Stream(device=self.device)
                self._aux_copy_stream = torch.cuda.Stream(device=self.device)
            else:
                self.copy_stream, self._aux_copy_stream = copy_streams
            self._own_copy_stream = self.copy_stream
            storage = torch.empty((slot_count, *shape), dtype=dtype, device=self.device)
            # The allocation may be recycled memory whose earlier readers are
            # still queued on the current stream: order the first copy after them.
            self.copy_stream.wait_stream(torch.cuda.current_stream(self.device))
            self._aux_copy_stream.wait_stream(torch.cuda.current_stream(self.device))
        if cache_id is None and copy_streams is not None:
            cache_id = f"cuda-{self.device.index}-cache-{next(_shared_stream_cache_ids)}"
        self.cache_id = cache_id or f"cuda-{self.device.index}-stream-{int(self.copy_stream.cuda_stream)}"
        self.queue_id = queue_id or f"{self.cache_id}-copy"
        self._storage = storage
        self._slots = [_Slot(i, storage[i]) for i in range(slot_count)]
        self._resident: dict[Hashable, int] = {}
        self._inflight: dict[Hashable, _Transfer] = {}
        self._outstanding_transfers: deque[_Transfer] = deque()
        self._stats = _Counters()
        self._sequence = 0
        self._submission_sequence = 0
        self._state_version = 0
        self._observer = observer
        self._source_owner = source_owner
        self._closed = False
        self._closing = False
        self._lock = RLock()

    # ------------------------------------------------------------ queries --
    @property
    def sources_are_pinned(self) -> bool:
        return not (self._closed or self._closing) and all(
            s.is_pinned() for s in self._sources.values())

    @property
    def closed(self) -> bool:
        with self._lock:
            return self._closed

    @property
    def active_lease_count(self) -> int:
        with self._lock:
            return sum(s.active_leases for s in self._slots)

    @property
    def slot_count(self) -> int:
        return len(self._slots)

    @property
    def storage(self) -> torch.Tensor:
        """The ``[slot_count, expert_numel]`` HBM slot tensor."""
        return self._storage

    def stats(self) -> ExpertCacheStats:
        with self._lock:
            self._reap_completed_use_guards()
            return self._stats_snapshot()

    def resident_expert_ids(self) -> tuple[Hashable, ...]:
        with self._lock:
            self._reap_completed_transfers()
            return tuple(sorted(self._resident, key=self._source_order.__getitem__))

    def _resident_key_set(self) -> frozenset:
        """The resident expert ids (unordered) after reaping."""
        with self._lock:
            self._reap_completed_transfers()
            return frozenset(self._resident)

    def _slot_table(self, keys) -> tuple[int, list[int], list[torch.cuda.Event]]:
        """(table version, slot of each key that is resident or in flight
        or -1, ready events of the in-flight ones: a reader waits on them).
        The version changes whenever an expert is assigned a slot or the
        cache is reset or restored; stays exact while the caller holds the
        lock."""
        with self._lock:
            self._reap_completed_transfers()
            inflight = self._inflight
            cached = self._slot_table_cache
            if (not inflight and cached is not None and cached[0] is keys
                    and cached[1] == self._table_version):
                return cached[1], cached[2], []
            resident = self._resident
            table = []
            pending = []
            for k in keys:
                slot = resident.get(k)
                if slot is None:
                    t = inflight.get(k)
                    if t is not None:
                        slot = t.slot_id
                        pending.append(t.ready_event)
                    else:
                        slot = -1
                table.append(slot)
            if not pending:  # reused while the version stands and nothing is in flight
                self._slot_table_cache = (keys, self._table_version, table)
            return self._table_version, table, pending

    def is_available(self, expert_id: Hashable) -> bool:
        """True when an acquire of ``expert_id`` would not choose a victim
        (resident or already in flight)."""
        with self._lock:
            self._reap_completed_transfers()
            return expert_id in self._resident or expert_id in self._inflight

    def has_unleased_slot(self) -> bool:
        """True when at least one slot holds no active lease (or pin)."""
        with self._lock:
            return any(s.active_leases == 0 for s in self._slots)

    # ----------------------------------------------------------- acquire --
    def acquire(self, expert_id: Hashable) -> ExpertLease:
        return self._acquire(expert_id, defer_touch=False)

    def _prefetch(self, expert_id: Hashable) -> ExpertLease:
        return self._acquire(expert_id, defer_touch=True)

    def _check_open_and_known(self, expert_id: Hashable) -> None:
        if self._closed or self._closing:
            raise RuntimeError("expert cache is closed")
        if expert_id not in self._sources:
            raise KeyError(f"unknown expert {expert_id!r}")

    def _prefetch_nonblocking(self, expert_id: Hashable, *, resident_only: bool = False,
                              eviction_probabilities: Mapping[Hashable, float] | None = None,
                              ) -> ExpertLease | None:
        """Lease without ever queueing a wait on a busy slot: returns None when
        no writable slot exists (or when ``resident_only`` and it would miss)."""
        with self._lock:
            self._check_open_and_known(expert_id)
            self._reap_completed_transfers()
            if expert_id in self._resident or expert_id in self._inflight:
                return self._acquire(expert_id, defer_touch=True)
            if resident_only:
                return None
            if eviction_probabilities is None:
                slot = self._choose_lru_slot(ready_only=True)
            else:
                slot = self._choose_probability_slot(expert_id, eviction_probabilities)
            if slot is None:
                return None
            self._assign_and_submit(slot, expert_id)
            return self._new_lease(slot, defer_touch=True)

    def _acquire(self, expert_id: Hashable, *, defer_touch: bool) -> ExpertLease:
        with self._lock:
            self._check_open_and_known(expert_id)
            self._reap_completed_transfers()
            transfer = self._inflight.get(expert_id)
            if transfer is not None:
                slot = self._slots[transfer.slot_id]
                if self._observer is not None:
                    self._record_transition(kind=RuntimeEventKind.INFLIGHT_JOIN,
                                            expert_id=expert_id, slot=slot,
                                            submission_sequence=transfer.submission_sequence,
                                            ready_event=transfer.ready_event)
                self._stats.inflight_joins += 1
                return self._new_lease(slot, defer_touch=defer_touch)
            slot_id = self._resident.get(expert_id)
            if slot_id is not None:
                slot = self._slots[slot_id]
                if self._observer is not None:
                    self._record_transition(kind=RuntimeEventKind.RESIDENT_HIT,
                                            expert_id=expert_id, slot=slot)
                self._stats.resident_hits += 1
                lease = self._new_lease(slot, defer_touch=defer_touch)
                # Residency is published only after the ready event completed,
                # so waiting on it again would be a no-op stream wait.
                lease._ready_known = True
                return lease
            slot = self._choose_lru_slot()
            if slot is None:
                raise NoEvictableSlotError("all GPU expert slots have active leases")
            self._assign_and_submit(slot, expert_id)
            return self._new_lease(slot, defer_touch=defer_touch)

    # ---------------------------------------------------------- snapshots --
    def snapshot(self) -> GpuExpertCacheSnapshot:
        with self._lock:
            done = {t.submission_sequence: t.ready_event.query()
                    for t in self._outstanding_transfers}
            guards = {s.slot_id: sum(not ev.query() for ev in s.use_events.values())
                      for s in self._slots}
            current = {(t.slot_id, t.generation): t for t in self._inflight.values()}
            slots = []
            for s in self._slots:
                t = current.get((s.slot_id, s.generation))
                if s.expert_id is None:
                    ready = False
                elif t is not None:
                    ready = done[t.submission_sequence]
                else:
                    ready = s.expert_id in self._resident
                slots.append(CacheSlotSnapshot(
                    slot_id=s.slot_id, expert_id=s.expert_id, generation=s.generation,
                    active_leases=s.active_leases, last_used_sequence=s.last_used_sequence,
                    ready=ready, pending_use_guards=guards[s.slot_id]))
            pending = tuple(
                PendingTransferSnapshot(expert_id=t.expert_id, slot_id=t.slot_id,
                                        generation=t.generation,
                                        submission_sequence=t.submission_sequence,
                                        ready_event=t.ready_event, ready_event_completed=False)
                for t in self._outstanding_transfers if not done[t.submission_sequence])
            return GpuExpertCacheSnapshot(
                cache_id=self.cache_id, queue_id=self.queue_id, capacity=len(self._slots),
                host_state_version=self._state_version, lru_sequence=self._sequence,
                submission_sequence=self._submission_sequence, slots=tuple(slots),
                pending_transfers=pending,
                stats=self._stats_snapshot(pending_use_guards=sum(guards.values())))

    def _gpu_quiescent(self) -> bool:
        return (all(t.ready_event.query() for t in self._outstanding_transfers)
                and all(ev.query() for s in self._slots for ev in s.use_events.values()))

    def cold_reset(self) -> None:
        """Forget every assignment and counter (needs a quiescent cache)."""
        with self._lock:
            if self._closed or self._closing:
                raise RuntimeError("expert cache is closed")
            if any(s.active_leases for s in self._slots):
                raise RuntimeError("cold reset cannot run while an active lease exists")
            if not self._gpu_quiescent():
                raise RuntimeError("cold reset requires explicit CUDA synchronization")
            self._resident.clear()
            self._inflight.clear()
            self._table_version += 1
            self._outstanding_transfers.clear()
            for s in self._slots:
                s.expert_id = None
                s.generation = 0
                s.active_leases = 0
                s.last_used_sequence = 0
                s.ready_event = None
                s.write_stream = None
                s.use_events.clear()
            self._stats = _Counters()
            self._sequence = 0
            self._submission_sequence = 0
            self._state_version = 0

    def _require_checkpoint_boundary(self) -> None:
        if self._closed or self._closing:
            raise RuntimeError("expert cache is closed")
        if self._observer is not None:
            raise RuntimeError("checkpoint restoration requires no active cache observer")
        if any(s.active_leases for s in self._slots):
            raise RuntimeError("checkpoint boundary cannot contain active leases")
        if not self._gpu_quiescent():
            raise RuntimeError("checkpoint boundary requires explicit CUDA synchronization")

    def _capture_checkpoint(self) -> _ExpertCacheCheckpoint:
        """Copy slot weights to pinned host memory together with all policy
        state (gpu_expert_cache.py:391-408)."""
        with self._lock:
            self._require_checkpoint_boundary()
            weights = torch.empty_like(self._storage, device="cpu", pin_memory=True)
            weights.copy_(self._storage.detach())
            return _ExpertCacheCheckpoint(
                owner=self, weights=weights,
                slots=tuple(replace(s, tensor=weights[s.slot_id], use_events=dict(s.use_events))
                            for s in self._slots),
                resident=dict(self._resident), inflight=dict(self._inflight),
                transfers=tuple(self._outstanding_transfers), stats=replace(self._stats),
                sequence=self._sequence, submission_sequence=self._submission_sequence,
                state_version=self._state_version)

    def _restore_checkpoint(self, checkpoint: _ExpertCacheCheckpoint) -> dict:
        started = perf_counter_ns()
        with self._lock:
            self._require_checkpoint_boundary()
            if checkpoint.owner is not self:
                raise ValueError("expert checkpoint belongs to a different cache instance")
            checked = perf_counter_ns()
            self._storage.copy_(checkpoint.weights)
            copied = perf_counter_ns()
            torch.cuda.current_stream(self.device).synchronize()
            synced = perf_counter_ns()
            self._slots = [replace(s, tensor=self._storage[s.slot_id], use_events=dict(s.use_events),
                                   write_stream=None)
                           for s in checkpoint.slots]
            self._resident = dict(checkpoint.resident)
            self._table_version += 1
            self._inflight = dict(checkpoint.inflight)
            self._outstanding_transfers = deque(checkpoint.transfers)
            self._stats = replace(checkpoint.stats)
            self._sequence = checkpoint.sequence
            self._submission_sequence = checkpoint.submission_sequence
            self._state_version = checkpoint.state_version
            finished = perf_counter_ns()
            return dict(weight_bytes=checkpoint.weights.numel() * checkpoint.weights.element_size(),
                        weights_pinned=checkpoint.weights.is_pinned(),
                        total_wall_ns=finished - started,
                        timings_ns=dict(boundary_check=checked - started,
                                        weight_copy_call=copied - checked,
                                        stream_synchronize=synced - copied,
                                        metadata_restore=finished - synced))

    def close(self) -> None:
        """Synchronise the device, drop all state and the sources, then close
        the source owner (idempotent)."""
        with self._lock:
            if self._closed:
                return
            if not self._closing and any(s.active_leases for s in self._slots):
                raise RuntimeError("expert cache cannot close while an active lease exists")
            self._closing = True
            torch.cuda.synchronize(self.device)
            self._resident.clear()
            self._inflight.clear()
            self._table_version += 1
            self._outstanding_transfers.clear()
            for s in self._slots:
                s.expert_id = None
                s.ready_event = None
                s.use_events.clear()
            self._sources.clear()
            self._canonical_keys.clear()
            owner, self._source_owner = self._source_owner, None
            if owner is not None:
                owner.close()
            self._closed = True
            self._closing = False

    # ------------------------------------------------------------- policy --
    def _new_lease(self, slot: _Slot, *, defer_touch: bool) -> ExpertLease:
        if slot.expert_id is None or slot.ready_event is None:
            raise RuntimeError("cannot lease an unassigned GPU slot")
        slot.active_leases += 1
        if defer_touch:
            self._state_version += 1
        else:
            self._touch(slot)
        return ExpertLease(self, slot.expert_id, slot.slot_id, slot.generation, slot.ready_event,
                           _defer_touch=defer_touch)

    @staticmethod
    def _writable(slot: _Slot, resident_slot: int | None) -> bool:
        """The slot's last H2D is complete and no reader guard is pending."""
        copied = (slot.ready_event is None or resident_slot == slot.slot_id
                  or slot.ready_event.query())
        return copied and all(ev.query() for ev in slot.use_events.values())

    def _choose_lru_slot(self, *, ready_only: bool = False) -> _Slot | None:
        free = [s for s in self._slots if s.active_leases == 0]
        if not ready_only:
            return min(free, key=_Slot.lru_key) if free else None
        # Probe in eviction order and stop at the first writable slot.
        for slot in sorted(free, key=_Slot.lru_key):
            if self._writable(slot, self._resident.get(slot.expert_id)):
                return slot
        return None

    def _choose_probability_slot(self, expert_id: Hashable,
                                 probabilities: Mapping[Hashable, float]) -> _Slot | None:
        """Admit a speculative expert only over a writable, unleased victim of
        strictly lower probability (empty slots first, then lower probability,
        then LRU, then slot id) -- gpu_expert_cache.py:520-541."""
        incoming = probabilities.get(expert_id, 0.0)
        free = [s for s in self._slots if s.active_leases == 0]
        order = sorted(free, key=lambda s: (s.expert_id is not None,
                                            probabilities.get(s.expert_id, 0.0),
                                            s.last_used_sequence, s.slot_id))
        for slot in order:
            if slot.expert_id is not None and probabilities.get(slot.expert_id, 0.0) >= incoming:
                break
            if self._writable(slot, self._resident.get(slot.expert_id)):
                return slot
        return None

    def _assign_and_submit(self, slot: _Slot, expert_id: Hashable) -> None:
        expert_id = self._canonical_keys.get(expert_id, expert_id)
        self._table_version += 1
        victim = slot.expert_id
        if victim is not None:
            self._resident.pop(victim, None)
            self._inflight.pop(victim, None)
            self._stats.evictions += 1
        slot.generation += 1
        slot.expert_id = expert_id
        guards = tuple(slot.use_events.values())
        slot.use_events.clear()
        stream = self._transfer_stream()
        if slot.ready_event is not None and slot.write_stream is not stream:
            # Writes of one slot stay in submission order even when the
            # previous one ran on the other stream (on the same stream the
            # stream order already keeps them).
            stream.wait_event(slot.ready_event)
        for guard in guards:
            self._await_reader(stream, guard)
        ops.copy_h2d(slot.tensor, self._sources[expert_id], stream)
        ready = torch.cuda.Event(blocking=False)
        ready.record(stream)
        slot.ready_event = ready
        slot.write_stream = stream
        transfer = _Transfer(expert_id, slot.slot_id, slot.generation,
                             self._submission_sequence, ready)
        self._inflight[expert_id] = transfer
        self._outstanding_transfers.append(transfer)
        self._stats.h2d_submissions += 1
        self._submission_sequence += 1
        if self._observer is not None:
            if victim is not None:
                self._record_transition(kind=RuntimeEventKind.EVICT, expert_id=expert_id,
                                        slot=slot, victim_expert_id=victim)
            self._record_transition(kind=RuntimeEventKind.H2D_SUBMIT, expert_id=expert_id,
                                    slot=slot, submission_sequence=transfer.submission_sequence,
                                    ready_event=ready)

    @staticmethod
    def _await_reader(stream: torch.cuda.Stream, guard: torch.cuda.Event) -> None:
        """Order a slot's next H2D after a kernel that read the slot.  The
        host waits for the reader (polling, at most _READER_POLL_S) rather
        than the copy stream: a copy stream that waits on compute-stream
        events while compute kernels wait on its own ready events stalls
        between copies on MI355X (9 MiB copies fell from 57 to 32-50 GB/s in
        that pattern, and back to 57 with the waits on the host).  A reader
        still running after the poll window gets the device-side wait."""
        if guard.query():
            return
        deadline = perf_counter_ns() + _READER_POLL_NS
        while perf_counter_ns() < deadline:
            if guard.query():
                return
        stream.wait_event(guard)

    def _transfer_stream(self) -> torch.cuda.Stream:
        """Stream of the next H2D: alternate the cache's two SDMA streams by
        submission sequence; a replaced copy_stream (a scheduler's shared
        queue) takes every transfer."""
        if self.copy_stream is not self._own_copy_stream or self._submission_sequence % 2 == 0:
            return self.copy_stream
        return self._aux_copy_stream

    def _reap_completed_transfers(self) -> None:
        """Publish completed transfers as resident, strictly in submission order."""
        changed = False
        queue = self._outstanding_transfers
        while queue and queue[0].ready_event.query():
            t = queue.popleft()
            slot = self._slots[t.slot_id]
            if slot.expert_id == t.expert_id and slot.generation == t.generation:
                self._resident[t.expert_id] = t.slot_id
            if self._inflight.get(t.expert_id) == t:
                del self._inflight[t.expert_id]
            changed = True
        if changed:
            self._state_version += 1

    def _reap_completed_use_guards(self) -> None:
        changed = False
        for slot in self._slots:
            done = [sid for sid, ev in slot.use_events.items() if ev.query()]
            for sid in done:
                del slot.use_events[sid]
            changed = changed or bool(done)
        if changed:
            self._state_version += 1

    def _touch(self, slot: _Slot) -> None:
        self._sequence += 1
        self._state_version += 1
        slot.last_used_sequence = self._sequence

    def _stats_snapshot(self, *, pending_use_guards: int | None = None) -> ExpertCacheStats:
        if pending_use_guards is None:
            pending_use_guards = sum(len(s.use_events) for s in self._slots)
        c = self._stats
        return ExpertCacheStats(h2d_submissions=c.h2d_submissions, resident_hits=c.resident_hits,
                                inflight_joins=c.inflight_joins, evictions=c.evictions,
                                pending_use_guards=pending_use_guards)

    def _validate_lease(self, slot: _Slot, expert_id: Hashable, generation: int) -> None:
        if ((slot.expert_id is not expert_id and slot.expert_id != expert_id)
                or slot.generation != generation or slot.active_leases <= 0):
            raise RuntimeError("expert lease refers to a reused GPU slot")

    def _lease_tensor(self, expert_id: Hashable, slot_id: int, generation: int, *,
                      touch: bool = False) -> torch.Tensor:
        with self._lock:
            slot = self._slots[slot_id]
            self._validate_lease(slot, expert_id, generation)
            if touch:
                self._touch(slot)
            return slot.tensor

    def _record_consume_wait(self, *, expert_id, slot_id, generation, ready_event, stream) -> None:
        if self._observer is None:
            return
        self._observer.record(kind=RuntimeEventKind.CONSUME_WAIT, cache_id=self.cache_id,
                              queue_id=self.queue_id, expert_id=expert_id, slot_id=slot_id,
                              generation=generation, ready_event=ready_event,
                              stream_ids=(int(stream.cuda_stream),))

    def _release(self, expert_id: Hashable, slot_id: int, generation: int,
                 used_streams: tuple, *, keep_pinned: bool = False) -> None:
        with self._lock:
            slot = self._slots[slot_id]
            self._validate_lease(slot, expert_id, generation)
            if not keep_pinned:
                self._record_use_guards(slot, used_streams)
            if self._observer is not None:
                self._record_transition(kind=RuntimeEventKind.RELEASE, expert_id=expert_id,
                                        slot=slot,
                                        stream_ids=tuple(sorted(int(s.cuda_stream)
                                                                for s in used_streams)))
            if not keep_pinned:
                slot.active_leases -= 1
            self._touch(slot)

    def _unpin(self, expert_id: Hashable, slot_id: int, generation: int,
               used_streams: tuple) -> None:
        """Second half of a release made with keep_pinned=True: the kernels
        reading the slot are enqueued, so record their guards and unpin."""
        with self._lock:
            slot = self._slots[slot_id]
            self._validate_lease(slot, expert_id, generation)
            self._record_use_guards(slot, used_streams)
            slot.active_leases -= 1

    def _unpin_run(self, run: _PinRun, used_streams: tuple) -> None:
        """``_unpin`` of every slot of a resident run: one use event per
        stream guards the run's slots."""
        with self._lock:
            guards = []
            for stream in used_streams:
                ev = torch.cuda.Event(blocking=False)
                ev.record(stream)
                guards.append((int(stream.cuda_stream), ev))
            slots = self._slots
            for key, slot_id, generation in zip(run.keys, run.slot_ids, run.generations):
                slot = slots[slot_id]
                self._validate_lease(slot, key, generation)
                for sid, ev in guards:
                    slot.use_events[sid] = ev
                slot.active_leases -= 1

    def _resident_steps(self, keys, index: int, current, stream, limit: int):
        """Run steps ``index`` .. of the layer's one-ahead lease sequence in
        one locked pass while both the step's expert and the next one are
        resident: for each step exactly what the caller's per-expert
        sequence does (acquire the expert when no lease is carried over,
        prefetch the next expert, wait on ``stream``, release keeping the
        slot pinned), with the same LRU touches, counters, state versions
        and observer events in the same order.  At most ``limit`` steps.
        Returns ([(expert_id, lease, weights)], next index, carried lease).
        If an observer raises, the leases this call took are unwound and the
        carried-in lease stays with the caller."""
        out = []
        made = []
        sid = int(stream.cuda_stream)
        obs = self._observer
        with self._lock:
            self._check_open_and_known(keys[index])
            self._reap_completed_transfers()
            if obs is None:
                return self._resident_run_unobserved(keys, index, current, stream, sid, limit)
            resident = self._resident
            n = len(keys)
            try:
                while index + 1 < n and len(out) < limit:
                    key, nxt = keys[index], keys[index + 1]
                    slot_id, next_id = resident.get(key), resident.get(nxt)
                    if slot_id is None or next_id is None:
                        break
                    slot = self._slots[slot_id]
                    if current is None:  # acquire: immediate touch
                        if obs is not None:
                            self._record_transition(kind=RuntimeEventKind.RESIDENT_HIT,
                                                    expert_id=key, slot=slot)
                        self._stats.resident_hits += 1
                        current = self._new_lease(slot, defer_touch=False)
                        current._ready_known = True
                        made.append(current)
                    # one-ahead prefetch of the next expert: deferred touch
                    nslot = self._slots[next_id]
                    if obs is not None:
                        self._record_transition(kind=RuntimeEventKind.RESIDENT_HIT,
                                                expert_id=nxt, slot=nslot)
                    self._stats.resident_hits += 1
                    ahead = self._new_lease(nslot, defer_touch=True)
                    ahead._ready_known = True
                    made.append(ahead)
                    # wait: the ready event is complete, so no stream wait
                    current._streams[sid] = stream
                    if current._touch_on_wait:
                        self._touch(slot)
                        current._touch_on_wait = False
                    if obs is not None:
                        self._record_consume_wait(expert_id=key, slot_id=slot.slot_id,
                                                  generation=current.generation,
                                                  ready_event=current.ready_event,
                                                  stream=stream)
                    # release, keeping the slot pinned until its launch
                    if obs is not None:
                        self._record_transition(kind=RuntimeEventKind.RELEASE, expert_id=key,
                                                slot=slot, stream_ids=(sid,))
                    self._touch(slot)
                    current._released = True
                    current._unpin_pending = True
                    out.append((key.expert_id, current, slot.tensor))
                    current = ahead
                    index += 1
            except BaseException:
                done = {id(lease) for _, lease, _ in out}
                for _, lease, _ in out:
                    lease._unpin()
                for lease in made:
                    if id(lease) not in done:
                        lease.release()
                raise
        return out, index, current

    def _resident_run_unobserved(self, keys, index: int, current, stream, sid: int,
                                 limit: int):
        """``_resident_steps`` without an observer (lock held).  Step j of the
        run (keys[index + j] and the next key both resident) does, per the
        per-expert sequence: acquire (first step, when no lease is carried
        in: pin + LRU touch), one-ahead prefetch of the next key (pin, hit,
        touch deferred to its wait), the wait's deferred touch (every step
        but a first one whose carried lease has no deferred touch), release
        (LRU touch, slot stays pinned).  Every slot of the run is distinct,
        so each step's slot ends with its release touch's sequence number;
        the counters take the totals.  The released entries share one
        ``_PinRun``; only the lease carried out of the run is an
        ``ExpertLease``.  Everything that allocates runs before the first
        change to the cache."""
        resident = self._resident
        ids = [resident.get(k) for k in keys[index:index + limit + 1]]
        if None in ids:
            del ids[ids.index(None):]
        steps = len(ids) - 1
        if steps <= 0:
            return [], index, current
        slots = self._slots
        run = [slots[i] for i in ids]
        end = index + steps
        last = run[steps]
        ahead = ExpertLease(self, keys[end], last.slot_id, last.generation, last.ready_event,
                            _defer_touch=True)
        ahead._ready_known = True
        first = 0 if current is None else 1
        out = []
        if current is not None:  # the lease carried in holds keys[index]
            out.append((keys[index].expert_id, current, run[0].tensor))
        if first < steps:
            run_keys = keys[index + first:end]
            pins = _PinRun(self, run_keys, ids[first:steps],
                           [slot.generation for slot in run[first:steps]], {sid: stream})
            out.extend([(k.expert_id, pins, slot.tensor)
                        for k, slot in zip(run_keys, run[first:steps])])
        fresh = current is None
        if fresh:
            deferred = False
            run[0].active_leases += 1
        else:
            deferred = current._touch_on_wait
            current._streams[sid] = stream
            current._touch_on_wait = False
            current._released = True
            current._unpin_pending = True
        seq = self._sequence + fresh + deferred
        for j in range(steps):
            if j:
                seq += 1  # the wait's deferred touch
            seq += 1      # the release touch
            run[j].last_used_sequence = seq
            run[j + 1].active_leases += 1
        self._sequence = seq
        self._state_version += fresh + 2 * steps + (steps - 1 + deferred)
        self._stats.resident_hits += fresh + steps
        return out, end, ahead

    def _unpin_many(self, leases) -> None:
        """``_unpin`` of leases (and resident runs) whose weights one launch
        read: a single use event per stream, recorded after that launch,
        guards every slot of the batch (it completes no earlier than
        per-lease events would).  A run listed once per expert is unpinned
        once."""
        with self._lock:
            events: dict[int, torch.cuda.Event] = {}
            slots = self._slots

            def guards_of(streams: dict) -> list:
                out = []
                for sid, stream in streams.items():
                    ev = events.get(sid)
                    if ev is None:
                        ev = torch.cuda.Event(blocking=False)
                        ev.record(stream)
                        events[sid] = ev
                    out.append((sid, ev))
                return out

            for lease in leases:
                if not lease._unpin_pending:
                    continue
                lease._unpin_pending = False
                guards = guards_of(lease._streams)
                if lease.__class__ is _PinRun:
                    for key, slot_id, generation in zip(lease.keys, lease.slot_ids,
                                                        lease.generations):
                        slot = slots[slot_id]
                        if ((slot.expert_id is not key and slot.expert_id != key)
                                or slot.generation != generation or slot.active_leases <= 0):
                            raise RuntimeError("expert lease refers to a reused GPU slot")
                        for sid, ev in guards:
                            slot.use_events[sid] = ev
                        slot.active_leases -= 1
                    continue
                slot = slots[lease.slot_id]
                self._validate_lease(slot, lease.expert_id, lease.generation)
                for sid, ev in guards:
                    slot.use_events[sid] = ev
                slot.active_leases -= 1

    @staticmethod
    def _record_use_guards(slot: _Slot, used_streams: tuple) -> None:
        for stream in used_streams:
            ev = torch.cuda.Event(blocking=False)
            ev.record(stream)
            slot.use_events[int(stream.cuda_stream)] = ev

    def _record_transition(self, *, kind, expert_id, slot, submission_sequence=None,
                           victim_expert_id=None, ready_event=None, stream_ids=()) -> None:
        if self._observer is None:
            return
        self._observer.record(kind=kind, cache_id=self.cache_id, queue_id=self.queue_id,
                              expert_id=expert_id, slot_id=slot.slot_id,
                              generation=slot.generation,
                              submission_sequence=submission_sequence,
                              victim_expert_id=victim_expert_id, ready_event=ready_event,
                              stream_ids=stream_ids)

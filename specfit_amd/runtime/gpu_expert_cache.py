"""Per-layer HBM expert cache in front of pinned host experts (gfx950).

Interface of src/specfit/runtime/gpu_expert_cache.py:75-745: the same
constructor, public methods, error types and messages, and the private
members other modules use (``_prefetch``, ``_prefetch_nonblocking``,
``_slots``, ``_sources``, ``_resident``, ``_inflight``,
``_outstanding_transfers``, ``_submission_sequence``, ``_state_version``,
``_lock``, ``_require_checkpoint_boundary``, ``_capture_checkpoint``,
``_restore_checkpoint``).

Policy (the reference's, gpu_expert_cache.py:195-266, 495-609, 684-718):

* a lookup joins an in-flight transfer, else hits a resident slot, else
  misses; a miss evicts the unleased slot with the smallest
  (occupied, last_used_sequence, slot_id) -- empty slots first, then LRU;
* every assignment bumps the slot's generation and a lease pins one
  generation; acquire touches the slot at once, a prefetch at its first wait;
* a slot's next H2D is ordered after its previous transfer and after every
  stream that read it (use guards recorded at release);
* transfers become resident only when reaped, strictly in submission order.

How the state is held here:

* Device: one contiguous ``[slot_count, expert_numel]`` bf16 tensor, so a
  slot is a 9 MiB row the grouped SwiGLU kernel addresses as
  ``base + slot * stride`` (the device slot table).
* Host experts: adopted page-locked tensors, or rows of ONE page-locked
  block the cache allocates for all the experts it has to pin itself (one
  pinned allocation per layer instead of one per expert).
* Transfers: ``sf_copy_h2d`` (hipMemcpyAsync, an SDMA copy that leaves the
  compute units to the GEMMs), alternating between two SDMA streams.
* ``_resident`` is a ``_ResidentMap``: every mutation takes a process-unique
  version, so the device slot table derived from it is rebuilt exactly when
  the map changed, whoever changed it.
* Pins: an ``ExpertLease`` pins one slot; a ``_RunPin`` pins a run of
  resident slots that one batched lease sequence took.  Both expose
  ``_pinned_slots()`` and are dropped by ``_unpin_many``.
"""
from __future__ import annotations

import ctypes
import itertools
from collections import deque
from dataclasses import dataclass, field
from threading import RLock
from time import perf_counter_ns
from typing import Hashable, Mapping, Protocol, Sequence

import torch

from .. import ops
from ..codec import CompressedExperts
from . import lease as _lease_mod
from .cache_observer import CacheTransitionObserver
from .cache_snapshot import CacheSlotSnapshot, GpuExpertCacheSnapshot, PendingTransferSnapshot
from .lease import ExpertCacheStats, ExpertLease, NoEvictableSlotError
from .trace import RuntimeEventKind as _K

_PINNED = _lease_mod._PINNED
_CLOSED = _lease_mod._CLOSED

# How long the host spins on a slot's last reader before a victim's H2D is
# submitted, before it hands the wait to the copy stream instead: about one
# 9 MiB expert copy at the host-link rate.  See _await_reader.
_READER_SPIN_NS = 200_000

_versions = itertools.count(1)

# Staging buffers of a cache with coded transfers: a buffer is reused four
# transfers later, by when its decode has long run unless it waits for a
# reader of its slot.
_STAGING_BUFFERS = 4


class _ResidentMap(dict):
    """expert -> slot of completed transfers.  Each mutation (including an
    in-place ``clear`` by code outside the cache) takes a fresh
    process-unique ``version``; reads stay plain dict operations."""

    __slots__ = ("version",)

    def __init__(self, *args) -> None:
        super().__init__(*args)
        self.version = next(_versions)

    def __setitem__(self, key, value) -> None:
        dict.__setitem__(self, key, value)
        self.version = next(_versions)

    def __delitem__(self, key) -> None:
        dict.__delitem__(self, key)
        self.version = next(_versions)

    def __ior__(self, other):
        dict.update(self, other)
        self.version = next(_versions)
        return self

    def pop(self, *args):
        value = dict.pop(self, *args)
        self.version = next(_versions)
        return value

    def popitem(self):
        item = dict.popitem(self)
        self.version = next(_versions)
        return item

    def setdefault(self, key, default=None):
        value = dict.setdefault(self, key, default)
        self.version = next(_versions)
        return value

    def update(self, *args, **kwargs) -> None:
        dict.update(self, *args, **kwargs)
        self.version = next(_versions)

    def clear(self) -> None:
        dict.clear(self)
        self.version = next(_versions)


@dataclass(slots=True)
class _Counters:
    h2d_submissions: int = 0
    resident_hits: int = 0
    inflight_joins: int = 0
    evictions: int = 0

    def copy(self) -> "_Counters":
        return _Counters(self.h2d_submissions, self.resident_hits, self.inflight_joins,
                         self.evictions)


@dataclass(slots=True, eq=False)
class _Slot:
    slot_id: int
    tensor: torch.Tensor
    expert_id: Hashable | None = None
    generation: int = 0
    active_leases: int = 0
    last_used_sequence: int = 0
    ready_event: torch.cuda.Event | None = None
    # raw handle of a stream that read the slot -> event after its last read
    use_events: dict = field(default_factory=dict)
    write_stream: torch.cuda.Stream | None = None  # stream of the last H2D into the slot
    ready_seq: int = -1  # submission sequence of that H2D (the one ready_event marks)

    def victim_rank(self) -> tuple:
        return (self.expert_id is not None, self.last_used_sequence, self.slot_id)


@dataclass(frozen=True, slots=True)
class _Transfer:
    expert_id: Hashable
    slot_id: int
    generation: int
    submission_sequence: int
    ready_event: torch.cuda.Event
    stream: int | None = None  # raw handle of the copy stream (None: unknown)


class _SourceOwner(Protocol):
    def close(self) -> None: ...


@dataclass(frozen=True)
class _PolicyImage:
    """Every piece of host policy state, detached from the live cache."""

    slots: tuple          # per slot: (expert_id, generation, last_used_sequence,
                          #            ready_event, use_events, active_leases)
    resident: dict
    inflight: dict
    transfers: tuple
    counters: _Counters
    sequence: int
    submission_sequence: int
    state_version: int


@dataclass(frozen=True)
class _ExpertCacheCheckpoint:
    owner: object
    weights: torch.Tensor  # pinned host image of the slot storage
    policy: _PolicyImage


class _RunPin:
    """Pins of a run of resident slots taken by one batched lease sequence
    (``_resident_run``): every slot stays pinned until the kernel reading
    the run is enqueued; ``_unpin_many`` then guards and unpins them all."""

    __slots__ = ("_cache", "_entries", "_readers", "_state")

    def __init__(self, cache: "GpuExpertCache", entries: tuple, readers: dict) -> None:
        self._cache = cache
        self._entries = entries  # [(slot id, key, generation), ...]
        self._readers = readers
        self._state = _PINNED

    def _pinned_slots(self):
        return self._entries

    def _unpin(self) -> None:
        if self._state == _PINNED:
            self._cache._unpin_many((self,))


def _stage_sources(cpu_sources: Mapping, adopt: bool, owned: bool,
                   coded: frozenset = frozenset()) -> tuple[dict, dict]:
    """(key -> page-locked tensor, key -> source order).  Adopted sources
    are used as they are; the others are copied into the rows of one
    page-locked block allocated here.  Experts in ``coded`` always move as
    coded records from their own page-locked blob, so their sources stay
    as they are, page-locked or not."""
    items = tuple(cpu_sources.items())
    shape, dtype = items[0][1].shape, items[0][1].dtype
    to_pin = []
    for key, src in items:
        if src.device.type != "cpu":
            raise ValueError(f"expert {key!r} source must be on CPU")
        if src.shape != shape:
            raise ValueError("all expert sources must have the same shape")
        if src.dtype != dtype:
            raise ValueError("all expert sources must have the same dtype")
        if not (adopt and src.is_pinned() and src.is_contiguous()) and key not in coded:
            if owned:
                raise ValueError("owned expert sources must be contiguous pinned CPU tensors")
            to_pin.append(key)
    pinned = {key: src.detach() for key, src in items}
    if to_pin:
        block = torch.empty((len(to_pin), *shape), dtype=dtype, pin_memory=True)
        for row, key in zip(block, to_pin):
            row.copy_(pinned[key])
            pinned[key] = row
    return pinned, {key: i for i, (key, _) in enumerate(items)}


_shared_stream_cache_ids = itertools.count()


class GpuExpertCache:
    """LRU cache of packed expert weights in HBM slots (one per layer)."""

    def __init__(self, cpu_sources: Mapping[Hashable, torch.Tensor], *, slot_count: int,
                 device: torch.device | str, adopt_pinned_sources: bool = False,
                 cache_id: str | None = None, queue_id: str | None = None,
                 observer: CacheTransitionObserver | None = None,
                 source_owner: _SourceOwner | None = None,
                 copy_streams: tuple[torch.cuda.Stream, torch.cuda.Stream] | None = None,
                 compressed_sources: CompressedExperts | None = None) -> None:
        """``copy_streams``: two SDMA streams the cache's transfers alternate
        between, instead of a pair of its own.  The layer caches of one
        model share a pair (layers copy one after another; per-cache pairs
        of 48 layers ran at ~89% of the link rate one shared pair reaches).
        ``compressed_sources``: exponent-coded records of (some of) the
        experts (specfit_amd.codec); their transfers copy the record into a
        device staging buffer and decode it into the slot on the same copy
        stream, and the slot then holds the same bytes as a raw copy of the
        source."""
        if not cpu_sources:
            raise ValueError("cpu_sources must contain at least one expert")
        if slot_count <= 0:
            raise ValueError("slot_count must be positive")
        if source_owner is not None and not adopt_pinned_sources:
            raise ValueError("source_owner requires adopt_pinned_sources=True")
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError("GpuExpertCache requires a CUDA device")
        self.device = dev if dev.index is not None else torch.device(
            "cuda", torch.cuda.current_device())
        for name, value in (("cache_id", cache_id), ("queue_id", queue_id)):
            if value is not None and not (isinstance(value, str) and value):
                raise ValueError(f"{name} must be a non-empty string")
        if copy_streams is not None and (
                len(copy_streams) != 2 or copy_streams[0] is copy_streams[1]
                or any(not isinstance(s, torch.cuda.Stream) or s.device != self.device
                       for s in copy_streams)):
            raise ValueError("copy_streams must be two distinct streams of the cache device")

        coded = frozenset()
        if compressed_sources is not None:
            if not isinstance(compressed_sources, CompressedExperts):
                raise ValueError("compressed_sources must be a CompressedExperts image")
            if compressed_sources.numel != next(iter(cpu_sources.values())).numel():
                raise ValueError("compressed_sources do not match the experts' size")
            if any(key not in cpu_sources for key in compressed_sources.records):
                raise ValueError("compressed_sources hold an expert the cache does not know")
            if compressed_sources.staging_bytes() and not compressed_sources.blob.is_pinned():
                raise ValueError("compressed_sources must be in page-locked memory")
            coded = frozenset(k for k, r in compressed_sources.records.items() if not r.raw)
        self._sources, self._source_order = _stage_sources(
            cpu_sources, adopt_pinned_sources, source_owner is not None, coded)
        # Each source key maps to itself: slots and maps hold these objects,
        # so lookups with them match by identity.
        self._key_objects = {key: key for key in self._sources}
        first = next(iter(self._sources.values()))
        shared = copy_streams is not None
        with torch.cuda.device(self.device):
            if not shared:
                copy_streams = (torch.cuda.Stream(device=self.device),
                                torch.cuda.Stream(device=self.device))
            self.copy_stream, self._aux_copy_stream = copy_streams
            self._own_copy_stream = self.copy_stream
            self._storage = torch.empty((slot_count, *first.shape), dtype=first.dtype,
                                        device=self.device)
            # A ring of staging buffers for coded transfers (by submission
            # sequence).
            staging = compressed_sources.staging_bytes() if compressed_sources else 0
            self._staging = [torch.empty(staging, dtype=torch.uint8, device=self.device)
                             for _ in range(_STAGING_BUFFERS if staging else 0)]
            # The allocation may be recycled memory that kernels queued on the
            # current stream still read: order the first copies after them.
            here = torch.cuda.current_stream(self.device)
            for s in copy_streams:
                s.wait_stream(here)
        if cache_id is None:
            # Caches sharing a stream pair are told apart by a counter.
            cache_id = (f"cuda-{self.device.index}-cache-{next(_shared_stream_cache_ids)}" if shared
                        else f"cuda-{self.device.index}-stream-{int(self.copy_stream.cuda_stream)}")
        self.cache_id = cache_id
        self.queue_id = queue_id or f"{cache_id}-copy"
        self._slots = [_Slot(i, self._storage[i]) for i in range(slot_count)]
        self._resident: dict = _ResidentMap()
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
        # (keys, resident-map version, table) of the last _slot_table.
        self._table_memo: tuple | None = None
        self._codec = compressed_sources
        # the (event, stream) after the decode that last read each staging buffer
        self._staging_reader: list = [None] * len(self._staging)
        # Per coded expert: (record pointer, bytes, list counts, ctypes
        # exponent table), checked here once instead of per transfer.
        self._coded_args: dict = {}
        if compressed_sources is not None:
            blob = compressed_sources.blob.data_ptr()
            for key, r in compressed_sources.records.items():
                if not r.raw:
                    self._coded_args[key] = (blob + r.offset, r.nbytes, tuple(r.counts),
                                             (ctypes.c_uint8 * 32).from_buffer_copy(r.table))
        self._staging_ptrs = [b.data_ptr() for b in self._staging]
        self.h2d_bytes = 0  # bytes moved over the host link

    # ------------------------------------------------------------- queries --
    @property
    def sources_are_pinned(self) -> bool:
        """Every host buffer a transfer copies from is page-locked (raw
        sources, and the record blob of coded experts)."""
        if self._closed or self._closing:
            return False
        codec = self._codec
        records = codec.records if codec is not None else {}
        return all(s.is_pinned() for k, s in self._sources.items()
                   if k not in records or records[k].raw)

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
            return self._counters_record()

    def resident_expert_ids(self) -> tuple[Hashable, ...]:
        with self._lock:
            self._reap_completed_transfers()
            order = self._source_order
            return tuple(sorted(self._resident, key=order.__getitem__))

    def _resident_key_set(self) -> frozenset:
        with self._lock:
            self._reap_completed_transfers()
            return frozenset(self._resident)

    def _slot_table(self, keys: Sequence[Hashable]) -> tuple[int | None, list[int]]:
        """(version, slot of each key whose transfer has completed, else -1).

        Experts still in flight get -1: a kernel launched over the table
        reads only completed slots, and those stay in place until their
        readers are guarded (resident experts are leased, in resident-first
        order, before any miss chooses a victim).  The version is the
        resident map's: equal versions mean equal tables."""
        with self._lock:
            self._reap_completed_transfers()
            resident = self._resident
            version = getattr(resident, "version", None)
            memo = self._table_memo
            if memo is not None and memo[0] is keys and version is not None and memo[1] == version:
                return version, memo[2]
            get = resident.get
            table = [get(k, -1) for k in keys]
            self._table_memo = (keys, version, table)
            return version, table

    def is_available(self, expert_id: Hashable) -> bool:
        """True when acquiring ``expert_id`` would choose no victim."""
        with self._lock:
            self._reap_completed_transfers()
            return expert_id in self._resident or expert_id in self._inflight

    def has_unleased_slot(self) -> bool:
        with self._lock:
            return any(s.active_leases == 0 for s in self._slots)

    # ------------------------------------------------------------- leasing --
    def acquire(self, expert_id: Hashable) -> ExpertLease:
        return self._acquire(expert_id, defer_touch=False)

    def _prefetch(self, expert_id: Hashable) -> ExpertLease:
        return self._acquire(expert_id, defer_touch=True)

    def _check_open_and_known(self, expert_id: Hashable) -> None:
        if self._closed or self._closing:
            raise RuntimeError("expert cache is closed")
        if expert_id not in self._sources:
            raise KeyError(f"unknown expert {expert_id!r}")

    def _join_or_hit(self, expert_id: Hashable, touch_now: bool) -> ExpertLease | None:
        """The lease of an expert that is in flight (join) or resident
        (hit), counted and observed; None for a miss.  Lock held, reaped."""
        transfer = self._inflight.get(expert_id)
        if transfer is not None:
            slot = self._slots[transfer.slot_id]
            if self._observer is not None:
                self._record_transition(_K.INFLIGHT_JOIN, expert_id, slot,
                                        submission_sequence=transfer.submission_sequence,
                                        ready_event=transfer.ready_event)
            self._stats.inflight_joins += 1
            return self._lease(slot, touch_now=touch_now, ready_known=False)
        slot_id = self._resident.get(expert_id)
        if slot_id is None:
            return None
        slot = self._slots[slot_id]
        if self._observer is not None:
            self._record_transition(_K.RESIDENT_HIT, expert_id, slot)
        self._stats.resident_hits += 1
        # Residency is published only after the transfer completed.
        return self._lease(slot, touch_now=touch_now, ready_known=True)

    def _acquire(self, expert_id: Hashable, *, defer_touch: bool) -> ExpertLease:
        with self._lock:
            self._check_open_and_known(expert_id)
            self._reap_completed_transfers()
            lease = self._join_or_hit(expert_id, not defer_touch)
            if lease is not None:
                return lease
            victim = self._choose_lru_slot()
            if victim is None:
                raise NoEvictableSlotError("all GPU expert slots have active leases")
            self._assign_and_submit(victim, expert_id)
            return self._lease(victim, touch_now=not defer_touch, ready_known=False)

    def _prefetch_nonblocking(self, expert_id: Hashable, *, resident_only: bool = False,
                              eviction_probabilities: Mapping[Hashable, float] | None = None,
                              ) -> ExpertLease | None:
        """A prefetch lease that never queues a wait on a busy slot: None
        when only a slot whose transfer or readers are pending could take
        the expert (or, with ``resident_only``, when it would miss)."""
        with self._lock:
            self._check_open_and_known(expert_id)
            self._reap_completed_transfers()
            lease = self._join_or_hit(expert_id, False)
            if lease is not None or resident_only:
                return lease
            if eviction_probabilities is None:
                victim = self._choose_lru_slot(ready_only=True)
            else:
                victim = self._choose_probability_slot(expert_id, eviction_probabilities)
            if victim is None:
                return None
            self._assign_and_submit(victim, expert_id)
            return self._lease(victim, touch_now=False, ready_known=False)

    def _lease(self, slot: _Slot, *, touch_now: bool, ready_known: bool) -> ExpertLease:
        if slot.expert_id is None or slot.ready_event is None:
            raise RuntimeError("cannot lease an unassigned GPU slot")
        slot.active_leases += 1
        if touch_now:
            self._touch(slot)
        else:
            self._state_version += 1
        lease = ExpertLease(self, slot.expert_id, slot.slot_id, slot.generation, slot.ready_event,
                            touch_pending=not touch_now, ready_known=ready_known)
        lease._ready_stream = slot.write_stream
        lease._ready_seq = slot.ready_seq
        return lease

    @staticmethod
    def _check_pin(slot: _Slot, key: Hashable, generation: int) -> None:
        if ((slot.expert_id is not key and slot.expert_id != key)
                or slot.generation != generation or slot.active_leases <= 0):
            raise RuntimeError("expert lease refers to a reused GPU slot")

    def _consume(self, lease: ExpertLease, stream: torch.cuda.Stream) -> torch.Tensor:
        """Lease wait: the deferred touch, the observer event, the weights."""
        with self._lock:
            slot = self._slots[lease.slot_id]
            self._check_pin(slot, lease._key, lease._generation)
            if lease._touch_pending:
                lease._touch_pending = False
                self._touch(slot)
            if self._observer is not None:
                self._observer.record(kind=_K.CONSUME_WAIT, cache_id=self.cache_id,
                                      queue_id=self.queue_id, expert_id=lease._key,
                                      slot_id=slot.slot_id, generation=slot.generation,
                                      ready_event=lease.ready_event,
                                      stream_ids=(int(stream.cuda_stream),))
            return slot.tensor

    def _finish(self, lease: ExpertLease, *, keep_pin: bool) -> None:
        """Lease release: guards on the reader streams (unless the pin is
        kept for a launch still to be enqueued), observer event, unpin,
        LRU touch."""
        with self._lock:
            slot = self._slots[lease.slot_id]
            self._check_pin(slot, lease._key, lease._generation)
            readers = lease._readers
            if not keep_pin:
                for sid, stream in readers.items():
                    ev = torch.cuda.Event(blocking=False)
                    ev.record(stream)
                    slot.use_events[sid] = ev
            if self._observer is not None:
                self._record_transition(_K.RELEASE, lease._key, slot,
                                        stream_ids=tuple(sorted(readers)))
            if not keep_pin:
                slot.active_leases -= 1
            self._touch(slot)

    def _unpin_many(self, pins) -> None:
        """Drop pins (leases released with the pin kept, and run pins) whose
        slots one just-enqueued launch read: one event per reader stream,
        recorded now, guards every slot of every pin."""
        with self._lock:
            events: dict[int, torch.cuda.Event] = {}
            slots = self._slots
            for pin in pins:
                if pin._state != _PINNED:
                    continue
                pin._state = _CLOSED
                guards = []
                for sid, stream in pin._readers.items():
                    ev = events.get(sid)
                    if ev is None:
                        ev = events[sid] = torch.cuda.Event(blocking=False)
                        ev.record(stream)
                    guards.append((sid, ev))
                # One loop per slot (the body of _check_pin inlined: this
                # runs once per expert of every launch).
                for slot_id, key, generation in pin._pinned_slots():
                    slot = slots[slot_id]
                    if ((slot.expert_id is not key and slot.expert_id != key)
                            or slot.generation != generation or slot.active_leases <= 0):
                        raise RuntimeError("expert lease refers to a reused GPU slot")
                    use = slot.use_events
                    for sid, ev in guards:
                        use[sid] = ev
                    slot.active_leases -= 1

    # -------------------------------------------------- batched lease runs --
    def _resident_steps(self, keys, index: int, current, stream, limit: int):
        """Steps ``index`` .. of the one-ahead lease sequence of a layer
        (acquire when no lease is carried in, prefetch the next expert,
        wait on ``stream``, release keeping the pin), taken in one locked
        pass while the step's expert and the next one are both resident:
        the same touches, counters, state versions and observer events in
        the same order as the per-expert sequence.  At most ``limit`` steps.
        Returns ([(expert id, pin, weights)], next index, lease carried out)."""
        with self._lock:
            self._check_open_and_known(keys[index])
            self._reap_completed_transfers()
            if self._observer is None:
                return self._resident_run(keys, index, current, stream, limit)
            return self._resident_run_observed(keys, index, current, stream, limit)

    def _resident_run_observed(self, keys, index, current, stream, limit):
        """``_resident_steps`` with an observer: step by step through the
        lease methods, so every event is recorded where the per-expert
        sequence records it.  If the observer raises, the leases taken here
        are released and the carried-in lease stays with the caller."""
        resident = self._resident
        taken, out = [], []
        try:
            while index + 1 < len(keys) and len(out) < limit:
                key, nxt = keys[index], keys[index + 1]
                if key not in resident or nxt not in resident:
                    break
                if current is None:
                    current = self._join_or_hit(key, True)
                    taken.append(current)
                ahead = self._join_or_hit(nxt, False)
                taken.append(ahead)
                weights = current.wait(stream)
                current._release_keep_pinned()
                out.append((key.expert_id, current, weights))
                current = ahead
                index += 1
        except BaseException:
            for _, pin, _ in out:
                pin._unpin()
            for lease in taken:
                lease.release()
            raise
        return out, index, current

    def _resident_run(self, keys, index, current, stream, limit):
        """``_resident_steps`` without an observer, in closed form.  Step j
        of a run of n steps does: acquire (first step, no lease carried in:
        pin + touch), prefetch the next key (pin, hit, touch deferred), the
        wait's deferred touch (all steps but a first one whose carried lease
        has none), release (touch, pin kept).  All slots of a run are
        distinct, so each ends at its release touch's sequence number."""
        get = self._resident.get
        ids = []
        for k in keys[index:index + limit + 1]:
            sid = get(k)
            if sid is None:
                break
            ids.append(sid)
        steps = len(ids) - 1
        if steps <= 0:
            return [], index, current
        slots = self._slots
        run = [slots[i] for i in ids]
        end = index + steps
        last = run[-1]
        carried_out = ExpertLease(self, keys[end], last.slot_id, last.generation, last.ready_event,
                                  touch_pending=True, ready_known=True)
        handle = int(stream.cuda_stream)
        out = []
        fresh = current is None
        if fresh:
            deferred = False
            run[0].active_leases += 1
            first_pinned = 0
        else:
            deferred = current._touch_pending
            current._touch_pending = False
            current._readers[handle] = stream
            current._state = _PINNED
            out.append((keys[index].expert_id, current, run[0].tensor))
            first_pinned = 1
        entries = []
        pin = _RunPin(self, entries, {handle: stream}) if first_pinned < steps else None
        seq = self._sequence + fresh + deferred
        # One pass per step: its touches, the next slot's pin, and (past a
        # carried-in lease) the run pin's entry and the caller's step.
        for j in range(steps):
            slot = run[j]
            seq += 2 if j else 1  # (the wait's deferred touch) + the release touch
            slot.last_used_sequence = seq
            run[j + 1].active_leases += 1
            if j >= first_pinned:
                key = keys[index + j]
                entries.append((slot.slot_id, key, slot.generation))
                out.append((key.expert_id, pin, slot.tensor))
        self._sequence = seq
        self._state_version += fresh + 3 * steps - 1 + deferred
        self._stats.resident_hits += fresh + steps
        return out, end, carried_out

    # --------------------------------------------------------- snapshots --
    def snapshot(self) -> GpuExpertCacheSnapshot:
        with self._lock:
            done = {t.submission_sequence: t.ready_event.query()
                    for t in self._outstanding_transfers}
            current = {(t.slot_id, t.generation): t for t in self._inflight.values()}
            slot_rows = []
            total_guards = 0
            for s in self._slots:
                guards = sum(not ev.query() for ev in s.use_events.values())
                total_guards += guards
                t = current.get((s.slot_id, s.generation))
                if s.expert_id is None:
                    ready = False
                elif t is not None:
                    ready = done[t.submission_sequence]
                else:
                    ready = s.expert_id in self._resident
                slot_rows.append(CacheSlotSnapshot(
                    slot_id=s.slot_id, expert_id=s.expert_id, generation=s.generation,
                    active_leases=s.active_leases, last_used_sequence=s.last_used_sequence,
                    ready=ready, pending_use_guards=guards))
            pending = tuple(
                PendingTransferSnapshot(expert_id=t.expert_id, slot_id=t.slot_id,
                                        generation=t.generation,
                                        submission_sequence=t.submission_sequence,
                                        ready_event=t.ready_event, ready_event_completed=False)
                for t in self._outstanding_transfers if not done[t.submission_sequence])
            return GpuExpertCacheSnapshot(
                cache_id=self.cache_id, queue_id=self.queue_id, capacity=len(self._slots),
                host_state_version=self._state_version, lru_sequence=self._sequence,
                submission_sequence=self._submission_sequence, slots=tuple(slot_rows),
                pending_transfers=pending,
                stats=self._counters_record(pending_use_guards=total_guards))

    # -------------------------------------------- reset, checkpoint, close --
    def _quiescent(self) -> bool:
        """No transfer and no slot reader is still pending on the GPU."""
        if not all(t.ready_event.query() for t in self._outstanding_transfers):
            return False
        return all(ev.query() for s in self._slots for ev in s.use_events.values())

    def _forget_assignments(self) -> None:
        self._resident.clear()
        self._inflight.clear()
        self._outstanding_transfers.clear()
        for s in self._slots:
            s.expert_id = None
            s.ready_event = None
            s.write_stream = None
            s.ready_seq = -1
            s.use_events.clear()

    def cold_reset(self) -> None:
        """Forget every assignment and counter (needs a quiescent cache)."""
        with self._lock:
            if self._closed or self._closing:
                raise RuntimeError("expert cache is closed")
            if any(s.active_leases for s in self._slots):
                raise RuntimeError("cold reset cannot run while an active lease exists")
            if not self._quiescent():
                raise RuntimeError("cold reset requires explicit CUDA synchronization")
            self._forget_assignments()
            for s in self._slots:
                s.generation = s.active_leases = s.last_used_sequence = 0
            self._stats = _Counters()
            self._sequence = self._submission_sequence = self._state_version = 0

    def _require_checkpoint_boundary(self) -> None:
        problem = None
        if self._closed or self._closing:
            problem = "expert cache is closed"
        elif self._observer is not None:
            problem = "checkpoint restoration requires no active cache observer"
        elif any(s.active_leases for s in self._slots):
            problem = "checkpoint boundary cannot contain active leases"
        elif not self._quiescent():
            problem = "checkpoint boundary requires explicit CUDA synchronization"
        if problem is not None:
            raise RuntimeError(problem)

    def _policy_image(self) -> _PolicyImage:
        return _PolicyImage(
            slots=tuple((s.expert_id, s.generation, s.last_used_sequence, s.ready_event,
                         dict(s.use_events), s.active_leases) for s in self._slots),
            resident=dict(self._resident), inflight=dict(self._inflight),
            transfers=tuple(self._outstanding_transfers), counters=self._stats.copy(),
            sequence=self._sequence, submission_sequence=self._submission_sequence,
            state_version=self._state_version)

    def _apply_policy_image(self, image: _PolicyImage) -> None:
        for s, (expert, gen, last, ready, guards, leases) in zip(self._slots, image.slots):
            s.expert_id, s.generation, s.last_used_sequence = expert, gen, last
            s.ready_event, s.use_events, s.active_leases = ready, dict(guards), leases
            s.write_stream, s.ready_seq = None, -1
        self._resident = _ResidentMap(image.resident)
        self._inflight = dict(image.inflight)
        self._outstanding_transfers = deque(image.transfers)
        self._stats = image.counters.copy()
        self._sequence = image.sequence
        self._submission_sequence = image.submission_sequence
        self._state_version = image.state_version

    def _capture_checkpoint(self) -> _ExpertCacheCheckpoint:
        """The slot weights (copied into page-locked host memory) and the
        complete host policy state, at a quiescent boundary."""
        with self._lock:
            self._require_checkpoint_boundary()
            image = torch.empty(self._storage.shape, dtype=self._storage.dtype,
                                pin_memory=True)
            image.copy_(self._storage)
            return _ExpertCacheCheckpoint(owner=self, weights=image, policy=self._policy_image())

    def _restore_checkpoint(self, checkpoint: _ExpertCacheCheckpoint) -> dict:
        """Put a checkpoint of this cache back; returns the timing record of
        src/specfit/runtime/gpu_expert_cache.py:410-431."""
        marks = [perf_counter_ns()]
        with self._lock:
            self._require_checkpoint_boundary()
            if checkpoint.owner is not self:
                raise ValueError("expert checkpoint belongs to a different cache instance")
            marks.append(perf_counter_ns())
            self._storage.copy_(checkpoint.weights)
            marks.append(perf_counter_ns())
            torch.cuda.current_stream(self.device).synchronize()
            marks.append(perf_counter_ns())
            self._apply_policy_image(checkpoint.policy)
            marks.append(perf_counter_ns())
        w = checkpoint.weights
        phases = ("boundary_check", "weight_copy_call", "stream_synchronize", "metadata_restore")
        return dict(weight_bytes=w.numel() * w.element_size(), weights_pinned=w.is_pinned(),
                    total_wall_ns=marks[-1] - marks[0],
                    timings_ns={name: marks[i + 1] - marks[i] for i, name in enumerate(phases)})

    def close(self) -> None:
        """Idempotent: synchronise the device, drop every assignment and the
        host experts, then close the source owner."""
        with self._lock:
            if self._closed:
                return
            if not self._closing and any(s.active_leases for s in self._slots):
                raise RuntimeError("expert cache cannot close while an active lease exists")
            self._closing = True
            torch.cuda.synchronize(self.device)
            self._forget_assignments()
            self._sources.clear()
            self._key_objects.clear()
            self._codec = None
            self._staging = []
            self._staging_reader = []
            self._staging_ptrs = []
            self._coded_args = {}
            owner, self._source_owner = self._source_owner, None
            if owner is not None:
                owner.close()
            self._closed, self._closing = True, False

    # -------------------------------------------------------------- policy --
    def _copy_done(self, slot: _Slot) -> bool:
        if slot.ready_event is None:
            return True
        if self._resident.get(slot.expert_id) == slot.slot_id:
            return True
        return slot.ready_event.query()

    def _writable(self, slot: _Slot) -> bool:
        """The slot's last H2D has completed and no reader is pending."""
        return self._copy_done(slot) and all(ev.query() for ev in slot.use_events.values())

    def _choose_lru_slot(self, *, ready_only: bool = False) -> _Slot | None:
        free = [s for s in self._slots if s.active_leases == 0]
        if not free:
            return None
        if not ready_only:
            return min(free, key=_Slot.victim_rank)
        free.sort(key=_Slot.victim_rank)
        return next((s for s in free if self._writable(s)), None)

    def _choose_probability_slot(self, expert_id: Hashable,
                                 probabilities: Mapping[Hashable, float]) -> _Slot | None:
        """Speculative admission (gpu_expert_cache.py:520-541): only over a
        writable, unleased victim of strictly lower probability; empty slots
        first, then lower probability, then LRU, then slot id."""
        score = probabilities.get
        incoming = score(expert_id, 0.0)
        ranked = sorted((s for s in self._slots if s.active_leases == 0),
                        key=lambda s: (s.expert_id is not None, score(s.expert_id, 0.0),
                                       s.last_used_sequence, s.slot_id))
        for s in ranked:
            if s.expert_id is not None and score(s.expert_id, 0.0) >= incoming:
                return None
            if self._writable(s):
                return s
        return None

    def _transfer_stream(self) -> torch.cuda.Stream:
        """Stream of the next H2D: the cache's two SDMA streams alternate by
        submission sequence; a replaced ``copy_stream`` (a scheduler's
        shared queue) takes every transfer."""
        if self.copy_stream is not self._own_copy_stream or self._submission_sequence % 2 == 0:
            return self.copy_stream
        return self._aux_copy_stream

    def _assign_and_submit(self, slot: _Slot, expert_id: Hashable) -> None:
        key = self._key_objects.get(expert_id, expert_id)
        victim = slot.expert_id
        if victim is not None:
            self._resident.pop(victim, None)
            self._inflight.pop(victim, None)
            self._stats.evictions += 1
        slot.generation += 1
        slot.expert_id = key
        readers = tuple(slot.use_events.values())
        slot.use_events.clear()
        stream = self._transfer_stream()
        record = self._coded_args.get(key)
        staged = None
        if record is None:
            if slot.ready_event is not None and slot.write_stream is not stream:
                # Writes of one slot stay in submission order across the two
                # streams (on one stream, stream order already keeps them).
                stream.wait_event(slot.ready_event)
            for guard in readers:
                self._await_reader(stream, guard)
            ops.copy_h2d(slot.tensor, self._sources[key], stream)
            self.h2d_bytes += slot.tensor.numel() * slot.tensor.element_size()
        else:
            staged = self._stage_record(record, stream)
            self._decode_into(slot, record, staged, stream, readers)
        ready = torch.cuda.Event(blocking=False)
        ready.record(stream)
        if staged is not None:
            self._staging_reader[staged] = (ready, stream)
        slot.ready_event = ready
        slot.write_stream = stream
        slot.ready_seq = self._submission_sequence
        transfer = _Transfer(key, slot.slot_id, slot.generation, self._submission_sequence, ready,
                             int(stream.cuda_stream))
        self._inflight[key] = transfer
        self._outstanding_transfers.append(transfer)
        self._stats.h2d_submissions += 1
        self._submission_sequence += 1
        if self._observer is not None:
            if victim is not None:
                self._record_transition(_K.EVICT, key, slot, victim_expert_id=victim)
            self._record_transition(_K.H2D_SUBMIT, key, slot,
                                    submission_sequence=transfer.submission_sequence,
                                    ready_event=ready)

    def _stage_record(self, record: tuple, stream: torch.cuda.Stream) -> int:
        """Enqueue the copy of a coded record into the next staging buffer
        on the copy stream; returns the buffer.  The copy touches no slot,
        so it waits for nothing but the decode that last read the buffer
        (already ordered when that decode ran on the same stream)."""
        j = self._submission_sequence % len(self._staging)
        last = self._staging_reader[j]
        if last is not None and last[1] is not stream and not last[0].query():
            stream.wait_event(last[0])
        ops.stage_record(self._staging_ptrs[j], record[0], record[1], stream)
        self.h2d_bytes += record[1]
        return j

    def _decode_into(self, slot: _Slot, record: tuple, j: int, stream: torch.cuda.Stream,
                     readers: tuple) -> None:
        """Enqueue the decode of staging buffer j into the slot on the copy
        stream, after the record's copy (stream order), the slot's previous
        write and every stream that read the slot."""
        if slot.ready_event is not None and slot.write_stream is not stream:
            stream.wait_event(slot.ready_event)
        for guard in readers:
            self._await_reader(stream, guard)
        ops.decode_staged(self._staging_ptrs[j], record[1], slot.tensor.numel(), record[3],
                          record[2], slot.tensor.data_ptr(), stream)

    @staticmethod
    def _await_reader(stream: torch.cuda.Stream, guard: torch.cuda.Event) -> None:
        """Order a slot's next H2D after a kernel that read the slot.  The
        host waits for the reader (spinning at most _READER_SPIN_NS) before
        it hands the wait to the copy stream: copy streams that wait on
        compute-stream events while compute kernels wait on their ready
        events stalled between copies on MI355X (9 MiB copies fell from 57 to
        32-50 GB/s in that pattern, and back to 57 with host-side waits).  A
        reader still running after the spin gets the device-side wait."""
        if guard.query():
            return
        deadline = perf_counter_ns() + _READER_SPIN_NS
        while perf_counter_ns() < deadline:
            if guard.query():
                return
        stream.wait_event(guard)

    def _reap_completed_transfers(self) -> None:
        """Publish completed transfers as resident, in submission order.
        When the oldest one has completed, the newest transfer of each copy
        stream in the queue is queried: if all of those completed, so did
        every transfer (each stream completes its copies in order), and the
        queue is published without querying each event."""
        queue = self._outstanding_transfers
        if not queue or not queue[0].ready_event.query():
            return
        slots, resident, inflight = self._slots, self._resident, self._inflight
        if len(queue) > 2 and self._newest_per_stream_done(queue):
            done = len(queue)
        else:
            done = 1
            while done < len(queue) and queue[done].ready_event.query():
                done += 1
        # A _ResidentMap takes one version for the whole batch (below).
        batched = type(resident) is _ResidentMap
        publish = dict.__setitem__ if batched else type(resident).__setitem__
        for _ in range(done):
            t = queue.popleft()
            key = t.expert_id
            slot = slots[t.slot_id]
            held = slot.expert_id
            if slot.generation == t.generation and (held is key or held == key):
                publish(resident, key, t.slot_id)
            current = inflight.get(key)
            if current is t or (current is not None and current == t):
                del inflight[key]
        if batched:
            resident.version = next(_versions)
        self._state_version += 1

    @staticmethod
    def _newest_per_stream_done(queue) -> bool:
        seen = set()
        for t in reversed(queue):
            if t.stream is None:
                return False
            if t.stream not in seen:
                if not t.ready_event.query():
                    return False
                seen.add(t.stream)
        return True

    def _reap_completed_use_guards(self) -> None:
        reaped = False
        for slot in self._slots:
            done = [sid for sid, ev in slot.use_events.items() if ev.query()]
            for sid in done:
                del slot.use_events[sid]
            reaped = reaped or bool(done)
        if reaped:
            self._state_version += 1

    def _touch(self, slot: _Slot) -> None:
        self._sequence += 1
        self._state_version += 1
        slot.last_used_sequence = self._sequence

    def _counters_record(self, *, pending_use_guards: int | None = None) -> ExpertCacheStats:
        if pending_use_guards is None:
            pending_use_guards = sum(len(s.use_events) for s in self._slots)
        c = self._stats
        return ExpertCacheStats(h2d_submissions=c.h2d_submissions, resident_hits=c.resident_hits,
                                inflight_joins=c.inflight_joins, evictions=c.evictions,
                                pending_use_guards=pending_use_guards)

    def _record_transition(self, kind, expert_id, slot, *, submission_sequence=None,
                           victim_expert_id=None, ready_event=None, stream_ids=()) -> None:
        self._observer.record(kind=kind, cache_id=self.cache_id, queue_id=self.queue_id,
                              expert_id=expert_id, slot_id=slot.slot_id,
                              generation=slot.generation,
                              submission_sequence=submission_sequence,
                              victim_expert_id=victim_expert_id, ready_event=ready_event,
                              stream_ids=stream_ids)

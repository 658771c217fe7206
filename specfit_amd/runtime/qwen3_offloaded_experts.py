"""Offloaded Qwen3-MoE expert operator on the gfx950 kernels.

Drop-in for src/specfit/runtime/qwen3_offloaded_experts.py:19-292
(``ReductionMode``, ``ExpertExecutionPolicy``, ``Qwen3OffloadedExperts`` with
the same constructor, ``forward`` signature and ValueErrors, and the
``_expert_forward`` seam).

One layer forward:

1. K2 ``sf_dispatch`` stably sorts the T*K routes by expert id on the device
   (replaces torch.sort / unique_consecutive / where, :111-122, :173-178) and
   also writes the [E+1] counts into the layer's pinned staging buffer; the
   host waits for K2 and reads them once (the layer's only device-to-host
   sync -- the reference has the same one) to know the active experts.
2. Experts are leased from the ``GpuExpertCache`` in the reference's order
   and with its acquire / one-ahead prefetch / release sequence
   (:205-230), so LRU state, generations, statistics and observer events
   evolve exactly as in the reference.  Consecutive experts that need no
   eviction (resident hits, in-flight joins) are computed by ONE grouped
   SwiGLU launch (K3); their slots stay pinned until that launch is
   enqueued, and the batch is always flushed before an acquisition that
   chooses a victim, so every eviction decision sees the same leased set as
   the reference.  A miss is computed by its own launch, ordered after its
   H2D ready event on the GPU only (no host wait), so later copies stream
   back to back on the copy stream while earlier experts compute.
3. K3 writes bf16(y * routing weight) per dispatched row; K4 ``sf_combine``
   adds each token's rows in canonical (ascending expert id) order with one
   fp32 accumulator (default) or, like the reference's sequence of bf16
   ``index_add_`` calls (:140-164), with bf16 rounding per addition --
   always so in arrival order.

Every expert's result is independent of how experts are grouped into
launches and of the execution order, so canonical outputs are bitwise
invariant to order, slot count and prefetch policy.
"""
from __future__ import annotations

from contextlib import closing
from dataclasses import dataclass, field
from enum import Enum
from itertools import compress
from typing import Sequence

import torch
from torch import nn

from .. import ops
from .gpu_expert_cache import GpuExpertCache
from .lease import ExpertLease, NoEvictableSlotError
from .state import ExpertKey


# Largest number of experts one K3 launch of the legacy path computes.
_MAX_BATCH = 64
# Misses share a K3 launch in groups of two thirds of the slots; among the
# last that many experts of a layer's order, in groups of half the slots, so
# that less K3 work is left after the layer's last copy.  Measured on MI355X
# against groups of half the slots throughout (same box, two runs each):
# the 48-layer forwards (12 slots) 189.6 / 111.0 against 186.8 – 187.9 /
# 107.9 – 108.1 tokens/s (cold / verification tree), fewer launches per
# layer; the 24-slot headline unchanged (19,910 – 19,947 tokens/s) with
# 0.486 of the HBM roofline in-step and 0.86 of K3 under the copies.
# Groups of two thirds without the tail groups reach 0.54 of the roofline
# but leave 26% of K3 after the last copy.
_MISS_GROUP_NUM, _MISS_GROUP_DEN = 2, 3
_TAIL_GROUP_DIVISOR = 2  # 0: no tail groups


class ReductionMode(str, Enum):
    CANONICAL = "canonical"
    ARRIVAL_ORDER = "arrival_order"


class ExpertExecutionPolicy(str, Enum):
    EXPERT_ID_ASCENDING = "expert_id_ascending"
    RESIDENT_FIRST = "resident_first"


@dataclass
class _GroupedRoutes:
    """Device buffers of one layer forward shared by its K3 launches."""

    hidden: torch.Tensor          # bf16 [T, H] contiguous
    plan: ops.DispatchPlan
    route_weights: torch.Tensor   # bf16 [T*K] contiguous
    act: torch.Tensor             # bf16 [T*K, I] scratch
    rows: torch.Tensor            # bf16 [T*K, H] scaled expert outputs
    expert_ids: Sequence[int] = ()
    tag: str = ""                 # "resident" or "miss": label of the launch
    storage: torch.Tensor | None = None  # the cache's [slots, 3*I*H] slot storage
    covered: frozenset = frozenset()  # experts whose rows a slot-table launch computed
    # Transfers the next launch must wait for: copy stream -> (sequence,
    # ready event) of the latest transfer of a batched lease on that stream.
    pending: dict = field(default_factory=dict)


def _dispatch(top_k_index: torch.Tensor, num_experts: int,
              host_meta: torch.Tensor | None = None) -> ops.DispatchPlan:
    """Seam: K2 dispatch of one layer's routes (with ``host_meta``, the
    kernel also writes the counts the layer reads into that pinned buffer)."""
    return ops.dispatch(top_k_index, num_experts, host_meta=host_meta)


def _expert_forward(hidden_states: torch.Tensor, packed_weights, *, hidden_size: int,
                    intermediate_size: int, routes: _GroupedRoutes | None = None) -> torch.Tensor:
    """Seam for every expert MLP launch (qwen3_offloaded_experts.py:38-62).

    Without ``routes``: the reference signature -- ``hidden_states`` are the
    gathered rows of one expert and ``packed_weights`` its packed
    ``[gate | up | down]`` tensor; returns the unscaled SwiGLU output.
    With ``routes``: ``packed_weights`` is a sequence of slot tensors for
    ``routes.expert_ids``; K3 writes their weighted rows into ``routes.rows``.
    """
    projection = hidden_size * intermediate_size
    if routes is None:
        if packed_weights.numel() != 3 * projection:
            raise ValueError(f"packed expert has {packed_weights.numel()} elements, "
                             f"expected {3 * projection}")
        return ops.expert_swiglu(hidden_states, packed_weights, hidden_size, intermediate_size)
    ops.grouped_swiglu(routes.hidden, routes.plan, routes.route_weights, routes.expert_ids,
                       packed_weights, hidden_size, intermediate_size, routes.act, routes.rows,
                       tag=routes.tag, slot_storage=routes.storage)
    return routes.rows


_DEFAULT_EXPERT_FORWARD = _expert_forward


class Qwen3OffloadedExperts(nn.Module):
    """Routed experts of one decoder layer served from a GpuExpertCache."""

    def __init__(self, *, layer_id: int, cache: GpuExpertCache, hidden_size: int,
                 intermediate_size: int,
                 reduction_mode: ReductionMode | str = ReductionMode.CANONICAL,
                 execution_policy: ExpertExecutionPolicy | str = (
                     ExpertExecutionPolicy.EXPERT_ID_ASCENDING),
                 h2d_prefetch: bool = True, combine_fp32: bool = True) -> None:
        super().__init__()
        if layer_id < 0:
            raise ValueError("layer_id must be non-negative")
        if hidden_size <= 0:
            raise ValueError("hidden_size must be positive")
        if intermediate_size <= 0:
            raise ValueError("intermediate_size must be positive")
        if type(h2d_prefetch) is not bool:
            raise ValueError("h2d_prefetch must be a boolean")
        if type(combine_fp32) is not bool:
            raise ValueError("combine_fp32 must be a boolean")
        self.layer_id = layer_id
        self.cache = cache
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.reduction_mode = ReductionMode(reduction_mode)
        self.execution_policy = ExpertExecutionPolicy(execution_policy)
        self.h2d_prefetch = h2d_prefetch
        # Canonical reduction accumulates in fp32 and rounds once (max error
        # against the fp32 layer ~6e-3 instead of ~1e-2 for per-addition bf16
        # rounding); arrival order always rounds every addition to bf16, the
        # order-dependent arithmetic that mode exists to reproduce.
        self.combine_fp32 = combine_fp32
        self._prediction_scheduler = None
        self._num_experts: int | None = None
        self._keys: tuple = ()  # ExpertKey of each expert id, set with _num_experts
        # Reused pinned staging of the per-forward [counts; offsets] read
        # (allocated once: growing the pinned pool can synchronise the device).
        self._host_counts: torch.Tensor | None = None
        # Device slot table (slot of each expert id or -1) and its pinned
        # staging, rewritten by every slot-table forward.
        self._table_host: torch.Tensor | None = None
        self._table_dev: torch.Tensor | None = None
        self._table_version: int | None = None  # cache table version on the device
        # Whether the layer's last legacy forward copied an expert in.
        self._last_forward_copied = True

    # -------------------------------------------------------------- forward --
    def forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                top_k_weights: torch.Tensor, *,
                execution_order: Sequence[int] | None = None) -> torch.Tensor:
        self._validate_inputs(hidden_states, top_k_index, top_k_weights)
        if self._prediction_scheduler is not None:
            if execution_order is not None:
                raise ValueError(
                    "explicit execution_order conflicts with dynamic predicted prefetch")
            return self._forward_prefetched(hidden_states, top_k_index, top_k_weights)
        if execution_order is None and self._uses_slot_table():
            return self._forward_slot_table(hidden_states, top_k_index, top_k_weights)
        routes, active = self._prepare(hidden_states, top_k_index, top_k_weights,
                                       idle=self._reap_while_routing)
        order = self._resolve_execution_order(active, execution_order)
        if routes is None:
            return torch.zeros_like(hidden_states)
        self._run_legacy(order, routes)
        return self._combine_rows(routes, top_k_index, order)

    def _uses_slot_table(self) -> bool:
        """The resident-first, one-ahead forward with the stock K3 seam and a
        [slots, 3*H*I] slot storage runs its resident experts from the
        device slot table when the layer's previous forward copied nothing
        in.  A layer that keeps missing takes the per-launch path instead:
        there the resident launch goes after the first miss copy is queued
        (the copies bound the step and the kernel hides under them), while
        the table launch would add its host cost before that copy."""
        storage = self.cache.storage
        return (not self._last_forward_copied
                and self.execution_policy is ExpertExecutionPolicy.RESIDENT_FIRST
                and self.h2d_prefetch and _expert_forward is _DEFAULT_EXPERT_FORWARD
                and storage.dim() == 2
                and storage.shape[1] == 3 * self.hidden_size * self.intermediate_size)

    def _forward_slot_table(self, hidden_states, top_k_index, top_k_weights):
        """Resident-first forward whose resident experts start before the
        routes reach the host: right after K2, one K3 launch over the device
        slot table (the slot of every expert whose transfer has completed,
        -1 otherwise) computes every resident expert that has rows while
        the host waits for the counts.  Then the reference lease sequence
        runs unchanged (resident hits, one-ahead prefetch, misses), with K3
        launches only for the experts the table launch did not cover:
        misses, transfers still in flight when the table was taken, and
        experts with more rows than tokens (repeated ids in a token's
        routes), whose rows the table launch computed with the split of a
        smaller expert.

        Why no table slot is overwritten while the table launch reads it:
        the launch reads only resident experts that have rows; in
        resident-first order every one of them is leased (and its lease
        records a use guard after the table launch on the compute stream)
        before the first miss chooses a victim, and the cache lock is held
        from the table to the end of the sequence."""
        T, K = top_k_index.shape
        if hidden_states.dtype != torch.bfloat16:
            raise ValueError("hidden_states must be bfloat16")
        if T == 0 or K == 0:
            return torch.zeros_like(hidden_states)
        num_experts = self.num_experts()
        cache = self.cache
        dev = hidden_states.device
        with cache._lock:
            # Host work before K2, so the table launch follows the counts
            # read without a host gap.
            version, slots = cache._slot_table(self._keys)
            table = self._upload_slot_table(version, slots, dev)
            routes = self._new_routes(hidden_states, top_k_weights, None)
            plan = _dispatch(top_k_index, num_experts, self._counts_staging(num_experts))
            routes.plan = plan
            entry = ops.grouped_swiglu_table(routes.hidden, plan, routes.route_weights, table,
                                             routes.storage, self.hidden_size,
                                             self.intermediate_size, routes.act, routes.rows,
                                             max_rows=T, tag="resident")
            counts = self._read_counts(plan, top_k_index, num_experts)
            active = tuple(compress(range(num_experts), counts))
            routes.covered = frozenset(e for e in active if slots[e] >= 0 and counts[e] <= T)
            if entry is not None:
                entry[0] = len(routes.covered)
                entry[1] = sum(counts[e] for e in routes.covered)
            order = self._resolve_execution_order(active, None)
            if len(routes.covered) == len(active):
                # The table launch computed every routed expert: the combine
                # needs nothing from the lease sequence, so it is enqueued
                # first and the host's bookkeeping (touches, counters, use
                # guards, all recorded after the table launch on this
                # stream) overlaps the device work instead of delaying it.
                out = self._combine_rows(routes, top_k_index, order)
                # Nothing is launched from this lease sequence, so the batch
                # cap of K3 launches does not apply: one run, one unpin.
                self._run_legacy(order, routes, batch_cap=len(order) + 1)
                return out
            self._run_legacy(order, routes)
        return self._combine_rows(routes, top_k_index, order)

    def _combine_rows(self, routes, top_k_index, order) -> torch.Tensor:
        if self.reduction_mode is ReductionMode.ARRIVAL_ORDER:
            return ops.combine(routes.rows, top_k_index, routes.plan, self.hidden_size,
                               expert_rank=self._arrival_ranks(order), accumulate_fp32=False)
        return ops.combine(routes.rows, top_k_index, routes.plan, self.hidden_size,
                           accumulate_fp32=self.combine_fp32)

    def _run_legacy(self, order, routes, batch_cap: int = _MAX_BATCH) -> None:
        before = self.cache._stats.h2d_submissions
        self._run_in_order(order, routes, batch_cap)
        self._last_forward_copied = self.cache._stats.h2d_submissions != before

    def _upload_slot_table(self, version: int | None, slots: list[int],
                           device: torch.device) -> torch.Tensor:
        """Copy the slot table to the device on the current stream, unless
        the table of this resident-map version is already there (``None``:
        an unversioned map, always uploaded).  The pinned staging is reused:
        the previous forward's upload was ordered before its counts read,
        which that forward waited for."""
        E = len(slots)
        if self._table_host is None or self._table_host.numel() != E:
            self._table_host = torch.empty(E, dtype=torch.int32, pin_memory=True)
            self._table_dev = torch.empty(E, dtype=torch.int32, device=device)
            self._table_version = None
        if version is None or version != self._table_version:
            self._table_host.numpy()[:] = slots
            self._table_dev.copy_(self._table_host, non_blocking=True)
            self._table_version = version
        return self._table_dev

    def _forward_prefetched(self, hidden_states, top_k_index, top_k_weights):
        """Scheduler-driven forward (qwen3_offloaded_experts.py:166-203): the
        scheduler hands out leased experts in the order it chooses (completed
        transfers first) in batches; each batch is computed by one grouped K3
        launch, enqueued before control returns to the scheduler, which then
        releases the batch's leases.  Outputs are reduced canonically."""
        scheduler = self._prediction_scheduler
        # While the device routes, the scheduler keeps placing copies as
        # queue credits free up (the copy link would otherwise idle until
        # the counts arrive).
        routes, active = self._prepare(hidden_states, top_k_index, top_k_weights,
                                       idle=scheduler._place_while_routing)
        batches = scheduler.expert_batches(self.layer_id, active)
        stream = torch.cuda.current_stream(self.cache.device)
        with closing(batches):
            for batch in batches:
                if routes is None:
                    raise RuntimeError("scheduler yielded an expert for an empty layer")
                routes.expert_ids = [e for e, _ in batch]
                routes.tag = "scheduled"
                _expert_forward(routes.hidden, [lease.wait(stream) for _, lease in batch],
                                hidden_size=self.hidden_size,
                                intermediate_size=self.intermediate_size, routes=routes)
        if routes is None:
            return torch.zeros_like(hidden_states)
        return ops.combine(routes.rows, top_k_index, routes.plan, self.hidden_size,
                           accumulate_fp32=self.combine_fp32)

    # ------------------------------------------------------------- helpers --
    def num_experts(self) -> int:
        """Expert count of this layer: 1 + the largest expert id among the
        cache's sources for this layer."""
        if self._num_experts is None:
            own = {k.expert_id: k for k in self.cache._sources
                   if isinstance(k, ExpertKey) and k.layer_id == self.layer_id}
            if not own:
                raise ValueError(f"cache holds no experts of layer {self.layer_id}")
            n = max(own) + 1
            if n > 256:
                raise ValueError("at most 256 experts per layer are supported")
            # The cache's own key objects: map lookups then hit by identity.
            self._keys = tuple(own.get(e) or ExpertKey(self.layer_id, e) for e in range(n))
            self._num_experts = n
        return self._num_experts

    def _prepare(self, hidden_states, top_k_index, top_k_weights, idle=None):
        """Dispatch on the device, read the active experts, allocate the
        layer's row buffers.  Returns (routes or None when there are no
        routes, active experts ascending).  ``idle``: host work to run while
        the counts are not there yet (``DispatchPlan.finish_counts``)."""
        T, K = top_k_index.shape
        if hidden_states.dtype != torch.bfloat16:
            raise ValueError("hidden_states must be bfloat16")
        if T == 0 or K == 0:
            return None, ()
        num_experts = self.num_experts()
        plan = _dispatch(top_k_index, num_experts, self._counts_staging(num_experts))
        # The row buffers do not depend on the counts: allocate them while
        # the device routes.
        routes = self._new_routes(hidden_states, top_k_weights, plan)
        counts = self._read_counts(plan, top_k_index, num_experts, idle)
        active = tuple(compress(range(num_experts), counts))
        return routes, active

    def _reap_while_routing(self) -> bool:
        """While the counts are on their way: publish the transfers that
        complete meanwhile (the previous forward's last copies), work the
        execution order would otherwise do after the counts arrive.  True
        while transfers are outstanding."""
        cache = self.cache
        with cache._lock:
            cache._reap_completed_transfers()
            return bool(cache._outstanding_transfers)

    def _counts_staging(self, num_experts: int) -> torch.Tensor:
        if self._host_counts is None:
            self._host_counts = torch.empty((2, num_experts + 1), dtype=torch.int32,
                                            pin_memory=True)
        return self._host_counts

    def _read_counts(self, plan, top_k_index, num_experts, idle=None) -> list:
        """The layer's one device-to-host read: routes per expert."""
        plan.fetch_counts(self._counts_staging(num_experts), idle=idle)
        counts = plan.count_list
        if counts[num_experts]:
            self._raise_invalid_index(top_k_index, num_experts)
        return counts

    def _new_routes(self, hidden_states, top_k_weights, plan) -> _GroupedRoutes:
        T, K = top_k_weights.shape
        dev = hidden_states.device
        N, I, H = T * K, self.intermediate_size, self.hidden_size
        work = torch.empty(N * (I + H), dtype=torch.bfloat16, device=dev)  # act, then rows
        routes = _GroupedRoutes(
            hidden=hidden_states.contiguous(),
            plan=plan,
            route_weights=top_k_weights.to(torch.bfloat16).contiguous().reshape(-1),
            act=work[:N * I].view(N, I),
            rows=work[N * I:].view(N, H))
        storage = self.cache.storage
        if storage.dim() == 2 and storage.shape[1] == 3 * self.hidden_size * self.intermediate_size:
            routes.storage = storage
        return routes

    def _raise_invalid_index(self, top_k_index, num_experts) -> None:
        values = top_k_index.flatten().tolist()
        bad = next(v for v in values if v < 0 or v >= num_experts)
        ExpertKey(self.layer_id, int(bad))  # negative ids raise ValueError here
        raise KeyError(f"unknown expert {ExpertKey(self.layer_id, int(bad))!r}")

    def _arrival_ranks(self, order: Sequence[int]) -> list[int]:
        """Execution position of each expert (combine order of ARRIVAL_ORDER)."""
        rank = [0] * self.num_experts()
        for position, expert in enumerate(order):
            rank[expert] = position
        return rank

    def _launch(self, routes: _GroupedRoutes, batch: list[tuple[int, ExpertLease, torch.Tensor]],
                tag: str = "") -> None:
        """One K3 launch for the batch's experts that a slot-table launch
        did not already compute, then unpin every lease of the batch (the
        use guard is recorded after both launches on the compute stream)."""
        try:
            covered = routes.covered
            todo = [(e, w) for e, _, w in batch if e not in covered] if covered else \
                [(e, w) for e, _, w in batch]
            pending = routes.pending
            if pending:
                stream = torch.cuda.current_stream(self.cache.device)
                for _, ready in pending.values():
                    stream.wait_event(ready)
                pending.clear()
            if todo:
                routes.expert_ids = [e for e, _ in todo]
                routes.tag = tag
                _expert_forward(routes.hidden, [w for _, w in todo],
                                hidden_size=self.hidden_size,
                                intermediate_size=self.intermediate_size, routes=routes)
        finally:
            self.cache._unpin_many([lease for _, lease, _ in batch])

    def _run_in_order(self, order: tuple[int, ...], routes: _GroupedRoutes,
                      batch_cap: int = _MAX_BATCH) -> None:
        """Reference lease sequence (acquire, optional one-ahead prefetch,
        wait, release) with the K3 launches batched.

        A released expert's slot stays pinned until its batch is launched.
        Pinned slots were all touched after every unpinned slot, so as long
        as one unleased, unpinned slot exists the LRU victim of the next
        miss is the same slot the reference would pick; otherwise the batch
        is launched first.  Batches are also capped at ``batch_cap``
        (``_MAX_BATCH`` experts per K3 launch unless the caller knows that
        no batch launches anything)."""
        cache = self.cache
        stream = torch.cuda.current_stream(cache.device)
        batch: list[tuple[int, ExpertLease, torch.Tensor]] = []
        # Misses are launched in groups of two thirds of the slots (the last
        # ones of the order in groups of half) so that the copy stream never
        # waits for the kernel of the group being filled.
        miss_group = max(1, cache.slot_count * _MISS_GROUP_NUM // _MISS_GROUP_DEN)
        tail_group = (max(1, cache.slot_count // _TAIL_GROUP_DIVISOR) if _TAIL_GROUP_DIVISOR
                      else miss_group)
        misses = 0

        def flush() -> None:
            nonlocal misses
            if batch:
                pending_batch = list(batch)
                tag = "miss" if misses else "resident"
                batch.clear()
                misses = 0
                self._launch(routes, pending_batch, tag)

        def before_acquire(k: ExpertKey, *, split_resident_run: bool) -> bool:
            """Flush if the eviction could differ (or, when asked, to keep a
            run of resident experts in its own launch); True when k misses."""
            if cache.is_available(k):
                return False
            if batch and ((split_resident_run and misses == 0) or not cache.has_unleased_slot()):
                flush()
            return True

        ahead: ExpertLease | None = None
        ahead_missed = False
        all_keys = self._keys
        keys = [all_keys[e] for e in order]
        n = len(order)
        index = 0
        try:
            while index < n:
                if self.h2d_prefetch and misses == 0 and not ahead_missed and index + 1 < n:
                    # Runs of resident experts: the same lease sequence in
                    # one locked pass (no miss can occur inside the run).
                    steps, index, ahead = cache._resident_steps(keys, index, ahead, stream,
                                                                batch_cap - len(batch))
                    if steps:
                        batch.extend(steps)
                        if len(batch) >= batch_cap:
                            flush()
                        continue
                expert_id = order[index]
                index += 1
                current, ahead = ahead, None
                missed, ahead_missed = ahead_missed, False
                if current is None:
                    k = keys[index - 1]
                    missed = before_acquire(k, split_resident_run=True)
                    current = cache.acquire(k)
                try:
                    if self.h2d_prefetch and index < n:
                        nxt = keys[index]
                        will_miss = before_acquire(nxt, split_resident_run=False)
                        try:
                            ahead = cache._prefetch(nxt)
                            ahead_missed = will_miss
                        except NoEvictableSlotError:
                            pass
                    weights = current._wait_pending(stream, routes.pending)
                except BaseException:
                    current.release()
                    raise
                batch.append((expert_id, current, weights))
                current._release_keep_pinned()
                misses += int(missed)
                group = tail_group if n - index <= miss_group else miss_group
                if (len(batch) >= batch_cap or misses >= group
                        or (misses == 0 and ahead_missed)):
                    flush()
            flush()
        except BaseException:
            for _, lease, _ in batch:
                lease._unpin()
            batch.clear()
            raise
        finally:
            if ahead is not None:
                ahead.release()

    def _validate_inputs(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                         top_k_weights: torch.Tensor) -> None:
        if hidden_states.ndim != 2:
            raise ValueError("hidden_states must have shape [tokens, hidden]")
        if hidden_states.shape[1] != self.hidden_size:
            raise ValueError(f"hidden_states width is {hidden_states.shape[1]}, "
                             f"expected {self.hidden_size}")
        if top_k_index.ndim != 2:
            raise ValueError("top_k_index must have shape [tokens, top_k]")
        if top_k_weights.shape != top_k_index.shape:
            raise ValueError("top_k_weights must match top_k_index shape")
        if top_k_index.shape[0] != hidden_states.shape[0]:
            raise ValueError("routing tensors must match the token count")
        if top_k_index.dtype is not torch.long:
            raise ValueError("top_k_index must use torch.long")
        if hidden_states.device != self.cache.device:
            raise ValueError("hidden_states must be on the cache device")
        if top_k_index.device != hidden_states.device:
            raise ValueError("top_k_index must be on the hidden-state device")
        if top_k_weights.device != hidden_states.device:
            raise ValueError("top_k_weights must be on the hidden-state device")

    def _resolve_execution_order(self, active_experts: tuple[int, ...],
                                 execution_order: Sequence[int] | None) -> tuple[int, ...]:
        if execution_order is not None:
            order = tuple(int(e) for e in execution_order)
            if len(order) != len(set(order)):
                raise ValueError("execution_order must not contain duplicates")
            if set(order) != set(active_experts):
                raise ValueError("execution_order must contain every active expert exactly once")
            return order
        if self.execution_policy is ExpertExecutionPolicy.EXPERT_ID_ASCENDING:
            return active_experts
        cache = self.cache
        keys = self._keys
        hits, misses = [], []
        with cache._lock:
            cache._reap_completed_transfers()
            resident = cache._resident
            for e in active_experts:
                (hits if keys[e] in resident else misses).append(e)
        return tuple(hits + misses)

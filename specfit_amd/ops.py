"""PyTorch-facing wrappers of the C-ABI kernels (K1-K4 and the H2D copy).

Tensors are plumbing: each wrapper checks dtype, device, shape and
contiguity on the host, allocates outputs with the caching allocator and
enqueues the HIP kernel on the caller's (default: current) stream through the
C-ABI.  There is no PyTorch or CPU fallback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import torch

from . import _native

_BF16 = torch.bfloat16


_HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h
_hip_runtime = None


def _hip():
    global _hip_runtime
    if _hip_runtime is None:
        lib = ctypes.CDLL("libamdhip64.so")
        lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                            ctypes.c_void_p]
        lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        lib.hipEventQuery.argtypes = [ctypes.c_void_p]
        _hip_runtime = lib
    return _hip_runtime


class TimingEvent:
    """A HIP timing event recorded without the system-scope fence that
    ordinary events perform (hipEventDisableSystemFence): no cache
    writeback/invalidate between the timed kernels, so bracketing every
    launch does not slow the launches it times.  Same interface as the
    parts of torch.cuda.Event used here."""

    def __init__(self) -> None:
        self._ev = ctypes.c_void_p()
        rc = _hip().hipEventCreateWithFlags(ctypes.byref(self._ev), _HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream: torch.cuda.Stream) -> None:
        rc = _hip().hipEventRecord(self._ev, ctypes.c_void_p(int(stream.cuda_stream)))
        if rc:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end: "TimingEvent") -> float:
        """Milliseconds from this event to ``end`` (both must have completed)."""
        ms = ctypes.c_float()
        rc = _hip().hipEventElapsedTime(ctypes.byref(ms), self._ev, end._ev)
        if rc:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)

    def __del__(self) -> None:
        if self._ev and _hip_runtime is not None:
            _hip_runtime.hipEventDestroy(self._ev)
            self._ev = ctypes.c_void_p()


_HIP_EVENT_DISABLE_TIMING = 0x2  # hip_runtime_api.h
_HIP_ERROR_NOT_READY = 600       # hipErrorNotReady


class HostWaitEvent:
    """A HIP event (no timing) recorded on a raw stream handle for the host
    to wait on, as torch.cuda.Event.record + synchronize but without a
    Stream object or a fresh event per record: handles come from a pool and
    go back to it when the wrapper is dropped (re-recording a handle whose
    earlier record is still pending is allowed)."""

    _pool: list = []
    __slots__ = ("_ev",)

    def __init__(self, stream_handle: int) -> None:
        self._ev = None
        ev = self._pool.pop() if self._pool else None
        if ev is None:
            ev = ctypes.c_void_p()
            rc = _hip().hipEventCreateWithFlags(ctypes.byref(ev), _HIP_EVENT_DISABLE_TIMING)
            if rc:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
        self._ev = ev
        rc = _hip().hipEventRecord(ev, ctypes.c_void_p(stream_handle))
        if rc:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def synchronize(self) -> None:
        rc = _hip().hipEventSynchronize(self._ev)
        if rc:
            raise RuntimeError(f"hipEventSynchronize failed ({rc})")

    def query(self) -> bool:
        """True once the recorded work has completed (does not block)."""
        rc = _hip().hipEventQuery(self._ev)
        if rc == _HIP_ERROR_NOT_READY:
            return False
        if rc:
            raise RuntimeError(f"hipEventQuery failed ({rc})")
        return True

    def __del__(self) -> None:
        if self._ev is not None:
            self._pool.append(self._ev)
            self._ev = None


class LaunchRecorder:
    """Collects HIP timing events around K3 launches and H2D copies, each on
    the stream the work runs on (enabled by ``record_launches``).  Events
    are TimingEvents; read them after the device has finished the work."""

    def __init__(self, *, copies: bool = True, park_cycles: int = 0,
                 per_copy: bool = False) -> None:
        self.k3: list[tuple[int, int, str, TimingEvent, TimingEvent]] = []
        # With park_cycles, a short device sleep is queued on the stream
        # before each launch's start event: a launch enqueued while its
        # stream is idle would otherwise have the host's enqueue latency
        # (the time between the start event and the kernels reaching the
        # device) counted as kernel time.
        self.park_cycles = park_cycles
        # Copies are timed per window (first copy start .. last copy end of a
        # window, per stream), not per copy: ``close_copy_window`` ends one.
        self.copies = copies
        self.h2d_bytes = 0
        self.h2d_count = 0
        # (record bytes, values, start, end) of each coded-transfer decode,
        # bracketed on its copy stream (start: after the record's copy).
        self.decodes: list[tuple[int, int, TimingEvent, TimingEvent]] = []
        self.windows: list[tuple[TimingEvent, TimingEvent]] = []
        self._open: dict[int, tuple[torch.cuda.Stream, TimingEvent]] = {}
        # With per_copy, a (start, end) event pair on the copy stream around
        # every copy, and ``mark`` events the caller records (e.g. at each
        # layer's router) to place the copies in the forward.
        self.per_copy = per_copy
        self.copy_spans: list[tuple[TimingEvent, TimingEvent]] = []
        self.marks: list[tuple[object, TimingEvent]] = []
        self._copy_start: TimingEvent | None = None

    def _copy_started(self, stream: torch.cuda.Stream, nbytes: int) -> None:
        self.h2d_bytes += nbytes
        self.h2d_count += 1
        key = int(stream.cuda_stream)
        if self.copies and key not in self._open:
            start = TimingEvent()
            start.record(stream)
            self._open[key] = (stream, start)
        if self.per_copy:
            self._copy_start = TimingEvent()
            self._copy_start.record(stream)

    def _copy_ended(self, stream: torch.cuda.Stream) -> None:
        if self.per_copy and self._copy_start is not None:
            end = TimingEvent()
            end.record(stream)
            self.copy_spans.append((self._copy_start, end))
            self._copy_start = None

    def mark(self, label, stream: torch.cuda.Stream) -> None:
        """Record an event labelled ``label`` on ``stream``."""
        ev = TimingEvent()
        ev.record(stream)
        self.marks.append((label, ev))

    def close_copy_window(self) -> None:
        for stream, start in self._open.values():
            end = TimingEvent()
            end.record(stream)
            self.windows.append((start, end))
        self._open.clear()

    def copy_busy_seconds(self) -> float:
        """Sum over windows of the copy-stream busy interval (windows of the
        two SDMA streams overlap in time; their union is returned)."""
        spans = []
        origin = None
        for start, end in self.windows:
            if origin is None:
                origin = start
            spans.append((origin.elapsed_time(start), origin.elapsed_time(end)))
        spans.sort()
        total, cur_s, cur_e = 0.0, None, None
        for s_, e_ in spans:
            if cur_e is None or s_ > cur_e:
                if cur_e is not None:
                    total += cur_e - cur_s
                cur_s, cur_e = s_, e_
            else:
                cur_e = max(cur_e, e_)
        if cur_e is not None:
            total += cur_e - cur_s
        return total * 1e-3

    def _events(self, stream):
        start = TimingEvent()
        end = TimingEvent()
        if self.park_cycles:
            with torch.cuda.stream(stream):
                torch.cuda._sleep(self.park_cycles)
        start.record(stream)
        return start, end


_recorder: LaunchRecorder | None = None


class record_launches:
    """Context manager: ``with record_launches() as rec: ...``."""

    def __init__(self, *, copies: bool = True, park_cycles: int = 0,
                 per_copy: bool = False) -> None:
        self._copies = copies
        self._park = park_cycles
        self._per_copy = per_copy

    def __enter__(self) -> LaunchRecorder:
        global _recorder
        if _recorder is not None:
            raise RuntimeError("launch recording is already active")
        _recorder = LaunchRecorder(copies=self._copies, park_cycles=self._park,
                                   per_copy=self._per_copy)
        return _recorder

    def __exit__(self, *exc) -> None:
        global _recorder
        _recorder = None


_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(stream: torch.cuda.Stream | None, device: torch.device) -> int:
    if stream is not None:
        return int(stream.cuda_stream)
    if _current_raw_stream is not None and device.index is not None:
        return _current_raw_stream(device.index)  # no Stream object on the hot path
    return int(torch.cuda.current_stream(device).cuda_stream)


def _require_cuda(name: str, t: torch.Tensor, dtype: torch.dtype | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a HIP device")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must have dtype {dtype}")


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------ K1 ----
def router_topk(hidden: torch.Tensor, weight: torch.Tensor, top_k: int,
                norm_topk_prob: bool, *, stream: torch.cuda.Stream | None = None):
    """(logits bf16 [T,E], weights bf16 [T,K], indices int64 [T,K]) of the
    fused router kernel.  Replaces Qwen3MoeTopKRouter.forward (tf:258-267)."""
    _require_cuda("hidden_states", hidden, _BF16)
    _require_cuda("router weight", weight, _BF16)
    if hidden.ndim != 2 or weight.ndim != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("router expects hidden [T,H] and weight [E,H]")
    if hidden.device != weight.device:
        raise ValueError("router inputs must share a device")
    hidden = hidden.contiguous()
    weight = weight.contiguous()
    T, H = hidden.shape
    E = weight.shape[0]
    # One allocation for the three outputs (indices first, 8-byte aligned).
    nk = T * top_k
    buf = torch.empty(nk + (T * E + nk + 3) // 4, dtype=torch.int64, device=hidden.device)
    idx = buf[:nk].view(T, top_k)
    halves = buf[nk:].view(_BF16)
    logits = halves[:T * E].view(T, E)
    w = halves[T * E:T * E + nk].view(T, top_k)
    rc = _native.lib().sf_router_topk(
        _ptr(hidden), _ptr(weight), T, H, E, int(top_k), int(bool(norm_topk_prob)),
        _ptr(logits), _ptr(w), _ptr(idx), _stream_handle(stream, hidden.device))
    _native.check(rc, "sf_router_topk")
    return logits, w, idx


# ------------------------------------------------------------------ K2 ----
@dataclass
class DispatchPlan:
    """Device-side dispatch of one layer's routes (output of K2).

    counts/offsets are int32 [E+1] (counts[E] = out-of-range entries),
    perm_pos/inv_perm int32 [T*K].  ``host_counts`` is filled by
    ``fetch_counts`` (the layer's one device-to-host read)."""

    tokens: int
    top_k: int
    num_experts: int
    meta: torch.Tensor            # int32 [2, E+1]: row 0 counts, row 1 offsets
    perm_pos: torch.Tensor
    inv_perm: torch.Tensor
    host_counts: torch.Tensor | None = None
    # Python copies of host_counts[0] (routes per expert) and [1] (offsets),
    # made with it.
    count_list: list | None = None
    offset_list: list | None = None
    _counts_event: tuple | None = None  # (event, staging) of a started read

    @property
    def counts(self) -> torch.Tensor:
        return self.meta[0]

    @property
    def offsets(self) -> torch.Tensor:
        return self.meta[1]

    def fetch_counts(self, staging: torch.Tensor | None = None, *, idle=None) -> torch.Tensor:
        """[counts; offsets] in pinned host memory: waits for dispatch when it
        wrote them there (``dispatch(..., host_meta=...)``), else copies them
        in one transfer and waits for it.  ``staging`` is a reusable pinned
        int32 [2, E+1] buffer for the copy; without one a pinned buffer is
        allocated (which may synchronise the device while the allocator
        grows, so hot paths pass one).  ``idle``: see ``finish_counts``."""
        if self.host_counts is None:
            self.start_counts(staging)
        return self.finish_counts(idle)

    def start_counts(self, staging: torch.Tensor | None = None) -> None:
        """Enqueue the [counts; offsets] copy on the current stream without
        waiting (``finish_counts`` waits).  Nothing to do when the read is
        already started, or when dispatch wrote the counts to host memory."""
        if self.host_counts is not None or self._counts_event is not None:
            return
        shape = (2, self.num_experts + 1)
        if staging is None:
            staging = torch.empty(shape, dtype=torch.int32, pin_memory=True)
        elif staging.shape != shape or staging.dtype != torch.int32 or not staging.is_pinned():
            raise ValueError("staging must be pinned int32 [2, num_experts + 1]")
        ev = torch.cuda.Event()
        staging.copy_(self.meta, non_blocking=True)
        ev.record(torch.cuda.current_stream(self.meta.device))
        self._counts_event = (ev, staging)

    def finish_counts(self, idle=None) -> torch.Tensor:
        """Wait for the counts.  ``idle``, when given, is called repeatedly
        while they are not there yet, as long as it returns True (host work
        that should not wait for the routes, e.g. submitting copies as copy
        credits free up); then the host blocks."""
        if self.host_counts is None:
            if self._counts_event is None:
                self.start_counts()
            ev, staging = self._counts_event
            if idle is not None:
                while not ev.query() and idle():
                    pass
            ev.synchronize()
            self._counts_event = None
            self.host_counts = staging
            self.count_list, self.offset_list = staging.tolist()
        return self.host_counts

    def active_experts(self) -> tuple[int, ...]:
        counts = self.fetch_counts()[0]
        if int(counts[self.num_experts]):
            raise KeyError("routing index outside the expert range")
        return tuple(int(e) for e in torch.nonzero(counts[: self.num_experts]).flatten().tolist())

    def host_offsets(self) -> list[int]:
        return self.fetch_counts()[1].tolist()


def dispatch(index: torch.Tensor, num_experts: int, *,
             stream: torch.cuda.Stream | None = None,
             host_meta: torch.Tensor | None = None) -> DispatchPlan:
    """Stable counting sort of the [T,K] routes by expert id (K2).

    ``host_meta``: a pinned int32 [2, num_experts + 1] buffer that the
    kernel also writes [counts; offsets] into; the plan's counts read then
    waits for the kernel instead of enqueuing a copy.  The caller keeps the
    buffer untouched until it has read the counts (``fetch_counts``)."""
    _require_cuda("top_k_index", index, torch.int64)
    if index.ndim != 2:
        raise ValueError("top_k_index must have shape [tokens, top_k]")
    shape = (2, num_experts + 1)
    if host_meta is not None and (host_meta.shape != shape or host_meta.dtype != torch.int32
                                  or not host_meta.is_pinned() or not host_meta.is_contiguous()):
        raise ValueError("host_meta must be pinned contiguous int32 [2, num_experts + 1]")
    index = index.contiguous()
    T, K = index.shape
    dev = index.device
    # [counts; offsets], perm_pos and inv_perm in one allocation.
    e1 = num_experts + 1
    buf = torch.empty(2 * e1 + 2 * T * K, dtype=torch.int32, device=dev)
    meta = buf[:2 * e1].view(2, e1)
    perm = buf[2 * e1:2 * e1 + T * K]
    inv = buf[2 * e1 + T * K:]
    plan = DispatchPlan(T, K, int(num_experts), meta, perm, inv)
    if T * K == 0:
        meta.zero_()
        if host_meta is not None:
            host_meta.zero_()
            plan.host_counts = host_meta
            plan.count_list, plan.offset_list = host_meta.tolist()
        return plan
    handle = _stream_handle(stream, dev)
    counts_ptr = meta.data_ptr()  # row 0; row 1 (offsets) follows E + 1 int32 later
    rc = _native.lib().sf_dispatch(_ptr(index), T, K, int(num_experts), counts_ptr,
                                   counts_ptr + 4 * (num_experts + 1), _ptr(perm), _ptr(inv),
                                   _ptr(host_meta), handle)
    _native.check(rc, "sf_dispatch")
    if host_meta is not None:
        plan._counts_event = (HostWaitEvent(handle), host_meta)
    return plan


# ------------------------------------------------------------------ K3 ----
def grouped_swiglu(hidden: torch.Tensor, plan: DispatchPlan, route_weights: torch.Tensor | None,
                   expert_ids: Sequence[int], expert_weights: Sequence[torch.Tensor],
                   hidden_size: int, intermediate_size: int, act: torch.Tensor,
                   out_rows: torch.Tensor, *, stream: torch.cuda.Stream | None = None,
                   tag: str = "", slot_storage: torch.Tensor | None = None) -> None:
    """Grouped SwiGLU over the dispatched rows of the listed experts (K3).
    ``expert_weights[i]`` is the packed [3*H*I] bf16 weight tensor of
    ``expert_ids[i]`` (a cache slot).  With ``slot_storage`` (the cache's
    [slots, 3*H*I] bf16 storage) each weight is checked to be one of its
    rows by address arithmetic instead of tensor property checks."""
    n = len(expert_ids)
    if n != len(expert_weights):
        raise ValueError("expert_ids and expert_weights differ in length")
    if n == 0 or plan.tokens == 0:
        return
    numel = 3 * hidden_size * intermediate_size
    N = plan.tokens * plan.top_k
    if act.shape != (N, intermediate_size) or out_rows.shape != (N, hidden_size):
        raise ValueError("workspace shapes do not match the dispatch plan")
    if hidden.shape != (plan.tokens, hidden_size) or not hidden.is_contiguous():
        raise ValueError("hidden_states must be contiguous [tokens, hidden]")
    if route_weights is not None and (route_weights.dtype != _BF16 or route_weights.numel() != N
                                      or not route_weights.is_contiguous()):
        raise ValueError("route weights must be contiguous bf16 [tokens*top_k]")
    E = plan.num_experts
    ids = [int(e) for e in expert_ids]
    weights = list(expert_weights)
    counts = plan.count_list
    if counts is not None and n > 1:
        # Experts with more rows take longer: give them the first workgroups
        # so they start first and the light ones fill in behind them.  An
        # expert's result does not depend on its position in the launch.
        order = sorted(range(n), key=lambda i: -counts[ids[i]])
        ids = [ids[i] for i in order]
        weights = [weights[i] for i in order]
    for e in ids:
        if not 0 <= e < E:
            raise KeyError(f"unknown expert {e}")
    if slot_storage is not None:
        if (slot_storage.dtype != _BF16 or slot_storage.dim() != 2
                or slot_storage.shape[1] != numel or not slot_storage.is_contiguous()
                or slot_storage.device != hidden.device):
            raise ValueError(f"slot storage must be contiguous bf16 [slots, {numel}]")
        base = slot_storage.data_ptr()
        row_bytes = numel * 2
        span = slot_storage.shape[0] * row_bytes
        ptrs = [w.data_ptr() for w in weights]
        for e, w, ptr in zip(ids, weights, ptrs):
            off = ptr - base
            if not (0 <= off < span and off % row_bytes == 0 and w.numel() == numel):
                raise ValueError(f"packed expert {e} is not a row of the slot storage")
    else:
        for e, w in zip(ids, weights):
            if (w.dtype != _BF16 or w.numel() != numel or not w.is_contiguous()
                    or w.device != hidden.device):
                raise ValueError(f"packed expert {e} must be contiguous bf16 with {numel} elements")
        ptrs = [w.data_ptr() for w in weights]
    id_arr = (ctypes.c_int32 * n)(*ids)
    w_arr = (ctypes.c_uint64 * n)(*ptrs)
    # Rows of each expert from the counts already on the host: the kernels
    # then start streaming weights without reading offsets first.
    row_begin = row_count = None
    offs = plan.offset_list
    if counts is not None and offs is not None:
        row_begin = ctypes.cast((ctypes.c_int32 * n)(*[offs[e] for e in ids]), ctypes.c_void_p)
        row_count = ctypes.cast((ctypes.c_int32 * n)(*[counts[e] for e in ids]), ctypes.c_void_p)
    max_rows = N
    if counts is not None:
        max_rows = max(1, max(counts[e] for e in ids))
    rec = _recorder
    if rec is not None:  # timing events bracket the C call only, not the host work above
        s = stream if stream is not None else torch.cuda.current_stream(hidden.device)
        start, end = rec._events(s)
    rc = _native.lib().sf_grouped_swiglu(
        _ptr(hidden), _ptr(plan.perm_pos), _ptr(plan.offsets), _ptr(route_weights),
        plan.tokens, plan.top_k, hidden_size, intermediate_size, n, max_rows,
        ctypes.cast(id_arr, ctypes.c_void_p), ctypes.cast(w_arr, ctypes.c_void_p),
        row_begin, row_count, _ptr(act), _ptr(out_rows), _stream_handle(stream, hidden.device))
    _native.check(rc, "sf_grouped_swiglu")
    if rec is not None:
        end.record(s)
        rows = 0
        if counts is not None:
            rows = int(sum(counts[int(e)] for e in expert_ids))
        rec.k3.append((n, rows, tag, start, end))


def grouped_swiglu_table(hidden: torch.Tensor, plan: DispatchPlan,
                         route_weights: torch.Tensor | None, slot_of_expert: torch.Tensor,
                         slot_storage: torch.Tensor, hidden_size: int, intermediate_size: int,
                         act: torch.Tensor, out_rows: torch.Tensor, *,
                         max_rows: int | None = None, stream: torch.cuda.Stream | None = None,
                         tag: str = "") -> list | None:
    """K3 over every expert whose device slot-table entry is >= 0 (no host
    knowledge of the active set needed).  ``max_rows`` bounds any expert's
    rows (default tokens * top_k; tokens when every token's experts are
    distinct).  While launches are recorded, returns the recorder's entry
    ``[experts, rows, tag, start, end]``: the caller fills in the first two
    once it knows which experts had rows."""
    if plan.tokens == 0:
        return None
    _require_cuda("slot_of_expert", slot_of_expert, torch.int32)
    if slot_of_expert.numel() != plan.num_experts or not slot_of_expert.is_contiguous():
        raise ValueError("slot_of_expert must be contiguous int32 [num_experts]")
    numel = 3 * hidden_size * intermediate_size
    if slot_storage.ndim != 2 or slot_storage.shape[1] != numel or slot_storage.dtype != _BF16:
        raise ValueError("slot storage must be bf16 [slots, 3*H*I]")
    N = plan.tokens * plan.top_k
    if act.shape != (N, intermediate_size) or out_rows.shape != (N, hidden_size):
        raise ValueError("workspace shapes do not match the dispatch plan")
    bound = N if max_rows is None else int(max_rows)
    if bound < 1:
        raise ValueError("max_rows must be positive")
    rec = _recorder
    entry = None
    if rec is not None:
        s = stream if stream is not None else torch.cuda.current_stream(hidden.device)
        start, end = rec._events(s)
    rc = _native.lib().sf_grouped_swiglu_table(
        _ptr(hidden), _ptr(plan.perm_pos), _ptr(plan.offsets), _ptr(route_weights),
        plan.tokens, plan.top_k, hidden_size, intermediate_size, plan.num_experts, bound,
        _ptr(slot_of_expert), _ptr(slot_storage), int(slot_storage.stride(0)),
        _ptr(act), _ptr(out_rows), _stream_handle(stream, hidden.device))
    _native.check(rc, "sf_grouped_swiglu_table")
    if rec is not None:
        end.record(s)
        entry = [0, 0, tag, start, end]
        rec.k3.append(entry)
    return entry


def expert_swiglu(rows: torch.Tensor, packed: torch.Tensor, hidden_size: int,
                  intermediate_size: int, *,
                  stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """y = SwiGLU expert MLP of already-gathered rows (no routing weight)."""
    _require_cuda("hidden_states", rows, _BF16)
    _require_cuda("packed expert", packed, _BF16)
    if rows.ndim != 2 or rows.shape[1] != hidden_size:
        raise ValueError("rows must have shape [m, hidden]")
    expected = 3 * hidden_size * intermediate_size
    if packed.numel() != expected:
        raise ValueError(f"packed expert has {packed.numel()} elements, expected {expected}")
    if rows.stride(1) != 1:
        rows = rows.contiguous()
    packed = packed.contiguous()
    m = rows.shape[0]
    out = torch.empty((m, hidden_size), dtype=_BF16, device=rows.device)
    if m == 0:
        return out
    act = torch.empty((m, intermediate_size), dtype=_BF16, device=rows.device)
    rc = _native.lib().sf_expert_swiglu(_ptr(rows), m, int(rows.stride(0)), hidden_size,
                                        intermediate_size, _ptr(packed), _ptr(act), _ptr(out),
                                        _stream_handle(stream, rows.device))
    _native.check(rc, "sf_expert_swiglu")
    return out


# ------------------------------------------------------------------ K4 ----
def combine(rows: torch.Tensor, index: torch.Tensor, plan: DispatchPlan, hidden_size: int,
            *, expert_rank: Sequence[int] | None = None, accumulate_fp32: bool = False,
            out: torch.Tensor | None = None,
            stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """out[t] = sum of token t's scaled expert rows in canonical (or
    ``expert_rank``) order (K4)."""
    T, K = plan.tokens, plan.top_k
    if out is None:
        out = torch.empty((T, hidden_size), dtype=_BF16, device=index.device)
    if T == 0:
        return out
    if rows.shape != (T * K, hidden_size) or rows.dtype != _BF16 or not rows.is_contiguous():
        raise ValueError("rows must be contiguous bf16 [tokens*top_k, hidden]")
    if out.shape != (T, hidden_size) or not out.is_contiguous() or out.dtype != _BF16:
        raise ValueError("out must be contiguous bf16 [tokens, hidden]")
    index = index.contiguous()
    rank_arg = None
    if expert_rank is not None:
        if len(expert_rank) != plan.num_experts:
            raise ValueError("expert_rank must hold one rank per expert")
        rank_arg = ctypes.cast((ctypes.c_int32 * plan.num_experts)(*expert_rank), ctypes.c_void_p)
    rc = _native.lib().sf_combine(_ptr(rows), _ptr(index), _ptr(plan.inv_perm), rank_arg, T, K,
                                  plan.num_experts, hidden_size, int(bool(accumulate_fp32)),
                                  _ptr(out), _stream_handle(stream, out.device))
    _native.check(rc, "sf_combine")
    return out


# ------------------------------------------------------------- H2D copy ----
def copy_h2d(dst: torch.Tensor, src: torch.Tensor, stream: torch.cuda.Stream) -> None:
    """Enqueue dst <- src (pinned host) on ``stream`` (hipMemcpyAsync/SDMA)."""
    if src.device.type != "cpu" or dst.device.type != "cuda":
        raise ValueError("copy_h2d copies host memory into a device tensor")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("copy_h2d needs contiguous tensors")
    nbytes = src.numel() * src.element_size()
    if nbytes != dst.numel() * dst.element_size():
        raise ValueError("copy_h2d size mismatch")
    rec = _recorder
    if rec is not None:
        rec._copy_started(stream, nbytes)
    rc = _native.lib().sf_copy_h2d(_ptr(dst), _ptr(src), nbytes, int(stream.cuda_stream))
    _native.check(rc, "sf_copy_h2d")
    if rec is not None:
        rec._copy_ended(stream)


def stage_record(staging_ptr: int, record_ptr: int, nbytes: int,
                 stream: torch.cuda.Stream) -> None:
    """sf_copy_h2d of a coded record (page-locked host) into a device
    staging buffer, from pointers the caller has validated once (the expert
    cache's per-transfer path; ``copy_h2d`` and ``expert_decode`` are the
    checked forms)."""
    rec = _recorder
    if rec is not None:
        rec._copy_started(stream, nbytes)
    rc = _native.lib().sf_copy_h2d(staging_ptr, record_ptr, nbytes, int(stream.cuda_stream))
    _native.check(rc, "sf_copy_h2d")
    if rec is not None:
        rec._copy_ended(stream)


def decode_staged(staging_ptr: int, nbytes: int, n_values: int, table_c, counts: tuple,
                  out_ptr: int, stream: torch.cuda.Stream) -> None:
    """sf_expert_decode of a staged record into a slot, from validated
    pointers, a ctypes uint8[32] exponent table and the record's
    (n_second, n_third, n_raw)."""
    rec = _recorder
    if rec is not None:
        start, end = TimingEvent(), TimingEvent()
        start.record(stream)
    rc = _native.lib().sf_expert_decode(staging_ptr, nbytes, n_values, table_c, counts[0],
                                        counts[1], counts[2], out_ptr, int(stream.cuda_stream))
    _native.check(rc, "sf_expert_decode")
    if rec is not None:
        end.record(stream)
        rec.decodes.append((nbytes, n_values, start, end))


def expert_decode(record: torch.Tensor, counts, table: bytes, out: torch.Tensor,
                  stream: torch.cuda.Stream | None = None) -> None:
    """out (bf16, on the device) <- the values of an exponent-coded expert
    record (uint8, on the device; layout and ``counts`` = (n_second,
    n_third, n_raw) as in specfit_amd.codec)."""
    _require_cuda("record", record, torch.uint8)
    _require_cuda("out", out, _BF16)
    if record.dim() != 1 or not record.is_contiguous() or not out.is_contiguous():
        raise ValueError("expert_decode needs a contiguous 1-D record and a contiguous output")
    if len(table) != 32:
        raise ValueError("the exponent table has 32 entries")
    if len(counts) != 3:
        raise ValueError("counts are (n_second, n_third, n_raw)")
    tbl = (ctypes.c_uint8 * 32).from_buffer_copy(bytes(table))
    n2, n3, nr = (int(c) for c in counts)
    rc = _native.lib().sf_expert_decode(_ptr(record), record.numel(), out.numel(), tbl,
                                        n2, n3, nr, _ptr(out), _stream_handle(stream, out.device))
    _native.check(rc, "sf_expert_decode")


# ------------------------------------------------------------------ K5 ----
def tree_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   mask: torch.Tensor | None, scale: float, *,
                   stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Grouped-query attention of the verification forward (K5).

    query [B, Hq, Q, D], key/value [B, Hkv, S, D] bf16 (any strides with a
    unit last stride), mask [B, 1 or Hq, Q, S] bool (True = attend; the first
    head's mask is used) or None for causal attention aligned to the end of
    the keys.  Returns [B, Q, Hq, D] bf16, the layout HF attention functions
    return."""
    for name, t in (("query", query), ("key", key), ("value", value)):
        _require_cuda(name, t, _BF16)
        if t.dim() != 4 or t.stride(-1) != 1:
            raise ValueError(f"{name} must be 4-D with a unit last stride")
    B, Hq, Q, D = query.shape
    Bk, Hkv, S, Dk = key.shape
    if key.shape != value.shape or Bk != B or Dk != D:
        raise ValueError("key/value shapes do not match the query")
    if Hkv < 1 or Hq % Hkv:
        raise ValueError("query heads must be a multiple of key/value heads")
    if mask is not None:
        if mask.dtype != torch.bool:
            raise TypeError("tree attention takes a bool mask (True = attend)")
        if mask.device != query.device or mask.dim() != 4 or mask.shape[0] not in (1, B) \
                or tuple(mask.shape[2:]) != (Q, S) or mask.stride(-1) != 1:
            raise ValueError(f"mask must be bool [B, 1, {Q}, {S}] with a unit last stride")
    out = torch.empty((B, Q, Hq, D), dtype=_BF16, device=query.device)
    if B == 0 or Q == 0:
        return out
    if S == 0:
        return out.zero_()
    lib = _native.lib()
    handle = _stream_handle(stream, query.device)
    for b in range(B):
        q, k, v = query[b], key[b], value[b]
        m = None if mask is None else mask[b if mask.shape[0] == B else 0, 0]
        rc = lib.sf_tree_attention(
            q.data_ptr(), q.stride(1), q.stride(0), k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1), None if m is None else m.data_ptr(),
            0 if m is None else m.stride(0), Q, S, Hq, Hkv, D, float(scale), out[b].data_ptr(),
            handle)
        _native.check(rc, "sf_tree_attention")
    return out


# ------------------------------------------------------------------ K6 ----
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, *,
             stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """RMSNorm over the last dimension (K6): bf16(weight * bf16(x * rsqrt(
    mean(x^2) + eps))) with the mean in fp32, as Qwen3MoeRMSNorm.forward.
    ``x`` is bf16 with a unit last stride and rows at a uniform stride (a
    contiguous tensor, or a view such as [..., heads, head_dim] of one);
    returns a new contiguous tensor of x's shape."""
    _require_cuda("x", x, _BF16)
    _require_cuda("weight", weight, _BF16)
    dim = x.shape[-1]
    if weight.dim() != 1 or weight.shape[0] != dim or weight.stride(0) != 1:
        raise ValueError(f"weight must be a contiguous bf16 [{dim}] tensor")
    if x.dim() == 0:
        raise ValueError("x must have at least one dimension")
    out = torch.empty(x.shape, dtype=_BF16, device=x.device)
    rows = out.numel() // dim if dim else 0
    if rows == 0:
        return out
    flat = x.reshape(rows, dim)  # a view whenever the rows share one stride
    if flat.stride(1) != 1:
        flat = flat.contiguous()
    rc = _native.lib().sf_rms_norm(flat.data_ptr(), flat.stride(0), rows, dim, weight.data_ptr(),
                                   float(eps), out.data_ptr(), dim,
                                   _stream_handle(stream, x.device))
    _native.check(rc, "sf_rms_norm")
    return out


# ------------------------------------------------------------------ K7 ----
def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                 k_weight: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor, *,
                 stream: torch.cuda.Stream | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Query/key RMSNorm + rotary embedding of one attention layer (K7).

    q [1, T, Hq, 128] and k [1, T, Hk, 128] bf16 (the projections viewed per
    head: heads contiguous within a token, tokens at any stride that is a
    multiple of 8, such as views into one fused q/k/v projection), norm
    weights bf16 [128], cos/sin bf16 [1, T, 128] contiguous.
    Returns (q, k) as [1, Hq, T, 128] and [1, Hk, T, 128] contiguous: the
    tensors Qwen3MoeAttention.forward has after its norms, transposes and
    apply_rotary_pos_emb, with the same bits when the norms are K6's."""
    for name, t in (("q", q), ("k", k), ("q_weight", q_weight), ("k_weight", k_weight),
                    ("cos", cos), ("sin", sin)):
        _require_cuda(name, t, _BF16)
    for name, t in (("q_weight", q_weight), ("k_weight", k_weight), ("cos", cos), ("sin", sin)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if q.dim() != 4 or k.dim() != 4 or q.shape[0] != 1 or k.shape[:2] != q.shape[:2]:
        raise ValueError("q and k must be [1, tokens, heads, head_dim] with the same tokens")
    _, T, Hq, D = q.shape
    Hk = k.shape[2]
    for name, t in (("q", q), ("k", k)):
        if t.stride(3) != 1 or t.stride(2) != D or (T > 1 and t.stride(1) % 8):
            raise ValueError(f"{name} must have contiguous heads and a token stride that is a "
                             "multiple of 8")
    if k.shape[3] != D or q_weight.shape != (D,) or k_weight.shape != (D,):
        raise ValueError("head dimensions do not match")
    if cos.shape != (1, T, D) or sin.shape != (1, T, D):
        raise ValueError(f"cos and sin must be [1, {T}, {D}]")
    q_out = torch.empty((1, Hq, T, D), dtype=_BF16, device=q.device)
    k_out = torch.empty((1, Hk, T, D), dtype=_BF16, device=q.device)
    q_tok = q.stride(1) if T > 1 else Hq * D
    k_tok = k.stride(1) if T > 1 else Hk * D
    rc = _native.lib().sf_qk_norm_rope(q.data_ptr(), q_tok, k.data_ptr(), k_tok, T, Hq, Hk, D,
                                       q_weight.data_ptr(), k_weight.data_ptr(), float(eps),
                                       cos.data_ptr(), sin.data_ptr(), q_out.data_ptr(),
                                       k_out.data_ptr(), _stream_handle(stream, q.device))
    _native.check(rc, "sf_qk_norm_rope")
    return q_out, k_out

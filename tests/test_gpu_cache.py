"""GpuExpertCache semantics on the device: the known answers of the
reference's cache tests (tests/gpu/test_gpu_expert_cache.py:28-480 and
tests/gpu/test_cache_observer.py:32-260), restated for this runtime.

Pending transfers / guards are forced from the host with torch.cuda._sleep,
a bounded spin kernel, enqueued on the copy stream or a use stream.
"""
import pytest
import torch
import torch.nn.functional as F

from specfit_amd.runtime import (GpuExpertCache, NoEvictableSlotError,
                                 RecordingCacheTransitionObserver, RuntimeEventKind,
                                 aggregate_cache_transition_counters)

pytestmark = pytest.mark.gpu


def _sources(n=3):
    base = torch.arange(64 * 96, dtype=torch.float32).reshape(64, 96)
    return {e: ((base.remainder(29) - 14) / (e + 17)).to(torch.bfloat16) for e in range(n)}


def test_one_slot_survives_102_switches(device):
    sources = _sources()
    x = torch.linspace(-1, 1, 4 * 96, device=device, dtype=torch.bfloat16).reshape(4, 96)
    expected = {e: F.linear(x, s.to(device)) for e, s in sources.items()}
    cache = GpuExpertCache(sources, slot_count=1, device=device)
    assert cache.sources_are_pinned
    assert cache.copy_stream.cuda_stream != torch.cuda.default_stream(device).cuda_stream
    outs = []
    for i in range(102):
        with cache.acquire(i % 3) as lease:
            outs.append((i % 3, F.linear(x, lease.wait()).clone()))
    torch.cuda.synchronize(device)
    for e, y in outs:
        torch.testing.assert_close(y, expected[e], rtol=1.6e-2, atol=1.6e-2)
    st = cache.stats()
    assert (st.h2d_submissions, st.evictions) == (102, 101)
    assert cache.resident_expert_ids() == (2,)
    cache.close()


def test_two_acquires_join_one_inflight_copy(device):
    cache = GpuExpertCache(_sources(), slot_count=1, device=device)
    with torch.cuda.stream(cache.copy_stream):
        torch.cuda._sleep(10_000_000)
    first, second = cache.acquire(0), cache.acquire(0)
    try:
        assert cache.stats().h2d_submissions == 1
        assert cache.stats().inflight_joins == 1
        assert first.slot_id == second.slot_id
        assert first.ready_event is second.ready_event
        assert first.wait().data_ptr() == second.wait().data_ptr()
    finally:
        second.release()
        first.release()
    torch.cuda.synchronize(device)
    with cache.acquire(0) as lease:
        lease.wait()
    assert cache.stats().resident_hits == 1 and cache.stats().inflight_joins == 1
    cache.close()


def test_active_lease_blocks_eviction_and_lru_order(device):
    cache = GpuExpertCache(_sources(), slot_count=1, device=device)
    lease = cache.acquire(0)
    with pytest.raises(NoEvictableSlotError):
        cache.acquire(1)
    lease.release()
    with cache.acquire(1) as l1:
        l1.wait()
    torch.cuda.synchronize(device)
    assert cache.resident_expert_ids() == (1,)
    cache.close()

    lru = GpuExpertCache(_sources(), slot_count=2, device=device)
    for e in (0, 1, 0, 2):
        with lru.acquire(e) as l2:
            l2.wait()
    torch.cuda.synchronize(device)
    assert lru.resident_expert_ids() == (0, 2)
    assert lru.stats().evictions == 1
    lru.close()


def test_completed_hits_leave_no_pending_guards(device):
    cache = GpuExpertCache(_sources(), slot_count=1, device=device)
    ones = torch.ones(1, 96, dtype=torch.bfloat16, device=device)
    for _ in range(64):
        with cache.acquire(0) as lease:
            F.linear(ones, lease.wait())
    torch.cuda.synchronize(device)
    assert cache.stats().pending_use_guards == 0
    cache.close()


def test_snapshot_tracks_cold_pending_resident_and_eviction(device):
    cache = GpuExpertCache(_sources(), slot_count=1, device=device, cache_id="test-layer-0")
    cold = cache.snapshot()
    assert (cold.cache_id, cold.queue_id, cold.capacity) == ("test-layer-0", "test-layer-0-copy", 1)
    assert (cold.host_state_version, cold.lru_sequence, cold.submission_sequence) == (0, 0, 0)
    assert cold.pending_transfers == () and cold.slots[0].expert_id is None
    with torch.cuda.stream(cache.copy_stream):
        torch.cuda._sleep(10_000_000)
    first, second = cache.acquire(0), cache.acquire(0)
    pending = cache.snapshot()
    assert pending.slots[0].expert_id == 0 and pending.slots[0].active_leases == 2
    assert len(pending.pending_transfers) == 1
    t = pending.pending_transfers[0]
    assert (t.expert_id, t.slot_id, t.generation, t.submission_sequence) == (0, 0, 1, 0)
    assert t.ready_event is first.ready_event
    assert pending.slots[0].ready == t.ready_event_completed
    assert (pending.stats.h2d_submissions, pending.stats.inflight_joins) == (1, 1)
    again = cache.snapshot()
    assert again.host_state_version == pending.host_state_version
    assert again.lru_sequence == pending.lru_sequence and again.submission_sequence == 1
    second.release()
    first.release()
    torch.cuda.synchronize(device)
    with cache.acquire(0) as lease:
        lease.wait()
    torch.cuda.synchronize(device)
    res = cache.snapshot()
    assert res.pending_transfers == () and res.slots[0].ready and res.stats.resident_hits == 1
    with cache.acquire(1) as lease:
        lease.wait()
    torch.cuda.synchronize(device)
    ev = cache.snapshot()
    assert (ev.slots[0].expert_id, ev.slots[0].generation, ev.submission_sequence,
            ev.stats.evictions) == (1, 2, 2, 1)
    cache.close()


def test_cold_reset_requires_quiescence(device):
    cache = GpuExpertCache(_sources(), slot_count=1, device=device, cache_id="reset-layer")
    with torch.cuda.stream(cache.copy_stream):
        torch.cuda._sleep(10_000_000)
    lease = cache.acquire(0)
    with pytest.raises(RuntimeError, match="active lease"):
        cache.cold_reset()
    lease.release()
    with pytest.raises(RuntimeError, match="CUDA synchronization"):
        cache.cold_reset()
    torch.cuda.synchronize(device)
    cache.cold_reset()
    cold = cache.snapshot()
    assert (cold.host_state_version, cold.lru_sequence, cold.submission_sequence) == (0, 0, 0)
    assert cold.slots[0].expert_id is None and cold.slots[0].generation == 0
    with cache.acquire(0) as fresh:
        fresh.wait()
    after = cache.snapshot()
    assert (after.slots[0].generation, after.submission_sequence, after.stats.h2d_submissions) == (1, 1, 1)
    torch.cuda.synchronize(device)
    cache.close()


def test_reused_slot_submission_queue(device):
    cache = GpuExpertCache(_sources(), slot_count=1, device=device, cache_id="queue-layer")
    with torch.cuda.stream(cache.copy_stream):
        torch.cuda._sleep(10_000_000)
    for e in (0, 1, 0):
        cache.acquire(e).release()
    q = cache.snapshot()
    assert tuple(t.submission_sequence for t in q.pending_transfers) == (0, 1, 2)
    assert tuple(t.expert_id for t in q.pending_transfers) == (0, 1, 0)
    assert tuple(t.generation for t in q.pending_transfers) == (1, 2, 3)
    assert (q.slots[0].expert_id, q.slots[0].generation, q.stats.h2d_submissions,
            q.stats.evictions) == (0, 3, 3, 2)
    torch.cuda.synchronize(device)
    with cache.acquire(0) as lease:
        lease.wait()
    torch.cuda.synchronize(device)
    r = cache.snapshot()
    assert r.pending_transfers == () and r.stats.resident_hits == 1 and r.slots[0].generation == 3
    cache.close()


def test_use_guard_observed_without_reaping(device):
    cache = GpuExpertCache(_sources(), slot_count=1, device=device, cache_id="guard-layer")
    torch.cuda.synchronize(device)
    use = torch.cuda.Stream(device=device)
    lease = cache.acquire(0)
    with torch.cuda.stream(use):
        lease.wait(use)
        torch.cuda._sleep(10_000_000)
    lease.release()
    g1, g2 = cache.snapshot(), cache.snapshot()
    assert g1.slots[0].pending_use_guards == 1 and g1.stats.pending_use_guards == 1
    assert g2.slots[0].pending_use_guards == 1 and g2.host_state_version == g1.host_state_version
    with pytest.raises(RuntimeError, match="CUDA synchronization"):
        cache.cold_reset()
    torch.cuda.synchronize(device)
    done = cache.snapshot()
    assert done.slots[0].pending_use_guards == 0 and done.host_state_version == g1.host_state_version
    cache.cold_reset()
    cache.close()


def test_cold_reset_replays_the_same_lru_state(device):
    cache = GpuExpertCache(_sources(), slot_count=2, device=device, cache_id="replay-layer")

    def run():
        for e in (0, 1, 0, 2):
            with cache.acquire(e) as lease:
                lease.wait()
        torch.cuda.synchronize(device)
        s = cache.snapshot()
        return (tuple((x.slot_id, x.expert_id, x.generation, x.last_used_sequence) for x in s.slots),
                s.lru_sequence, s.submission_sequence, s.stats)

    first = run()
    cache.cold_reset()
    assert run() == first
    # Same final state as the CPU LRU restatement of the access sequence.
    from oracle.lru import LayerLRU
    ref = LayerLRU(2)
    for e in (0, 1, 0, 2):
        ref.access(e)
    assert first[0] == ref.state() and first[1] == ref.lru_sequence
    cache.close()


def test_close_rejects_active_lease_and_closes_owner(device):
    class Owner:
        calls = 0
        ready = None

        def close(self):
            assert self.ready is not None and self.ready.query()
            Owner.calls += 1

    owner = Owner()
    sources = {e: s.pin_memory() for e, s in _sources().items()}
    cache = GpuExpertCache(sources, slot_count=1, device=device, adopt_pinned_sources=True,
                           source_owner=owner)
    with torch.cuda.stream(cache.copy_stream):
        torch.cuda._sleep(10_000_000)
    lease = cache.acquire(0)
    owner.ready = lease.ready_event
    with pytest.raises(RuntimeError, match="active lease"):
        cache.close()
    assert not cache.closed and Owner.calls == 0
    lease.release()
    cache.close()
    cache.close()
    assert cache.closed and Owner.calls == 1
    with pytest.raises(RuntimeError, match="closed"):
        cache.acquire(0)


def test_adopt_unpinned_sources_copies(device):
    sources = _sources()
    cache = GpuExpertCache(sources, slot_count=1, device=device, adopt_pinned_sources=True)
    assert cache.sources_are_pinned
    with cache.acquire(0) as lease:
        assert torch.equal(lease.wait().cpu(), sources[0])
    cache.close()


def test_observer_known_sequence(device):
    obs = RecordingCacheTransitionObserver(run_id="run-0")
    src = {e: torch.full((32, 32), float(e + 1), dtype=torch.bfloat16) for e in range(3)}
    cache = GpuExpertCache(src, slot_count=1, device=device, cache_id="layer-0",
                           queue_id="layer-0-copy", observer=obs)
    with torch.cuda.stream(cache.copy_stream):
        torch.cuda._sleep(10_000_000)
    first, second = cache.acquire(0), cache.acquire(0)
    first.wait()
    second.wait()
    second.release()
    first.release()
    torch.cuda.synchronize(device)
    with cache.acquire(0) as lease:
        lease.wait()
    with cache.acquire(1) as lease:
        lease.wait()
    torch.cuda.synchronize(device)
    events = obs.events()
    K = RuntimeEventKind
    assert tuple(e.kind for e in events) == (
        K.H2D_SUBMIT, K.INFLIGHT_JOIN, K.CONSUME_WAIT, K.CONSUME_WAIT, K.RELEASE, K.RELEASE,
        K.RESIDENT_HIT, K.CONSUME_WAIT, K.RELEASE, K.EVICT, K.H2D_SUBMIT, K.CONSUME_WAIT,
        K.RELEASE)
    assert tuple(e.sequence for e in events) == tuple(range(len(events)))
    assert [e.submission_sequence for e in events if e.kind is K.H2D_SUBMIT] == [0, 1]
    evict = next(e for e in events if e.kind is K.EVICT)
    assert (evict.victim_expert_id, evict.expert_id) == (0, 1)
    counted = aggregate_cache_transition_counters(events)
    st = cache.stats()
    assert (counted.h2d_submissions, counted.resident_hits, counted.inflight_joins,
            counted.evictions) == (st.h2d_submissions, st.resident_hits, st.inflight_joins,
                                   st.evictions)
    cache.close()


def test_checkpoint_capture_restore_roundtrip(device):
    cache = GpuExpertCache(_sources(), slot_count=2, device=device)
    for e in (0, 1):
        with cache.acquire(e) as lease:
            lease.wait()
    torch.cuda.synchronize(device)
    cache.resident_expert_ids()
    before = cache.snapshot()
    ckpt = cache._capture_checkpoint()
    with cache.acquire(2) as lease:
        lease.wait()
    torch.cuda.synchronize(device)
    info = cache._restore_checkpoint(ckpt)
    assert info["weights_pinned"]
    after = cache.snapshot()
    assert [(s.expert_id, s.generation, s.last_used_sequence) for s in after.slots] == \
        [(s.expert_id, s.generation, s.last_used_sequence) for s in before.slots]
    with cache.acquire(1) as lease:
        assert torch.equal(lease.wait().cpu(), _sources()[1])
    cache.close()

"""Logical replay of the expert caches on the host.

Known answer: the reference's replay fixture
(tests/unit/test_logical_replay.py:288-316, 446-509): a 2-slot layer holding
expert 0 (generation 1, last used 4, LRU sequence 4, one H2D so far)
replays accesses (0, 1, 2) to slots ((0, 0, 2, 2, 10), (0, 1, 1, 1, 8)) with
2 H2D, 1 hit, 1 eviction, 3 waits, 3 releases (10 events) and occupancy
1 -> 2.  Random sequences are checked against the oracle's LRU
(oracle/lru.py, itself pinned by the reference's replay known answers).
"""
import random

import pytest

from oracle.lru import LayerLRU
from specfit_amd.runtime import ExpertKey
from specfit_amd.runtime.cache_snapshot import CacheSlotSnapshot, GpuExpertCacheSnapshot
from specfit_amd.runtime.lease import ExpertCacheStats
from specfit_amd.runtime.replay import (LogicalReplayError, ReplayCounters,
                                        replay_qwen3_access_cycles, replay_qwen3_accesses)
from specfit_amd.runtime.trace import RuntimeEventKind


def _snapshot(slots, lru, submission, h2d=0, hits=0, evictions=0, layer=0):
    return GpuExpertCacheSnapshot(
        cache_id=f"layer-{layer}", queue_id=f"layer-{layer}-copy", capacity=len(slots),
        host_state_version=lru, lru_sequence=lru, submission_sequence=submission,
        slots=tuple(CacheSlotSnapshot(slot_id=i, expert_id=e, generation=g, active_leases=a,
                                      last_used_sequence=u, ready=e is not None,
                                      pending_use_guards=0)
                    for i, (e, g, a, u) in enumerate(slots)),
        pending_transfers=(),
        stats=ExpertCacheStats(h2d_submissions=h2d, resident_hits=hits, inflight_joins=0,
                               evictions=evictions, pending_use_guards=0))


def test_reference_fixture_known_answer():
    before = _snapshot([(ExpertKey(0, 0), 1, 0, 4), (None, 0, 0, 0)], lru=4, submission=1, h2d=1)
    r = replay_qwen3_accesses((before,), ((0, 1, 2),))
    assert r.counters == ReplayCounters(h2d_submissions=2, resident_hits=1, inflight_joins=0,
                                         evictions=1, consume_waits=3, releases=3)
    assert r.counters.acquisitions == 3 and r.counters.event_count == 10 == len(r.events)
    assert (r.initial_occupancy, r.final_occupancy) == (1, 2)
    assert tuple((s.layer_id, s.slot_id, s.expert_id, s.generation, s.last_used_sequence)
                 for s in r.final_slots) == ((0, 0, 2, 2, 10), (0, 1, 1, 1, 8))
    assert r.final_lru_sequences == (10,) and r.final_submission_sequences == (3,)
    accesses = [e.expert_id for e in r.events if e.kind in (
        RuntimeEventKind.H2D_SUBMIT, RuntimeEventKind.RESIDENT_HIT, RuntimeEventKind.INFLIGHT_JOIN)]
    assert accesses == [0, 1, 2]
    evict = [e for e in r.events if e.kind is RuntimeEventKind.EVICT]
    assert len(evict) == 1 and evict[0].victim_expert_id == 0 and evict[0].expert_id == 2
    assert r.initial_resident_reload_h2d == 0


def test_boundary_and_input_validation():
    busy = _snapshot([(0, 1, 1, 4), (None, 0, 0, 0)], lru=4, submission=1, h2d=1)
    with pytest.raises(LogicalReplayError, match="active lease"):
        replay_qwen3_accesses((busy,), ((0,),))
    ok = _snapshot([(0, 1, 0, 4), (None, 0, 0, 0)], lru=4, submission=1, h2d=1)
    for bad in (((1, 0),), ((0, 0),), ((-1,),), ((True,),)):
        with pytest.raises(LogicalReplayError, match="ascending"):
            replay_qwen3_accesses((ok,), bad)
    with pytest.raises(LogicalReplayError, match="layer count"):
        replay_qwen3_accesses((ok,), ((0,), (1,)))
    with pytest.raises(LogicalReplayError, match="must not be empty"):
        replay_qwen3_access_cycles((ok,), ())


def test_resident_first_runs_residents_before_misses():
    before = _snapshot([(5, 1, 0, 2), (9, 1, 0, 3)], lru=3, submission=2, h2d=2)
    r = replay_qwen3_access_cycles((before,), (((1, 5, 9),),), resident_first=True)[0]
    order = [e.expert_id for e in r.events if e.kind in (RuntimeEventKind.H2D_SUBMIT,
                                                         RuntimeEventKind.RESIDENT_HIT)]
    assert order == [5, 9, 1]
    # expert 1 then evicts the older of the two just-touched residents (5)
    evict = next(e for e in r.events if e.kind is RuntimeEventKind.EVICT)
    assert evict.victim_expert_id == 5


@pytest.mark.parametrize("seed", range(8))
def test_random_cycles_match_the_oracle_lru(seed):
    rng = random.Random(seed)
    slots = rng.randint(1, 6)
    E = 12
    lrus = [LayerLRU(slots) for _ in range(2)]
    before = tuple(_snapshot([(None, 0, 0, 0)] * slots, lru=0, submission=0, layer=l)
                   for l in range(2))
    cycles = tuple(tuple(tuple(sorted(rng.sample(range(E), rng.randint(0, 7)))) for _ in range(2))
                   for _ in range(5))
    results = replay_qwen3_access_cycles(before, cycles)
    for cycle, result in zip(cycles, results):
        h2d = 0
        for l, experts in enumerate(cycle):
            for e in experts:
                h2d += int(lrus[l].access(e) != "hit")
        assert result.counters.h2d_submissions == h2d
        got = [[(s.expert_id, s.generation, s.last_used_sequence) for s in result.final_slots
                if s.layer_id == l] for l in range(2)]
        want = [[(s.expert_id, s.generation, s.last_used_sequence) for s in lru.slots]
                for lru in lrus]
        assert got == want

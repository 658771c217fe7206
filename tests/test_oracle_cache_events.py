"""Pins the cache-event replayer (oracle/cache_events.py) on hand-built
event sequences: known post-states for the demand, one-ahead and scheduler
touch rules, and each inconsistency it must reject."""
import pytest

from oracle.cache_events import replay_events


def _pre(slots=2, layers=1):
    return dict(layers=[dict(layer_id=l, capacity=slots, lru_sequence=0, submission_sequence=0,
                             counters=dict(h2d_submissions=0, resident_hits=0, inflight_joins=0,
                                           evictions=0, pending_use_guards=0),
                             slots=[dict(slot_id=s, expert_id=None, generation=0,
                                         active_leases=0, last_used_sequence=0, ready=False,
                                         pending_use_guards=0) for s in range(slots)])
                        for l in range(layers)])


def _use(expert, slot, gen, *, sub=None, victim=None, join=False, hit=False):
    """Events of one expert use: (evict), submit / hit / join, wait, release."""
    out = []
    if victim is not None:
        out.append(("evict", 0, expert, slot, gen, None, victim))
    kind = "resident_hit" if hit else "inflight_join" if join else "h2d_submit"
    out.append((kind, 0, expert, slot, gen, sub, None))
    out.append(("consume_wait", 0, expert, slot, gen, None, None))
    out.append(("release", 0, expert, slot, gen, None, None))
    return out




def test_demand_and_one_ahead_touch_rules():
    events = _use(3, 0, 1, sub=0) + _use(5, 1, 1, sub=1) + _use(7, 0, 2, sub=2, victim=3)
    post = replay_events(_pre(), events, {(0, 3), (0, 5), (0, 7)}, "demand")
    layer = post["layers"][0]
    assert [(s["expert_id"], s["generation"], s["last_used_sequence"]) for s in layer["slots"]] \
        == [(7, 2, 6), (5, 1, 4)]
    assert layer["lru_sequence"] == 6 and layer["submission_sequence"] == 3
    assert layer["counters"] == dict(h2d_submissions=3, resident_hits=0, inflight_joins=0,
                                     evictions=1, pending_use_guards=0)
    # one-ahead: the first lease touches at once, the later ones at their wait
    post = replay_events(_pre(), events, {(0, 3), (0, 5), (0, 7)}, "one_ahead")
    assert post["layers"][0]["lru_sequence"] == 6
    interleaved = [("h2d_submit", 0, 3, 0, 1, 0, None), ("h2d_submit", 0, 5, 1, 1, 1, None),
                   ("consume_wait", 0, 3, 0, 1, None, None), ("release", 0, 3, 0, 1, None, None),
                   ("consume_wait", 0, 5, 1, 1, None, None), ("release", 0, 5, 1, 1, None, None)]
    post = replay_events(_pre(), interleaved, {(0, 3), (0, 5)}, "one_ahead")
    # touches: acquire 3 (1), release 3 (2), wait 5 (3), release 5 (4)
    assert [s["last_used_sequence"] for s in post["layers"][0]["slots"]] == [2, 4]
    post = replay_events(_pre(), interleaved, {(0, 3), (0, 5)}, "ready_demand")
    # every lease deferred: wait 3 (1), release 3 (2), wait 5 (3), release 5 (4)
    assert [s["last_used_sequence"] for s in post["layers"][0]["slots"]] == [2, 4]
    post = replay_events(_pre(), interleaved, {(0, 3), (0, 5)}, "demand")
    # immediate touches: acquire 3, acquire 5, release 3 (3), release 5 (4)
    assert [s["last_used_sequence"] for s in post["layers"][0]["slots"]] == [3, 4]


@pytest.mark.parametrize("events,actual,variant,message", [
    ([("resident_hit", 0, 3, 0, 5, None, None)], set(), "demand", "stale"),
    (_use(3, 0, 1, sub=0)[:1] + [("release", 0, 3, 0, 1, None, None)] * 2, {(0, 3)}, "demand",
     "release without a live lease"),
    (_use(3, 0, 1, sub=0), {(0, 4)}, "demand", "non-router expert"),
    (_use(3, 0, 1, sub=1), {(0, 3)}, "demand", "invalid copy"),
    (_use(3, 0, 2, sub=0), {(0, 3)}, "demand", "invalid copy"),
    (_use(3, 0, 1, sub=0)[:2] + [("evict", 0, 5, 0, 2, None, 3)], {(0, 3)}, "demand",
     "leased victim"),
    (_use(3, 0, 1, sub=0)[:1], {(0, 3)}, "demand", "incomplete"),
    ([("bogus", 0, 3, 0, 1, None, None)], set(), "demand", "unknown cache event"),
    (_use(3, 0, 1, sub=0), {(0, 3)}, "nope", "unknown runtime variant"),
])
def test_inconsistent_decisions_are_rejected(events, actual, variant, message):
    with pytest.raises(ValueError, match=message):
        replay_events(_pre(), events, actual, variant)


def test_accurate_prediction_must_not_evict_an_unconsumed_routed_expert():
    # routed {3, 5} fit in 2 of 3 slots: the layer is accurate; evicting 3
    # before it was consumed is a wrong speculative decision
    events = [("h2d_submit", 0, 3, 0, 1, 0, None), ("release", 0, 3, 0, 1, None, None),
              ("evict", 0, 9, 0, 2, None, 3)]
    with pytest.raises(ValueError, match="accurate prefetch"):
        replay_events(_pre(slots=3), events, {(0, 3), (0, 5)}, "predicted_same_layer")


def test_logical_state_reads_snapshots_into_the_replay_format():
    """A two-slot snapshot (one slot empty, one holding expert 3 of layer 0)
    becomes the state dict the replay consumes, and an empty snapshot is
    exactly the hand-built pre-state above."""
    from oracle.cache_events import logical_state
    from specfit_amd.runtime import (CacheSlotSnapshot, ExpertCacheStats, ExpertKey,
                                     GpuExpertCacheSnapshot)

    def snap(slots, **seq):
        return GpuExpertCacheSnapshot(
            cache_id="qwen3-layer-0", queue_id="layer-0-copy", capacity=len(slots),
            host_state_version=0, slots=tuple(slots), pending_transfers=(),
            stats=ExpertCacheStats(h2d_submissions=seq.get("sub", 0), resident_hits=0,
                                   inflight_joins=0, evictions=0, pending_use_guards=0),
            lru_sequence=seq.get("lru", 0), submission_sequence=seq.get("sub", 0))

    empty = [CacheSlotSnapshot(slot_id=s, expert_id=None, generation=0, active_leases=0,
                               last_used_sequence=0, ready=False, pending_use_guards=0)
             for s in range(2)]
    assert logical_state([snap(empty)]) == _pre()
    held = CacheSlotSnapshot(slot_id=1, expert_id=ExpertKey(0, 3), generation=1,
                             active_leases=0, last_used_sequence=2, ready=True,
                             pending_use_guards=0)
    state = logical_state([snap([empty[0], held], lru=2, sub=1)])
    layer = state["layers"][0]
    assert layer["slots"][1] == dict(slot_id=1, expert_id=3, generation=1, active_leases=0,
                                     last_used_sequence=2, ready=True, pending_use_guards=0)
    assert (layer["lru_sequence"], layer["submission_sequence"]) == (2, 1)
    assert layer["counters"]["h2d_submissions"] == 1
    # the replay continues from it: evict 3, copy 7 into slot 1
    events = [("evict", 0, 7, 1, 2, None, 3), ("h2d_submit", 0, 7, 1, 2, 1, None),
              ("consume_wait", 0, 7, 1, 2, None, None), ("release", 0, 7, 1, 2, None, None)]
    post = replay_events(state, events, {(0, 7)}, "demand")
    assert post["layers"][0]["slots"][1]["expert_id"] == 7
    assert post["layers"][0]["counters"]["evictions"] == 1

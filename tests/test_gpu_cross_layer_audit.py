"""Cross-layer prefetch audit on the device.

For every runtime variant (``oracle.cache_events.VARIANTS``: demand,
one-ahead, the ready-first scheduler without predictions, predicted
same-layer and cross-layer, wrong cross-layer predictions), slot count and
starting state, one forward of the toy target (tests/_toy_target.py) runs
with a compact observer on every layer cache.  The recorded transitions,
replayed by the oracle's independent restatement of the reference's audit
(src/specfit/cross_layer_prefetch.py:49-142) from the caches' logical state
before the forward, must give exactly their logical state after it: slots,
generations, LRU and submission sequences and counters.  The variants and
the predictions they run with are the reference audit's
(tests/gpu/test_cross_layer_prefetch_audit.py).
"""
from __future__ import annotations

from contextlib import nullcontext

import pytest
import torch

from _toy_target import ROUTES, toy_case
from oracle.cache_events import VARIANTS, CompactTransitions, logical_state, replay_events

pytestmark = pytest.mark.gpu

LAYERS = 2
ROUTED = sorted({e for row in ROUTES for e in row})  # experts 0..4; 5 is never routed

# variant -> (one-ahead H2D prefetch, scheduler predictions or None, lookahead)
HOW = {
    "demand": (False, None, 0),
    "one_ahead": (True, None, 0),
    "ready_demand": (False, {}, 0),
    "predicted_same_layer": (False, dict.fromkeys(range(LAYERS), ROUTED), 0),
    "predicted_cross_layer": (False, dict.fromkeys(range(LAYERS), ROUTED), 1),
    "wrong_cross_layer": (False, dict.fromkeys(range(LAYERS), [5]), 1),
}


def test_every_variant_has_a_way_to_run():
    assert set(HOW) == set(VARIANTS)


def _audited_forward(case, variant: str):
    """(logical state before, transitions, logical state after) of one
    forward run the way ``variant`` runs it."""
    one_ahead, predictions, lookahead = HOW[variant]
    before = logical_state(case.loaded.cache_snapshots())
    recorder = CompactTransitions()
    for cache in case.caches:
        cache._observer = recorder
    try:
        case.loaded.set_expert_h2d_prefetch(one_ahead)
        scheduling = (nullcontext() if predictions is None else
                      case.loaded.prefetch_experts(predictions, lookahead_layers=lookahead))
        with torch.inference_mode(), scheduling:
            case.forward()
        torch.cuda.synchronize()
    finally:
        for cache in case.caches:
            cache._observer = None
    return before, recorder.events, logical_state(case.loaded.cache_snapshots())


@pytest.mark.parametrize("start", ["cold", "two_resident"])
@pytest.mark.parametrize("slots", [2, 6])
@pytest.mark.parametrize("variant", VARIANTS)
def test_recorded_transitions_replay_to_the_live_caches(device, variant, slots, start):
    case = toy_case(slots=slots, layers=LAYERS)
    try:
        case.loaded.cold_reset_expert_caches()
        if start == "two_resident":
            case.make_resident((0, 5))  # one routed expert and one never routed
        torch.cuda.synchronize()
        before, events, after = _audited_forward(case, variant)
        print(f"audit {variant} slots={slots} {start}: {len(events)} transitions", flush=True)
        routed = {(lid, e) for lid in range(LAYERS) for e in ROUTED}
        assert replay_events(before, events, routed, variant) == after
    finally:
        case.close()

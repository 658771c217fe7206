"""Cross-layer prefetch audit on the device (the reference's
tests/gpu/test_cross_layer_prefetch_audit.py restated): for each runtime
variant -- demand, one-ahead, the ready-first scheduler without predictions,
predicted same-layer and cross-layer, and wrong cross-layer predictions --
from a cold and from a partly filled cache, the cache transitions the live
caches record must replay (oracle/cache_events.py, an independent
restatement of the reference's audit) to exactly the caches' final logical
state: slots, generations, LRU and submission sequences and counters."""
from contextlib import nullcontext
from dataclasses import asdict

import pytest
import torch

from oracle.cache_events import VARIANTS, CompactTransitions, replay_events
from specfit_amd.runtime import ExpertKey
from test_gpu_prefetch_model import _case, _close

pytestmark = pytest.mark.gpu


def _logical(caches):
    layers = []
    for lid, cache in enumerate(caches):
        snap = cache.snapshot()
        slots = []
        for s in snap.slots:
            row = asdict(s)
            row["expert_id"] = None if s.expert_id is None else s.expert_id.expert_id
            slots.append(row)
        layers.append(dict(layer_id=lid, capacity=snap.capacity, lru_sequence=snap.lru_sequence,
                           submission_sequence=snap.submission_sequence,
                           counters=asdict(snap.stats), slots=slots))
    return dict(layers=layers)


@pytest.mark.parametrize("slots", [2, 6])
def test_observed_events_reconstruct_the_live_caches_for_all_variants(device, slots):
    loaded, _, inputs = _case(slots=slots)
    try:
        for variant in VARIANTS:
            for natural in (False, True):
                loaded.cold_reset_expert_caches()
                if natural:
                    for lid, cache in enumerate(loaded.expert_caches):
                        for e in (0, 5):
                            with cache.acquire(ExpertKey(lid, e)) as lease:
                                lease.wait()
                torch.cuda.synchronize()
                pre = _logical(loaded.expert_caches)
                observer = CompactTransitions()
                for cache in loaded.expert_caches:
                    cache._observer = observer
                loaded.set_expert_h2d_prefetch(variant == "one_ahead")
                if variant == "ready_demand":
                    predictions = {}
                elif variant == "wrong_cross_layer":
                    predictions = {lid: [5] for lid in range(2)}
                else:
                    predictions = {lid: list(range(5)) for lid in range(2)}
                if variant in VARIANTS[:2]:
                    context = nullcontext()
                else:
                    context = loaded.prefetch_experts(
                        predictions, lookahead_layers=int(variant in VARIANTS[4:]))
                with torch.inference_mode(), context:
                    loaded.model(*inputs)
                torch.cuda.synchronize()
                for cache in loaded.expert_caches:
                    cache._observer = None
                actual = {(lid, e) for lid in range(2) for e in range(5)}
                post = _logical(loaded.expert_caches)
                print(f"audit slots={slots} {variant} natural={natural}: "
                      f"{len(observer.events)} transitions", flush=True)
                assert replay_events(pre, observer.events, actual, variant) == post, \
                    (slots, variant, natural)
    finally:
        for cache in loaded.expert_caches:
            cache._observer = None
        _close(loaded)

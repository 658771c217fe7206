"""Logical replay vs the live expert caches on the device.

The replay (src/specfit/replay.py:217-455 restated) must predict the
runtime's cache state exactly: for random routings through a small
offloaded layer stack (one-ahead prefetch off, so every access is the
acquire -> wait -> release sequence the replay models), the replayed final
slots, LRU and submission sequences and counter deltas equal the live
snapshots after the forward, for both execution policies.
"""
import pytest
import torch

from specfit_amd.runtime import (ExpertKey, GpuExpertCache, Qwen3OffloadedExperts)
from specfit_amd.runtime.replay import replay_qwen3_access_cycles

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("policy", ["expert_id_ascending", "resident_first"])
@pytest.mark.parametrize("slots", [1, 3, 5])
def test_replay_predicts_live_cache_state(device, policy, slots):
    g = torch.Generator().manual_seed(slots * 7 + len(policy))
    E, H, I, K, L = 8, 32, 16, 2, 2
    caches, layers = [], []
    for lid in range(L):
        sources = {ExpertKey(lid, e): (torch.randn(3 * I * H, generator=g) / 8).to(torch.bfloat16)
                   for e in range(E)}
        cache = GpuExpertCache(sources, slot_count=slots, device=device,
                               cache_id=f"layer-{lid}", queue_id=f"layer-{lid}-copy")
        caches.append(cache)
        layers.append(Qwen3OffloadedExperts(layer_id=lid, cache=cache, hidden_size=H,
                                            intermediate_size=I, execution_policy=policy,
                                            h2d_prefetch=False))
    for step in range(6):
        T = int(torch.randint(1, 6, (1,), generator=g))
        routes = [torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
                  for _ in range(L)]
        torch.cuda.synchronize()
        before = tuple(c.snapshot() for c in caches)
        accessed = tuple(tuple(sorted(set(r.flatten().tolist()))) for r in routes)
        predicted = replay_qwen3_access_cycles(before, (accessed,),
                                               resident_first=policy == "resident_first")[0]
        h = (torch.randn(T, H, generator=g)).to(torch.bfloat16).to(device)
        for layer, r in zip(layers, routes):
            w = torch.full((T, K), 0.5, dtype=torch.bfloat16, device=device)
            h = layer(h, r.to(device), w)
        torch.cuda.synchronize()
        after = tuple(c.snapshot() for c in caches)
        live_slots = tuple((lid, s.slot_id, None if s.expert_id is None else s.expert_id.expert_id,
                            s.generation, s.last_used_sequence)
                           for lid, snap in enumerate(after) for s in snap.slots)
        replay_slots = tuple((s.layer_id, s.slot_id, s.expert_id, s.generation,
                              s.last_used_sequence) for s in predicted.final_slots)
        assert replay_slots == live_slots, (step, policy, slots)
        assert predicted.final_lru_sequences == tuple(s.lru_sequence for s in after)
        assert predicted.final_submission_sequences == tuple(s.submission_sequence for s in after)
        for field in ("h2d_submissions", "resident_hits", "evictions"):
            live = sum(getattr(a.stats, field) - getattr(b.stats, field)
                       for a, b in zip(after, before))
            assert getattr(predicted.counters, field) == live, field
    for c in caches:
        c.close()

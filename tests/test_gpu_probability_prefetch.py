"""Probability-scored speculation and eviction of the prefetch scheduler.

Restates the reference's tests
(tests/gpu/test_qwen3_probability_prefetch.py:28-193) for this runtime:
probabilities rank and cap a layer's predictions; with
``eviction_policy="probability"`` a speculative copy replaces the writable,
unleased victim of lowest predicted probability (and none of equal or higher
probability, while routed demand still progresses); invalid scores fail
before any cache changes; the scored context snapshots its inputs; real
Qwen3 logits are unchanged by scheduling.  The victim rule restated is
src/specfit/runtime/gpu_expert_cache.py:520-541.
"""
from __future__ import annotations

import tempfile
from contextlib import ExitStack
from fractions import Fraction
from types import MappingProxyType

import pytest
import torch

from specfit_amd.runtime import ExpertKey, RuntimeEventKind, load_offloaded_qwen3
from test_gpu_prefetch_model import (_assert_restored, _case, _close,
                                     _save_qwen3_style_checkpoint, _tiny_config)

pytestmark = pytest.mark.gpu


def _fill(cache, experts):
    for e in experts:
        with cache.acquire(ExpertKey(0, e)) as lease:
            lease.wait()
    torch.cuda.synchronize()


def test_probabilities_rank_and_limit_attention_prefetch_for_both_policies(device):
    loaded, _, inputs = _case(slots=3, layers=1)
    expected = loaded.model(*inputs)
    for policy in ("lru", "probability"):
        loaded.cold_reset_expert_caches()
        with loaded.prefetch_experts({0: (0, 1, 2, 3, 4)},
                                     prediction_probabilities={0: {0: .7, 1: .8, 2: 0., 3: .1,
                                                                   4: .9}},
                                     eviction_policy=policy, lookahead_layers=0,
                                     trace=True) as sched:
            copies = [row["expert_id"] for row in sched.events() if row["action"] == "copy"]
            assert copies == [4, 1], policy  # highest first, capped at slots - 1
            actual = loaded.model(*inputs)
        torch.cuda.synchronize()
        assert torch.equal(actual, expected)
        assert sched.stats()["layers"][0]["predicted_experts"] == 2
        assert sched.stats()["peak_inflight"] <= 2
    _close(loaded)


def test_probability_eviction_chooses_lower_probability_instead_of_lru(device):
    loaded, observer, inputs = _case(slots=3, layers=1)
    cache = loaded.expert_caches[0]
    expected = loaded.model(*inputs)
    for policy, victim in (("lru", 0), ("probability", 1)):
        loaded.cold_reset_expert_caches()
        _fill(cache, (0, 1, 2))
        begin = len(observer.events())
        with loaded.prefetch_experts({0: (4,)},
                                     prediction_probabilities={0: {0: .6, 1: .1, 2: .4, 4: .9}},
                                     eviction_policy=policy, lookahead_layers=0):
            evicted = [e.victim_expert_id.expert_id for e in observer.events()[begin:]
                       if e.kind is RuntimeEventKind.EVICT]
            assert evicted == [victim], policy
            actual = loaded.model(*inputs)
        torch.cuda.synchronize()
        assert torch.equal(actual, expected)
    _close(loaded)


def test_equal_or_lower_probability_skips_speculation_but_real_demand_progresses(device):
    loaded, _, inputs = _case(slots=3, layers=1)
    cache = loaded.expert_caches[0]
    expected = loaded.model(*inputs)
    for incoming in (.5, .4):
        loaded.cold_reset_expert_caches()
        _fill(cache, (0, 1, 2))
        before = cache.stats().h2d_submissions
        streams = (cache.copy_stream,)
        with loaded.prefetch_experts({0: (4,)},
                                     prediction_probabilities={0: {0: .8, 1: .6, 2: .5,
                                                                   4: incoming}},
                                     eviction_policy="probability", lookahead_layers=0) as sched:
            assert cache.stats().h2d_submissions == before  # no victim of lower probability
            actual = loaded.model(*inputs)
        _assert_restored(loaded, streams)
        assert torch.equal(actual, expected)
        row = sched.stats()["layers"][0]
        assert row["prediction_copies"] == 0 and row["demand_copies"] == 2, incoming
    _close(loaded)


@pytest.mark.parametrize("protected", ["leased", "busy"])
def test_probability_eviction_skips_busy_and_leased_victims(device, protected):
    loaded, _, _ = _case(slots=3, layers=1)
    cache = loaded.expert_caches[0]
    probabilities = {ExpertKey(0, e): p for e, p in ((0, .2), (1, .1), (2, .3), (4, .9))}
    _fill(cache, (0, 1, 2))
    use_stream = torch.cuda.Stream()
    held = cache.acquire(ExpertKey(0, 1))
    try:
        with torch.cuda.stream(use_stream):
            torch.cuda._sleep(100_000_000)
            preserved = held.wait(use_stream).clone()
        if protected == "busy":
            held.release()  # unleased, but its reader is still running
        copied = cache._prefetch_nonblocking(ExpertKey(0, 4), eviction_probabilities=probabilities)
        assert copied is not None
        with copied:
            assert copied.slot_id == 0  # expert 0: next lowest probability, writable
            actual = copied.wait().clone()
    finally:
        held.release()
    torch.cuda.synchronize()
    assert torch.equal(preserved.cpu(), cache._sources[ExpertKey(0, 1)])
    assert torch.equal(actual.cpu(), cache._sources[ExpertKey(0, 4)])
    _close(loaded)


def test_bad_probabilities_and_policy_fail_before_cache_mutation(device):
    loaded, _, _ = _case(slots=3, layers=1)
    cache = loaded.expert_caches[0]
    module = loaded.model.model.layers[0].mlp.experts
    cases = [dict(eviction_policy="unknown"), dict(eviction_policy="probability"),
             dict(prediction_probabilities=[]), dict(prediction_probabilities={0: []}),
             dict(prediction_probabilities={1: {0: .5}}),
             dict(prediction_probabilities={0: {6: .5}}),
             dict(prediction_probabilities={0: {0: .5, 6: 0.}}),
             dict(prediction_probabilities={0: {True: .5}}),
             dict(prediction_probabilities={0: {1: .5}})]
    cases += [dict(prediction_probabilities={0: {0: p}})
              for p in (float("nan"), float("inf"), -.1, 1.1, True, "0.5")]
    before = cache.stats()
    for kwargs in cases:
        with pytest.raises((ValueError, TypeError)):
            loaded.prefetch_experts({0: (0,)}, **kwargs)
        assert cache.stats() == before, kwargs
        assert module._prediction_scheduler is None
    for expert in (True, -1, 6, "0", 0.):
        with pytest.raises((ValueError, TypeError)):
            loaded.prefetch_experts({0: (expert,)}, prediction_probabilities={0: {0: .5}})
        assert cache.stats() == before, expert
        assert module._prediction_scheduler is None
    _close(loaded)


def test_scored_context_snapshots_inputs_and_preserves_ties_and_non_candidates(device):
    loaded, _, inputs = _case(slots=3, layers=2)
    expected = loaded.model(*inputs)
    streams = tuple(c.copy_stream for c in loaded.expert_caches)
    for policy in ("lru", "probability"):
        loaded.cold_reset_expert_caches()
        predictions = {lid: [4, 0, 4, 1, 2] for lid in range(2)}
        scores = {lid: {0: Fraction(1, 2), 1: Fraction(1, 2), 2: 0., 4: .9, 5: 1.}
                  for lid in range(2)}
        sched = loaded.prefetch_experts(
            MappingProxyType(predictions),
            prediction_probabilities=MappingProxyType({lid: MappingProxyType(row)
                                                       for lid, row in scores.items()}),
            eviction_policy=policy, lookahead_layers=0, trace=True)
        # duplicates folded, zero dropped, equal scores -> lower id, cap 2
        assert sched.predictions == ((4, 0), (4, 0))
        for lid in range(2):  # the context holds its own copy of the inputs
            predictions[lid][:] = [5]
            scores[lid].clear()
        with sched:
            copies = [row["expert_id"] for row in sched.events() if row["action"] == "copy"]
            assert copies == [4, 0], policy
            actual = loaded.model(*inputs)
        assert torch.equal(actual, expected)
        _assert_restored(loaded, streams)
    _close(loaded)


def test_real_qwen3_scored_predictions_preserve_complete_logits(device):
    from transformers import Qwen3MoeForCausalLM

    torch.manual_seed(909)
    source = Qwen3MoeForCausalLM(_tiny_config(2)).to(torch.bfloat16)
    with tempfile.TemporaryDirectory() as root:
        _save_qwen3_style_checkpoint(source, root)
        with load_offloaded_qwen3(root, device=device, slots_per_layer=2,
                                  h2d_prefetch=False) as loaded:
            ids = torch.tensor([[1, 7, 11, 19]], device=device)
            predictions = {}

            def hook(lid):
                def record(module, inputs, output):
                    predictions[lid] = torch.unique(output[2]).cpu().tolist()
                return record

            with torch.inference_mode(), ExitStack() as stack:
                for lid, layer in enumerate(loaded.model.model.layers):
                    stack.callback(layer.mlp.gate.register_forward_hook(hook(lid)).remove)
                expected = loaded.model(ids, use_cache=False).logits
            probabilities = {lid: {e: 1 / (e + 1) for e in experts}
                             for lid, experts in predictions.items()}
            for policy in ("lru", "probability"):
                for depth in (0, 1):
                    loaded.cold_reset_expert_caches()
                    with torch.inference_mode(), loaded.prefetch_experts(
                            predictions, prediction_probabilities=probabilities,
                            eviction_policy=policy, lookahead_layers=depth) as sched:
                        actual = loaded.model(ids, use_cache=False).logits
                    assert torch.equal(actual, expected), (policy, depth)
                    assert sched.stats()["complete"]

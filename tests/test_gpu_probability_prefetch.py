"""Probability-scored speculation and eviction of the prefetch scheduler.

Behaviour checked (the reference's scored-prefetch cases, whose inputs and
expected copies and victims are kept here as data:
tests/gpu/test_qwen3_probability_prefetch.py:28-193; the victim rule is
src/specfit/runtime/gpu_expert_cache.py:520-541):

* probabilities rank a layer's predictions (highest first, zero dropped,
  equal scores to the lower id) and cap them at slots - 1;
* with ``eviction_policy="probability"`` a speculative copy replaces the
  writable, unleased slot of lowest predicted probability, and only one of
  strictly lower probability than the incoming expert; routed demand still
  gets its copies;
* leased slots and slots still being read are never victims;
* invalid scores and policies fail before any cache changes;
* the context keeps its own copy of the scores it was given;
* scheduling never changes what the model computes, on the toy target and
  on a real tiny Qwen3-MoE checkpoint.

Each scored speculation case is one row of ``SPECULATION``: the experts
made resident first, the layer-0 predictions and scores, and what must
happen under each eviction policy.  ``_run_scored`` runs a row and reports
what the caches did.
"""
from __future__ import annotations

import tempfile
from contextlib import ExitStack
from dataclasses import dataclass, field
from fractions import Fraction
from types import MappingProxyType

import pytest
import torch

from _toy_target import save_per_expert_checkpoint, tiny_qwen3_config, toy_case
from specfit_amd.runtime import ExpertKey, RuntimeEventKind, load_offloaded_qwen3

pytestmark = pytest.mark.gpu


@dataclass(frozen=True)
class Scored:
    name: str
    resident: tuple                 # layer-0 experts made resident before the context
    predicted: tuple                # layer-0 predictions, as given
    scores: dict                    # layer-0 probabilities, as given
    policy: str                     # eviction policy
    copies_at_entry: tuple | None = None   # expected speculative copies, in order
    victims_at_entry: tuple | None = None  # expected evictions before the forward
    counts: dict = field(default_factory=dict)  # expected per-layer stats entries


SPECULATION = [
    # Ranked by score, 2 (score 0) dropped, capped at slots - 1 = 2.
    *(Scored(f"rank-and-cap-{p}", (), (0, 1, 2, 3, 4),
             {0: .7, 1: .8, 2: 0., 3: .1, 4: .9}, p, copies_at_entry=(4, 1),
             counts={"predicted_experts": 2}) for p in ("lru", "probability")),
    # A full cache: LRU evicts the oldest (0), probability the least likely (1).
    Scored("victim-lru", (0, 1, 2), (4,), {0: .6, 1: .1, 2: .4, 4: .9}, "lru",
           victims_at_entry=(0,)),
    Scored("victim-probability", (0, 1, 2), (4,), {0: .6, 1: .1, 2: .4, 4: .9}, "probability",
           victims_at_entry=(1,)),
    # No resident expert is strictly less likely than the incoming one: no
    # speculative copy, and the forward's two misses are demand copies.
    *(Scored(f"no-lower-victim-{x}", (0, 1, 2), (4,), {0: .8, 1: .6, 2: .5, 4: x},
             "probability", copies_at_entry=(), victims_at_entry=(),
             counts={"prediction_copies": 0, "demand_copies": 2}) for x in (.5, .4)),
]


def _run_scored(row: Scored) -> dict:
    case = toy_case(slots=3, layers=1)
    try:
        reference = case.forward()
        case.loaded.cold_reset_expert_caches()
        case.make_resident(row.resident)
        mark = len(case.observer.events())
        streams = case.copy_streams()
        with case.loaded.prefetch_experts({0: row.predicted},
                                          prediction_probabilities={0: row.scores},
                                          eviction_policy=row.policy, lookahead_layers=0,
                                          trace=True) as sched:
            # What entering the context did, before any forward ran.
            at_entry = case.observer.events()[mark:]
            copies = tuple(r["expert_id"] for r in sched.events() if r["action"] == "copy")
            output = case.forward()
        case.assert_quiet(streams)
        return dict(same_output=torch.equal(output, reference), copies=copies,
                    submitted=sum(e.kind is RuntimeEventKind.H2D_SUBMIT for e in at_entry),
                    victims=tuple(e.victim_expert_id.expert_id for e in at_entry
                                  if e.kind is RuntimeEventKind.EVICT),
                    stats=sched.stats())
    finally:
        case.close()


@pytest.mark.parametrize("row", SPECULATION, ids=lambda r: r.name)
def test_scored_speculation(device, row):
    got = _run_scored(row)
    print(f"{row.name}: copies {got['copies']} victims {got['victims']}", flush=True)
    assert got["same_output"]
    if row.copies_at_entry is not None:
        assert got["copies"] == row.copies_at_entry
        assert got["submitted"] == len(row.copies_at_entry)
    if row.victims_at_entry is not None:
        assert got["victims"] == row.victims_at_entry
    layer = got["stats"]["layers"][0]
    for key, value in row.counts.items():
        assert layer[key] == value, key
    assert got["stats"]["complete"] and got["stats"]["peak_inflight"] <= 2


@pytest.mark.parametrize("protection", ["active lease", "pending reader"])
def test_protected_slot_is_never_the_probability_victim(device, protection):
    """Expert 1 has the lowest score but its slot is leased, or unleased with
    a reader still running on another stream: the copy of expert 4 takes
    the next least likely slot (expert 0's), and expert 1's bytes survive."""
    case = toy_case(slots=3, layers=1)
    cache = case.caches[0]
    try:
        case.make_resident((0, 1, 2))
        score = {ExpertKey(0, e): p for e, p in {0: .2, 1: .1, 2: .3, 4: .9}.items()}
        reader = torch.cuda.Stream()
        lease = cache.acquire(ExpertKey(0, 1))
        with torch.cuda.stream(reader):
            torch.cuda._sleep(100_000_000)
            kept = lease.wait(reader).clone()
        if protection == "pending reader":
            lease.release()
        incoming = cache._prefetch_nonblocking(ExpertKey(0, 4), eviction_probabilities=score)
        assert incoming is not None
        with incoming:
            assert incoming.slot_id == 0
            landed = incoming.wait().clone()
        lease.release()
        torch.cuda.synchronize()
        assert torch.equal(kept.cpu(), cache._sources[ExpertKey(0, 1)])
        assert torch.equal(landed.cpu(), cache._sources[ExpertKey(0, 4)])
    finally:
        case.close()


_NAN, _INF = float("nan"), float("inf")
# (predictions, keyword arguments) that must be refused before anything runs.
BAD_SCORED = {
    "unknown-policy": ({0: (0,)}, dict(eviction_policy="unknown")),
    "probability-without-scores": ({0: (0,)}, dict(eviction_policy="probability")),
    "scores-not-a-mapping": ({0: (0,)}, dict(prediction_probabilities=[])),
    "layer-scores-not-a-mapping": ({0: (0,)}, dict(prediction_probabilities={0: []})),
    "scored-layer-outside-model": ({0: (0,)}, dict(prediction_probabilities={1: {0: .5}})),
    "scored-expert-unknown": ({0: (0,)}, dict(prediction_probabilities={0: {6: .5}})),
    "scored-expert-unknown-zero": ({0: (0,)}, dict(prediction_probabilities={0: {0: .5, 6: 0.}})),
    "scored-expert-bool": ({0: (0,)}, dict(prediction_probabilities={0: {True: .5}})),
    "predicted-expert-unscored": ({0: (0,)}, dict(prediction_probabilities={0: {1: .5}})),
    **{f"score-{v!r}": ({0: (0,)}, dict(prediction_probabilities={0: {0: v}}))
       for v in (_NAN, _INF, -.1, 1.1, True, "0.5")},
    **{f"predicted-{e!r}": ({0: (e,)}, dict(prediction_probabilities={0: {0: .5}}))
       for e in (True, -1, 6, "0", 0.)},
}


@pytest.mark.parametrize("name", sorted(BAD_SCORED))
def test_invalid_scored_context_changes_nothing(device, name):
    predictions, kwargs = BAD_SCORED[name]
    case = toy_case(slots=3, layers=1)
    try:
        cache, module = case.caches[0], case.loaded.model.model.layers[0].mlp.experts
        before = cache.stats()
        with pytest.raises((ValueError, TypeError)):
            case.loaded.prefetch_experts(predictions, **kwargs)
        assert cache.stats() == before
        assert module._prediction_scheduler is None
    finally:
        case.close()


@pytest.mark.parametrize("policy", ["lru", "probability"])
def test_scored_context_owns_its_inputs(device, policy):
    """Read-only views of mutable predictions and scores (with Fraction
    scores) are folded on construction: duplicates once, zero dropped, ties
    to the lower id, at most 2 per layer.  Changing the caller's objects
    afterwards changes nothing."""
    case = toy_case(slots=3, layers=2)
    try:
        reference = case.forward()
        case.loaded.cold_reset_expert_caches()
        mine = {lid: [4, 0, 4, 1, 2] for lid in range(2)}
        my_scores = {lid: {0: Fraction(1, 2), 1: Fraction(1, 2), 2: 0., 4: .9, 5: 1.}
                     for lid in range(2)}
        sched = case.loaded.prefetch_experts(
            MappingProxyType(mine),
            prediction_probabilities=MappingProxyType(
                {lid: MappingProxyType(s) for lid, s in my_scores.items()}),
            eviction_policy=policy, lookahead_layers=0, trace=True)
        assert sched.predictions == ((4, 0), (4, 0))
        for lid in range(2):
            mine[lid][:] = [5]
            my_scores[lid].clear()
        streams = case.copy_streams()
        with sched:
            assert [r["expert_id"] for r in sched.events() if r["action"] == "copy"] == [4, 0]
            output = case.forward()
        assert torch.equal(output, reference)
        case.assert_quiet(streams)
    finally:
        case.close()


@pytest.fixture(scope="module")
def tiny_qwen3_root():
    from transformers import Qwen3MoeForCausalLM

    torch.manual_seed(909)
    model = Qwen3MoeForCausalLM(tiny_qwen3_config(2)).to(torch.bfloat16)
    with tempfile.TemporaryDirectory() as root:
        save_per_expert_checkpoint(model, root)
        yield root


@pytest.mark.parametrize("policy,lookahead", [(p, d) for p in ("lru", "probability")
                                              for d in (0, 1)])
def test_scored_predictions_keep_real_qwen3_logits(device, tiny_qwen3_root, policy, lookahead):
    """A real (tiny) Qwen3-MoE checkpoint with 2 slots per layer: the routed
    experts of an unscheduled forward, scored 1 / (id + 1), as predictions;
    the scheduled forward's logits are bitwise the unscheduled ones."""
    with load_offloaded_qwen3(tiny_qwen3_root, device=device, slots_per_layer=2,
                              h2d_prefetch=False) as loaded:
        ids = torch.tensor([[1, 7, 11, 19]], device=device)
        routed = {}
        with torch.inference_mode(), ExitStack() as hooks:
            for lid, layer in enumerate(loaded.model.model.layers):
                hooks.callback(layer.mlp.gate.register_forward_hook(
                    lambda mod, inp, out, lid=lid: routed.__setitem__(
                        lid, sorted(set(out[2].flatten().tolist())))).remove)
            reference = loaded.model(ids, use_cache=False).logits
        scores = {lid: {e: 1 / (e + 1) for e in experts} for lid, experts in routed.items()}
        loaded.cold_reset_expert_caches()
        with torch.inference_mode(), loaded.prefetch_experts(
                routed, prediction_probabilities=scores, eviction_policy=policy,
                lookahead_layers=lookahead) as sched:
            logits = loaded.model(ids, use_cache=False).logits
        assert torch.equal(logits, reference)
        assert sched.stats()["complete"]

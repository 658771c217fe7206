"""Qwen3OffloadedExperts + router on the device: the reference operator
tests (tests/gpu/test_qwen3_offloaded_experts.py:60-458,
test_qwen3_expert_prefetch.py:102-121) restated, plus whole-layer parity
with the oracle at the Qwen3-30B-A3B shape.
"""
from unittest.mock import patch

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from specfit_amd.runtime import (ExpertExecutionPolicy, ExpertKey, GpuExpertCache,
                                 Qwen3MoeTopKRouterHip, Qwen3OffloadedExperts,
                                 RecordingCacheTransitionObserver, ReductionMode,
                                 RuntimeEventKind)
from specfit_amd.runtime import qwen3_offloaded_experts as implementation
from specfit_amd import ops
from specfit_amd.workloads import make_hidden, make_layer

pytestmark = pytest.mark.gpu


def _pack(gate, up, down):
    return torch.cat((gate.flatten(), up.flatten(), down.flatten()))


def _hf_experts(gate_up, down, H, I):
    """transformers' eager Qwen3MoeExperts on the CPU in bf16 (tf:222-246)."""
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeExperts
    cfg = Qwen3MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=gate_up.shape[0],
                         hidden_act="silu")
    ref = Qwen3MoeExperts(cfg).to(dtype=torch.bfloat16)
    with torch.no_grad():
        ref.gate_up_proj.copy_(gate_up)
        ref.down_proj.copy_(down)
    return ref


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_canonical_output_is_invariant_to_execution_order(device):
    H, I = 4, 3
    g = torch.Generator().manual_seed(29)
    gate_up = torch.randn(3, 2 * I, H, dtype=torch.bfloat16, generator=g)
    down = torch.randn(3, H, I, dtype=torch.bfloat16, generator=g)
    sources = {ExpertKey(0, e): _pack(gate_up[e, :I], gate_up[e, I:], down[e]) for e in range(3)}
    hidden = torch.randn(2, H, dtype=torch.bfloat16, generator=g).to(device)
    idx = torch.tensor([[0, 1, 2], [2, 0, 1]], dtype=torch.long, device=device)
    w = torch.tensor([[0.50, 0.30, 0.20], [0.45, 0.35, 0.20]], dtype=torch.bfloat16, device=device)
    cache = GpuExpertCache(sources, slot_count=1, device=device)
    experts = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H, intermediate_size=I,
                                    reduction_mode=ReductionMode.CANONICAL)
    fwd = experts(hidden, idx, w, execution_order=(0, 1, 2))
    torch.cuda.synchronize(device)
    assert cache.resident_expert_ids() == (ExpertKey(0, 2),)
    rev = experts(hidden, idx, w, execution_order=(2, 1, 0))
    torch.cuda.synchronize(device)
    assert cache.resident_expert_ids() == (ExpertKey(0, 0),)
    ref = _hf_experts(gate_up, down, H, I)(hidden.cpu(), idx.cpu(), w.cpu())
    assert torch.equal(fwd, rev)
    torch.testing.assert_close(fwd.cpu(), ref, rtol=1.6e-2, atol=1.6e-2)
    cache.close()


def test_resident_first_avoids_eviction_before_first_use(device):
    H, I = 4, 3
    g = torch.Generator().manual_seed(101)
    sources = {ExpertKey(0, e): torch.randn(3 * H * I, dtype=torch.bfloat16, generator=g)
               for e in range(3)}
    hidden = torch.randn(2, H, dtype=torch.bfloat16, generator=g).to(device)
    idx = torch.tensor([[0, 1, 2], [2, 0, 1]], dtype=torch.long, device=device)
    w = torch.tensor([[0.50, 0.30, 0.20], [0.45, 0.35, 0.20]], dtype=torch.bfloat16, device=device)

    def case(policy):
        obs = RecordingCacheTransitionObserver(run_id=f"rf-{policy}")
        cache = GpuExpertCache(sources, slot_count=2, device=device, observer=obs)
        for e in (1, 2):
            with cache.acquire(ExpertKey(0, e)) as lease:
                lease.wait()
        torch.cuda.synchronize(device)
        obs.reset()
        kw = {} if policy is None else {"execution_policy": policy}
        return cache, Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H,
                                            intermediate_size=I, **kw), obs

    legacy = case(None)
    resident = case(ExpertExecutionPolicy.RESIDENT_FIRST)
    explicit = case(ExpertExecutionPolicy.RESIDENT_FIRST)
    assert legacy[1].execution_policy is ExpertExecutionPolicy.EXPERT_ID_ASCENDING
    before = [c[0].stats() for c in (legacy, resident, explicit)]
    out_l = legacy[1](hidden, idx, w)
    out_r = resident[1](hidden, idx, w)
    out_e = explicit[1](hidden, idx, w, execution_order=(0, 1, 2))
    torch.cuda.synchronize(device)
    after = [c[0].stats() for c in (legacy, resident, explicit)]
    kinds = {RuntimeEventKind.H2D_SUBMIT, RuntimeEventKind.RESIDENT_HIT}
    assert tuple(e.expert_id.expert_id for e in legacy[2].events() if e.kind in kinds) == (0, 1, 2)
    assert tuple((e.kind, e.expert_id.expert_id) for e in resident[2].events() if e.kind in kinds) == (
        (RuntimeEventKind.RESIDENT_HIT, 1), (RuntimeEventKind.RESIDENT_HIT, 2),
        (RuntimeEventKind.H2D_SUBMIT, 0))
    assert tuple(e.expert_id.expert_id for e in explicit[2].events() if e.kind in kinds) == (0, 1, 2)

    def delta(b, a):
        return (a.h2d_submissions - b.h2d_submissions, a.resident_hits - b.resident_hits,
                a.inflight_joins - b.inflight_joins, a.evictions - b.evictions)

    assert delta(before[0], after[0]) == (3, 0, 0, 3)
    assert delta(before[1], after[1]) == (1, 2, 0, 1)
    assert delta(before[2], after[2]) == (3, 0, 0, 3)
    assert torch.equal(out_l, out_r) and torch.equal(out_l, out_e)
    for c in (legacy, resident, explicit):
        c[0].close()


def test_expert_math_at_qwen3_shape_matches_hf_eager(device):
    H, I = 2048, 768
    g = torch.Generator().manual_seed(41)
    gate_up = torch.randn(1, 2 * I, H, dtype=torch.bfloat16, generator=g)
    down = torch.randn(1, H, I, dtype=torch.bfloat16, generator=g)
    source = _pack(gate_up[0, :I], gate_up[0, I:], down[0])
    hidden = torch.randn(8, H, dtype=torch.bfloat16, generator=g)
    idx = torch.zeros(8, 1, dtype=torch.long)
    w = torch.ones(8, 1, dtype=torch.bfloat16)
    cache = GpuExpertCache({ExpertKey(0, 0): source}, slot_count=1, device=device)
    experts = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H, intermediate_size=I)
    got = experts(hidden.to(device), idx.to(device), w.to(device)).cpu()
    ref = _hf_experts(gate_up, down, H, I)(hidden, idx, w)
    # The reference compares bitwise against cuBLAS; a different GEMM
    # summation order moves some bf16 outputs by one ulp, so the bar is the
    # reference tolerance plus the fp32 closed form at 1e-2.
    scale = ref.float().abs().max()
    assert ((got.float() - ref.float()).abs().max() / scale).item() <= 1e-2
    y32 = oracle.expert_forward_fp32(hidden.float().numpy(), source.float().numpy(), H, I)
    assert np.abs(got.float().numpy() - y32).max() / np.abs(y32).max() <= 1e-2
    cache.close()


def test_arrival_order_known_answer(device):
    silu_one = F.silu(torch.tensor(1.0, dtype=torch.bfloat16)).item()
    desired = (1.0, 2.0 ** -8, -1.0)
    one = torch.tensor([[1.0]], dtype=torch.bfloat16)
    sources = {ExpertKey(0, e): _pack(one, one, torch.tensor([[v / silu_one]], dtype=torch.bfloat16))
               for e, v in enumerate(desired)}
    hidden = torch.ones(1, 1, dtype=torch.bfloat16, device=device)
    idx = torch.tensor([[0, 1, 2]], dtype=torch.long, device=device)
    w = torch.ones(1, 3, dtype=torch.bfloat16, device=device)
    caches = {m: GpuExpertCache(sources, slot_count=1, device=device) for m in ReductionMode}
    experts = {m: Qwen3OffloadedExperts(layer_id=0, cache=caches[m], hidden_size=1,
                                        intermediate_size=1, reduction_mode=m) for m in ReductionMode}
    lost = experts[ReductionMode.ARRIVAL_ORDER](hidden, idx, w, execution_order=(0, 1, 2))
    experts[ReductionMode.CANONICAL](hidden, idx, w, execution_order=(0, 1, 2))
    torch.cuda.synchronize(device)
    assert caches[ReductionMode.ARRIVAL_ORDER].stats() == caches[ReductionMode.CANONICAL].stats()
    kept = experts[ReductionMode.ARRIVAL_ORDER](hidden, idx, w, execution_order=(0, 2, 1))
    assert float(lost.item()) == 0.0
    assert float(kept.item()) == 2.0 ** -8
    for c in caches.values():
        c.close()


def _small_case(device, slots):
    g = torch.Generator().manual_seed(909)
    sources = {ExpertKey(0, e): torch.randn(3 * 16 * 12, generator=g, dtype=torch.bfloat16) / 16
               for e in range(6)}
    cache = GpuExpertCache(sources, slot_count=slots, device=device)
    hidden = torch.randn(4, 16, generator=g, dtype=torch.bfloat16).to(device)
    idx = torch.tensor([[4, 0, 2], [1, 4, 3], [2, 0, 1], [4, 3, 0]], device=device)
    w = torch.rand(4, 3, generator=g, dtype=torch.bfloat16).to(device)
    return cache, (hidden, idx, w)


def test_noncontiguous_repeated_and_empty_inputs(device):
    outputs = {}
    for tokens in (0, 1, 4):
        for slots in (1, 6):
            for prefetch in (False, True):
                cache, (hidden, idx, w) = _small_case(device, slots)
                idx[0, 2] = idx[0, 0]
                inputs = tuple(t[:tokens].t().contiguous().t() for t in (hidden, idx, w))
                originals = tuple(t.clone() for t in inputs)
                mod = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=16,
                                            intermediate_size=12, h2d_prefetch=prefetch)
                out = mod(*inputs)
                torch.cuda.synchronize(device)
                for a, b in zip(inputs, originals):
                    assert torch.equal(a, b)
                assert cache.active_lease_count == 0
                outputs.setdefault(tokens, []).append(out.cpu())
                if tokens:
                    x = inputs[0].float().cpu().numpy()
                    ex = {e: cache._sources[ExpertKey(0, e)].float().numpy() for e in range(6)}
                    ref = oracle.moe_forward_bf16(x, inputs[1].cpu().numpy(),
                                                  inputs[2].float().cpu().numpy(), ex, 16, 12, 6,
                                                  accumulate_fp32=True)
                    np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=1.6e-2,
                                               atol=1.6e-2)
                cache.close()
    for tokens, outs in outputs.items():
        assert all(torch.equal(o, outs[0]) for o in outs), tokens
        assert outs[0].shape == (tokens, 16)


def test_injected_failure_releases_every_lease(device):
    cache, inputs = _small_case(device, 3)
    mod = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=16, intermediate_size=12)
    expected = mod(*inputs)
    for name in ("_expert_forward", "_dispatch"):
        with patch.object(implementation, name, side_effect=RuntimeError("injected")):
            with pytest.raises(RuntimeError, match="injected"):
                mod(*inputs)
        assert cache.active_lease_count == 0
    assert torch.equal(mod(*inputs), expected)
    torch.cuda.synchronize(device)
    cache.close()


def test_validation_errors(device):
    cache, (hidden, idx, w) = _small_case(device, 2)
    mod = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=16, intermediate_size=12)
    with pytest.raises(ValueError, match="shape"):
        mod(hidden[0], idx, w)
    with pytest.raises(ValueError, match="width"):
        mod(hidden[:, :8], idx, w)
    with pytest.raises(ValueError, match="torch.long"):
        mod(hidden, idx.int(), w)
    with pytest.raises(ValueError, match="match"):
        mod(hidden, idx, w[:, :2])
    with pytest.raises(ValueError, match="duplicates"):
        mod(hidden, idx, w, execution_order=(0, 0, 1, 2, 3, 4))
    with pytest.raises(ValueError, match="exactly once"):
        mod(hidden, idx, w, execution_order=(0, 1, 2))
    with pytest.raises(KeyError):
        mod(hidden, torch.full_like(idx, 7), w)
    with pytest.raises(ValueError):
        Qwen3OffloadedExperts(layer_id=-1, cache=cache, hidden_size=16, intermediate_size=12)
    with pytest.raises(ValueError):
        Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=16, intermediate_size=12,
                              h2d_prefetch=1)
    assert cache.active_lease_count == 0
    cache.close()


def _qwen3_layer(device, num_experts, tokens, slots, seed=0, zipf=1.1):
    layer = make_layer(seed=seed, num_experts=num_experts, zipf_s=zipf, pin_memory=True)
    hidden = make_hidden(tokens, seed=seed + 100, zipf_fold=zipf is not None)
    router = Qwen3MoeTopKRouterHip(num_experts=num_experts, hidden_size=2048, top_k=8,
                                   norm_topk_prob=True, device=device)
    with torch.no_grad():
        router.weight.copy_(layer.router)
    sources = {ExpertKey(0, e): layer.experts[e] for e in range(num_experts)}
    cache = GpuExpertCache(sources, slot_count=slots, device=device, adopt_pinned_sources=True)
    return layer, hidden.to(device), router, cache


def test_qwen3_layer_matches_fp32_oracle_and_is_schedule_invariant(device):
    E, T = 32, 64
    layer, hidden, router, cache = _qwen3_layer(device, E, T, slots=6)
    _, w, idx = router(hidden)
    outs = []
    for slots, policy, prefetch in ((6, "resident_first", True), (6, "expert_id_ascending", False),
                                    (E, "expert_id_ascending", True), (2, "resident_first", False)):
        c = cache if slots == 6 else GpuExpertCache(cache._sources, slot_count=slots, device=device,
                                                    adopt_pinned_sources=True)
        mod = Qwen3OffloadedExperts(layer_id=0, cache=c, hidden_size=2048, intermediate_size=768,
                                    execution_policy=policy, h2d_prefetch=prefetch)
        for _ in range(2):
            outs.append(mod(hidden, idx, w))
        torch.cuda.synchronize(device)
        assert c.active_lease_count == 0
        if c is not cache:
            c.close()
    assert all(torch.equal(o, outs[0]) for o in outs)
    x = oracle.bf16_float(_bits(hidden))
    ex = {e: oracle.bf16_float(_bits(layer.experts[e])) for e in range(E)}
    wf = oracle.bf16_float(_bits(w))
    y32 = oracle.moe_forward_fp32(x, idx.cpu().numpy(), wf, ex, 2048, 768)
    got = oracle.bf16_float(_bits(outs[0]))
    err = np.abs(got - y32).max() / np.abs(y32).max()
    print(f"layer max normalised error vs fp32 oracle: {err:.3e}", flush=True)
    assert err <= 1e-2
    yb = oracle.moe_forward_bf16(x, idx.cpu().numpy(), wf, ex, 2048, 768, E, accumulate_fp32=True)
    np.testing.assert_allclose(got, yb, rtol=1.6e-2, atol=1.6e-2)
    # the bf16-per-addition combine (reference index_add_ arithmetic) also
    # stays within the reference tolerance of its oracle
    mod = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=2048, intermediate_size=768,
                                combine_fp32=False)
    got16 = oracle.bf16_float(_bits(mod(hidden, idx, w)))
    yb16 = oracle.moe_forward_bf16(x, idx.cpu().numpy(), wf, ex, 2048, 768, E)
    np.testing.assert_allclose(got16, yb16, rtol=1.6e-2, atol=1.6e-2)
    cache.close()


@pytest.mark.parametrize("name", ["router_hf_t256_h2048_e128_k8_uniform.npz",
                                  "router_hf_t256_h2048_e128_k8_zipf.npz"])
def test_router_module_agrees_with_hf_router_row_by_row(device, name):
    """The HIP router module at the Qwen3-30B-A3B shape (256 tokens) on the
    inputs of a transformers golden fixture: bit-exact with the oracle, and
    row by row against transformers' router (tf:258-267): rows with equal
    logits select the same experts unless the 8th logit is tied (lower id
    kept here, torch.topk picks another), and rows whose logits differ by
    one ulp differ only through a flip at the boundary."""
    from _router_agreement import classify
    from test_oracle_router import real_shape_case

    f, h_bits, w_bits = real_shape_case(name)
    h = torch.from_numpy(h_bits.view(np.int16)).view(torch.bfloat16)
    w = torch.from_numpy(w_bits.view(np.int16)).view(torch.bfloat16)
    ours = Qwen3MoeTopKRouterHip(num_experts=128, hidden_size=2048, top_k=8, norm_topk_prob=True,
                                 device=device)
    with torch.no_grad():
        ours.weight.copy_(w)
    lg, tw, ti = ours(h.to(device))
    torch.cuda.synchronize()
    o_lg, o_tw, o_ti, _ = oracle.router(h_bits, w_bits, 8, True)
    assert np.array_equal(_bits(lg), o_lg) and np.array_equal(_bits(tw), o_tw)
    assert np.array_equal(ti.cpu().numpy(), o_ti)
    a = classify(_bits(lg), ti.cpu().numpy(), f["logits"], f["index"], 8)
    print(f"{name}: {a.same_set_rows}/{a.rows} rows select transformers' experts; "
          f"{a.tie_rows} boundary ties, {a.flip_set_rows} one-ulp flips", flush=True)
    assert a.agreement >= 0.95


def test_batched_resident_runs_keep_the_reference_lease_sequence(device):
    """Runs of resident experts are leased in one locked pass (a lean form
    without an observer, a per-event form with one).  Both must leave the
    cache exactly where the per-expert lease sequence (acquire, one-ahead
    prefetch, wait, release) leaves it: slot contents, generations, LRU
    sequence numbers and counters after every step, and the same output."""
    E, H, I, K, slots = 12, 32, 16, 3, 8
    g = torch.Generator().manual_seed(41)
    sources = {e: (torch.randn(3 * I * H, generator=g) / 8).to(torch.bfloat16) for e in range(E)}

    def stack(observer):
        cache = GpuExpertCache({ExpertKey(0, e): t for e, t in sources.items()},
                               slot_count=slots, device=device, observer=observer)
        return cache, Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H,
                                            intermediate_size=I,
                                            execution_policy="resident_first", h2d_prefetch=True)

    lean = stack(None)
    observed = stack(RecordingCacheTransitionObserver(run_id="resident-runs"))
    per_expert = stack(None)

    def state(cache):
        snap = cache.snapshot()
        return (tuple((s.slot_id, s.expert_id, s.generation, s.last_used_sequence,
                       s.active_leases) for s in snap.slots),
                snap.lru_sequence, snap.submission_sequence, cache.stats())

    for step in range(12):
        T = int(torch.randint(1, 7, (1,), generator=g))
        h = torch.randn(T, H, generator=g).to(torch.bfloat16).to(device)
        idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(device)
        w = torch.rand(T, K, generator=g).to(torch.bfloat16).to(device)
        y_lean = lean[1](h, idx, w)
        y_obs = observed[1](h, idx, w)
        with patch.object(GpuExpertCache, "_resident_steps",
                          lambda self, keys, index, current, stream, limit: ([], index, current)):
            y_ref = per_expert[1](h, idx, w)
        torch.cuda.synchronize()
        print(f"resident-run step {step} T={T} stats {lean[0].stats()}", flush=True)
        assert state(lean[0]) == state(per_expert[0]), step
        assert state(observed[0]) == state(per_expert[0]), step
        assert torch.equal(y_lean, y_ref) and torch.equal(y_obs, y_ref)
    assert lean[0].stats().resident_hits > 20  # the runs were exercised
    for cache, _ in (lean, observed, per_expert):
        cache.close()


@pytest.mark.parametrize("shape", ["tiny", "qwen3"])
def test_slot_table_forward_matches_the_launch_path(device, shape):
    """After a forward that copied nothing in, a resident-first layer runs
    its resident experts from the device slot table.  Output bits, cache
    slots, LRU and submission sequences, counters and (tiny shape, with
    observers) the recorded cache transitions must equal those of the
    per-launch path (the same order passed explicitly), also when the table
    forward misses and when a token repeats an expert (an expert with more
    rows than tokens)."""
    if shape == "tiny":
        E, H, I, K, slots = 12, 32, 16, 3, 10
    else:
        E, H, I, K, slots = 12, 2048, 768, 3, 10
    g = torch.Generator().manual_seed(77)
    sources = {e: (torch.randn(3 * I * H, generator=g) * 0.02).to(torch.bfloat16)
               for e in range(E)}

    observers = {}

    def stack(name):
        observers[name] = RecordingCacheTransitionObserver(run_id=name) if shape == "tiny" else None
        cache = GpuExpertCache({ExpertKey(0, e): t for e, t in sources.items()},
                               slot_count=slots, device=device, cache_id="layer-0",
                               queue_id="layer-0-copy", observer=observers[name])
        return cache, Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H,
                                            intermediate_size=I,
                                            execution_policy="resident_first", h2d_prefetch=True)

    (ca, la), (cb, lb) = stack("table"), stack("launch")

    def events(name):  # the cache transitions, without stream ids and timings
        if observers[name] is None:
            return ()
        return tuple((e.kind, e.expert_id, e.slot_id, e.generation, e.submission_sequence,
                      e.victim_expert_id) for e in observers[name].events())

    def state(cache):
        snap = cache.snapshot()
        return (tuple((s.slot_id, s.expert_id, s.generation, s.last_used_sequence)
                      for s in snap.slots), snap.lru_sequence, snap.submission_sequence,
                cache.stats())

    def resident_ids():
        return sorted(k.expert_id for k in cb._resident_key_set())

    def from_pool(T, pool):
        pool = torch.tensor(pool)
        return torch.stack([pool[torch.randperm(len(pool), generator=g)[:K]] for _ in range(T)])

    # (kind, tokens): load all of 0..9; resident experts only; a token that
    # repeats an expert; one expert outside the cache (a miss)
    steps = [("load", 4), ("resident", 5), ("resident", 6), ("repeat", 2), ("miss", 6),
             ("resident", 5), ("resident", 7)]
    real = ops.grouped_swiglu_table
    table_calls = []

    def spy(*args, **kwargs):
        table_calls.append(kwargs.get("max_rows"))
        return real(*args, **kwargs)

    for step, (kind, T) in enumerate(steps):
        if kind == "load":
            idx = torch.tensor([[0, 1, 2], [3, 4, 5], [6, 7, 8], [9, 0, 1]])
        elif kind == "resident":
            idx = from_pool(T, resident_ids())
        elif kind == "repeat":
            r = resident_ids()
            idx = torch.tensor([[r[0], r[0], r[1]], [r[0], r[2], r[3]]])
        else:
            outside = [e for e in range(E) if e not in resident_ids()]
            idx = from_pool(T, resident_ids())
            idx[0, 0] = outside[0]
        h = (torch.randn(T, H, generator=g)).to(torch.bfloat16).to(device)
        w = torch.rand(T, K, generator=g).to(torch.bfloat16).to(device)
        idx = idx.to(device)
        uses_table = la._uses_slot_table()
        active = sorted(set(idx.flatten().tolist()))
        resident = cb._resident_key_set()
        order = ([e for e in active if ExpertKey(0, e) in resident]
                 + [e for e in active if ExpertKey(0, e) not in resident])
        calls = len(table_calls)
        with patch.object(ops, "grouped_swiglu_table", spy):
            ya = la(h, idx, w)
        yb = lb(h, idx, w, execution_order=order)
        torch.cuda.synchronize()
        print(f"slot-table case {shape} step {step} T={T} table={uses_table} "
              f"stats {ca.stats()}", flush=True)
        assert (len(table_calls) > calls) == uses_table
        assert torch.equal(ya, yb), step
        assert state(ca) == state(cb), step
        assert events("table") == events("launch"), step
    assert len(table_calls) == 4  # hits only (twice), repeated expert, a miss
    if shape == "tiny":  # the tiny stacks record their cache transitions
        assert len(events("table")) > 100
    ca.close()
    cb.close()


def _table_stacks(device, E=12, slots=6, seed=78):
    """A resident-first layer (slot-table eligible) and an identical second
    stack that computes the same routes on the per-launch path."""
    H, I = 2048, 768
    g = torch.Generator().manual_seed(seed)
    sources = {e: (torch.randn(3 * I * H, generator=g) * 0.02).to(torch.bfloat16)
               for e in range(E)}

    def stack():
        cache = GpuExpertCache({ExpertKey(0, e): t for e, t in sources.items()},
                               slot_count=slots, device=device)
        return cache, Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H,
                                            intermediate_size=I,
                                            execution_policy="resident_first", h2d_prefetch=True)

    return sources, g, stack(), stack()


def _routes(device, g, rows, K):
    idx = torch.tensor(rows, device=device)
    T = idx.shape[0]
    h = torch.randn(T, 2048, generator=g).to(torch.bfloat16).to(device)
    w = torch.rand(T, K, generator=g).to(torch.bfloat16).to(device)
    return h, idx, w


def _spy_table():
    calls = []
    real = ops.grouped_swiglu_table

    def spy(*args, **kwargs):
        calls.append(1)
        return real(*args, **kwargs)

    return calls, patch.object(ops, "grouped_swiglu_table", spy)


def _oracle_check(sources, h, idx, w, out, where):
    x = oracle.bf16_float(_bits(h))
    ex = {e: oracle.bf16_float(_bits(t)) for e, t in sources.items()}
    y32 = oracle.moe_forward_fp32(x, idx.cpu().numpy(), oracle.bf16_float(_bits(w)), ex, 2048, 768)
    err = np.abs(oracle.bf16_float(_bits(out)) - y32).max() / np.abs(y32).max()
    print(f"{where}: max normalised error vs fp32 oracle {err:.3e}", flush=True)
    assert err <= 1e-2


def test_slot_table_forward_with_a_copy_in_flight_and_a_lower_id_miss(device):
    """A slot-table forward that starts while a copy is still in flight, and
    in which a lower-id miss takes that in-flight slot as its LRU victim:
    the table launch must not read the in-flight slot (its expert is
    computed by its own launch after its transfer), so no H2D overwrites a
    slot the table kernel reads.  Output bits equal the per-launch path's
    and the oracle's within tolerance."""
    sources, g, (ca, la), (cb, lb) = _table_stacks(device)
    K = 4
    residents = [6, 7, 8, 9, 10]
    # 1. five residents, then a forward over them that copies nothing
    for rows in ([[6, 7, 8, 9], [10, 6, 7, 8]], [[9, 8, 7, 6], [6, 10, 9, 8]]):
        h, idx, w = _routes(device, g, rows, K)
        la(h, idx, w)
        lb(h, idx, w)
    torch.cuda.synchronize()
    assert sorted(k.expert_id for k in ca._resident_key_set()) == residents
    assert la._uses_slot_table()
    # 2. hold both copy streams, prefetch expert 11 into the free slot, make
    #    that slot the least recently used one
    for s in {id(ca.copy_stream): ca.copy_stream,
              id(ca._aux_copy_stream): ca._aux_copy_stream}.values():
        with torch.cuda.stream(s):
            torch.cuda._sleep(100_000_000)
    ca._prefetch(ExpertKey(0, 11)).release()
    for e in residents:
        ca.acquire(ExpertKey(0, e)).release()
    assert ExpertKey(0, 11) in ca._inflight
    eleven = ca._inflight[ExpertKey(0, 11)].slot_id
    lru = min((s for s in ca._slots if s.active_leases == 0), key=lambda s: s.last_used_sequence)
    assert lru.slot_id == eleven
    # 3. a forward over residents, expert 11 (in flight) and expert 2 (a miss
    #    whose victim is 11's slot)
    h, idx, w = _routes(device, g, [[6, 2, 11, 7], [11, 8, 9, 2]], K)
    calls, spy = _spy_table()
    with spy:
        ya = la(h, idx, w)
    yb = lb(h, idx, w, execution_order=[6, 7, 8, 9, 2, 11])
    torch.cuda.synchronize()
    assert calls == [1], "the forward did not take the slot-table path"
    assert torch.equal(ya, yb)
    _oracle_check(sources, h, idx, w, ya, "in-flight table case")
    ca.close()
    cb.close()


def _discard_completed_experts(caches):
    """What the reference's cache-off intervention does to each cache
    (src/specfit/main_comparison_runtime.py:7-32), written out for this
    test: after a device synchronisation and a boundary check, every
    assignment is dropped behind the cache's back -- resident and in-flight
    maps and the transfer queue cleared, every slot emptied with its
    generation bumped -- and the host state version bumped."""
    torch.cuda.synchronize()
    for cache in caches:
        with cache._lock:
            cache._require_checkpoint_boundary()
            cache._resident.clear()
            cache._inflight.clear()
            cache._outstanding_transfers.clear()
            for slot in cache._slots:
                slot.expert_id, slot.ready_event = None, None
                slot.generation += 1
                slot.last_used_sequence = 0
                slot.use_events.clear()
            cache._state_version += 1


def test_discard_completed_experts_between_slot_table_forwards(device):
    """discard_completed_experts (called by the reference before non-decode
    forwards) empties the cache without going through it; the next
    slot-table forward must see the empty cache (no stale device table),
    copy every expert in and match the per-launch path bitwise."""
    sources, g, (ca, la), (cb, lb) = _table_stacks(device, slots=8)
    K = 4
    rows = [[0, 1, 2, 3], [4, 5, 0, 1]]
    h, idx, w = _routes(device, g, rows, K)
    for _ in range(2):  # the first copies the experts in, the second nothing
        la(h, idx, w)
        lb(h, idx, w)
    calls, spy = _spy_table()
    with spy:
        la(h, idx, w)  # after a forward that copied nothing: the slot table
    lb(h, idx, w)
    torch.cuda.synchronize()
    assert calls == [1]
    _discard_completed_experts([ca, cb])
    assert not ca.resident_expert_ids()
    before = ca.stats().h2d_submissions
    h, idx, w = _routes(device, g, [[5, 4, 3, 2], [1, 0, 6, 7]], K)
    with spy:
        ya = la(h, idx, w)
    yb = lb(h, idx, w, execution_order=list(range(8)))
    torch.cuda.synchronize()
    assert calls == [1, 1], "the forward after the discard did not take the slot-table path"
    assert ca.stats().h2d_submissions - before == 8  # every expert copied in again
    assert torch.equal(ya, yb)
    _oracle_check(sources, h, idx, w, ya, "after discard")
    ca.close()
    cb.close()

"""CPU checks of the C-ABI library and of the host-side runtime logic.

The library must load without a GPU and export every function that
include/specfit_amd.h declares; argument validation happens on the host
before any HIP call, so invalid calls are rejected here without a device.
"""
import ctypes
import os
import re

import pytest
import torch

from specfit_amd import _native
from specfit_amd.runtime import (CacheSlotSnapshot, ExpertCacheStats, ExpertKey,
                                 GpuExpertCacheSnapshot, RecordingCacheTransitionObserver,
                                 RuntimeEventKind, aggregate_cache_transition_counters)
from specfit_amd.workloads import expected_distinct_uniform, make_hidden, make_layer, zipf_bias

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "specfit_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sf_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    names = _declared_functions()
    assert "sf_router_topk" in names and "sf_copy_h2d" in names
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, name
    assert set(_native.SIGNATURES) == set(names)


def test_version_and_error_strings():
    assert _native.lib().sf_abi_version() == _native.SF_ABI_VERSION == 13
    assert _native.error_string(0) == "success"
    assert _native.error_string(1) == "invalid argument"
    assert _native.error_string(12345) != ""
    assert "scratch" in _native.error_string(5)
    with pytest.raises(RuntimeError, match="invalid argument"):
        _native.check(1, "probe")


def test_host_side_validation_needs_no_device():
    lib = _native.lib()
    null = None
    # experts out of range / top-k larger than experts / negative tokens
    assert lib.sf_router_topk(null, null, 4, 32, 0, 1, 1, null, null, null, null) == 1
    assert lib.sf_router_topk(null, null, 4, 32, 4, 5, 1, null, null, null, null) == 1
    assert lib.sf_router_topk(null, null, -1, 32, 4, 2, 1, null, null, null, null) == 1
    assert lib.sf_router_topk(null, null, 0, 32, 4, 2, 1, null, null, null, null) == 0
    assert lib.sf_dispatch(null, 4, 8, 300, null, null, null, null, null, null) == 1
    assert lib.sf_combine(null, null, null, null, 4, 64, 128, 2048, 0, null, null) == 1
    assert lib.sf_grouped_swiglu(null, null, null, null, 4, 8, 2048, 768, -1, 1, null, null, null,
                                 null, null, null, null) == 1
    assert lib.sf_expert_swiglu(null, 4, 10, 2048, 768, null, null, null, null) == 1
    # tree attention: bad counts, heads not a multiple, head dim, misaligned keys
    fake = 4096  # never dereferenced: every case below fails before a launch
    args = dict(qs=(4096, 128), ks=(1 << 20, 128), mask=(None, 0))

    def attn(q_heads, kv_heads, head_dim, queries=4, keys=8, k=fake):
        return lib.sf_tree_attention(fake, *args["qs"], k, *args["ks"], fake, *args["ks"],
                                     *args["mask"], queries, keys, q_heads, kv_heads, head_dim,
                                     0.1, fake, null)
    assert attn(32, 4, 128, queries=0) == 1
    assert attn(32, 5, 128) == 2
    assert attn(32, 4, 12) == 2
    assert attn(32, 4, 512) == 2
    assert attn(96, 4, 128) == 2          # 24 query heads per key/value head
    assert attn(32, 4, 128, k=fake + 8) == 3
    # query/key norm + rotary: head dim, token strides shorter than the heads or unaligned
    def qk(q_tok, k_tok, head_dim=128, tokens=2):
        return lib.sf_qk_norm_rope(fake, q_tok, fake, k_tok, tokens, 32, 4, head_dim, fake, fake,
                                   1e-6, fake, fake, fake, fake, null)
    assert qk(4096, 512, head_dim=64) == 2
    assert qk(4095, 512) == 1
    assert qk(4096, 511) == 1
    assert qk(5124, 5120) == 1
    assert qk(5120, 5120, tokens=0) == 0
    assert lib.sf_copy_h2d(null, null, 0, null) == 0
    assert lib.sf_copy_h2d(null, null, 16, null) == 1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setenv("SPECFIT_AMD_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(_native.NativeLibraryError, match="not found"):
        _native.lib()


def test_expert_key_and_snapshot_validation():
    assert ExpertKey(0, 3) < ExpertKey(1, 0)
    with pytest.raises(ValueError):
        ExpertKey(0, -1)
    stats = ExpertCacheStats(0, 0, 0, 0, 0)
    with pytest.raises(ValueError, match="empty slot"):
        CacheSlotSnapshot(0, None, 0, 0, 0, True, 0)
    slot = CacheSlotSnapshot(0, None, 0, 0, 0, False, 0)
    snap = GpuExpertCacheSnapshot("c", "q", 1, 0, 0, 0, (slot,), (), stats)
    assert snap.capacity == 1
    with pytest.raises(ValueError, match="every cache slot"):
        GpuExpertCacheSnapshot("c", "q", 2, 0, 0, 0, (slot,), (), stats)
    dup = (CacheSlotSnapshot(0, 5, 1, 0, 1, True, 0), CacheSlotSnapshot(1, 5, 1, 0, 2, True, 0))
    with pytest.raises(ValueError, match="unique"):
        GpuExpertCacheSnapshot("c", "q", 2, 0, 0, 0, dup, (), stats)


def test_observer_records_and_aggregates():
    obs = RecordingCacheTransitionObserver(run_id="r")
    for kind in (RuntimeEventKind.RESIDENT_HIT, RuntimeEventKind.RESIDENT_HIT,
                 RuntimeEventKind.INFLIGHT_JOIN):
        obs.record(kind=kind, cache_id="c", queue_id="q", expert_id=1, slot_id=0, generation=1)
    obs.record(kind=RuntimeEventKind.EVICT, cache_id="c", queue_id="q", expert_id=2, slot_id=0,
               generation=2, victim_expert_id=1)
    with pytest.raises(ValueError, match="sequence and ready event"):
        obs.record(kind=RuntimeEventKind.H2D_SUBMIT, cache_id="c", queue_id="q", expert_id=2,
                   slot_id=0, generation=2)
    events = obs.events()
    assert [e.sequence for e in events] == [0, 1, 2, 3]
    c = aggregate_cache_transition_counters(events)
    assert (c.resident_hits, c.inflight_joins, c.evictions, c.h2d_submissions) == (2, 1, 1, 0)
    obs.reset(run_id="r2")
    assert obs.cursor() == 0 and obs.run_id == "r2"


def test_workload_generator_is_seeded_and_zipf_skewed():
    a = make_layer(seed=3, num_experts=8, hidden_size=64, intermediate_size=32, zipf_s=1.1)
    b = make_layer(seed=3, num_experts=8, hidden_size=64, intermediate_size=32, zipf_s=1.1)
    assert torch.equal(a.experts, b.experts) and torch.equal(a.router, b.router)
    assert a.experts.shape == (8, 3 * 64 * 32) and a.expert_bytes == 3 * 64 * 32 * 2
    bias = zipf_bias(128, 1.1, 1.0, 0)
    p = torch.exp(bias.double())
    assert abs(p.sum().item() - 1.0) < 1e-9
    assert sorted(p.tolist(), reverse=True)[0] / sorted(p.tolist(), reverse=True)[1] == pytest.approx(2 ** 1.1)
    h = make_hidden(4, 64, seed=1, zipf_fold=True)
    assert torch.all(h[:, 0] == 1.0)
    assert expected_distinct_uniform(16) == pytest.approx(82.4, abs=0.1)

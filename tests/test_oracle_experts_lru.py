"""Pins the oracle's expert math and LRU restatement on the CPU.

Expert math: the bf16 eager restatement against transformers' eager
Qwen3MoeExperts on torch CPU (golden fixture + the reference's real-shape
case, hidden 2048 / intermediate 768 / 8 tokens / seed 41,
tests/gpu/test_qwen3_offloaded_experts.py:314-377), and the fp32 form
against an independent float64 torch evaluation.  LRU: the reference's known
answers (tests/unit/test_logical_replay.py:446-509,
tests/gpu/test_gpu_expert_cache.py:28-69,140-153,
tests/gpu/test_qwen3_offloaded_experts.py:158-312).
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

import oracle
from oracle.lru import LayerLRU, Slot

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_moe_bf16_oracle_against_transformers_golden():
    f = np.load(os.path.join(GOLDEN, "experts_hf_t6_h64_i32_e8_k3.npz"))
    H, I = int(f["hidden_size"]), int(f["intermediate_size"])
    packed = oracle.bf16_float(f["packed"])
    experts = {e: packed[e] for e in range(packed.shape[0])}
    got = oracle.moe_forward_bf16(oracle.bf16_float(f["hidden"]), f["index"],
                                  oracle.bf16_float(f["weights"]), experts, H, I, packed.shape[0])
    hf = oracle.bf16_float(f["out"])
    np.testing.assert_allclose(got, hf, rtol=1.6e-2, atol=1.6e-2)
    assert np.mean(got == hf) >= 0.9  # same rounding points: mostly bitwise


def _hf_eager_expert(x, gate_up, down):
    gate, up = F.linear(x, gate_up).chunk(2, dim=-1)
    return F.linear(F.silu(gate) * up, down)


def test_expert_bf16_oracle_at_qwen3_shape_against_torch_eager():
    H, I = 2048, 768
    g = torch.Generator().manual_seed(41)
    gate_up = torch.randn(2 * I, H, dtype=torch.bfloat16, generator=g)
    down = torch.randn(H, I, dtype=torch.bfloat16, generator=g)
    x = torch.randn(8, H, dtype=torch.bfloat16, generator=g)
    ref = _hf_eager_expert(x, gate_up, down).float().numpy()
    packed = torch.cat((gate_up.flatten(), down.flatten())).float().numpy()
    got = oracle.expert_forward_bf16(x.float().numpy(), packed, H, I)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() / scale <= 1e-2
    assert np.mean(got == ref) >= 0.9
    y32 = oracle.expert_forward_fp32(x.float().numpy(), packed, H, I)
    y64 = _hf_eager_expert(x.double(), gate_up.double(), down.double()).numpy()
    assert np.abs(y32 - y64).max() / np.abs(y64).max() <= 1e-6
    assert np.abs(got - y64).max() / np.abs(y64).max() <= 1e-2


def test_fp32_layer_is_the_weighted_sum_of_experts():
    rng = np.random.default_rng(1)
    H, I, E, T, K = 16, 8, 5, 4, 3
    experts = {e: (rng.standard_normal(3 * H * I) * 0.3).astype(np.float32) for e in range(E)}
    x = rng.standard_normal((T, H)).astype(np.float32)
    idx = np.array([[0, 1, 2], [4, 4, 1], [3, 0, 2], [1, 3, 4]], np.int64)
    w = rng.random((T, K)).astype(np.float32)
    out = oracle.moe_forward_fp32(x, idx, w, experts, H, I)
    for t in range(T):
        want = sum(w[t, j] * oracle.expert_forward_fp32(x[t:t + 1], experts[int(idx[t, j])], H, I)[0]
                   for j in range(K))
        np.testing.assert_allclose(out[t], want, rtol=1e-5, atol=1e-6)


def test_lru_replay_known_answer():
    state = LayerLRU(2, slots=[Slot(0, 0, 1, 0, 4), Slot(1)], lru_sequence=4,
                     submission_sequence=1, h2d_submissions=1)
    assert [state.access(e) for e in (0, 1, 2)] == ["hit", "miss", "miss"]
    assert (state.h2d_submissions, state.resident_hits, state.evictions) == (3, 1, 1)
    assert state.state() == ((0, 2, 2, 10), (1, 1, 1, 8))
    assert state.lru_sequence == 10 and state.submission_sequence == 3


def test_lru_switches_and_order():
    one = LayerLRU(1)
    for i in range(102):
        one.access(i % 3)
    assert (one.h2d_submissions, one.evictions, one.resident()) == (102, 101, {2})
    two = LayerLRU(2)
    for e in (0, 1, 0, 2):
        two.access(e)
    assert two.resident() == {0, 2} and two.evictions == 1


def test_resident_first_stats_deltas():
    def run(order_fn):
        lru = LayerLRU(2)
        for e in (1, 2):
            lru.access(e)
        before = (lru.h2d_submissions, lru.resident_hits, lru.evictions)
        for e in order_fn(lru):
            lru.access(e)
        return tuple(a - b for a, b in zip((lru.h2d_submissions, lru.resident_hits, lru.evictions),
                                            before))

    assert run(lambda lru: (0, 1, 2)) == (3, 0, 3)
    assert run(lambda lru: lru.resident_first((0, 1, 2))) == (1, 2, 1)

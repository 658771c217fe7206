"""Pins the oracle's dispatch and combine on the CPU.

Dispatch against numpy's stable argsort / bincount (a library routine) and
the reference edge cases (duplicated expert in a row, T = 0, 1, out-of-range
ids); combine against the reference test's known answer
(1 + 2^-8 - 1 in bf16, tests/gpu/test_qwen3_offloaded_experts.py:379-458),
against torch CPU's bf16 index_add_ applied expert by expert (the
reference's reduction, qwen3_offloaded_experts.py:155-164) and against an
fp64 sum for the fp32 mode.
"""
import numpy as np
import pytest
import torch

import oracle


@pytest.mark.parametrize("T,K,E,seed", [(64, 8, 128, 0), (1, 8, 128, 1), (300, 8, 3, 2),
                                        (17, 5, 256, 3), (4, 2, 4, 4)])
def test_dispatch_is_a_stable_sort(T, K, E, seed):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, E, size=(T, K)).astype(np.int64)
    idx[0, -1] = idx[0, 0]
    counts, offsets, perm, inv = oracle.dispatch(idx, E)
    flat = idx.reshape(-1)
    np.testing.assert_array_equal(perm, np.argsort(flat, kind="stable"))
    np.testing.assert_array_equal(counts[:E], np.bincount(flat, minlength=E))
    assert counts[E] == 0
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts[:E])]))
    np.testing.assert_array_equal(inv[perm], np.arange(T * K))


def test_dispatch_empty_and_invalid():
    counts, offsets, perm, inv = oracle.dispatch(np.zeros((0, 8), np.int64), 128)
    assert counts.sum() == 0 and offsets[-1] == 0 and perm.size == 0
    bad = np.array([[0, 5], [130, 2], [-1, 1]], np.int64)
    counts, offsets, perm, inv = oracle.dispatch(bad, 128)
    assert counts[128] == 2 and offsets[128] == 4
    assert inv.tolist()[2] == -1 and inv.tolist()[4] == -1
    np.testing.assert_array_equal(perm[:4], [0, 5, 3, 1])


def test_combine_known_answer():
    idx = np.array([[0, 1, 2]], np.int64)
    _, _, _, inv = oracle.dispatch(idx, 3)
    rows = oracle.bf16_bits(np.array([[1.0], [2.0 ** -8], [-1.0]], np.float32))
    assert oracle.bf16_float(oracle.combine(rows, idx, inv, 3))[0, 0] == 0.0
    assert oracle.bf16_float(oracle.combine(rows, idx, inv, 3, [0, 2, 1]))[0, 0] == 2.0 ** -8
    assert oracle.bf16_float(oracle.combine(rows, idx, inv, 3, accumulate_fp32=True))[0, 0] == 2.0 ** -8


def test_combine_matches_torch_bf16_index_add_per_expert():
    rng = np.random.default_rng(9)
    T, K, E, H = 20, 8, 32, 64
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    idx[3, 5] = idx[3, 2]
    counts, offsets, perm, inv = oracle.dispatch(idx, E)
    rows = oracle.bf16_bits(rng.standard_normal((T * K, H)).astype(np.float32))
    rows_t = torch.from_numpy(rows.view(np.int16)).view(torch.bfloat16)
    for order in (list(range(E)), list(rng.permutation(E))):
        out = torch.zeros(T, H, dtype=torch.bfloat16)
        for e in order:
            a, b = offsets[e], offsets[e + 1]
            if a == b:
                continue
            tokens = torch.from_numpy(perm[a:b] // K).long()
            for r, t in zip(range(a, b), tokens):  # rows of one expert in position order
                out.index_add_(0, t.view(1), rows_t[r:r + 1])
        rank = [0] * E
        for pos, e in enumerate(order):
            rank[e] = pos
        got = oracle.combine(rows, idx, inv, E, rank)
        np.testing.assert_array_equal(got, out.view(torch.int16).numpy().view(np.uint16))
    want64 = np.zeros((T, H))
    for i in range(T * K):
        want64[i // K] += oracle.bf16_float(rows[inv[i]]).astype(np.float64)
    got32 = oracle.bf16_float(oracle.combine(rows, idx, inv, E, accumulate_fp32=True))
    assert np.all(np.abs(got32 - want64) <= np.abs(want64) * 2.0 ** -8 + 1e-6)

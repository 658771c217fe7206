"""Draft-tree verification inputs on the host.

Known answers restate the reference's tests
(tests/gpu/test_eagle3_tree.py:517-561, 1000-1036, 1144-1152); the masks of
random trees are checked against a direct ancestor walk, the definition
used by eagle3_types.py:450-473.
"""
import math

import numpy as np
import pytest
import torch

from specfit_amd.runtime import Eagle3DraftTree, compact_tree_cache, synthetic_tree


def _tree():
    return Eagle3DraftTree(
        token_ids=(7, 2, 6, 3), parent_ids=(0, 0, 1, 2), depths=(1, 1, 2, 2),
        conditional_probabilities=(0.4, 0.6, 0.5, 0.7),
        cumulative_log_probabilities=(math.log(0.4), math.log(0.6), math.log(0.4 * 0.5),
                                      math.log(0.6 * 0.7)))


def test_attention_positions_and_non_left_acceptance():
    tree = _tree()
    mask = tree.verification_attention_mask(base_kv_length=2, device=torch.device("cpu"))
    expected = torch.tensor(((1, 0, 0, 0, 0), (1, 1, 0, 0, 0), (1, 0, 1, 0, 0),
                             (1, 1, 0, 1, 0), (1, 0, 1, 0, 1)), dtype=torch.bool)
    assert mask.shape == (1, 1, 5, 7) and mask.dtype == torch.bool
    assert mask[..., :2].all()
    assert torch.equal(mask[0, 0, :, 2:], expected)
    assert torch.equal(tree.verification_position_ids(base_kv_length=2, device="cpu"),
                       torch.tensor([[2, 3, 3, 4, 4]]))
    assert tree.accepted_path(torch.tensor([[2, 0, 3, 0, 4]])) == (2, 4)
    assert tree.source_raw_ids == (1, 2, 3, 4)
    assert tree.verification_raw_ids == (0, 1, 2, 3, 4)
    assert tree.raw_ids_for_verification_positions((0, 2, 4)) == (0, 2, 4)
    with pytest.raises(ValueError):
        tree.raw_ids_for_verification_positions((5,))
    assert torch.equal(tree.verification_token_ids(torch.tensor([[9]])),
                       torch.tensor([[9, 7, 2, 6, 3]]))


def test_seed_only_tree():
    seed_only = Eagle3DraftTree((), (), (), (), ())
    assert seed_only.draft_node_count == 0
    assert torch.equal(seed_only.verification_token_ids(torch.tensor([[13]])), torch.tensor([[13]]))
    assert torch.equal(seed_only.verification_position_ids(base_kv_length=2, device="cpu"),
                       torch.tensor([[2]]))
    assert seed_only.verification_attention_mask(base_kv_length=2, device="cpu").all()
    assert seed_only.accepted_path(torch.tensor([[14]])) == ()


def test_validation_errors():
    with pytest.raises(ValueError, match="cumulative"):
        Eagle3DraftTree((7,), (0,), (1,), (0.4,), (-0.4,))
    with pytest.raises(ValueError, match="precede"):
        Eagle3DraftTree((7,), (1,), (1,), (0.4,), (math.log(0.4),))
    with pytest.raises(ValueError, match="depth"):
        Eagle3DraftTree((7,), (0,), (2,), (0.4,), (math.log(0.4),))
    with pytest.raises(ValueError, match="distinct"):
        Eagle3DraftTree((7, 7), (0, 0), (1, 1), (0.4, 0.5), (math.log(0.4), math.log(0.5)))
    with pytest.raises(ValueError, match="equal lengths"):
        Eagle3DraftTree((7, 8), (0,), (1,), (0.4,), (math.log(0.4),))
    with pytest.raises(ValueError, match="probabilities must be in"):
        Eagle3DraftTree((7,), (0,), (1,), (1.5,), (math.log(1.5),))
    with pytest.raises(ValueError, match="shape"):
        _tree().verification_token_ids(torch.tensor([1, 2]))
    with pytest.raises(ValueError, match="do not match"):
        _tree().accepted_path(torch.tensor([[1, 2]]))


def _walk_mask(tree, base):
    q = 1 + tree.draft_node_count
    m = torch.zeros((1, 1, q, base + q), dtype=torch.bool)
    m[..., :base] = True
    for node in range(q):
        a = node
        while True:
            m[0, 0, node, base + a] = True
            if a == 0:
                break
            a = tree.parent_ids[a - 1]
    return m


@pytest.mark.parametrize("nodes,depth,seed", [(60, 6, 0), (13, 3, 1), (7, 7, 2), (40, 2, 3)])
def test_synthetic_tree_masks_match_an_ancestor_walk(nodes, depth, seed):
    tree = synthetic_tree(nodes, depth, seed=seed, vocab=1000)
    assert tree.draft_node_count == nodes and max(tree.depths) == depth
    for base in (0, 3, 1024):
        assert torch.equal(tree.verification_attention_mask(base_kv_length=base, device="cpu"),
                           _walk_mask(tree, base))
    # a chain path through the tree is accepted exactly when the verifier
    # predicts each node's token at its parent
    deepest = max(range(1, nodes + 1), key=lambda n: tree.depths[n - 1])
    path = []
    n = deepest
    while n:
        path.append(n)
        n = tree.parent_ids[n - 1]
    path.reverse()
    verifier = np.full(1 + nodes, -1)
    parent = 0
    for n in path:
        verifier[parent] = tree.token_ids[n - 1]
        parent = n
    assert tree.accepted_path(torch.tensor(verifier).unsqueeze(0)) == tuple(path)


def test_compact_tree_cache_keeps_prefix_and_selected_positions():
    from transformers import DynamicCache

    cache = DynamicCache()
    g = torch.Generator().manual_seed(3)
    base, nodes = 5, 6
    for layer in range(3):
        k = torch.randn(1, 2, base + 1 + nodes, 4, generator=g)
        v = torch.randn(1, 2, base + 1 + nodes, 4, generator=g)
        cache.update(k, v, layer)
    keys = [layer.keys.clone() for layer in cache.layers]
    positions = (0, 2, 5)
    compact_tree_cache(cache, base_kv_length=base, verification_positions=positions,
                       verification_node_count=1 + nodes)
    assert cache.get_seq_length() == base + len(positions)
    for layer, before in zip(cache.layers, keys):
        assert torch.equal(layer.keys[..., :base, :], before[..., :base, :])
        assert torch.equal(layer.keys[..., base:, :],
                           before[..., [base + p for p in positions], :])
    with pytest.raises(RuntimeError, match="unexpected length"):
        compact_tree_cache(cache, base_kv_length=base, verification_positions=positions,
                           verification_node_count=1 + nodes)

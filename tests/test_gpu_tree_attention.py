"""K5 tree attention and the verify-subtree forward on the device.

K5 is a floating-point kernel: it is compared with a torch fp32 reference of
the same masked grouped-query attention (the math of transformers'
sdpa_attention_forward, which the reference's target uses).  The model-level
tests restate tests/gpu/test_eagle3_tree.py:1435-1530 (each tree node's
logits equal an independent causal decode of its path) on a bf16 offloaded
model, so the tolerance is bf16's rather than fp32's.
"""
import math

import pytest
import torch

from specfit_amd import ops
from specfit_amd.runtime import (TREE_ATTENTION, Eagle3DraftTree, build_offloaded_qwen3,
                                 register_tree_attention, synthetic_tree, verify_draft_tree)

pytestmark = pytest.mark.gpu


def _reference(q, k, v, mask, scale):
    """fp32 masked GQA attention: q [B,Hq,Q,D], k/v [B,Hkv,S,D], mask
    [B,1,Q,S] bool or None (causal aligned to the end)."""
    B, Hq, Q, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    G = Hq // Hkv
    kf = k.float().repeat_interleave(G, dim=1)
    vf = v.float().repeat_interleave(G, dim=1)
    s = torch.matmul(q.float(), kf.transpose(-1, -2).contiguous()) * scale
    if mask is None:
        qi = torch.arange(Q, device=q.device)[:, None]
        si = torch.arange(S, device=q.device)[None, :]
        mask = (si <= S - Q + qi).view(1, 1, Q, S)
    s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)
    return torch.matmul(p, vf).transpose(1, 2)  # [B, Q, Hq, D]


def _check(out, ref):
    assert out.shape == ref.shape and out.dtype == torch.bfloat16
    err = (out.float() - ref).abs()
    scale = ref.abs().max().clamp_min(1e-6)
    assert (err.max() / scale).item() <= 1e-2, (err.max() / scale).item()
    assert torch.all(err <= 8e-3 * ref.abs() + 2e-3 * scale)


def _rand(shape, device, g, std=1.0):
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16).to(device)


def test_verification_shape_with_tree_mask(device):
    g = torch.Generator().manual_seed(11)
    tree = synthetic_tree(60, 6, seed=5, vocab=151936)
    base, Q, Hq, Hkv, D = 1024, 61, 32, 4, 128
    S = base + Q
    q = _rand((1, Q, Hq, D), device, g).transpose(1, 2)  # HF layout: a transposed view
    k = _rand((1, Hkv, S, D), device, g)
    v = _rand((1, Hkv, S, D), device, g)
    mask = tree.verification_attention_mask(base_kv_length=base, device=device)
    scale = D ** -0.5
    out = ops.tree_attention(q, k, v, mask, scale)
    _check(out, _reference(q, k, v, mask, scale))
    again = ops.tree_attention(q, k, v, mask, scale)
    assert torch.equal(out, again)  # run-to-run identical


@pytest.mark.parametrize("Hq,Hkv,D", [(4, 4, 8), (4, 2, 8), (8, 2, 64), (16, 4, 128),
                                      (16, 1, 128), (32, 4, 96), (8, 2, 256),
                                      (32, 4, 128), (8, 4, 64), (8, 4, 128), (32, 2, 64),
                                      (64, 4, 128)])  # the last: Qwen3-235B-A22B attention
@pytest.mark.parametrize("Q,S", [(1, 1), (1, 300), (7, 7), (61, 1085), (130, 130)])
def test_shapes_causal_and_masked(device, Hq, Hkv, D, Q, S):
    if D == 256 and Hq // Hkv > 4:
        pytest.skip("exceeds the kernel's LDS budget")
    g = torch.Generator().manual_seed(Hq * 1000 + D + Q + S)
    q = _rand((1, Hq, Q, D), device, g)
    k = _rand((1, Hkv, S, D), device, g)
    v = _rand((1, Hkv, S, D), device, g)
    scale = 1.0 / math.sqrt(D)
    _check(ops.tree_attention(q, k, v, None, scale), _reference(q, k, v, None, scale))
    gm = torch.Generator().manual_seed(S)
    mask = (torch.rand((1, 1, Q, S), generator=gm) < 0.3).to(device)
    mask[..., 0] = True
    _check(ops.tree_attention(q, k, v, mask, scale), _reference(q, k, v, mask, scale))


def test_mfma_and_loop_kernels_agree(device):
    """The verification shape through the MFMA kernel (16-byte aligned rows)
    and through the loop kernel (a query view one element off alignment):
    both within the fp32 reference's tolerance, and within bf16 rounding of
    each other."""
    g = torch.Generator().manual_seed(12)
    tree = synthetic_tree(60, 6, seed=6, vocab=151936)
    base, Q, Hq, Hkv, D = 1024, 61, 32, 4, 128
    S = base + Q
    qbuf = _rand((1, Q, Hq, D + 8), device, g)
    q_aligned = qbuf[..., :D].transpose(1, 2)
    q_shifted = torch.empty((1, Q, Hq, D + 1), dtype=torch.bfloat16, device=device)
    q_shifted[..., 1:] = qbuf[..., :D]
    q_off = q_shifted[..., 1:].transpose(1, 2)  # same values, rows 2 bytes off alignment
    k = _rand((1, Hkv, S, D), device, g)
    v = _rand((1, Hkv, S, D), device, g)
    mask = tree.verification_attention_mask(base_kv_length=base, device=device)
    scale = D ** -0.5
    ref = _reference(q_aligned, k, v, mask, scale)
    fast = ops.tree_attention(q_aligned, k, v, mask, scale)
    loop = ops.tree_attention(q_off, k, v, mask, scale)
    _check(fast, ref)
    _check(loop, ref)
    assert ((fast.float() - loop.float()).abs().max() / ref.abs().max()).item() <= 1e-2


def test_fully_masked_row_is_zero_and_large_logits_are_stable(device):
    g = torch.Generator().manual_seed(2)
    q = _rand((1, 8, 5, 128), device, g, std=30.0)
    k = _rand((1, 2, 200, 128), device, g, std=30.0)
    v = _rand((1, 2, 200, 128), device, g)
    mask = torch.ones((1, 1, 5, 200), dtype=torch.bool, device=device)
    mask[0, 0, 3] = False
    out = ops.tree_attention(q, k, v, mask, 0.088)
    assert torch.count_nonzero(out[0, 3]) == 0
    ref = _reference(q, k, v, mask, 0.088)
    keep = [0, 1, 2, 4]
    _check(out[:, keep], ref[:, keep])
    assert torch.isfinite(out.float()).all()


def test_argument_errors(device):
    q = torch.zeros((1, 4, 2, 8), dtype=torch.bfloat16, device=device)
    k = torch.zeros((1, 3, 5, 8), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="multiple"):
        ops.tree_attention(q, k, k, None, 1.0)
    k = torch.zeros((1, 2, 5, 8), dtype=torch.bfloat16, device=device)
    with pytest.raises(TypeError, match="bool"):
        ops.tree_attention(q, k, k, torch.zeros((1, 1, 2, 5), device=device), 1.0)
    with pytest.raises(ValueError, match="mask"):
        ops.tree_attention(q, k, k, torch.ones((1, 1, 2, 4), dtype=torch.bool, device=device), 1.0)


# ------------------------------------------------------------ model level --
def _tiny_model(layers=2, seed=7):
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    torch.manual_seed(seed)
    config = Qwen3MoeConfig(vocab_size=64, hidden_size=32, intermediate_size=48,
                            moe_intermediate_size=16, num_hidden_layers=layers,
                            num_attention_heads=4, num_key_value_heads=2, num_experts=4,
                            num_experts_per_tok=2, max_position_embeddings=64, bos_token_id=1,
                            eos_token_id=63, pad_token_id=62, norm_topk_prob=True)
    return Qwen3MoeForCausalLM(config).to(torch.bfloat16).eval()


def _offloaded(model, device, attn):
    register_tree_attention()
    model.config._attn_implementation = attn
    return build_offloaded_qwen3(model, device=device, slots_per_layer=2)


def _tree():
    return Eagle3DraftTree(
        token_ids=(5, 6, 9, 10), parent_ids=(0, 0, 1, 2), depths=(1, 1, 2, 2),
        conditional_probabilities=(0.6, 0.4, 0.5, 0.5),
        cumulative_log_probabilities=(math.log(0.6), math.log(0.4), math.log(0.6 * 0.5),
                                      math.log(0.4 * 0.5)))


@torch.inference_mode()
def test_each_tree_node_matches_an_independent_causal_path(device):
    loaded = _offloaded(_tiny_model(1), device, TREE_ATTENTION)
    target = loaded.model
    prefix = torch.tensor([[1, 7, 11]], device=device)
    tree = _tree()
    prefill = target(input_ids=prefix, attention_mask=torch.ones_like(prefix), use_cache=True,
                     logits_to_keep=1)
    seed = prefill.logits.argmax(dim=-1)
    verify_ids = tree.verification_token_ids(seed)
    tree_out = target(input_ids=verify_ids,
                      attention_mask=tree.verification_attention_mask(
                          base_kv_length=prefix.shape[1], device=device),
                      position_ids=tree.verification_position_ids(
                          base_kv_length=prefix.shape[1], device=device),
                      past_key_values=prefill.past_key_values, use_cache=True, logits_to_keep=0)
    for node in range(1 + tree.draft_node_count):
        path = []
        cur = node
        while cur:
            path.append(tree.token_ids[cur - 1])
            cur = tree.parent_ids[cur - 1]
        path.reverse()
        ids = torch.cat((prefix, seed, prefix.new_tensor(path).unsqueeze(0)), dim=1)
        expected = target(input_ids=ids, attention_mask=torch.ones_like(ids), use_cache=False,
                          logits_to_keep=1).logits[0, -1].float()
        actual = tree_out.logits[0, node].float()
        torch.testing.assert_close(actual, expected, atol=3e-2 * expected.abs().max().item(),
                                   rtol=3e-2)
        top2 = expected.topk(2).values
        if (top2[0] - top2[1]).item() > 0.05 * expected.abs().max().item():
            assert int(actual.argmax()) == int(expected.argmax())
    loaded.close()


@torch.inference_mode()
def test_tree_attention_model_matches_sdpa_model(device):
    base = _tiny_model(2, seed=9)
    state = {k: v.clone() for k, v in base.state_dict().items()}
    ours = _offloaded(base, device, TREE_ATTENTION)
    ref_model = _tiny_model(2, seed=9)
    ref_model.load_state_dict(state)
    theirs = _offloaded(ref_model, device, "sdpa")
    ids = torch.tensor([[1, 5, 9, 12, 3, 44, 21]], device=device)
    a = ours.model(input_ids=ids, attention_mask=torch.ones_like(ids)).logits.float()
    b = theirs.model(input_ids=ids, attention_mask=torch.ones_like(ids)).logits.float()
    torch.testing.assert_close(a, b, atol=3e-2 * b.abs().max().item(), rtol=3e-2)
    ours.close()
    theirs.close()


@torch.inference_mode()
def test_verify_draft_tree_commits_the_accepted_path(device):
    from transformers import DynamicCache

    loaded = _offloaded(_tiny_model(2, seed=4), device, TREE_ATTENTION)
    target = loaded.model
    prefix = torch.tensor([[1, 7, 11, 19]], device=device)
    cache = DynamicCache()
    prefill = target(input_ids=prefix, attention_mask=torch.ones_like(prefix),
                     past_key_values=cache, use_cache=True, logits_to_keep=1)
    seed = prefill.logits.argmax(dim=-1)
    # A chain that follows the target's own greedy decode is accepted whole
    # (up to bf16 near-ties), plus distractor siblings that never are.
    chain, ids = [], torch.cat((prefix, seed), dim=1)
    for _ in range(3):
        nxt = int(target(input_ids=ids, attention_mask=torch.ones_like(ids),
                         use_cache=False, logits_to_keep=1).logits[0, -1].argmax())
        chain.append(nxt)
        ids = torch.cat((ids, ids.new_tensor([[nxt]])), dim=1)
    tokens, parents, depths, probs = [], [], [], []
    parent = 0
    for depth, tok in enumerate(chain, start=1):
        tokens += [tok, (tok + 1) % 61]
        parents += [parent, parent]
        depths += [depth, depth]
        probs += [0.7, 0.3]
        parent = len(tokens) - 1
    cums, cum = [], {0: 0.0}
    for node, (p, par) in enumerate(zip(probs, parents), start=1):
        cum[node] = cum[par] + math.log(p)
        cums.append(cum[node])
    tree = Eagle3DraftTree(tuple(tokens), tuple(parents), tuple(depths), tuple(probs), tuple(cums))
    base = cache.get_seq_length()
    result = verify_draft_tree(target, tree, seed, cache)
    assert result.base_kv_length == base
    assert result.verification_positions == (0,) + result.accepted_node_ids
    assert cache.get_seq_length() == base + len(result.verification_positions)
    assert result.accepted_node_ids == tree.accepted_path(result.verifier_tokens)
    assert torch.equal(result.committed, result.verify_ids[:, result.verification_positions])
    last = result.verification_positions[-1]
    assert torch.equal(result.pending_seed, result.verifier_tokens[:, last:last + 1])
    # The seed's verification logits equal a causal forward of [prefix, seed].
    ids = torch.cat((prefix, seed), dim=1)
    expected = target(input_ids=ids, attention_mask=torch.ones_like(ids), use_cache=False,
                      logits_to_keep=1).logits[0, -1].float()
    torch.testing.assert_close(result.logits[0, 0].float(), expected,
                               atol=3e-2 * expected.abs().max().item(), rtol=3e-2)
    # The committed cache continues decoding: one more step runs on it.
    nxt = target(input_ids=result.pending_seed, past_key_values=cache, use_cache=True)
    assert cache.get_seq_length() == base + len(result.verification_positions) + 1
    assert torch.isfinite(nxt.logits.float()).all()
    loaded.close()

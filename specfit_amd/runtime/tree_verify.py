"""Draft-tree verification: the verify-subtree forward of the target model.

Restates the reference's verification inputs and step:
- ``Eagle3DraftTree`` and its verification helpers
  (src/specfit/runtime/eagle3_types.py:312-473): same fields, validation
  errors, raw ids, token ids, position ids, ancestor mask and accepted path;
- ``verify_draft_tree``: the verification call of
  ``ShallowTreeSpeculator._generate`` (eagle3_tree.py:1202-1290): one target
  forward over [pending seed, draft nodes] with the tree mask and depth
  positions against the cached prefix, greedy verifier tokens, the accepted
  path and its EOS cut;
- ``compact_tree_cache`` (eagle3_tree.py:833-858): keep the prefix plus the
  verified positions in the KV cache.

The target's attention layers run the HIP tree-attention kernel when the
model's attention implementation is ``TREE_ATTENTION`` (see
``tree_attention.register_tree_attention``) and its MoE blocks run the
offloaded HIP experts.
"""
from __future__ import annotations

from dataclasses import dataclass
from math import isclose, isfinite, log

import numpy as np
import torch


@dataclass(frozen=True, slots=True)
class Eagle3DraftTree:
    """A draft tree of ``len(token_ids)`` nodes (node ids 1..N; 0 is the
    pending seed).  Field meaning and validation as eagle3_types.py:312-401."""

    token_ids: tuple[int, ...]
    parent_ids: tuple[int, ...]
    depths: tuple[int, ...]
    conditional_probabilities: tuple[float, ...]
    cumulative_log_probabilities: tuple[float, ...]
    source_raw_ids: tuple[int, ...] = ()

    def __post_init__(self) -> None:
        size = len(self.token_ids)
        if not self.source_raw_ids and size:
            object.__setattr__(self, "source_raw_ids", tuple(range(1, size + 1)))
        if any(len(f) != size for f in (self.parent_ids, self.depths,
                                         self.conditional_probabilities,
                                         self.cumulative_log_probabilities,
                                         self.source_raw_ids)):
            raise ValueError("draft tree fields must have equal lengths")
        if any(isinstance(r, bool) or not isinstance(r, int) or r <= 0
               for r in self.source_raw_ids):
            raise ValueError("source raw IDs must be positive integers")
        if len(set(self.source_raw_ids)) != size:
            raise ValueError("source raw IDs must be unique")
        siblings: dict[int, set[int]] = {}
        cumulative = {0: 0.0}
        for node, (tok, parent, depth, prob, cum) in enumerate(
                zip(self.token_ids, self.parent_ids, self.depths,
                    self.conditional_probabilities, self.cumulative_log_probabilities), start=1):
            if isinstance(tok, bool) or not isinstance(tok, int) or tok < 0:
                raise ValueError("tree token IDs must be non-negative integers")
            if isinstance(parent, bool) or not isinstance(parent, int) or not 0 <= parent < node:
                raise ValueError("tree parents must precede their children")
            if isinstance(depth, bool) or not isinstance(depth, int):
                raise ValueError("tree depths must contain integers")
            if depth != (0 if parent == 0 else self.depths[parent - 1]) + 1:
                raise ValueError("tree node depth differs from its parent")
            if not isfinite(prob) or not 0.0 < prob <= 1.0:
                raise ValueError("conditional probabilities must be in (0, 1]")
            if not isfinite(cum):
                raise ValueError("cumulative log probabilities must be finite")
            if not isclose(cum, cumulative[parent] + log(prob), rel_tol=1e-5, abs_tol=1e-6):
                raise ValueError("cumulative score differs from its parent and conditional "
                                 "probability")
            seen = siblings.setdefault(parent, set())
            if tok in seen:
                raise ValueError("siblings must use distinct token IDs")
            seen.add(tok)
            cumulative[node] = cum

    @property
    def draft_node_count(self) -> int:
        return len(self.token_ids)

    @property
    def verification_raw_ids(self) -> tuple[int, ...]:
        return (0,) + self.source_raw_ids

    def raw_ids_for_verification_positions(self, verification_positions) -> tuple[int, ...]:
        if any(isinstance(p, bool) or not isinstance(p, int) or not 0 <= p <= self.draft_node_count
               for p in verification_positions):
            raise ValueError("verification positions are outside the draft tree")
        raw = self.verification_raw_ids
        return tuple(raw[p] for p in verification_positions)

    def verification_token_ids(self, pending_seed: torch.Tensor) -> torch.Tensor:
        """[1, 1 + N]: the pending seed followed by the draft tokens."""
        if pending_seed.shape != (1, 1):
            raise ValueError("pending_seed must have shape [1, 1]")
        return torch.cat((pending_seed, pending_seed.new_tensor(self.token_ids).unsqueeze(0)), dim=1)

    def verification_position_ids(self, *, base_kv_length: int, device) -> torch.Tensor:
        """[1, 1 + N]: base for the seed, base + depth for node."""
        if base_kv_length < 0:
            raise ValueError("base_kv_length must be non-negative")
        return torch.tensor((base_kv_length,) + tuple(base_kv_length + d for d in self.depths),
                            dtype=torch.long, device=device).unsqueeze(0)

    def ancestor_matrix(self) -> np.ndarray:
        """bool [1 + N, 1 + N]: row n admits n and its ancestors (0 included)."""
        q = 1 + self.draft_node_count
        m = np.zeros((q, q), dtype=bool)
        m[:, 0] = True
        for node in range(1, q):
            m[node] = m[self.parent_ids[node - 1]]
            m[node, node] = True
        return m

    def verification_attention_mask(self, *, base_kv_length: int, device) -> torch.Tensor:
        """bool [1, 1, 1 + N, base + 1 + N]: the whole prefix plus each
        node's ancestor chain (eagle3_types.py:450-473).  Built on the host
        and copied once."""
        if base_kv_length < 0:
            raise ValueError("base_kv_length must be non-negative")
        q = 1 + self.draft_node_count
        host = np.zeros((q, base_kv_length + q), dtype=bool)
        host[:, :base_kv_length] = True
        host[:, base_kv_length:] = self.ancestor_matrix()
        return torch.from_numpy(host).to(device).view(1, 1, q, base_kv_length + q)

    def accepted_path(self, verifier_token_ids: torch.Tensor) -> tuple[int, ...]:
        """Greedy acceptance: from the seed, follow the child whose token is
        the verifier's prediction at its parent (eagle3_types.py:475-502)."""
        if verifier_token_ids.shape != (1, 1 + self.draft_node_count):
            raise ValueError("verifier tokens do not match the draft tree")
        verifier = tuple(int(v) for v in verifier_token_ids[0].tolist())
        children: dict[int, list[int]] = {}
        for node, parent in enumerate(self.parent_ids, start=1):
            children.setdefault(parent, []).append(node)
        accepted = []
        parent = 0
        while True:
            predicted = verifier[parent]
            matching = tuple(n for n in children.get(parent, ())
                             if self.token_ids[n - 1] == predicted)
            if not matching:
                break
            if len(matching) != 1:
                raise RuntimeError("target token matches multiple sibling nodes")
            parent = matching[0]
            accepted.append(parent)
        return tuple(accepted)


@dataclass(frozen=True)
class TreeVerification:
    """Result of one verification forward."""

    verify_ids: torch.Tensor            # [1, 1 + N]
    logits: torch.Tensor                # [1, 1 + N, V]
    verifier_tokens: torch.Tensor       # [1, 1 + N] greedy target tokens
    accepted_node_ids: tuple[int, ...]
    verification_positions: tuple[int, ...]  # (0,) + accepted, cut at EOS
    committed: torch.Tensor             # verify_ids at verification_positions
    base_kv_length: int
    stopped_on_eos: bool
    pending_seed: torch.Tensor          # [1, 1] next seed


def _first_eos_position(committed: torch.Tensor, eos_token_ids) -> int | None:
    if not eos_token_ids:
        return None
    for i, tok in enumerate(committed[0].tolist()):
        if int(tok) in eos_token_ids:
            return i
    return None


def compact_tree_cache(cache, *, base_kv_length: int, verification_positions: tuple[int, ...],
                       verification_node_count: int) -> None:
    """Keep the prefix and the verified positions of every cache layer
    (eagle3_tree.py:833-858)."""
    expected = base_kv_length + verification_node_count
    index = None
    dest = slice(base_kv_length, base_kv_length + len(verification_positions))
    for layer in cache.layers:
        if layer.get_seq_length() != expected:
            raise RuntimeError("target cache layer has an unexpected length")
        if index is None or index.device != layer.keys.device:
            index = torch.tensor(tuple(base_kv_length + p for p in verification_positions),
                                 dtype=torch.long, device=layer.keys.device)
        keys = layer.keys.index_select(-2, index)
        values = layer.values.index_select(-2, index)
        layer.keys[..., dest, :].copy_(keys)
        layer.values[..., dest, :].copy_(values)
    cache.crop(base_kv_length + len(verification_positions))


def verify_draft_tree(target, tree: Eagle3DraftTree, pending_seed: torch.Tensor, cache, *,
                      eos_token_ids=(), commit: bool = True) -> TreeVerification:
    """One verification forward of ``tree`` against ``cache`` (a HF
    DynamicCache holding the committed prefix), as eagle3_tree.py:1202-1290:
    target(input_ids=[seed, drafts], attention_mask=tree mask,
    position_ids=base + depth, past_key_values=cache, use_cache=True,
    logits_to_keep=0); greedy verifier tokens; accepted path; EOS cut; and,
    when ``commit``, the KV compaction to the verified positions."""
    verify_ids = tree.verification_token_ids(pending_seed)
    base = cache.get_seq_length()
    device = verify_ids.device
    mask = tree.verification_attention_mask(base_kv_length=base, device=device)
    positions = tree.verification_position_ids(base_kv_length=base, device=device)
    outputs = target(input_ids=verify_ids, attention_mask=mask, position_ids=positions,
                     past_key_values=cache, use_cache=True, logits_to_keep=0)
    verifier = outputs.logits.argmax(dim=-1)
    accepted = tree.accepted_path(verifier)
    vpos = (0,) + accepted
    committed = verify_ids[:, vpos]
    stopped = False
    eos = _first_eos_position(committed, set(eos_token_ids))
    if eos is not None:
        vpos = vpos[:eos + 1]
        accepted = vpos[1:]
        committed = verify_ids[:, vpos]
        stopped = True
    if commit:
        compact_tree_cache(cache, base_kv_length=base, verification_positions=vpos,
                           verification_node_count=verify_ids.shape[1])
    last = vpos[-1]
    return TreeVerification(verify_ids=verify_ids, logits=outputs.logits,
                            verifier_tokens=verifier, accepted_node_ids=accepted,
                            verification_positions=vpos, committed=committed,
                            base_kv_length=base, stopped_on_eos=stopped,
                            pending_seed=verifier[:, last:last + 1])


def synthetic_tree(nodes: int, depth: int, *, seed: int, vocab: int) -> Eagle3DraftTree:
    """A seeded draft tree of exactly ``nodes`` nodes and depth ``depth``
    (each level gets nodes/depth nodes, the first levels take the remainder;
    parents are drawn from the previous level, sibling tokens are distinct
    and probabilities are consistent)."""
    if nodes < depth or depth < 1:
        raise ValueError("need nodes >= depth >= 1")
    rng = np.random.default_rng(seed)
    per = [nodes // depth + (1 if i < nodes % depth else 0) for i in range(depth)]
    token_ids, parent_ids, depths, probs, cums = [], [], [], [], []
    cum_of = {0: 0.0}
    prev = [0]
    used: dict[int, set[int]] = {}
    for level, count in enumerate(per, start=1):
        cur = []
        for _ in range(count):
            parent = int(prev[rng.integers(len(prev))])
            taken = used.setdefault(parent, set())
            tok = int(rng.integers(vocab))
            while tok in taken:
                tok = int(rng.integers(vocab))
            taken.add(tok)
            p = float(rng.uniform(0.05, 0.95))
            node = len(token_ids) + 1
            token_ids.append(tok)
            parent_ids.append(parent)
            depths.append(level)
            probs.append(p)
            cums.append(cum_of[parent] + log(p))
            cum_of[node] = cums[-1]
            cur.append(node)
        prev = cur
    return Eagle3DraftTree(tuple(token_ids), tuple(parent_ids), tuple(depths), tuple(probs),
                           tuple(cums))

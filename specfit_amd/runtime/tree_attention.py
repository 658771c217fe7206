"""The HIP tree-attention kernel as a transformers attention implementation.

``register_tree_attention()`` registers ``TREE_ATTENTION`` in transformers'
``AttentionInterface`` (with the sdpa mask builder, so masks stay 4-D bool
and pure-causal prefixes may arrive as ``None``).  A Qwen3-MoE model whose
``config._attn_implementation`` is ``TREE_ATTENTION`` then runs K5
(``sf_tree_attention``) in every attention layer, in place of
``sdpa_attention_forward`` (transformers/integrations/sdpa_attention.py),
which is what the reference's target model uses for the verification
forward (``load_offloaded_qwen3(..., attn_implementation="sdpa")``,
src/specfit/runtime/qwen3_offloaded_model.py:667-682).
"""
from __future__ import annotations

import torch

from .. import ops

TREE_ATTENTION = "specfit_tree"


def tree_attention_forward(module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                           value: torch.Tensor, attention_mask: torch.Tensor | None,
                           dropout: float = 0.0, scaling: float | None = None,
                           is_causal: bool | None = None, **kwargs) -> tuple[torch.Tensor, None]:
    """Same contract as sdpa_attention_forward: query [B, Hq, Q, D],
    key/value [B, Hkv, S, D], a 4-D bool mask or None (causal, aligned to
    the end of the keys); returns ([B, Q, Hq, D], None)."""
    if dropout:
        raise ValueError("tree attention is inference-only (dropout must be 0)")
    if kwargs.get("position_bias") is not None:
        raise ValueError("tree attention does not take a position bias")
    if attention_mask is None and is_causal is False and query.shape[2] > 1:
        raise ValueError("tree attention without a mask is causal")
    scale = scaling if scaling is not None else query.shape[-1] ** -0.5
    return ops.tree_attention(query, key, value, attention_mask, scale), None


def register_tree_attention() -> str:
    """Register K5 with transformers; returns the implementation name."""
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask

    AttentionInterface.register(TREE_ATTENTION, tree_attention_forward)
    ALL_MASK_ATTENTION_FUNCTIONS.register(TREE_ATTENTION, sdpa_mask)
    return TREE_ATTENTION

"""Qwen3-MoE attention layer with the fused query/key norm + rotary kernel.

Drop-in for transformers' ``Qwen3MoeAttention`` (tf:121-190, forward
tf:151-190): the same projections, norms, attributes and forward signature,
and the same attention-implementation dispatch (the tree-attention kernel
K5 when the config selects it).  For batch 1 with head_dim 128 the query and
key norms and ``apply_rotary_pos_emb`` (tf:162-167) run as one kernel (K7)
instead of twelve; other shapes take the module's own norms and the eager
rotary function.  With the norms on K6 both paths give the same bits.

When the three projections have no bias and one dtype and device, their
weights are moved into one [q; k; v] buffer (each projection's weight
becomes a view of its rows) and the forward runs one GEMM over it instead of
three; K7 reads the query and key heads straight out of the fused rows.  A
projection whose weight was replaced afterwards (``module.to``, a new
Parameter) turns the fused GEMM off for that layer.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import ops


class Qwen3AttentionHip(nn.Module):
    def __init__(self, attention: nn.Module) -> None:
        super().__init__()
        for name in ("config", "layer_idx", "head_dim", "num_key_value_groups", "scaling",
                     "attention_dropout", "is_causal", "sliding_window"):
            setattr(self, name, getattr(attention, name))
        self.q_proj, self.k_proj = attention.q_proj, attention.k_proj
        self.v_proj, self.o_proj = attention.v_proj, attention.o_proj
        self.q_norm, self.k_norm = attention.q_norm, attention.k_norm
        self._qkv = None
        self._qkv_rows = ()
        self._qkv_ptrs = ()
        self._fuse_projections()

    def _fuse_projections(self) -> None:
        projections = (self.q_proj, self.k_proj, self.v_proj)
        weights = [p.weight for p in projections]
        if (any(p.bias is not None for p in projections)
                or len({(w.dtype, w.device, w.shape[1:]) for w in weights}) != 1
                or weights[0].dim() != 2 or weights[0].is_meta):
            return
        fused = torch.cat([w.detach() for w in weights])
        rows = tuple(w.shape[0] for w in weights)
        for projection, view in zip(projections, fused.split(rows)):
            projection.weight = nn.Parameter(view, requires_grad=projection.weight.requires_grad)
        self._qkv, self._qkv_rows = fused, rows
        self._qkv_ptrs = tuple(p.weight.data_ptr() for p in projections)

    def _fused_projection(self) -> bool:
        return (self._qkv is not None and (self.q_proj.weight.data_ptr(),
                                           self.k_proj.weight.data_ptr(),
                                           self.v_proj.weight.data_ptr()) == self._qkv_ptrs)

    @classmethod
    def from_module(cls, attention: nn.Module) -> "Qwen3AttentionHip":
        """Wrap an HF ``Qwen3MoeAttention`` (shares its submodules)."""
        return cls(attention)

    def _fused(self, hidden_states: torch.Tensor, cos: torch.Tensor) -> bool:
        return (hidden_states.dim() == 3 and hidden_states.shape[0] == 1
                and self.head_dim == 128 and hidden_states.dtype == torch.bfloat16
                and cos.dtype == torch.bfloat16
                and self.q_norm.variance_epsilon == self.k_norm.variance_epsilon
                and self.q_norm.weight.dtype == torch.bfloat16
                and self.k_norm.weight.dtype == torch.bfloat16)

    def forward(self, hidden_states: torch.Tensor, position_embeddings, attention_mask,
                past_key_values=None, **kwargs):
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        from transformers.models.qwen3_moe.modeling_qwen3_moe import (apply_rotary_pos_emb,
                                                                        eager_attention_forward)

        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        cos, sin = position_embeddings
        fused_projection = self._fused_projection()
        if fused_projection:
            nq, nk, _ = self._qkv_rows
            qkv = F.linear(hidden_states, self._qkv)
            q = qkv[..., :nq].view(hidden_shape)
            k = qkv[..., nq:nq + nk].view(hidden_shape)
        else:
            q = self.q_proj(hidden_states).view(hidden_shape)
            k = self.k_proj(hidden_states).view(hidden_shape)
        if self._fused(hidden_states, cos):
            query_states, key_states = ops.qk_norm_rope(
                q, k, self.q_norm.weight, self.k_norm.weight, self.q_norm.variance_epsilon,
                cos.contiguous(), sin.contiguous())
        else:
            query_states = self.q_norm(q).transpose(1, 2)
            key_states = self.k_norm(k).transpose(1, 2)
            query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin)
        if fused_projection:
            value_states = qkv[..., nq + nk:].view(hidden_shape).transpose(1, 2)
        else:
            value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        if past_key_values is not None:
            key_states, value_states = past_key_values.update(key_states, value_states,
                                                              self.layer_idx)
        attention_interface = ALL_ATTENTION_FUNCTIONS.get_interface(
            self.config._attn_implementation, eager_attention_forward)
        attn_output, attn_weights = attention_interface(
            self, query_states, key_states, value_states, attention_mask,
            dropout=0.0 if not self.training else self.attention_dropout,
            scaling=self.scaling, sliding_window=self.sliding_window, **kwargs)
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), attn_weights


def install_hip_attention(model: nn.Module) -> int:
    """Replace every ``Qwen3MoeAttention`` of ``model`` with a
    ``Qwen3AttentionHip`` sharing its submodules; returns how many."""
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeAttention

    count = 0
    for layer in model.model.layers:
        if isinstance(layer.self_attn, Qwen3MoeAttention):
            layer.self_attn = Qwen3AttentionHip.from_module(layer.self_attn)
            count += 1
    return count

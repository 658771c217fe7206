"""Router module backed by the fused gfx950 router kernel (K1).

Drop-in for transformers' ``Qwen3MoeTopKRouter`` (tf:249-267): an
``nn.Module`` with a ``weight`` parameter [num_experts, hidden] whose
``forward(hidden) -> (router_logits bf16 [T,E], router_scores bf16 [T,K],
router_indices int64 [T,K])`` keeps the triple that forward hooks read
(the reference's route capture hooks ``output[2]``).  Top-k ties resolve to
the lower expert id.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import ops


class Qwen3MoeTopKRouterHip(nn.Module):
    def __init__(self, *, num_experts: int, hidden_size: int, top_k: int,
                 norm_topk_prob: bool, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str | None = None) -> None:
        super().__init__()
        if not 1 <= top_k <= min(num_experts, 32) or num_experts > 256:
            raise ValueError("unsupported router shape")
        self.top_k = top_k
        self.num_experts = num_experts
        self.norm_topk_prob = bool(norm_topk_prob)
        self.hidden_dim = hidden_size
        self.weight = nn.Parameter(torch.zeros(num_experts, hidden_size, dtype=dtype,
                                               device=device), requires_grad=False)

    @classmethod
    def from_config(cls, config, **kwargs) -> "Qwen3MoeTopKRouterHip":
        return cls(num_experts=config.num_experts, hidden_size=config.hidden_size,
                   top_k=config.num_experts_per_tok, norm_topk_prob=config.norm_topk_prob,
                   **kwargs)

    @classmethod
    def from_module(cls, router: nn.Module) -> "Qwen3MoeTopKRouterHip":
        """Wrap an HF ``Qwen3MoeTopKRouter`` (shares no storage with it)."""
        out = cls(num_experts=router.num_experts, hidden_size=router.hidden_dim,
                  top_k=router.top_k, norm_topk_prob=router.norm_topk_prob,
                  dtype=router.weight.dtype, device=router.weight.device)
        with torch.no_grad():
            out.weight.copy_(router.weight)
        return out

    def forward(self, hidden_states: torch.Tensor):
        hidden_states = hidden_states.reshape(-1, self.hidden_dim)
        return ops.router_topk(hidden_states, self.weight, self.top_k, self.norm_topk_prob)

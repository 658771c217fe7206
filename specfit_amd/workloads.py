"""Seeded synthetic inputs of the MoE verification workloads.

Shapes are those of a Qwen3-30B-A3B MoE block: hidden 2048, 128 experts,
top-8 softmax routing with renormalised weights, expert intermediate 768,
SwiGLU.  Random-init bf16 weights N(0, 0.02) for the router and the experts
and N(0, 1) hidden states, all drawn from ``torch.Generator('cpu')`` in a
fixed order: router first, then experts 0..E-1 as gate, up, down.

Skewed expert popularity: a seeded permutation pi ranks the experts and a
Zipf(s) law p_r ~ r^-s over the ranks gives each expert the logit bias
b_e = lam * log p_{pi(e)}.  The bias is folded into the router as a rank-1
term (hidden feature 0 := 1, router column 0 := b), so the router itself is
unchanged.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

QWEN3_30B_A3B = dict(hidden_size=2048, num_experts=128, top_k=8, intermediate_size=768)


@dataclass
class MoELayerWeights:
    router: torch.Tensor           # bf16 [E, H] (CPU)
    experts: torch.Tensor          # bf16 [E, 3*I*H] packed [gate | up | down] (CPU)
    hidden_size: int
    intermediate_size: int
    top_k: int
    zipf_bias: torch.Tensor | None  # fp32 [E] bias folded into router column 0

    @property
    def num_experts(self) -> int:
        return self.router.shape[0]

    @property
    def expert_bytes(self) -> int:
        return self.experts.shape[1] * self.experts.element_size()


def zipf_bias(num_experts: int, s: float, lam: float, seed: int) -> torch.Tensor:
    """b_e = lam * log p_{pi(e)} with p_r proportional to r^-s, r = 1..E."""
    g = torch.Generator("cpu").manual_seed(seed)
    perm = torch.randperm(num_experts, generator=g)
    ranks = torch.arange(1, num_experts + 1, dtype=torch.float64)
    p = ranks.pow(-s)
    p = p / p.sum()
    bias = torch.empty(num_experts, dtype=torch.float64)
    bias[perm] = lam * torch.log(p)
    return bias.float()


def make_layer(*, seed: int = 0, hidden_size: int = 2048, num_experts: int = 128,
               intermediate_size: int = 768, top_k: int = 8, std: float = 0.02,
               zipf_s: float | None = None, zipf_lambda: float = 1.0,
               pin_memory: bool = False) -> MoELayerWeights:
    """Router + packed experts of one MoE layer (CPU tensors, optionally in
    page-locked memory for the expert cache)."""
    g = torch.Generator("cpu").manual_seed(seed)
    H, I, E = hidden_size, intermediate_size, num_experts
    router = (torch.randn(E, H, generator=g) * std).to(torch.bfloat16)
    experts = torch.empty((E, 3 * I * H), dtype=torch.bfloat16, pin_memory=pin_memory)
    for e in range(E):
        for part in range(3):  # gate, up, down
            chunk = torch.randn(I * H, generator=g) * std
            experts[e, part * I * H:(part + 1) * I * H] = chunk.to(torch.bfloat16)
    bias = None
    if zipf_s is not None:
        bias = zipf_bias(E, zipf_s, zipf_lambda, seed + 7919)
        router[:, 0] = bias.to(torch.bfloat16)
    return MoELayerWeights(router, experts, H, I, top_k, bias)


def make_hidden(tokens: int, hidden_size: int = 2048, *, seed: int,
                zipf_fold: bool = False) -> torch.Tensor:
    """bf16 [tokens, hidden] ~ N(0, 1); feature 0 := 1 when the Zipf bias is
    folded into the router."""
    g = torch.Generator("cpu").manual_seed(seed)
    h = torch.randn(tokens, hidden_size, generator=g)
    if zipf_fold:
        h[:, 0] = 1.0
    return h.to(torch.bfloat16)


def expected_distinct_uniform(tokens: int, num_experts: int = 128, top_k: int = 8) -> float:
    """E[U] of distinct experts under uniform top-k routing."""
    return num_experts * (1.0 - (1.0 - top_k / num_experts) ** tokens)

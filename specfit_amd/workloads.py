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


def make_layer_sources(layers: int, *, device, seed: int = 0, hidden_size: int = 2048,
                       num_experts: int = 128, intermediate_size: int = 768,
                       std: float = 0.02, pin_memory: bool = True) -> list[torch.Tensor]:
    """Distinct packed experts for each of ``layers`` MoE layers in host
    memory (page-locked unless ``pin_memory`` is False): bf16 [E, 3*I*H]
    N(0, std) per layer (1.125 GiB at the Qwen3-30B-A3B shape), drawn on
    ``device`` from a generator seeded with seed + layer and copied to the
    host one expert block at a time."""
    device = torch.device(device)
    E, row = num_experts, 3 * intermediate_size * hidden_size
    chunk = 16  # experts per device draw: 302 MB of fp32 at the 30B shape
    out = []
    for layer in range(layers):
        gen = torch.Generator(device=device).manual_seed(seed + layer)
        host = torch.empty((E, row), dtype=torch.bfloat16, pin_memory=pin_memory)
        for e0 in range(0, E, chunk):
            n = min(chunk, E - e0)
            block = torch.empty((n, row), dtype=torch.float32, device=device)
            block.normal_(0.0, std, generator=gen)
            host[e0:e0 + n].copy_(block.to(torch.bfloat16))
        out.append(host)
    torch.cuda.synchronize(device)
    return out


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


QWEN3_30B_A3B_MODEL = dict(vocab_size=151936, hidden_size=2048, intermediate_size=6144,
                           moe_intermediate_size=768, num_hidden_layers=48,
                           num_attention_heads=32, num_key_value_heads=4, head_dim=128,
                           num_experts=128, num_experts_per_tok=8, norm_topk_prob=True,
                           rms_norm_eps=1e-6, max_position_embeddings=40960,
                           tie_word_embeddings=False, decoder_sparse_step=1, mlp_only_layers=[],
                           rope_parameters={"rope_type": "default", "rope_theta": 1e6})


def make_verify_model(*, device, layers: int = 48, slots_per_layer: int = 12, seed: int = 0,
                      experts: MoELayerWeights | None = None, std: float = 0.02,
                      expert_execution_policy: str = "resident_first",
                      layer_sources: list[torch.Tensor] | None = None,
                      compress_expert_sources: bool = False):
    """A Qwen3-30B-A3B-shaped target for the verification forward, random
    init: every non-expert weight N(0, std) bf16 (norm weights 1), drawn on
    the device from a seeded generator.  The routed experts of layer l are
    ``layer_sources[l]`` (distinct pinned packed experts per layer, see
    make_layer_sources) or, without them, the pinned packed experts of
    ``experts`` (one MoE layer's worth shared by all layers, so the host
    holds 1.2 GB instead of 54 GB; every layer still has its own slot cache
    and copies its own misses).  The attention layers run the HIP
    tree-attention kernel.  Returns the LoadedOffloadedQwen3."""
    from accelerate import init_empty_weights
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeRotaryEmbedding

    from .runtime import build_offloaded_qwen3, register_tree_attention

    device = torch.device(device)
    cfg = dict(QWEN3_30B_A3B_MODEL, num_hidden_layers=layers)
    config = Qwen3MoeConfig(**cfg)
    config._attn_implementation = register_tree_attention()
    with init_empty_weights():
        model = Qwen3MoeForCausalLM(config)
    for layer in model.model.layers:
        layer.mlp.experts = torch.nn.Identity()
    model.to_empty(device=device)
    gen = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=gen)
    model.to(torch.bfloat16)
    model.model.rotary_emb = Qwen3MoeRotaryEmbedding(config).to(device)
    if layer_sources is not None:
        if len(layer_sources) != layers:
            raise ValueError("layer_sources needs one tensor per layer")
        sources = {l: layer_sources[l] for l in range(layers)}
    else:
        if experts is None:
            experts = make_layer(seed=seed, pin_memory=True)
        sources = {l: experts.experts for l in range(layers)}
    return build_offloaded_qwen3(model, device=device, slots_per_layer=slots_per_layer,
                                 layer_experts=sources,
                                 compress_expert_sources=compress_expert_sources,
                                 expert_execution_policy=expert_execution_policy)


def make_kv_context(config, length: int, *, device, seed: int):
    """A DynamicCache holding ``length`` random (N(0, 1) bf16) key/value
    positions for every layer: the committed context the tree verifies
    against."""
    from transformers import DynamicCache

    head_dim = getattr(config, "head_dim", config.hidden_size // config.num_attention_heads)
    shape = (1, config.num_key_value_heads, length, head_dim)
    gen = torch.Generator(device=device).manual_seed(seed)
    cache = DynamicCache()
    for layer in range(config.num_hidden_layers):
        k = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
        v = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
        cache.update(k, v, layer)
    return cache

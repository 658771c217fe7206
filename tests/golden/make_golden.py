"""Writes the golden fixtures of this directory from transformers' Qwen3-MoE
router and eager experts (the third-party code the reference's MoE block
calls: transformers/models/qwen3_moe/modeling_qwen3_moe.py:222-267), run on
torch CPU.  The installed transformers is used; the reference pins 5.6.0.

    python tests/golden/make_golden.py

Fixtures are .npz files (no pickles): inputs and expected outputs only; the
real-shape router fixtures store the input recipe (inputs.py) and the
SHA-256 of the inputs instead of the inputs.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch
import transformers
from transformers import Qwen3MoeConfig
from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeExperts, Qwen3MoeTopKRouter

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from inputs import input_digest, real_shape_inputs  # noqa: E402


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def router_fixture(name: str, T: int, H: int, E: int, K: int, norm: bool, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    cfg = Qwen3MoeConfig(hidden_size=H, num_experts=E, num_experts_per_tok=K, norm_topk_prob=norm)
    router = Qwen3MoeTopKRouter(cfg).to(torch.bfloat16)
    with torch.no_grad():
        router.weight.copy_((torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16))
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        logits, weights, index = router(hidden)
    np.savez_compressed(os.path.join(HERE, name), hidden=bits(hidden), router=bits(router.weight),
                        logits=bits(logits), weights=bits(weights), index=index.numpy(),
                        top_k=np.int64(K), norm=np.int64(int(norm)),
                        transformers_version=np.array(transformers.__version__))


def real_shape_router_fixture(name: str, T: int, seed: int, zipf_s: float | None) -> None:
    """transformers' router at the Qwen3-30B-A3B shape (H 2048, E 128, top-8,
    renormalised).  Stores the input recipe and digest, not the inputs."""
    H, E, K = 2048, 128, 8
    hidden, weight = real_shape_inputs(T, H, E, seed, zipf_s)
    cfg = Qwen3MoeConfig(hidden_size=H, num_experts=E, num_experts_per_tok=K, norm_topk_prob=True)
    router = Qwen3MoeTopKRouter(cfg).to(torch.bfloat16)
    with torch.no_grad():
        router.weight.copy_(weight)
        logits, weights, index = router(hidden)
    np.savez_compressed(os.path.join(HERE, name), tokens=np.int64(T), seed=np.int64(seed),
                        zipf_s=np.float64(-1.0 if zipf_s is None else zipf_s),
                        input_sha256=np.array(input_digest(hidden, weight)),
                        logits=bits(logits), weights=bits(weights), index=index.numpy(),
                        top_k=np.int64(K), norm=np.int64(1),
                        transformers_version=np.array(transformers.__version__))


def experts_fixture(name: str, T: int, H: int, I: int, E: int, K: int, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    cfg = Qwen3MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, hidden_act="silu")
    experts = Qwen3MoeExperts(cfg).to(torch.bfloat16)
    gate_up = (torch.randn(E, 2 * I, H, generator=g) * 0.1).to(torch.bfloat16)
    down = (torch.randn(E, H, I, generator=g) * 0.1).to(torch.bfloat16)
    with torch.no_grad():
        experts.gate_up_proj.copy_(gate_up)
        experts.down_proj.copy_(down)
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    index = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    index[0, -1] = index[0, 0]  # a duplicated expert within one row
    weights = torch.rand(T, K, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        out = experts(hidden, index, weights)
    packed = torch.cat([gate_up.reshape(E, -1), down.reshape(E, -1)], dim=1)  # [gate|up|down]
    np.savez_compressed(os.path.join(HERE, name), hidden=bits(hidden), packed=bits(packed),
                        index=index.numpy(), weights=bits(weights), out=bits(out),
                        hidden_size=np.int64(H), intermediate_size=np.int64(I),
                        transformers_version=np.array(transformers.__version__))


if __name__ == "__main__":
    router_fixture("router_hf_t16_h256_e64_k8.npz", 16, 256, 64, 8, True, 0)
    router_fixture("router_hf_t8_h32_e4_k2_nonorm.npz", 8, 32, 4, 2, False, 1)
    experts_fixture("experts_hf_t6_h64_i32_e8_k3.npz", 6, 64, 32, 8, 3, 2)
    real_shape_router_fixture("router_hf_t256_h2048_e128_k8_uniform.npz", 256, 11, None)
    real_shape_router_fixture("router_hf_t256_h2048_e128_k8_zipf.npz", 256, 12, 1.1)
    print("fixtures written to", HERE)

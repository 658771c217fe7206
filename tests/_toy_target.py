"""A toy offloaded target for the prefetch-scheduler tests.

The scheduler (Qwen3ExpertPrefetch) and LoadedOffloadedQwen3 only touch a
target's ``model.layers[i].self_attn`` (a forward pre-hook marks the start
of layer i) and ``model.layers[i].mlp.experts`` (the offloaded expert
module), plus ``config.num_hidden_layers``.  ``ToyTarget`` is that and no
more: each layer passes its input through an identity "attention" and then
through its offloaded experts with routes fixed by the caller, so every
test controls exactly which experts each layer needs.

``toy_case`` builds one: ``layers`` layer caches of 6 tiny experts
(hidden 16, intermediate 12) under one recording observer, and a 4-token
input whose routes use experts 0-4 of every layer (expert 5 is never
routed).
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from types import SimpleNamespace

import torch
from torch import nn

from specfit_amd.runtime import (ExpertKey, GpuExpertCache, LoadedOffloadedQwen3,
                                 Qwen3OffloadedExperts, RecordingCacheTransitionObserver)

HIDDEN, INTERMEDIATE, EXPERTS = 16, 12, 6
# Top-3 routes of the 4 tokens: experts 0..4 appear, 5 never does.
ROUTES = ((4, 0, 2), (1, 4, 3), (2, 0, 1), (4, 3, 0))


class ToyDecoderLayer(nn.Module):
    """Identity attention (the scheduler's hook point), then the layer's
    offloaded experts over the caller's routes."""

    def __init__(self, experts: Qwen3OffloadedExperts) -> None:
        super().__init__()
        self.self_attn = nn.Identity()
        self.mlp = nn.ModuleDict({"experts": experts})

    def forward(self, hidden, routes, route_weights):
        return self.mlp["experts"](self.self_attn(hidden), routes, route_weights)


class ToyTarget(nn.Module):
    def __init__(self, expert_modules) -> None:
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList(ToyDecoderLayer(m) for m in expert_modules)
        self.config = SimpleNamespace(num_hidden_layers=len(self.model.layers))

    def forward(self, hidden, routes, route_weights):
        for layer in self.model.layers:
            hidden = layer(hidden, routes, route_weights)
        return hidden


@dataclass
class ToyCase:
    loaded: LoadedOffloadedQwen3
    observer: RecordingCacheTransitionObserver
    inputs: tuple  # hidden [4, 16] bf16, routes [4, 3] int64, route weights [4, 3] bf16

    @property
    def caches(self) -> tuple:
        return self.loaded.expert_caches

    def forward(self, inputs=None):
        return self.loaded.model(*(self.inputs if inputs is None else inputs))

    def copy_streams(self) -> tuple:
        return tuple(c.copy_stream for c in self.caches)

    def make_resident(self, experts, layers=None) -> None:
        """Acquire and wait for ``experts`` in each of ``layers`` (default
        all), then let the device finish."""
        for lid in (range(len(self.caches)) if layers is None else layers):
            for e in experts:
                with self.caches[lid].acquire(ExpertKey(lid, e)) as lease:
                    lease.wait()
        torch.cuda.synchronize()

    def assert_quiet(self, streams) -> None:
        assert_quiet(self.loaded, streams)

    def close(self) -> None:
        close_loaded(self.loaded)


def assert_quiet(loaded, streams) -> None:
    """After a scheduling context: each cache has its own copy stream back,
    no scheduler is installed, and no transfer, lease or use guard is left
    pending."""
    torch.cuda.synchronize()
    for layer, cache, stream in zip(loaded.model.model.layers, loaded.expert_caches, streams):
        assert cache.copy_stream is stream
        assert layer.mlp.experts._prediction_scheduler is None
        snap = cache.snapshot()
        assert not snap.pending_transfers
        assert not any(s.active_leases or s.pending_use_guards for s in snap.slots)


def close_loaded(loaded) -> None:
    torch.cuda.synchronize()
    loaded.close()


def toy_case(slots: int = 3, layers: int = 2, *, seed: int = 909) -> ToyCase:
    g = torch.Generator().manual_seed(seed)
    observer = RecordingCacheTransitionObserver(run_id="predicted-prefetch")
    caches, modules = [], []
    width = 3 * HIDDEN * INTERMEDIATE
    for lid in range(layers):
        packed = torch.randn(EXPERTS, width, generator=g).to(torch.bfloat16) / 16
        cache = GpuExpertCache({ExpertKey(lid, e): packed[e] for e in range(EXPERTS)},
                               slot_count=slots, device="cuda:0",
                               cache_id=f"qwen3-layer-{lid}", queue_id=f"layer-{lid}-copy",
                               observer=observer)
        caches.append(cache)
        modules.append(Qwen3OffloadedExperts(layer_id=lid, cache=cache, hidden_size=HIDDEN,
                                             intermediate_size=INTERMEDIATE, h2d_prefetch=False))
    tokens = len(ROUTES)
    hidden = torch.randn(tokens, HIDDEN, generator=g).to(torch.bfloat16).cuda()
    routes = torch.tensor(ROUTES, device="cuda:0")
    weights = torch.rand(tokens, len(ROUTES[0]), generator=g).to(torch.bfloat16).cuda()
    loaded = LoadedOffloadedQwen3(ToyTarget(modules), tuple(caches), None)
    return ToyCase(loaded, observer, (hidden, routes, weights))


# ------------------------------------------------ tiny real Qwen3-MoE model --
def tiny_qwen3_config(layers: int = 1):
    from transformers import Qwen3MoeConfig
    return Qwen3MoeConfig(dtype=torch.bfloat16, vocab_size=64, hidden_size=32,
                          intermediate_size=48, moe_intermediate_size=16,
                          num_hidden_layers=layers, num_attention_heads=4,
                          num_key_value_heads=2, num_experts=4, num_experts_per_tok=2,
                          max_position_embeddings=64, bos_token_id=1, eos_token_id=2,
                          pad_token_id=0, use_cache=True)


def save_per_expert_checkpoint(model, root) -> None:
    """Write ``model`` as an original Qwen3-MoE checkpoint directory: config,
    one safetensors shard with per-expert gate/up/down keys, and the index."""
    from safetensors.torch import save_file
    root = Path(root)
    model.config.save_pretrained(root)
    inter = model.config.moe_intermediate_size
    tensors = {}
    for name, value in model.state_dict().items():
        base, _, leaf = name.rpartition(".")
        if base.endswith(".experts") and leaf in ("gate_up_proj", "down_proj"):
            for e in range(value.shape[0]):
                if leaf == "gate_up_proj":
                    tensors[f"{base}.{e}.gate_proj.weight"] = value[e, :inter].contiguous()
                    tensors[f"{base}.{e}.up_proj.weight"] = value[e, inter:].contiguous()
                else:
                    tensors[f"{base}.{e}.down_proj.weight"] = value[e].contiguous()
        else:
            tensors[name] = value.contiguous()
    shard = "model-00001-of-00001.safetensors"
    save_file(tensors, root / shard)
    index = {"metadata": {"total_size": sum(t.numel() * t.element_size()
                                            for t in tensors.values())},
             "weight_map": dict.fromkeys(tensors, shard)}
    (root / "model.safetensors.index.json").write_text(json.dumps(index), encoding="utf-8")

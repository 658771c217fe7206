"""Offloaded Qwen3-MoE model assembly.

Drop-in for src/specfit/runtime/qwen3_offloaded_model.py:127-260,667-840
(``LoadedOffloadedQwen3`` and ``load_offloaded_qwen3``): an HF
``Qwen3MoeForCausalLM`` whose routed experts live in pinned host memory
behind one ``GpuExpertCache`` per decoder layer, with every layer's
``mlp.gate`` replaced by the fused router module and ``mlp.experts`` by
``Qwen3OffloadedExperts``.  Non-expert weights are loaded to the device.

Checkpoints: a directory with ``config.json`` and safetensors shards whose
expert tensors are either per expert
(``...mlp.experts.{e}.{gate,up,down}_proj.weight``, the original Qwen3 layout)
or fused (``...mlp.experts.gate_up_proj`` [E, 2I, H] and ``down_proj``
[E, H, I]).  Each layer's experts are packed into one pinned
``[E, 3*I*H]`` bf16 tensor in the reference's ``[gate | up | down]`` order.
"""
from __future__ import annotations

import json
import logging
import re
import time
from dataclasses import dataclass
from enum import Enum
from pathlib import Path

import torch

from ..codec import CompressedExperts
from .cache_observer import CacheTransitionObserver
from .gpu_expert_cache import GpuExpertCache
from .lease import ExpertCacheStats
from .qwen3_offloaded_experts import ExpertExecutionPolicy, Qwen3OffloadedExperts, ReductionMode
from .qwen3_attention import install_hip_attention
from .qwen3_norm import install_hip_norms
from .qwen3_router import Qwen3MoeTopKRouterHip
from .state import ExpertKey

_LOG = logging.getLogger(__name__)


class PackedExpertBackingMode(str, Enum):
    """How a packed-v1 checkpoint's expert layers become pinned sources
    (qwen3_offloaded_model.py:46-49).  Both are served by reading each layer
    file straight into page-locked memory here: registering an existing file
    mapping with the runtime is not available on this platform, so
    REGISTERED_MMAP maps no file and registers nothing (its mapped and
    registered byte counts stay 0)."""

    PINNED_COPY = "pinned_copy"
    REGISTERED_MMAP = "registered_mmap"


@dataclass(frozen=True, slots=True)
class Qwen3LoadTimings:
    """Wall time of the load stages (seconds) and bytes moved; the
    reference's fields (qwen3_offloaded_model.py:52-73)."""

    checkpoint_format: str = "original"
    expert_backing_mode: str = "original_pinned_copy"
    checkpoint_inspection_seconds: float = 0.0
    model_initialization_seconds: float = 0.0
    expert_pinned_allocation_seconds: float = 0.0
    expert_weight_read_seconds: float = 0.0
    expert_mmap_seconds: float = 0.0
    expert_host_registration_seconds: float = 0.0
    expert_view_seconds: float = 0.0
    expert_cache_initialization_seconds: float = 0.0
    nonexpert_read_seconds: float = 0.0
    nonexpert_h2d_seconds: float = 0.0
    finalization_seconds: float = 0.0
    total_seconds: float = 0.0
    expert_bytes_read: int = 0
    expert_bytes_mapped: int = 0
    expert_bytes_registered: int = 0
    nonexpert_bytes_read: int = 0


@dataclass
class LoadedOffloadedQwen3:
    model: object
    expert_caches: tuple
    load_timings: Qwen3LoadTimings | None

    def layer_cache_stats(self) -> tuple[ExpertCacheStats, ...]:
        return tuple(cache.stats() for cache in self.expert_caches)

    def cache_snapshots(self) -> tuple:
        snapshots = tuple(cache.snapshot() for cache in self.expert_caches)
        expected = tuple(f"qwen3-layer-{i}" for i in range(self.model.config.num_hidden_layers))
        if tuple(s.cache_id for s in snapshots) != expected:
            raise RuntimeError("expert cache order does not match Qwen3 decoder layers")
        queue_ids = tuple(s.queue_id for s in snapshots)
        if len(queue_ids) != len(set(queue_ids)):
            raise RuntimeError("expert cache queue IDs must be unique")
        return snapshots

    def cold_reset_expert_caches(self) -> None:
        if any(cache.active_lease_count for cache in self.expert_caches):
            raise RuntimeError("cold reset cannot run while an active lease exists")
        for device in {cache.device for cache in self.expert_caches}:
            torch.cuda.synchronize(device)
        for cache in self.expert_caches:
            cache.cold_reset()

    def cache_stats(self) -> ExpertCacheStats:
        stats = self.layer_cache_stats()
        return ExpertCacheStats(
            h2d_submissions=sum(s.h2d_submissions for s in stats),
            resident_hits=sum(s.resident_hits for s in stats),
            inflight_joins=sum(s.inflight_joins for s in stats),
            evictions=sum(s.evictions for s in stats),
            pending_use_guards=sum(s.pending_use_guards for s in stats))

    def _expert_modules(self, message: str) -> tuple:
        modules = tuple(layer.mlp.experts for layer in self.model.model.layers)
        if not all(isinstance(m, Qwen3OffloadedExperts) for m in modules):
            raise RuntimeError(message)
        return modules

    def set_expert_execution_policy(self, execution_policy) -> None:
        policy = ExpertExecutionPolicy(execution_policy)
        modules = self._expert_modules(
            "loaded Qwen3 does not contain an offloaded expert module in every decoder layer")
        if any(m._prediction_scheduler is not None for m in modules):
            raise RuntimeError("cannot switch execution policy during predicted prefetch")
        for m in modules:
            m.execution_policy = policy

    def set_expert_h2d_prefetch(self, enabled: bool) -> None:
        if type(enabled) is not bool:
            raise ValueError("h2d_prefetch must be a boolean")
        modules = self._expert_modules("every decoder layer must contain offloaded experts")
        if any(m._prediction_scheduler is not None for m in modules):
            raise RuntimeError("cannot switch H2D policy during predicted prefetch")
        if any(c.closed or c.active_lease_count for c in self.expert_caches):
            raise RuntimeError("prefetch switching requires open caches without active leases")
        for m in modules:
            m.h2d_prefetch = enabled

    def prefetch_experts(self, predictions, *, lookahead_layers: int = 1, max_inflight: int = 2,
                         max_prefetch_per_layer: int | None = None, trace: bool = False,
                         prediction_probabilities=None, eviction_policy: str = "lru"):
        from .qwen3_expert_prefetch import Qwen3ExpertPrefetch

        return Qwen3ExpertPrefetch(self, predictions, lookahead_layers=lookahead_layers,
                                   max_inflight=max_inflight,
                                   max_prefetch_per_layer=max_prefetch_per_layer, trace=trace,
                                   prediction_probabilities=prediction_probabilities,
                                   eviction_policy=eviction_policy)

    @property
    def closed(self) -> bool:
        return all(cache.closed for cache in self.expert_caches)

    def close(self) -> None:
        if any(getattr(layer.mlp.experts, "_prediction_scheduler", None) is not None
               for layer in self.model.model.layers):
            raise RuntimeError("cannot close the model during predicted prefetch")
        if sum(cache.active_lease_count for cache in self.expert_caches):
            raise RuntimeError("loaded Qwen3 cannot close while an active lease exists")
        for cache in reversed(self.expert_caches):
            cache.close()

    def __enter__(self) -> "LoadedOffloadedQwen3":
        if self.closed:
            raise RuntimeError("loaded Qwen3 is closed")
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        self.close()


# ------------------------------------------------------------ checkpoint --
_PER_EXPERT = re.compile(r"^(.*\.mlp\.experts)\.(\d+)\.(gate|up|down)_proj\.weight$")
_FUSED = re.compile(r"^(.*\.mlp\.experts)\.(gate_up_proj|down_proj)$")
_LAYER = re.compile(r"\.layers\.(\d+)\.")


def _tensor_files(root: Path) -> dict[str, Path]:
    index = root / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        return {name: root / shard for name, shard in weight_map.items()}
    files = sorted(root.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no safetensors checkpoint under {root}")
    from safetensors import safe_open

    out = {}
    for f in files:
        with safe_open(str(f), framework="pt") as handle:
            for name in handle.keys():
                out[name] = f
    return out


def _pack_layer_experts(get, names: dict, E: int, H: int, I: int) -> torch.Tensor:
    """Pinned [E, 3*I*H] bf16 packed experts of one layer."""
    packed = torch.empty((E, 3 * I * H), dtype=torch.bfloat16, pin_memory=True)
    if "gate_up_proj" in names:
        gu = get(names["gate_up_proj"]).to(torch.bfloat16)
        down = get(names["down_proj"]).to(torch.bfloat16)
        if gu.shape != (E, 2 * I, H) or down.shape != (E, H, I):
            raise ValueError("fused expert tensors have unexpected shapes")
        packed[:, : 2 * I * H].copy_(gu.reshape(E, -1))
        packed[:, 2 * I * H:].copy_(down.reshape(E, -1))
        return packed
    for e in range(E):
        parts = [get(names[(e, p)]).to(torch.bfloat16) for p in ("gate", "up", "down")]
        if parts[0].shape != (I, H) or parts[1].shape != (I, H) or parts[2].shape != (H, I):
            raise ValueError(f"expert {e} has unexpected projection shapes")
        packed[e, : I * H].copy_(parts[0].reshape(-1))
        packed[e, I * H: 2 * I * H].copy_(parts[1].reshape(-1))
        packed[e, 2 * I * H:].copy_(parts[2].reshape(-1))
    return packed


def _install(model, *, layer_packed: dict[int, torch.Tensor], device: torch.device,
             slots_per_layer: int, reduction_mode, expert_execution_policy,
             h2d_prefetch: bool, cache_observer, compress_expert_sources: bool = False,
             hip_dense_kernels: bool = True) -> tuple:
    config = model.config
    caches = []
    # One pair of SDMA streams for every layer cache (layers copy in turn).
    copy_streams = (torch.cuda.Stream(device=device), torch.cuda.Stream(device=device))
    coded: dict[int, CompressedExperts] = {}  # layers sharing a source share its records
    try:
        for layer_id, layer in enumerate(model.model.layers):
            packed = layer_packed[layer_id]
            sources = {ExpertKey(layer_id, e): packed[e] for e in range(packed.shape[0])}
            image = None
            if compress_expert_sources:
                shared = coded.get(id(packed))
                if shared is None:
                    shared = coded[id(packed)] = CompressedExperts.encode(
                        {e: packed[e] for e in range(packed.shape[0])}, device=device)
                image = CompressedExperts(shared.blob, {ExpertKey(layer_id, e): r for e, r
                                                        in shared.records.items()}, shared.numel)
            cache = GpuExpertCache(sources,
                                   slot_count=slots_per_layer, device=device,
                                   adopt_pinned_sources=True, cache_id=f"qwen3-layer-{layer_id}",
                                   queue_id=f"layer-{layer_id}-copy", observer=cache_observer,
                                   copy_streams=copy_streams, compressed_sources=image)
            caches.append(cache)
            layer.mlp.experts = Qwen3OffloadedExperts(
                layer_id=layer_id, cache=cache, hidden_size=config.hidden_size,
                intermediate_size=config.moe_intermediate_size, reduction_mode=reduction_mode,
                execution_policy=expert_execution_policy, h2d_prefetch=h2d_prefetch)
            layer.mlp.gate = Qwen3MoeTopKRouterHip.from_module(layer.mlp.gate)
        # The dense layers' RMSNorms run as one kernel each (K6), and each
        # attention layer's query/key norms and rotary embedding as one (K7);
        # without hip_dense_kernels they stay HF's eager modules.
        if hip_dense_kernels:
            install_hip_norms(model)
            install_hip_attention(model)
    except BaseException:
        for cache in reversed(caches):
            cache.close()
        raise
    return tuple(caches)


def load_offloaded_qwen3(model_root, *, device, slots_per_layer: int,
                         packed_checkpoint_root=None,
                         packed_expert_backing: PackedExpertBackingMode | str | None = None,
                         verify_packed_hashes: bool = False,
                         reduction_mode=ReductionMode.CANONICAL,
                         expert_execution_policy=ExpertExecutionPolicy.EXPERT_ID_ASCENDING,
                         attn_implementation: str = "sdpa",
                         cache_observer: CacheTransitionObserver | None = None,
                         h2d_prefetch: bool = True,
                         compress_expert_sources: bool = False,
                         hip_dense_kernels: bool = True) -> LoadedOffloadedQwen3:
    """Load a Qwen3-MoE checkpoint with offloaded experts
    (qwen3_offloaded_model.py:667-840).  ``model_root`` holds config.json
    and the original safetensors (per-expert or fused expert tensors); with
    ``packed_checkpoint_root`` the experts and non-experts come from that
    packed-v1 checkpoint instead, validated against ``model_root``'s
    config/index hashes (the weight shards need not exist).
    ``compress_expert_sources`` (an extension beyond the reference): every layer's
    misses move exponent-coded records (specfit_amd.codec) over the host
    link and are decoded into the slots, which hold the same bytes.
    ``hip_dense_kernels`` (default True): the dense layers' RMSNorms and the
    attention layers' query/key norms and rotary embedding run as HIP
    kernels, which may differ from HF eager by a last-place rounding of the
    variance; False keeps HF's eager modules (for equivalence checks)."""
    from accelerate import init_empty_weights
    from safetensors import safe_open
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    from ..checkpoint import PackedQwen3Checkpoint, read_expert_layer_pinned

    start = time.perf_counter()
    t = {}
    if type(h2d_prefetch) is not bool:
        raise ValueError("h2d_prefetch must be a boolean")
    if type(hip_dense_kernels) is not bool:
        raise ValueError("hip_dense_kernels must be a boolean")
    policy = ExpertExecutionPolicy(expert_execution_policy)
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("offloaded Qwen3 requires a CUDA device")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    root = Path(model_root).resolve()
    if packed_expert_backing is None:
        mode = (PackedExpertBackingMode.REGISTERED_MMAP if packed_checkpoint_root is not None
                else PackedExpertBackingMode.PINNED_COPY)
    else:
        mode = PackedExpertBackingMode(packed_expert_backing)
    if packed_checkpoint_root is None and mode is not PackedExpertBackingMode.PINNED_COPY:
        raise ValueError("registered_mmap requires packed_checkpoint_root")
    config = Qwen3MoeConfig.from_pretrained(root, local_files_only=True)
    config._attn_implementation = attn_implementation
    E, H, I = config.num_experts, config.hidden_size, config.moe_intermediate_size
    if not 1 <= slots_per_layer <= E:
        raise ValueError(f"slots_per_layer must be in [1, {E}]")

    handles: dict[Path, object] = {}

    def get(name: str, files: dict) -> torch.Tensor:
        path = files[name]
        if path not in handles:
            handles[path] = safe_open(str(path), framework="pt")
        return handles[path].get_tensor(name)

    t0 = time.perf_counter()
    layer_packed: dict[int, torch.Tensor] = {}
    if packed_checkpoint_root is not None:
        packed = PackedQwen3Checkpoint.open(packed_checkpoint_root, source_metadata_root=root,
                                            verify_hashes=verify_packed_hashes)
        census = packed.census
        if (census.num_hidden_layers, census.num_experts, census.hidden_size,
                census.moe_intermediate_size) != (config.num_hidden_layers, E, H, I):
            raise ValueError("packed checkpoint census does not match the model config")
        with safe_open(str(packed.nonexpert_path), framework="pt") as h:
            nonexpert_files = {name: packed.nonexpert_path for name in h.keys()}
        t["checkpoint_inspection_seconds"] = time.perf_counter() - t0
        fmt = "packed-v1"
        read_s = 0.0
        read_bytes = 0
        t1 = time.perf_counter()
        for lid in range(census.num_hidden_layers):
            tensor, seconds = read_expert_layer_pinned(packed.layer_path(lid),
                                                       (E, packed.packed_expert_elements))
            layer_packed[lid] = tensor
            read_s += seconds
            read_bytes += tensor.numel() * tensor.element_size()
        t["expert_weight_read_seconds"] = read_s
        t["expert_pinned_allocation_seconds"] = time.perf_counter() - t1 - read_s
        t["expert_bytes_read"] = read_bytes
    else:
        files = _tensor_files(root)
        expert_names: dict[int, dict] = {}
        nonexpert_files = {}
        for name, path in files.items():
            m = _PER_EXPERT.match(name)
            f = _FUSED.match(name)
            if m or f:
                entry = expert_names.setdefault(int(_LAYER.search(name).group(1)), {})
                if m:
                    entry[(int(m.group(2)), m.group(3))] = name
                else:
                    entry[f.group(2)] = name
            else:
                nonexpert_files[name] = path
        if sorted(expert_names) != list(range(config.num_hidden_layers)):
            raise ValueError("checkpoint does not hold routed experts for every decoder layer")
        t["checkpoint_inspection_seconds"] = time.perf_counter() - t0
        fmt = "original"
        t1 = time.perf_counter()
        layer_packed = {lid: _pack_layer_experts(lambda n: get(n, files), names, E, H, I)
                        for lid, names in expert_names.items()}
        t["expert_weight_read_seconds"] = time.perf_counter() - t1
        t["expert_bytes_read"] = sum(p.numel() * 2 for p in layer_packed.values())

    t2 = time.perf_counter()
    with init_empty_weights():
        model = Qwen3MoeForCausalLM(config)
    for layer in model.model.layers:
        layer.mlp.experts = torch.nn.Identity()
    t["model_initialization_seconds"] = time.perf_counter() - t2
    t3 = time.perf_counter()
    host = {name: get(name, nonexpert_files) for name in nonexpert_files}
    t["nonexpert_read_seconds"] = time.perf_counter() - t3
    t["nonexpert_bytes_read"] = sum(v.numel() * v.element_size() for v in host.values())
    t4 = time.perf_counter()
    state = {name: v.to(device=device, dtype=torch.bfloat16) for name, v in host.items()}
    missing, unexpected = model.load_state_dict(state, strict=False, assign=True)
    if unexpected:
        raise ValueError(f"unexpected checkpoint tensors: {unexpected[:5]}")
    if "lm_head.weight" in missing and getattr(config, "tie_word_embeddings", False):
        model.tie_weights()
    handles.clear()
    model.model.rotary_emb.to(device)
    torch.cuda.synchronize(device)
    t["nonexpert_h2d_seconds"] = time.perf_counter() - t4
    t5 = time.perf_counter()
    caches = _install(model, layer_packed=layer_packed, device=device,
                      slots_per_layer=slots_per_layer, reduction_mode=reduction_mode,
                      expert_execution_policy=policy, h2d_prefetch=h2d_prefetch,
                      cache_observer=cache_observer,
                      compress_expert_sources=compress_expert_sources,
                      hip_dense_kernels=hip_dense_kernels)
    t["expert_cache_initialization_seconds"] = time.perf_counter() - t5
    t6 = time.perf_counter()
    meta = [n for n, p in model.named_parameters() if p.is_meta]
    if meta:
        for cache in reversed(caches):
            cache.close()
        raise RuntimeError(f"model still has meta parameters: {meta[:5]}")
    model.requires_grad_(False)
    model.eval()
    torch.cuda.synchronize(device)
    t["finalization_seconds"] = time.perf_counter() - t6
    timings = Qwen3LoadTimings(
        checkpoint_format=fmt,
        expert_backing_mode=mode.value if fmt == "packed-v1" else "original_pinned_copy",
        total_seconds=time.perf_counter() - start, **t)
    _LOG.info("offloaded Qwen3 loaded: %s", timings)
    return LoadedOffloadedQwen3(model=model, expert_caches=caches, load_timings=timings)


def build_offloaded_qwen3(model, *, device, slots_per_layer: int,
                          reduction_mode=ReductionMode.CANONICAL,
                          expert_execution_policy=ExpertExecutionPolicy.EXPERT_ID_ASCENDING,
                          cache_observer: CacheTransitionObserver | None = None,
                          h2d_prefetch: bool = True,
                          layer_experts: dict[int, torch.Tensor] | None = None,
                          compress_expert_sources: bool = False,
                          hip_dense_kernels: bool = True
                          ) -> LoadedOffloadedQwen3:
    """Offload the experts of an in-memory HF ``Qwen3MoeForCausalLM``.

    The model's non-expert parameters move to ``device``; its fused expert
    parameters are packed into pinned memory (or ``layer_experts[l]``, a
    pinned ``[E, 3*I*H]`` bf16 tensor per layer, is used directly).
    ``hip_dense_kernels`` as for ``load_offloaded_qwen3``."""
    if type(hip_dense_kernels) is not bool:
        raise ValueError("hip_dense_kernels must be a boolean")
    device = torch.device(device)
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    config = model.config
    E, H, I = config.num_experts, config.hidden_size, config.moe_intermediate_size
    packed = {}
    for lid, layer in enumerate(model.model.layers):
        if layer_experts is not None:
            packed[lid] = layer_experts[lid]
        else:
            experts = layer.mlp.experts
            tensors = {"gate_up_proj": experts.gate_up_proj.detach(),
                       "down_proj": experts.down_proj.detach()}
            packed[lid] = _pack_layer_experts(
                tensors.__getitem__, {"gate_up_proj": "gate_up_proj", "down_proj": "down_proj"},
                E, H, I)
        layer.mlp.experts = torch.nn.Identity()
    model.to(device=device, dtype=torch.bfloat16)
    caches = _install(model, layer_packed=packed, device=device, slots_per_layer=slots_per_layer,
                      reduction_mode=reduction_mode,
                      expert_execution_policy=ExpertExecutionPolicy(expert_execution_policy),
                      h2d_prefetch=h2d_prefetch, cache_observer=cache_observer,
                      compress_expert_sources=compress_expert_sources,
                      hip_dense_kernels=hip_dense_kernels)
    model.requires_grad_(False)
    model.eval()
    return LoadedOffloadedQwen3(model=model, expert_caches=caches, load_timings=None)

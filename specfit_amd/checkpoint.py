"""Qwen3-MoE checkpoint layouts: the original HF layout and packed-v1.

Restates, with the same file format, fields and errors:
- ``CheckpointLayout`` / ``ModelCensus`` (src/specfit/adapters/qwen3_checkpoint.py:35-271):
  the census of an original checkpoint (``config.json``,
  ``model.safetensors.index.json``, per-expert
  ``model.layers.{l}.mlp.experts.{e}.{gate,up,down}_proj.weight`` tensors);
- the packed-v1 checkpoint (src/specfit/adapters/qwen3_packed_checkpoint.py):
  ``manifest.json`` (schema ``specfit.qwen3_packed_checkpoint`` version 1),
  ``experts/layer-NNN.safetensors`` holding one ``experts`` tensor
  ``[E, 3*I*H]`` per layer in ``[gate | up | down]`` order, and
  ``nonexperts.safetensors``; ``pack_qwen3_checkpoint`` writes it (source
  shards read in physical order, staged then renamed) and
  ``PackedQwen3Checkpoint.open`` validates it.

``read_expert_layer_pinned`` loads one packed layer straight from the file
into page-locked host memory (one allocation, reads into it, no staging
copy).  The reference maps the file and registers the mapping with the
runtime (registered_mmap.py:13-99); registering existing host memory is not
available on this platform, so the packed loader reads into memory the
runtime allocated as pinned instead.
"""
from __future__ import annotations

import hashlib
import json
import os
import re
import struct
import time
import uuid
from dataclasses import dataclass
from math import prod
from pathlib import Path
from typing import Any

import numpy as np
import torch

from .runtime.state import ExpertKey

PACKED_CHECKPOINT_SCHEMA = "specfit.qwen3_packed_checkpoint"
PACKED_CHECKPOINT_VERSION = 1
PACKED_MANIFEST_FILENAME = "manifest.json"
PACKED_EXPERT_LAYOUT = ("gate_proj", "up_proj", "down_proj")

_EXPERT_KEY = re.compile(r"^model\.layers\.(?P<layer>\d+)\.mlp\.experts\.(?P<expert>\d+)\."
                         r"(?P<projection>gate_proj|up_proj|down_proj)\.weight$")
_DTYPES = {"BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32,
           "F64": torch.float64, "I8": torch.int8, "U8": torch.uint8, "I16": torch.int16,
           "I32": torch.int32, "I64": torch.int64, "BOOL": torch.bool}


class PackedCheckpointError(ValueError):
    """A packed checkpoint (or its source) failed validation."""


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as fh:
        while chunk := fh.read(8 << 20):
            h.update(chunk)
    return h.hexdigest()


# ------------------------------------------------------------ safetensors --
def _read_header(path: Path) -> tuple[int, dict[str, dict[str, Any]]]:
    """(data start offset, tensor entries) of a safetensors file."""
    size = path.stat().st_size
    with path.open("rb") as fh:
        raw = fh.read(8)
        if len(raw) != 8:
            raise PackedCheckpointError(f"safetensors header length is missing: {path}")
        n = struct.unpack("<Q", raw)[0]
        if n <= 0 or n > size - 8:
            raise PackedCheckpointError(f"invalid safetensors header length in {path}")
        text = fh.read(n)
    try:
        header = json.loads(text)
    except (UnicodeDecodeError, json.JSONDecodeError) as error:
        raise PackedCheckpointError(f"invalid safetensors header JSON in {path}") from error
    if not isinstance(header, dict):
        raise PackedCheckpointError(f"safetensors header must be an object: {path}")
    entries = {}
    for name, entry in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(name, str) or not isinstance(entry, dict):
            raise PackedCheckpointError(f"invalid tensor header entry in {path}")
        off = entry.get("data_offsets")
        if (not isinstance(off, list) or len(off) != 2 or not all(isinstance(v, int) for v in off)
                or off[0] < 0 or off[1] < off[0]):
            raise PackedCheckpointError(f"invalid data_offsets for {name} in {path}")
        entries[name] = entry
    return 8 + n, entries


def _tensor_names_in_storage_order(path: Path) -> tuple[str, ...]:
    """Tensor names of a shard by data offset (overlaps rejected)."""
    _, entries = _read_header(path)
    ordered = sorted(entries.items(),
                     key=lambda kv: (kv[1]["data_offsets"][0], kv[1]["data_offsets"][1], kv[0]))
    end = 0
    for name, entry in ordered:
        if entry["data_offsets"][0] < end:
            raise PackedCheckpointError(f"overlapping data_offsets before {name} in {path}")
        end = entry["data_offsets"][1]
    return tuple(name for name, _ in ordered)


def _read_source_tensor(handle: Any, name: str) -> torch.Tensor:
    return handle.get_tensor(name)


def read_expert_layer_pinned(path: str | Path, expected_shape: tuple[int, int], *,
                             pin_memory: bool = True) -> tuple[torch.Tensor, float]:
    """The ``experts`` tensor of a packed layer file as a pinned bf16
    tensor, read directly into the pinned allocation.  Returns (tensor,
    read seconds).  ``pin_memory=False`` reads into ordinary memory (hosts
    without a GPU runtime)."""
    path = Path(path)
    start, entries = _read_header(path)
    if tuple(entries) != ("experts",):
        raise ValueError(f"packed expert layer must contain only 'experts': {path}")
    entry = entries["experts"]
    if entry.get("dtype") != "BF16":
        raise ValueError("packed expert layer must use BF16")
    if tuple(entry.get("shape", ())) != tuple(expected_shape):
        raise ValueError(f"packed expert layer has shape {tuple(entry.get('shape', ()))}, "
                         f"expected {tuple(expected_shape)}")
    lo, hi = entry["data_offsets"]
    nbytes = prod(expected_shape) * 2
    if hi - lo != nbytes:
        raise ValueError(f"packed expert layer byte count does not match its shape: {path}")
    out = torch.empty(expected_shape, dtype=torch.bfloat16, pin_memory=pin_memory)
    view = out.view(-1).view(torch.uint8).numpy()
    t0 = time.perf_counter()
    with path.open("rb", buffering=0) as fh:
        fh.seek(start + lo)
        pos = 0
        step = 64 << 20
        while pos < nbytes:
            got = fh.readinto(memoryview(view[pos:pos + step]))
            if not got:
                raise ValueError(f"packed expert layer is truncated: {path}")
            pos += got
    return out, time.perf_counter() - t0


# ------------------------------------------------------- original layout --
@dataclass(frozen=True, slots=True)
class TensorLocation:
    name: str
    shard: str
    shape: tuple[int, ...]
    dtype: str
    nbytes: int


@dataclass(frozen=True, slots=True)
class ExpertSpec:
    key: ExpertKey
    gate_proj: TensorLocation
    up_proj: TensorLocation
    down_proj: TensorLocation

    @property
    def nbytes(self) -> int:
        return self.gate_proj.nbytes + self.up_proj.nbytes + self.down_proj.nbytes


@dataclass(frozen=True, slots=True)
class ModelCensus:
    model_type: str
    torch_dtype: str
    num_hidden_layers: int
    num_experts: int
    num_experts_per_tok: int
    hidden_size: int
    moe_intermediate_size: int
    shared_expert_tensor_count: int
    checkpoint_total_bytes: int
    routed_expert_bytes: int
    nonexpert_bytes: int
    expert_bytes: int
    expert_count: int

    def as_dict(self) -> dict[str, int | str]:
        return {f: getattr(self, f) for f in self.__slots__}


@dataclass(frozen=True, slots=True)
class CheckpointLayout:
    model_root: Path
    config_sha256: str
    index_sha256: str
    census: ModelCensus
    experts: tuple[ExpertSpec, ...]

    @classmethod
    def from_pretrained(cls, model_root: str | Path) -> "CheckpointLayout":
        root = Path(model_root).resolve()
        config_path = root / "config.json"
        index_path = root / "model.safetensors.index.json"
        config = json.loads(config_path.read_text())
        index = json.loads(index_path.read_text())
        weight_map: dict[str, str] = index["weight_map"]
        by_shard: dict[str, list[str]] = {}
        for name, shard in weight_map.items():
            if _EXPERT_KEY.match(name):
                by_shard.setdefault(shard, []).append(name)
        found: dict[tuple[int, int], dict[str, TensorLocation]] = {}
        for shard, names in sorted(by_shard.items()):
            _, entries = _read_header(root / shard)
            for name in names:
                m = _EXPERT_KEY.match(name)
                entry = entries.get(name)
                if entry is None:
                    raise ValueError(f"{name} is missing from {shard}")
                dtype = entry["dtype"]
                if dtype not in _DTYPES:
                    raise ValueError(f"unsupported tensor dtype {dtype!r} for {name}")
                shape = tuple(entry["shape"])
                found.setdefault((int(m["layer"]), int(m["expert"])), {})[m["projection"]] = (
                    TensorLocation(name=name, shard=shard, shape=shape, dtype=dtype,
                                   nbytes=prod(shape) * _DTYPES[dtype].itemsize))
        L = int(config["num_hidden_layers"])
        E = int(config.get("num_experts") or config["num_local_experts"])
        H = int(config["hidden_size"])
        I = int(config["moe_intermediate_size"])
        if len(found) != L * E:
            raise ValueError(f"found {len(found)} routed experts, expected {L * E}")
        shapes = {"gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
        experts = []
        for layer in range(L):
            for expert in range(E):
                proj = found[(layer, expert)]
                if set(proj) != set(shapes):
                    raise ValueError(f"expert {(layer, expert)} has projections {sorted(proj)}")
                for p, shape in shapes.items():
                    if proj[p].shape != shape:
                        raise ValueError(f"{proj[p].name} has shape {proj[p].shape}, "
                                         f"expected {shape}")
                experts.append(ExpertSpec(ExpertKey(layer, expert), proj["gate_proj"],
                                          proj["up_proj"], proj["down_proj"]))
        sizes = {e.nbytes for e in experts}
        if len(sizes) != 1:
            raise ValueError(f"expert sizes are not uniform: {sizes}")
        routed = sum(e.nbytes for e in experts)
        total = int(index["metadata"]["total_size"])
        if routed > total:
            raise ValueError("routed expert bytes exceed checkpoint total size")
        census = ModelCensus(
            model_type=str(config["model_type"]),
            torch_dtype=str(config.get("dtype") or config.get("torch_dtype")),
            num_hidden_layers=L, num_experts=E,
            num_experts_per_tok=int(config["num_experts_per_tok"]), hidden_size=H,
            moe_intermediate_size=I,
            shared_expert_tensor_count=sum(".shared_expert." in n for n in weight_map),
            checkpoint_total_bytes=total, routed_expert_bytes=routed,
            nonexpert_bytes=total - routed, expert_bytes=next(iter(sizes)),
            expert_count=len(experts))
        return cls(model_root=root, config_sha256=_sha256(config_path),
                   index_sha256=_sha256(index_path), census=census, experts=tuple(experts))

    def expert(self, key: ExpertKey) -> ExpertSpec:
        try:
            spec = self.experts[key.layer_id * self.census.num_experts + key.expert_id]
        except IndexError as error:
            raise KeyError(key) from error
        if spec.key != key:
            raise KeyError(key)
        return spec

    def expert_cache_bytes(self, slots_per_layer: int) -> int:
        if not 0 <= slots_per_layer <= self.census.num_experts:
            raise ValueError(f"slots_per_layer must be in [0, {self.census.num_experts}]")
        return slots_per_layer * self.census.num_hidden_layers * self.census.expert_bytes


# ---------------------------------------------------------------- packed --
def _field(c: dict, key: str, kind: str):
    v = c.get(key)
    if kind == "mapping":
        if not isinstance(v, dict):
            raise PackedCheckpointError(f"packed checkpoint manifest field {key!r} must be an object")
    elif kind == "string":
        if not isinstance(v, str) or not v:
            raise PackedCheckpointError(
                f"packed checkpoint manifest field {key!r} must be a nonempty string")
    elif kind == "sha256":
        v = _field(c, key, "string")
        if len(v) != 64 or any(ch not in "0123456789abcdef" for ch in v):
            raise PackedCheckpointError(
                f"packed checkpoint manifest field {key!r} must be a lowercase SHA256")
    else:  # "positive" / "nonnegative" integers
        lo = 1 if kind == "positive" else 0
        if not isinstance(v, int) or isinstance(v, bool) or v < lo:
            word = "a positive" if lo else "a nonnegative"
            raise PackedCheckpointError(
                f"packed checkpoint manifest field {key!r} must be {word} integer")
    return v


def _census_from(raw: dict) -> ModelCensus:
    kinds = dict(model_type="string", torch_dtype="string", num_hidden_layers="positive",
                 num_experts="positive", num_experts_per_tok="positive", hidden_size="positive",
                 moe_intermediate_size="positive", shared_expert_tensor_count="nonnegative",
                 checkpoint_total_bytes="positive", routed_expert_bytes="positive",
                 nonexpert_bytes="nonnegative", expert_bytes="positive", expert_count="positive")
    return ModelCensus(**{k: _field(raw, k, kind) for k, kind in kinds.items()})


@dataclass(frozen=True, slots=True)
class _FileRecord:
    filename: str
    size_bytes: int
    sha256: str


def _file_record_from(raw: dict, label: str) -> _FileRecord:
    name = _field(raw, "filename", "string")
    rel = Path(name)
    if rel.is_absolute() or ".." in rel.parts or rel == Path("."):
        raise PackedCheckpointError(f"packed checkpoint {label} file name must stay under root")
    digest = _field(raw, "sha256", "sha256")
    return _FileRecord(filename=name, size_bytes=_field(raw, "size_bytes", "positive"),
                       sha256=digest)


@dataclass(frozen=True, slots=True)
class PackedQwen3Checkpoint:
    root: Path
    manifest: dict[str, Any]
    census: ModelCensus
    packed_expert_elements: int
    _layer_files: tuple[_FileRecord, ...]
    _nonexpert_file: _FileRecord

    @property
    def nonexpert_path(self) -> Path:
        return self.root / self._nonexpert_file.filename

    def layer_path(self, layer_id: int) -> Path:
        if not 0 <= layer_id < len(self._layer_files):
            raise IndexError(f"layer_id must be in [0, {len(self._layer_files) - 1}]")
        return self.root / self._layer_files[layer_id].filename

    @classmethod
    def open(cls, root: str | Path, *, source_layout: CheckpointLayout | None = None,
             source_metadata_root: str | Path | None = None,
             verify_hashes: bool = False) -> "PackedQwen3Checkpoint":
        """Validate and open a packed checkpoint (qwen3_packed_checkpoint.py:155-374)."""
        if source_layout is not None and source_metadata_root is not None:
            raise ValueError("source_layout and source_metadata_root are mutually exclusive")
        root = Path(root).resolve()
        mpath = root / PACKED_MANIFEST_FILENAME
        if not mpath.is_file():
            raise PackedCheckpointError(f"packed checkpoint manifest is missing: {mpath}")
        try:
            manifest = json.loads(mpath.read_text(encoding="utf-8"))
        except (OSError, json.JSONDecodeError) as error:
            raise PackedCheckpointError(
                f"packed checkpoint manifest is unreadable: {mpath}") from error
        if not isinstance(manifest, dict):
            raise PackedCheckpointError("packed checkpoint manifest must be an object")
        if manifest.get("complete") is not True:
            raise PackedCheckpointError("packed checkpoint manifest must declare complete=true")
        if manifest.get("schema") != PACKED_CHECKPOINT_SCHEMA:
            raise PackedCheckpointError("packed checkpoint manifest schema does not match")
        if manifest.get("schema_version") != PACKED_CHECKPOINT_VERSION:
            raise PackedCheckpointError(
                "packed checkpoint manifest schema version does not match")
        source = _field(manifest, "source", "mapping")
        if _field(source, "config_filename", "string") != "config.json":
            raise PackedCheckpointError("source config filename does not match")
        if _field(source, "index_filename", "string") != "model.safetensors.index.json":
            raise PackedCheckpointError("source index filename does not match")
        config_sha = _field(source, "config_sha256", "sha256")
        index_sha = _field(source, "index_sha256", "sha256")
        for key in ("repo_id", "revision"):
            if key in source:
                _field(source, key, "string")
        model = _field(manifest, "model", "mapping")
        census = _census_from(_field(model, "census", "mapping"))
        elements = _field(model, "packed_expert_elements", "positive")
        dtype = _field(model, "expert_dtype", "string")
        if dtype not in _DTYPES:
            raise PackedCheckpointError(f"unsupported packed expert dtype: {dtype}")
        if model.get("expert_layout") != list(PACKED_EXPERT_LAYOUT):
            raise PackedCheckpointError("packed checkpoint expert layout does not match")
        if elements != 3 * census.hidden_size * census.moe_intermediate_size:
            raise PackedCheckpointError(
                "packed expert element count does not match model dimensions")
        if elements * _DTYPES[dtype].itemsize != census.expert_bytes:
            raise PackedCheckpointError("packed expert byte count does not match census")
        if census.expert_count != census.num_hidden_layers * census.num_experts:
            raise PackedCheckpointError("packed expert count does not match census dimensions")
        if census.routed_expert_bytes != census.expert_count * census.expert_bytes:
            raise PackedCheckpointError("routed expert byte count does not match census")
        if census.checkpoint_total_bytes != census.routed_expert_bytes + census.nonexpert_bytes:
            raise PackedCheckpointError("checkpoint byte count does not match census")
        files = _field(manifest, "files", "mapping")
        nonexpert = _file_record_from(_field(files, "nonexperts", "mapping"), "nonexperts")
        raw_layers = files.get("layers")
        if not isinstance(raw_layers, list):
            raise PackedCheckpointError("packed checkpoint layer files must be a list")
        if len(raw_layers) != census.num_hidden_layers:
            raise PackedCheckpointError(
                "packed checkpoint layer file count does not match census")
        layers = []
        for lid, rec in enumerate(raw_layers):
            if not isinstance(rec, dict):
                raise PackedCheckpointError(
                    "packed checkpoint layer file record must be an object")
            if rec.get("layer_id") != lid:
                raise PackedCheckpointError("packed checkpoint layer IDs must be contiguous")
            if rec.get("tensor_name") != "experts":
                raise PackedCheckpointError(
                    "packed checkpoint layer tensor name must be experts")
            if rec.get("shape") != [census.num_experts, elements]:
                raise PackedCheckpointError(
                    "packed checkpoint layer tensor shape does not match")
            if rec.get("dtype") != dtype:
                raise PackedCheckpointError(
                    "packed checkpoint layer tensor dtype does not match")
            layers.append(_file_record_from(rec, f"layer {lid}"))
        records = (nonexpert, *layers)
        if len({r.filename for r in records}) != len(records):
            raise PackedCheckpointError("packed checkpoint file names must be unique")
        for rec in records:
            path = root / rec.filename
            if not path.is_file():
                raise PackedCheckpointError(f"packed checkpoint file is missing: {path}")
            if path.stat().st_size != rec.size_bytes:
                raise PackedCheckpointError(f"packed checkpoint file size does not match: {path}")
            if verify_hashes and _sha256(path) != rec.sha256:
                raise PackedCheckpointError(
                    f"packed checkpoint file SHA256 does not match: {path}")
        if source_layout is not None:
            if config_sha != source_layout.config_sha256:
                raise PackedCheckpointError(
                    "source config SHA256 does not match packed checkpoint")
            if index_sha != source_layout.index_sha256:
                raise PackedCheckpointError(
                    "source index SHA256 does not match packed checkpoint")
            if census.as_dict() != source_layout.census.as_dict():
                raise PackedCheckpointError("source census does not match packed checkpoint")
        elif source_metadata_root is not None:
            meta = Path(source_metadata_root).resolve()
            cfg, idx = meta / "config.json", meta / "model.safetensors.index.json"
            if not cfg.is_file() or not idx.is_file():
                raise PackedCheckpointError("source config or index metadata is missing")
            if _sha256(cfg) != config_sha:
                raise PackedCheckpointError(
                    "source config SHA256 does not match packed checkpoint")
            if _sha256(idx) != index_sha:
                raise PackedCheckpointError(
                    "source index SHA256 does not match packed checkpoint")
        return cls(root=root, manifest=manifest, census=census, packed_expert_elements=elements,
                   _layer_files=tuple(layers), _nonexpert_file=nonexpert)


def _expert_destinations(layout: CheckpointLayout):
    """tensor name -> (layer, expert, element offset, elements) in the
    packed ``[gate | up | down]`` row; plus the row length and dtype."""
    dtypes = {loc.dtype for e in layout.experts for loc in (e.gate_proj, e.up_proj, e.down_proj)}
    if len(dtypes) != 1:
        raise PackedCheckpointError(f"routed expert dtypes are not uniform: {dtypes}")
    dtype = next(iter(dtypes))
    if dtype not in _DTYPES:
        raise PackedCheckpointError(f"unsupported routed expert dtype: {dtype}")
    item = _DTYPES[dtype].itemsize
    row = 3 * layout.census.hidden_size * layout.census.moe_intermediate_size
    dest = {}
    for e in layout.experts:
        off = 0
        for loc in (e.gate_proj, e.up_proj, e.down_proj):
            n = loc.nbytes // item
            dest[loc.name] = (e.key.layer_id, e.key.expert_id, off, n)
            off += n
        if off != row:
            raise PackedCheckpointError(f"packed size does not match expert {e.key}")
    return dest, row, dtype


def _read_sources(src: Path, buffers: list[torch.Tensor], dest: dict) -> dict[str, torch.Tensor]:
    """Read every source shard in physical tensor order, scattering expert
    tensors into their packed rows; returns the non-expert tensors."""
    from safetensors import safe_open

    index = json.loads((src / "model.safetensors.index.json").read_text(encoding="utf-8"))
    weight_map = index.get("weight_map")
    if not isinstance(weight_map, dict) or not weight_map:
        raise PackedCheckpointError("source checkpoint weight_map must be a nonempty object")
    if not all(isinstance(k, str) and isinstance(v, str) for k, v in weight_map.items()):
        raise PackedCheckpointError("source checkpoint weight_map entries must be strings")
    by_shard: dict[str, set[str]] = {}
    for name, shard in weight_map.items():
        by_shard.setdefault(shard, set()).add(name)
    nonexperts: dict[str, torch.Tensor] = {}
    seen: set[str] = set()
    for shard in sorted(by_shard):
        order = _tensor_names_in_storage_order(src / shard)
        if set(order) != by_shard[shard]:
            missing = sorted(by_shard[shard] - set(order))
            unexpected = sorted(set(order) - by_shard[shard])
            raise PackedCheckpointError(f"source shard index mismatch for {shard}: "
                                        f"missing={missing[:5]}, unexpected={unexpected[:5]}")
        with safe_open(src / shard, framework="pt", device="cpu") as handle:
            for name in order:
                value = _read_source_tensor(handle, name)
                d = dest.get(name)
                if d is None:
                    nonexperts[name] = value.clone()
                else:
                    layer, expert, off, n = d
                    if value.numel() != n:
                        raise PackedCheckpointError(f"source tensor element count changed: {name}")
                    buffers[layer][expert, off:off + n].copy_(value.reshape(-1))
                seen.add(name)
    if seen != set(weight_map):
        raise PackedCheckpointError(
            f"source checkpoint tensors were not all read: {sorted(set(weight_map) - seen)[:5]}")
    if set(nonexperts) != set(weight_map) - set(dest):
        raise PackedCheckpointError("source nonexpert tensor collection is incomplete")
    if not nonexperts:
        raise PackedCheckpointError("source checkpoint contains no nonexpert tensors")
    return nonexperts


def _record(path: Path, root: Path) -> dict[str, Any]:
    return {"filename": path.relative_to(root).as_posix(), "size_bytes": path.stat().st_size,
            "sha256": _sha256(path)}


def pack_qwen3_checkpoint(source_root: str | Path, output_root: str | Path, *,
                          source_repo_id: str | None = None,
                          source_revision: str | None = None) -> PackedQwen3Checkpoint:
    """Write the packed-v1 form of an original checkpoint
    (qwen3_packed_checkpoint.py:650-795): built in a staging directory next
    to ``output_root`` and renamed into place when complete."""
    from safetensors.torch import save_file

    src = Path(source_root).resolve()
    dst = Path(output_root).resolve()
    for label, value in (("source_repo_id", source_repo_id), ("source_revision", source_revision)):
        if value is not None and (not isinstance(value, str) or not value):
            raise ValueError(f"{label} must be a nonempty string when provided")
    if dst.exists():
        raise FileExistsError(f"packed checkpoint destination already exists: {dst}")
    dst.parent.mkdir(parents=True, exist_ok=True)
    staging = dst.parent / f".{dst.name}.partial-{uuid.uuid4().hex}"
    staging.mkdir()
    layout = CheckpointLayout.from_pretrained(src)
    dest, row, dtype = _expert_destinations(layout)
    c = layout.census
    buffers = [torch.empty((c.num_experts, row), dtype=_DTYPES[dtype])
               for _ in range(c.num_hidden_layers)]
    nonexperts = _read_sources(src, buffers, dest)
    (staging / "experts").mkdir()
    width = max(3, len(str(c.num_hidden_layers - 1)))
    layer_records = []
    for lid, experts in enumerate(buffers):
        path = staging / "experts" / f"layer-{lid:0{width}d}.safetensors"
        save_file({"experts": experts}, path,
                  metadata={"format": "pt", "layer_id": str(lid),
                            "expert_layout": "|".join(PACKED_EXPERT_LAYOUT)})
        rec = _record(path, staging)
        rec.update({"layer_id": lid, "tensor_name": "experts", "shape": [c.num_experts, row],
                    "dtype": dtype})
        layer_records.append(rec)
    nonexpert_path = staging / "nonexperts.safetensors"
    save_file(nonexperts, nonexpert_path,
              metadata={"format": "pt", "source_config_sha256": layout.config_sha256,
                        "source_index_sha256": layout.index_sha256})
    nonexpert_record = _record(nonexpert_path, staging)
    nonexpert_record["tensor_count"] = len(nonexperts)
    source = {"config_filename": "config.json", "config_sha256": layout.config_sha256,
              "index_filename": "model.safetensors.index.json",
              "index_sha256": layout.index_sha256}
    if source_repo_id is not None:
        source["repo_id"] = source_repo_id
    if source_revision is not None:
        source["revision"] = source_revision
    manifest = {"schema": PACKED_CHECKPOINT_SCHEMA, "schema_version": PACKED_CHECKPOINT_VERSION,
                "complete": True, "source": source,
                "model": {"census": c.as_dict(), "packed_expert_elements": row,
                          "expert_layout": list(PACKED_EXPERT_LAYOUT), "expert_dtype": dtype},
                "files": {"nonexperts": nonexpert_record, "layers": layer_records}}
    tmp = staging / (PACKED_MANIFEST_FILENAME + ".partial")
    with tmp.open("w", encoding="utf-8") as fh:
        fh.write(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
        fh.flush()
        os.fsync(fh.fileno())
    os.replace(tmp, staging / PACKED_MANIFEST_FILENAME)
    os.rename(staging, dst)
    return PackedQwen3Checkpoint.open(dst, source_layout=layout)


__all__ = ["CheckpointLayout", "ExpertSpec", "ModelCensus", "PACKED_CHECKPOINT_SCHEMA",
           "PACKED_CHECKPOINT_VERSION", "PACKED_EXPERT_LAYOUT", "PACKED_MANIFEST_FILENAME",
           "PackedCheckpointError", "PackedQwen3Checkpoint", "TensorLocation",
           "pack_qwen3_checkpoint", "read_expert_layer_pinned"]

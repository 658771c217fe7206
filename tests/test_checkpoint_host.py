"""Original-layout census and the packed-v1 checkpoint on the host.

Restates the reference's tests (tests/unit/test_qwen3_packed_checkpoint.py:
the same fixture checkpoint of 2 layers x 2 experts, hidden 2, intermediate
3, split over two shards) for specfit_amd.checkpoint's writer and reader, plus the
direct pinned-layer reader.
"""
import hashlib
import json
from pathlib import Path
from unittest import mock

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

import specfit_amd.checkpoint as ckpt
from specfit_amd.checkpoint import (CheckpointLayout, PackedCheckpointError,
                                    PackedQwen3Checkpoint, pack_qwen3_checkpoint,
                                    read_expert_layer_pinned)


def _sha256(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def _write_source(root: Path, dtype=torch.float32) -> dict:
    config = {"model_type": "qwen3_moe", "torch_dtype": "float32", "num_hidden_layers": 2,
              "num_experts": 2, "num_experts_per_tok": 1, "hidden_size": 2,
              "moe_intermediate_size": 3}
    (root / "config.json").write_text(json.dumps(config, sort_keys=True), encoding="utf-8")
    tensors, nxt = {}, 1
    for layer in range(2):
        for expert in range(2):
            prefix = f"model.layers.{layer}.mlp.experts.{expert}"
            for proj, shape in (("gate_proj", (3, 2)), ("up_proj", (3, 2)), ("down_proj", (2, 3))):
                tensors[f"{prefix}.{proj}.weight"] = torch.arange(
                    nxt, nxt + 6, dtype=torch.float32).reshape(shape).to(dtype)
                nxt += 6
    tensors["model.embed_tokens.weight"] = torch.arange(8, dtype=torch.float32).reshape(4, 2)
    tensors["model.norm.weight"] = torch.tensor([0.25, 0.5])
    names = tuple(tensors)
    shards = ("model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors")
    save_file({n: tensors[n] for n in names[::2]}, root / shards[0])
    save_file({n: tensors[n] for n in names[1::2]}, root / shards[1])
    index = {"metadata": {"total_size": sum(t.numel() * t.element_size() for t in tensors.values())},
             "weight_map": {n: shards[i % 2] for i, n in enumerate(names)}}
    (root / "model.safetensors.index.json").write_text(json.dumps(index, sort_keys=True),
                                                       encoding="utf-8")
    return tensors


@pytest.fixture
def source(tmp_path):
    src = tmp_path / "source"
    src.mkdir()
    return src, _write_source(src), tmp_path / "packed"


def test_pack_preserves_expert_layout_and_nonexpert_tensors(source):
    src, tensors, out = source
    layout = CheckpointLayout.from_pretrained(src)
    assert layout.census.expert_count == 4 and layout.census.expert_bytes == 18 * 4
    packed = pack_qwen3_checkpoint(src, out, source_repo_id="fixture/Qwen3-MoE",
                                   source_revision="fixture-revision")
    reopened = PackedQwen3Checkpoint.open(out, source_layout=layout, verify_hashes=True)
    assert packed == reopened
    assert reopened.census.num_hidden_layers == 2 and reopened.census.num_experts == 2
    assert reopened.packed_expert_elements == 18 and reopened.manifest["complete"]
    for layer in range(2):
        with safe_open(reopened.layer_path(layer), framework="pt", device="cpu") as h:
            assert tuple(h.keys()) == ("experts",)
            actual = h.get_tensor("experts")
        rows = [torch.cat([tensors[f"model.layers.{layer}.mlp.experts.{e}.{p}.weight"].reshape(-1)
                           for p in ("gate_proj", "up_proj", "down_proj")]) for e in range(2)]
        torch.testing.assert_close(actual, torch.stack(rows))
    with safe_open(reopened.nonexpert_path, framework="pt", device="cpu") as h:
        assert set(h.keys()) == {"model.embed_tokens.weight", "model.norm.weight"}
        for name in h.keys():
            torch.testing.assert_close(h.get_tensor(name), tensors[name])
    m = reopened.manifest
    assert m["source"]["config_sha256"] == _sha256(src / "config.json")
    assert m["source"]["index_sha256"] == _sha256(src / "model.safetensors.index.json")
    assert m["source"]["repo_id"] == "fixture/Qwen3-MoE"
    assert m["source"]["revision"] == "fixture-revision"
    for rec in [m["files"]["nonexperts"], *m["files"]["layers"]]:
        path = out / rec["filename"]
        assert rec["size_bytes"] == path.stat().st_size and rec["sha256"] == _sha256(path)


def test_source_tensors_are_read_shard_first_in_physical_order(source):
    src, _, out = source
    index = json.loads((src / "model.safetensors.index.json").read_text(encoding="utf-8"))
    expected = []
    for shard in sorted(set(index["weight_map"].values())):
        expected.extend(ckpt._tensor_names_in_storage_order(src / shard))
    observed = []
    original = ckpt._read_source_tensor

    def recording(handle, name):
        observed.append(name)
        return original(handle, name)

    with mock.patch.object(ckpt, "_read_source_tensor", side_effect=recording):
        pack_qwen3_checkpoint(src, out)
    assert observed == expected


def test_open_rejects_missing_or_incomplete_manifest(tmp_path):
    d = tmp_path / "incomplete"
    d.mkdir()
    with pytest.raises(PackedCheckpointError, match="manifest"):
        PackedQwen3Checkpoint.open(d)
    (d / "manifest.json").write_text(json.dumps({"schema": ckpt.PACKED_CHECKPOINT_SCHEMA,
                                                 "schema_version": ckpt.PACKED_CHECKPOINT_VERSION,
                                                 "complete": False}), encoding="utf-8")
    with pytest.raises(PackedCheckpointError, match="complete"):
        PackedQwen3Checkpoint.open(d)


def test_open_rejects_source_hash_mismatch(source):
    src, _, out = source
    pack_qwen3_checkpoint(src, out)
    before = CheckpointLayout.from_pretrained(src)
    cfg = json.loads((src / "config.json").read_text(encoding="utf-8"))
    cfg["fixture_revision"] = 2
    (src / "config.json").write_text(json.dumps(cfg, sort_keys=True), encoding="utf-8")
    changed = CheckpointLayout.from_pretrained(src)
    assert before.config_sha256 != changed.config_sha256
    with pytest.raises(PackedCheckpointError, match="config SHA256"):
        PackedQwen3Checkpoint.open(out, source_layout=changed)


def test_open_validates_source_metadata_without_weight_shards(source):
    src, _, out = source
    pack_qwen3_checkpoint(src, out)
    for shard in src.glob("model-*.safetensors"):
        shard.unlink()
    reopened = PackedQwen3Checkpoint.open(out, source_metadata_root=src)
    assert reopened.census.num_hidden_layers == 2 and reopened.census.num_experts == 2


def test_source_metadata_validation_rejects_hash_mismatch(source):
    src, _, out = source
    pack_qwen3_checkpoint(src, out)
    cfg = json.loads((src / "config.json").read_text(encoding="utf-8"))
    cfg["fixture_revision"] = 3
    (src / "config.json").write_text(json.dumps(cfg, sort_keys=True), encoding="utf-8")
    with pytest.raises(PackedCheckpointError, match="config SHA256"):
        PackedQwen3Checkpoint.open(out, source_metadata_root=src)


def test_explicit_hash_verification_detects_same_size_corruption(source):
    src, _, out = source
    packed = pack_qwen3_checkpoint(src, out)
    path = packed.layer_path(0)
    with path.open("r+b") as fh:
        fh.seek(-1, 2)
        b = fh.read(1)
        fh.seek(-1, 2)
        fh.write(bytes((b[0] ^ 0xFF,)))
    PackedQwen3Checkpoint.open(out, verify_hashes=False)
    with pytest.raises(PackedCheckpointError, match="SHA256"):
        PackedQwen3Checkpoint.open(out, verify_hashes=True)


def test_pack_refuses_existing_destination(source):
    src, _, out = source
    out.mkdir()
    with pytest.raises(FileExistsError, match="already exists"):
        pack_qwen3_checkpoint(src, out)


def test_manifest_field_validation(source):
    src, _, out = source
    pack_qwen3_checkpoint(src, out)
    good = json.loads((out / "manifest.json").read_text())
    cases = [
        (lambda m: m.update(schema="other"), "schema does not match"),
        (lambda m: m["model"].update(expert_layout=["up_proj", "gate_proj", "down_proj"]),
         "expert layout"),
        (lambda m: m["model"].update(packed_expert_elements=17), "element count"),
        (lambda m: m["files"]["layers"][1].update(layer_id=0), "contiguous"),
        (lambda m: m["files"]["layers"][0].update(filename="../x.safetensors"), "under root"),
        (lambda m: m["source"].update(config_sha256="ABC"), "lowercase SHA256"),
        (lambda m: m["model"]["census"].update(nonexpert_bytes=-1), "nonnegative"),
    ]
    for change, message in cases:
        m = json.loads(json.dumps(good))
        change(m)
        (out / "manifest.json").write_text(json.dumps(m))
        with pytest.raises(PackedCheckpointError, match=message):
            PackedQwen3Checkpoint.open(out)


def test_pinned_layer_reader_matches_safetensors(tmp_path):
    src = tmp_path / "source"
    src.mkdir()
    _write_source(src, dtype=torch.bfloat16)
    packed = pack_qwen3_checkpoint(src, tmp_path / "packed")
    for layer in range(2):
        with safe_open(packed.layer_path(layer), framework="pt", device="cpu") as h:
            expected = h.get_tensor("experts")
        got, seconds = read_expert_layer_pinned(packed.layer_path(layer), (2, 18),
                                                pin_memory=False)
        assert torch.equal(got, expected) and seconds >= 0
    with pytest.raises(ValueError, match="shape"):
        read_expert_layer_pinned(packed.layer_path(0), (2, 17), pin_memory=False)
    f32 = pack_qwen3_checkpoint(*(lambda d: (d, tmp_path / "packed32"))(
        (lambda s: (s.mkdir(), _write_source(s), s)[2])(tmp_path / "src32")))
    with pytest.raises(ValueError, match="BF16"):
        read_expert_layer_pinned(f32.layer_path(0), (2, 18), pin_memory=False)

"""The reference's on-disk weight formats on the CPU: the FP8 pack writer and
reader (tools/pack_fp8.py, src/pcketlm/core/runtime/fp8_pack.py; the cases of
tests/test_fp8_pack_writer_reader.py), the row8 artifact
(tools/pack_weights_row8.py; tests/test_packed_weight_artifact.py) and the Q4
shards (src/pcketlm/core/model_import/q4_quantize.py), plus the library's
host file mapping (row8_artifact_cache.cpp:66-147)."""

from __future__ import annotations

import ctypes
import gc
import json
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from pocketlm_amd import formats, packs


def _pack_fixture(tmp_path: Path) -> Path:
    """The reference test's model directory: one safetensors shard of raw
    payloads (tests/test_fp8_pack_writer_reader.py:107-132)."""
    model_dir = tmp_path / "model"
    model_dir.mkdir()
    shard = model_dir / "model-00001-of-00001.safetensors"
    tensors = {
        "model.layers.0.mlp.experts.0.gate_proj.weight": ("F8_E4M3", [2, 4], b"abcdefgh"),
        "model.layers.0.mlp.experts.0.gate_proj.weight_scale_inv": ("F32", [1, 1], b"SCAL"),
        "model.layers.0.self_attn.q_a_proj.weight": ("F8_E4M3", [2, 4], b"ABCDEFGH"),
        "model.layers.0.self_attn.q_a_proj.weight_scale_inv": ("F32", [1, 1], b"scal"),
        "lm_head.weight": ("BF16", [2, 2], b"LMHD"),
    }
    header, payload, offset = {}, bytearray(), 0
    for name, (dtype, shape, raw) in tensors.items():
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [offset, offset + len(raw)]}
        payload.extend(raw)
        offset += len(raw)
    blob = json.dumps(header).encode("utf-8")
    shard.write_bytes(struct.pack("<Q", len(blob)) + blob + payload)
    (model_dir / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {name: shard.name for name in tensors}}), encoding="utf-8")
    return model_dir


GATE = "model.layers.0.mlp.experts.0.gate_proj.weight"
GATE_SCALE = GATE + "_scale_inv"


def test_pack_writer_preserves_bytes_and_reader_returns_views(tmp_path):
    model_dir = _pack_fixture(tmp_path)
    manifest = packs.pack_model_dir_to_fp8(model_dir, model_dir / "artifacts" / "fp8_pack", pack_bytes=128)
    reader = packs.FP8PackReader(model_dir)
    tensor = reader.get_tensor(GATE)
    assert manifest["format"] == "pcketlm-fp8-pack-v1" and len(manifest["tensors"]) == 5
    assert bytes(tensor.fp8_bytes) == b"abcdefgh"
    assert bytes(tensor.scale_bytes) == b"SCAL"
    assert tensor.scale_name == GATE_SCALE and tensor.scale_shape == [1, 1] and tensor.shape == [2, 4]
    assert reader.telemetry()["sequential_reads"] == 1
    assert bytes(reader.get_tensor("lm_head.weight").fp8_bytes) == b"LMHD"


def test_pack_order_and_scale_links(tmp_path):
    """The writer's order: top-level tensors, then per layer attention before
    routed experts; each weight directly followed by its scale, the two
    entries cross-linked."""
    model_dir = _pack_fixture(tmp_path)
    manifest = packs.pack_model_dir_to_fp8(model_dir, pack_bytes=128)
    order = sorted(manifest["tensors"].values(), key=lambda e: e["pack_order"])
    assert [e["name"] for e in order] == [
        "lm_head.weight", "model.layers.0.self_attn.q_a_proj.weight",
        "model.layers.0.self_attn.q_a_proj.weight_scale_inv", GATE, GATE_SCALE]
    assert [e["byte_offset"] for e in order] == [0, 4, 12, 16, 24]
    gate, scale = manifest["tensors"][GATE], manifest["tensors"][GATE_SCALE]
    assert gate["scale_byte_offset"] == scale["byte_offset"] == 24 and gate["scale_byte_length"] == 4
    assert scale["tensor_role"] == "scale_companion" and scale["weight_name"] == GATE
    assert gate["layer_index"] == 0 and gate["expert_index"] == 0
    assert manifest["pack_files"] == [{"index": 0, "file_name": "pack_0000.bin", "byte_length": 28}]


def test_pack_reader_reports_slice_and_span_locations(tmp_path):
    model_dir = _pack_fixture(tmp_path)
    packs.pack_model_dir_to_fp8(model_dir, pack_bytes=128)
    reader = packs.FP8PackReader(model_dir)
    sl = reader.get_tensor_slice_location(GATE, 2, 3)
    sp = reader.get_tensor_span_location([GATE, GATE_SCALE])
    with sl.path.open("rb") as handle:
        handle.seek(sl.byte_offset)
        assert handle.read(sl.byte_length) == b"cde"
    with sp.path.open("rb") as handle:
        handle.seek(sp.byte_offset)
        assert handle.read(sp.byte_length) == b"abcdefghSCAL"
    assert sp.tensor_slices == {GATE: (0, 8), GATE_SCALE: (8, 4)}
    assert bytes(reader.get_tensor_span_bytes([GATE, GATE_SCALE]).bytes) == b"abcdefghSCAL"
    assert bytes(reader.get_tensor_slice_bytes(GATE, 6, 2)) == b"gh"
    assert reader.telemetry()["sequential_reads"] == 4
    with pytest.raises(ValueError, match="exceeds"):
        reader.get_tensor_slice_location(GATE, 6, 3)
    with pytest.raises(KeyError, match="not present"):
        reader.get_tensor("missing.weight")


def test_pack_reader_releases_maps_once_views_are_gone(tmp_path):
    model_dir = _pack_fixture(tmp_path)
    packs.pack_model_dir_to_fp8(model_dir, pack_bytes=128)
    reader = packs.FP8PackReader(model_dir)
    tensor = reader.get_tensor(GATE)
    assert reader.telemetry()["mmap_bytes_mapped"] == 28
    reader.close()  # a live view keeps its map
    assert reader.telemetry()["pack_files_open"] == 1
    del tensor
    gc.collect()
    reader.close()
    assert reader.telemetry()["mmap_bytes_mapped"] == 0 and reader.telemetry()["pack_files_open"] == 0


def test_pack_rollover_and_cross_file_spans(tmp_path):
    """A tensor that would overflow pack_bytes starts a new pack file; spans
    across files are refused; tensors come back byte for byte."""
    g = torch.Generator().manual_seed(3)
    tensors = {}
    for e in range(3):
        for proj, shape in (("gate_proj", (8, 16)), ("up_proj", (8, 16)), ("down_proj", (16, 8))):
            name = f"model.layers.2.mlp.experts.{e}.{proj}.weight"
            tensors[name] = (torch.randn(shape, generator=g) * 0.1).to(torch.float8_e4m3fn)
            tensors[name + "_scale_inv"] = torch.rand((1, 1), generator=g)
    manifest = packs.write_fp8_pack(tensors, tmp_path / "m" / "artifacts" / "fp8_pack", pack_bytes=300)
    assert len(manifest["pack_files"]) > 1
    assert all(f["byte_length"] <= 300 for f in manifest["pack_files"])
    reader = packs.FP8PackReader(tmp_path / "m")
    for name, t in tensors.items():
        assert bytes(reader.get_tensor(name).fp8_bytes) == t.view(torch.uint8).numpy().tobytes()
    first, last = "model.layers.2.mlp.experts.0.gate_proj.weight", "model.layers.2.mlp.experts.2.down_proj.weight"
    assert manifest["tensors"][first]["pack_file_index"] != manifest["tensors"][last]["pack_file_index"]
    with pytest.raises(ValueError, match="crosses pack files"):
        reader.get_tensor_span_location([first, last])
    experts = reader.get_layer_experts(2, [1, 2])
    assert [v.name.split(".")[5] for v in experts] == ["1", "1", "1", "2", "2", "2"]
    assert [v.name.split(".")[6] for v in experts[:3]] == ["gate_proj", "up_proj", "down_proj"]


def test_pack_dir_override(tmp_path, monkeypatch):
    monkeypatch.setenv("PCKETLM_FP8_PACK_DIR", str(tmp_path / "elsewhere"))
    packs._pack_dir.cache_clear()
    try:
        assert packs.default_fp8_pack_dir(tmp_path / "model") == (tmp_path / "elsewhere").resolve()
        assert not packs.fp8_pack_available(tmp_path / "model")
        with pytest.raises(FileNotFoundError):
            packs.FP8PackReader(tmp_path / "model")
    finally:
        packs._pack_dir.cache_clear()


def test_row8_artifact_manifest_and_bytes(tmp_path):
    """tests/test_packed_weight_artifact.py:23-36 on the CPU: the manifest
    entry and the packed bytes of a 10 x 13 fp16 tensor."""
    from safetensors.torch import save_file

    model_dir = tmp_path / "source"
    model_dir.mkdir()
    down = torch.arange(130, dtype=torch.float32).reshape(10, 13).to(torch.float16)
    save_file({"model.layers.0.mlp.down_proj.weight": down,
               "model.layers.0.mlp.up_proj.weight": torch.ones((10, 13), dtype=torch.float16)},
              str(model_dir / "model-00001-of-00001.safetensors"))
    (model_dir / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {
        "model.layers.0.mlp.down_proj.weight": "model-00001-of-00001.safetensors",
        "model.layers.0.mlp.up_proj.weight": "model-00001-of-00001.safetensors"}}), encoding="utf-8")
    manifest = packs.build_row8_packed_artifact(model_dir, tmp_path / "row8", include_patterns=["down_proj"])
    entry = manifest["tensors"]["model.layers.0.mlp.down_proj.weight"]
    assert manifest["format"] == "pcketlm-row8-packed-gemv" and manifest["tensor_count"] == 1
    assert entry["shape"] == [10, 13] and entry["dtype"] == "F16" and entry["offset"] == 0
    data = (tmp_path / "row8" / "row8_packed.bin").read_bytes()
    assert len(data) == entry["nbytes"] == 2 * 16 * 13
    assert data == formats.pack_rows8_tensor(down).numpy().tobytes()
    packed = torch.frombuffer(bytearray(data), dtype=torch.uint16)
    assert torch.equal(formats.unpack_rows8_tensor(packed, 10, 13, dtype=torch.float16), down)


def test_q4_artifact_shards_hold_the_quantized_tensors(tmp_path):
    from safetensors import safe_open

    g = torch.Generator().manual_seed(8)
    w = torch.randn((48, 40), generator=g).to(torch.bfloat16)
    manifest = packs.quantize_tensors_to_q4_artifact({"model.layers.0.mlp.gate_proj.weight": w,
                                                      "model.layers.0.step": torch.arange(3)}, tmp_path)
    entry = manifest["tensors"]["model.layers.0.mlp.gate_proj.weight"]
    assert list(manifest["tensors"]) == ["model.layers.0.mlp.gate_proj.weight"]
    assert manifest["format"] == "pcketlm-q4" and entry["scheme"] == "per-channel-symmetric-v1"
    want_p, want_s, _meta = formats.quantize_tensor_to_q4(w)
    with safe_open(str(tmp_path / entry["q4_shard"]), framework="pt") as f:
        assert torch.equal(f.get_tensor("model.layers.0.mlp.gate_proj.weight"), want_p)
    with safe_open(str(tmp_path / entry["scale_shard"]), framework="pt") as f:
        assert torch.equal(f.get_tensor("model.layers.0.mlp.gate_proj.weight"), want_s)
    header, base = packs.read_safetensors_header(tmp_path / entry["q4_shard"])
    start, end = header["model.layers.0.mlp.gate_proj.weight"]["data_offsets"]
    raw = (tmp_path / entry["q4_shard"]).read_bytes()[base + start:base + end]
    assert raw == want_p.numpy().tobytes()


def test_row8_mapped_file_gives_host_views(tmp_path):
    """row8_artifact_map_file / mapped_data (row8_artifact_cache.cpp:66-147)
    on the CPU: whole-file mapping, bounds and alignment checks."""
    from pocketlm_amd import native

    payload = np.arange(32, dtype=np.uint16).tobytes()
    path = tmp_path / "packed.bin"
    path.write_bytes(payload)
    mapped = native.map_native_row8_file(path)
    try:
        assert mapped.nbytes == 64
        assert ctypes.string_at(mapped.data_ptr(0, 64), 64) == payload
        assert ctypes.string_at(mapped.data_ptr(10, 6), 6) == payload[10:16]
        for off, n in ((1, 2), (0, 3), (62, 4), (66, 0)):
            with pytest.raises(ValueError):
                mapped.data_ptr(off, n)
    finally:
        mapped.close()
    with pytest.raises(OSError):
        native.map_native_row8_file(tmp_path / "missing.bin")


def _q4_golden_cases(golden):
    g = golden("q4")
    for i in range(int(g["count"])):
        shape = tuple(int(v) for v in g[f"t{i}_shape"])
        t = torch.from_numpy(g[f"t{i}_in"].view(np.int16).copy()).view(torch.float16).reshape(shape)
        yield i, t, g[f"t{i}_packed"], g[f"t{i}_scales"]


def test_product_q4_quantizer_matches_golden(golden):
    """formats.quantize_tensor_to_q4 (the quantizer that builds Q4 artifacts
    and the bench's Q4 weights) gives the golden nibbles and fp16 scales of
    the reference's torch arithmetic (q4_quantize.py:48-71), bit for bit,
    on the 102 tensors of tests/golden/q4.npz (0-d, 1-d, 3-d and odd sizes
    included)."""
    for i, t, want_packed, want_scales in _q4_golden_cases(golden):
        packed, scales, meta = formats.quantize_tensor_to_q4(t)
        assert np.array_equal(packed.numpy(), want_packed), i
        assert np.array_equal(scales.view(torch.int16).numpy().view(np.uint16), want_scales), i
        assert meta["shape"] == list(t.shape) and meta["numel"] == t.numel()


@pytest.mark.gpu
def test_product_q4_quantizer_matches_golden_on_device(golden):
    """The same quantizer run on the GPU (as the bench runs it)."""
    for i, t, want_packed, want_scales in _q4_golden_cases(golden):
        packed, scales, _meta = formats.quantize_tensor_to_q4(t.cuda())
        assert np.array_equal(packed.cpu().numpy(), want_packed), i
        assert np.array_equal(scales.cpu().view(torch.int16).numpy().view(np.uint16), want_scales), i

"""The reference's on-disk weight artifacts streamed into HBM
(pocketlm_file_spans_to_device and the readers of pocketlm_amd.packs): the
device bytes equal the file bytes, and kernels fed from the loaded tensors
give the results of the same tensors placed in memory directly."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from pocketlm_amd import formats, native, packs

pytestmark = pytest.mark.gpu

MB = 1 << 20


def test_file_spans_reach_device_memory_bit_exact(tmp_path):
    """Spans at odd offsets and lengths, smaller and larger than one 8 MiB
    staging buffer, the whole 40 MiB file across all reader threads, an empty
    span; out-of-range spans and missing files are errors."""
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, size=40 * MB + 12345, dtype=np.uint8)
    path = tmp_path / "blob.bin"
    data.tofile(path)
    spans = [(0, 17), (5, 8 * MB), (3 * MB + 1, 9 * MB + 7), (len(data) - 100, 100), (123, 0), (0, len(data))]
    outs = [torch.empty(n, dtype=torch.uint8, device="cuda") for _o, n in spans]
    native.file_spans_to_device(path, [(o, t) for (o, _n), t in zip(spans, outs)])
    for (o, n), t in zip(spans, outs):
        assert np.array_equal(t.cpu().numpy(), data[o:o + n]), (o, n)
    with pytest.raises(RuntimeError, match="code -2"):
        native.file_spans_to_device(path, [(len(data) - 10, torch.empty(11, dtype=torch.uint8, device="cuda"))])
    with pytest.raises(RuntimeError, match="code -5"):
        native.file_spans_to_device(tmp_path / "missing.bin", [(0, torch.empty(4, dtype=torch.uint8, device="cuda"))])


def _experts(n, inter, hid, seed):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for e in range(n):
        for proj, shape in (("gate_proj", (inter, hid)), ("up_proj", (inter, hid)), ("down_proj", (hid, inter))):
            name = f"model.layers.3.mlp.experts.{e}.{proj}.weight"
            out[name] = (torch.randn(shape, generator=g) * 0.02).to(torch.float8_e4m3fn)
            out[name + "_scale_inv"] = torch.rand(((shape[0] + 127) // 128, (shape[1] + 127) // 128), generator=g) * 9e-3 + 1e-3
    return out


def test_fp8_pack_experts_load_to_device_and_feed_the_moe(tmp_path):
    """Three experts written as an FP8 pack that rolls over several files,
    loaded to the device by layer and expert id: the bytes match and the
    weighted MoE over the loaded experts equals the one over the originals."""
    inter, hid = 256, 512
    tensors = _experts(3, inter, hid, 11)
    manifest = packs.write_fp8_pack(tensors, tmp_path / "model" / "artifacts" / "fp8_pack", pack_bytes=400_000)
    assert len(manifest["pack_files"]) >= 2
    reader = packs.FP8PackReader(tmp_path / "model")
    loaded = reader.load_layer_experts(3, [0, 1, 2])
    originals = {}
    for e in range(3):
        parts = []
        for proj in ("gate_proj", "up_proj", "down_proj"):
            w = f"model.layers.3.mlp.experts.{e}.{proj}.weight"
            parts += [tensors[w].view(torch.uint8).cuda(), tensors[w + "_scale_inv"].cuda()]
        originals[e] = tuple(parts)
        for got, want in zip(loaded[e], parts):
            assert got.dtype == want.dtype and got.shape == want.shape and torch.equal(got, want)
    x = torch.randn((1, hid), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    route = torch.tensor([0.5, 0.25, 0.125], device="cuda")
    y_loaded = native.fp8_e4m3_block_mlp_many_weighted_f32([loaded[e] for e in range(3)], x, route)
    y_orig = native.fp8_e4m3_block_mlp_many_weighted_f32([originals[e] for e in range(3)], x, route)
    assert torch.equal(y_loaded, y_orig)
    assert reader.telemetry()["device_bytes_loaded"] == sum(t.numel() * t.element_size() for t in tensors.values())


def _hip_to_host(ptr: int, nbytes: int) -> bytes:
    hip = ctypes.CDLL("libamdhip64.so")
    buf = ctypes.create_string_buffer(nbytes)
    assert hip.hipMemcpy(buf, ctypes.c_void_p(ptr), ctypes.c_size_t(nbytes), 2) == 0  # device to host
    return buf.raw


def test_row8_artifact_loads_to_device_and_feeds_the_gemv(tmp_path):
    g = torch.Generator().manual_seed(4)
    a = (torch.randn((40, 72), generator=g) * 0.1).to(torch.float16)
    b = (torch.randn((24, 72), generator=g) * 0.1).to(torch.bfloat16)
    manifest = packs.build_row8_artifact_from_tensors({"a.weight": a, "b.weight": b}, tmp_path)
    for name, w in (("a.weight", a), ("b.weight", b)):
        packed, entry = packs.load_row8_packed_tensor(tmp_path, name)
        assert packed.device.type == "cuda" and packed.dtype == torch.uint16
        assert torch.equal(packed.cpu(), formats.pack_rows8_tensor(w))
        assert torch.equal(packs.load_row8_unpacked_tensor(tmp_path, name).cpu(), w)
        x = (torch.randn(72, generator=g) * 0.5).to(w.dtype).cuda()
        y = native.packed_gemv_rows8(x, packed, rows=w.shape[0], cols=72)
        y_mem = native.packed_gemv_rows8(x, formats.pack_rows8_tensor(w).cuda(), rows=w.shape[0], cols=72)
        assert torch.equal(y, y_mem)
        # the reference's handle API: the bytes sit in device memory
        handle = native.load_native_row8_tensor(tmp_path / manifest["data_file"], entry["offset"], entry["nbytes"])
        try:
            assert handle.nbytes == entry["nbytes"]
            assert _hip_to_host(handle.ptr, handle.nbytes) == formats.pack_rows8_tensor(w).numpy().tobytes()
        finally:
            handle.close()
    with pytest.raises(OSError):
        native.load_native_row8_tensor(tmp_path / manifest["data_file"], 0, 3)  # odd byte count


def test_q4_artifact_loads_to_device_and_feeds_the_gemv(tmp_path):
    g = torch.Generator().manual_seed(6)
    w = (torch.randn((96, 256), generator=g) * 0.02).to(torch.float16)
    packs.quantize_tensors_to_q4_artifact({"model.layers.0.mlp.up_proj.weight": w}, tmp_path)
    packed, scales, entry = packs.load_q4_tensor(tmp_path, "model.layers.0.mlp.up_proj.weight")
    want_p, want_s, _meta = formats.quantize_tensor_to_q4(w)
    assert packed.device.type == "cuda" and torch.equal(packed.cpu(), want_p) and torch.equal(scales.cpu(), want_s)
    assert entry["shape"] == [96, 256]
    x = (torch.randn(256, generator=g) * 0.5).to(torch.float16).cuda()
    y = native.q4_gemv_f16_f32(packed, scales, x, rows=96, cols=256)
    assert torch.equal(y, native.q4_gemv_f16_f32(want_p.cuda(), want_s.cuda(), x, rows=96, cols=256))

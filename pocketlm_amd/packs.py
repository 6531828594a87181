"""The reference's on-disk weight artifacts, read straight into HBM.

* FP8 pack ("pcketlm-fp8-pack-v1"): tools/pack_fp8.py writes pack_NNNN.bin
  files and pack_manifest.json from a safetensors model directory;
  src/pcketlm/core/runtime/fp8_pack.py:54-241 reads them through mmap.
  FP8PackReader offers that reader's views, slice and span locations and
  layer experts, and load_to_device moves named tensors (with their scale
  companions) into device tensors, one native transfer per pack file.
  pack_model_dir_to_fp8 / write_fp8_pack lay tensors out as the writer does
  (its order, pack rollover and manifest fields) without its resume state.
* row8 artifact ("pcketlm-row8-packed-gemv"): tools/pack_weights_row8.py:83-141
  writes row8_packed.bin and row8_manifest.json; build_row8_packed_artifact
  and load_row8_packed_tensor do the same, the load landing in HBM.
* Q4 shards ("pcketlm-q4", src/pcketlm/core/model_import/q4_quantize.py:92-168):
  .q4.safetensors / .scales.safetensors shards and q4_manifest.json;
  quantize_tensors_to_q4_artifact writes them and load_q4_tensor moves one
  tensor's packed nibbles and fp16 scales into HBM, located through the
  shards' safetensors headers.

The transfers go through pocketlm_file_spans_to_device: reader threads fill
pinned staging buffers while earlier chunks are copied, so page-cache reads
and PCIe transfers overlap (no host tensor is built on the way).
"""

from __future__ import annotations

import json
import mmap
import os
import re
import struct
from dataclasses import dataclass
from datetime import datetime, timezone
from functools import lru_cache
from pathlib import Path
from typing import Callable, Mapping

import torch

from . import formats, native

__all__ = [
    "FP8_PACK_FORMAT", "ROW8_FORMAT", "Q4_FORMAT", "FP8PackReader", "PackedTensorView", "PackedSliceLocation",
    "PackedSpanLocation", "PackedSpanView", "default_fp8_pack_dir", "fp8_pack_enabled", "fp8_pack_available",
    "pack_model_dir_to_fp8", "write_fp8_pack", "build_row8_packed_artifact", "build_row8_artifact_from_tensors",
    "load_row8_packed_tensor", "load_row8_unpacked_tensor", "quantize_tensors_to_q4_artifact", "load_q4_tensor",
    "read_safetensors_header",
]

FP8_PACK_FORMAT = "pcketlm-fp8-pack-v1"        # tools/pack_fp8.py:34
ROW8_FORMAT = "pcketlm-row8-packed-gemv"      # tools/pack_weights_row8.py:13
Q4_FORMAT = "pcketlm-q4"                      # src/pcketlm/core/model_import/q4_plan.py:13
Q4_SCHEME = "per-channel-symmetric-v1"        # q4_plan.py:14
DEFAULT_PACK_BYTES = 16 * 1024 ** 3
SCALE_SUFFIXES = (".scale_inv", "_scale_inv", ".scale", "_scale")

# safetensors dtype names -> torch dtypes of the device tensors (FP8 stays raw bytes)
_DTYPES = {
    "F8_E4M3": torch.uint8, "F8_E4M3FN": torch.uint8, "F8_E5M2": torch.uint8, "U8": torch.uint8, "I8": torch.int8,
    "BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32, "F64": torch.float64,
    "I16": torch.int16, "U16": torch.uint16, "I32": torch.int32, "I64": torch.int64, "BOOL": torch.bool,
}
_NAMES_OF = {torch.float8_e4m3fn: "F8_E4M3", torch.uint8: "F8_E4M3", torch.float32: "F32",
             torch.bfloat16: "BF16", torch.float16: "F16"}
_LAYER_EXPERT = re.compile(r"(?:^|\.)layers\.(\d+)\..*\.experts\.(\d+)\.")
_LAYER = re.compile(r"(?:^|\.)layers\.(\d+)\.")


def _device(device) -> torch.device:
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device(device)


def _empty_on(dtype_name: str, shape, nbytes: int, device: torch.device) -> torch.Tensor:
    dtype = _DTYPES.get(str(dtype_name).upper())
    if dtype is None:
        raise ValueError(f"unsupported tensor dtype {dtype_name}")
    flat = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
    if dtype == torch.uint8:
        return flat.view(*[int(v) for v in shape]) if shape else flat
    return flat.view(dtype).view(*[int(v) for v in shape]) if shape else flat.view(dtype)


def read_safetensors_header(path: Path) -> tuple[dict, int]:
    """(header, data start): the JSON header of a safetensors file and the
    file offset its data_offsets are relative to."""
    with Path(path).open("rb") as handle:
        (size,) = struct.unpack("<Q", handle.read(8))
        header = json.loads(handle.read(size).decode("utf-8"))
    return header, 8 + int(size)


# =========================================================================== FP8 pack

@dataclass(slots=True)
class PackedTensorView:
    """Memory views of one packed tensor and its optional scale companion."""

    name: str
    dtype: str
    shape: list[int]
    fp8_bytes: memoryview
    scale_bytes: memoryview | None = None
    scale_name: str | None = None
    scale_dtype: str | None = None
    scale_shape: list[int] | None = None


@dataclass(frozen=True, slots=True)
class PackedSliceLocation:
    path: Path
    byte_offset: int
    byte_length: int


@dataclass(frozen=True, slots=True)
class PackedSpanLocation:
    path: Path
    byte_offset: int
    byte_length: int
    tensor_slices: dict[str, tuple[int, int]]


@dataclass(slots=True)
class PackedSpanView:
    bytes: memoryview
    tensor_slices: dict[str, tuple[int, int]]


def fp8_pack_enabled() -> bool:
    return os.environ.get("PCKETLM_DISABLE_FP8_PACK", "").strip().lower() not in {"1", "true", "yes", "on"}


@lru_cache(maxsize=64)
def _pack_dir(model_dir: Path) -> Path:
    override = os.environ.get("PCKETLM_FP8_PACK_DIR", "").strip()
    return Path(override).resolve() if override else Path(model_dir).resolve() / "artifacts" / "fp8_pack"


def default_fp8_pack_dir(model_dir: Path) -> Path:
    """fp8_pack.py:289-294: PCKETLM_FP8_PACK_DIR, else <model>/artifacts/fp8_pack."""
    return _pack_dir(Path(model_dir))


def fp8_pack_available(model_dir: Path) -> bool:
    return fp8_pack_enabled() and (default_fp8_pack_dir(model_dir) / "pack_manifest.json").exists()


@dataclass(frozen=True, slots=True)
class _Extent:
    """Where one tensor's bytes sit: pack file number, offset, length."""

    file: int
    offset: int
    length: int

    @property
    def end(self) -> int:
        return self.offset + self.length


@dataclass(frozen=True, slots=True)
class _Record:
    """One manifest entry, parsed once."""

    name: str
    dtype: str
    shape: tuple[int, ...]
    at: _Extent
    scale_name: str | None
    scale_dtype: str | None
    scale_shape: tuple[int, ...] | None
    scale_at: _Extent | None
    expert: int | None
    companion: bool
    order: int

    @classmethod
    def parse(cls, name: str, e: dict) -> "_Record":
        scale_at = None
        if e.get("scale_name") and e.get("scale_byte_length") is not None:
            scale_at = _Extent(int(e["scale_pack_file_index"]), int(e["scale_byte_offset"]),
                               int(e["scale_byte_length"]))
        shape = e.get("scale_shape")
        return cls(name, str(e["dtype"]), tuple(int(v) for v in e.get("shape", [])),
                   _Extent(int(e["pack_file_index"]), int(e["byte_offset"]), int(e["byte_length"])),
                   e.get("scale_name"), e.get("scale_dtype"), None if shape is None else tuple(int(v) for v in shape),
                   scale_at, None if e.get("expert_index") is None else int(e["expert_index"]),
                   e.get("tensor_role") == "scale_companion", int(e.get("pack_order", 0)))


class _PackFiles:
    """The pack files of one pack directory: read-only maps opened on first
    use and kept, plus the numbers of files handed out by path."""

    def __init__(self, pack_dir: Path):
        self.pack_dir = pack_dir
        self.maps: dict[int, tuple[object, mmap.mmap]] = {}
        self.located: set[int] = set()

    def path(self, file: int) -> Path:
        return self.pack_dir / f"pack_{int(file):04d}.bin"

    def view(self, x: _Extent) -> memoryview:
        if x.file not in self.maps:
            handle = self.path(x.file).open("rb")
            self.maps[x.file] = (handle, mmap.mmap(handle.fileno(), 0, access=mmap.ACCESS_READ))
        return memoryview(self.maps[x.file][1])[x.offset:x.end]

    def release(self) -> None:
        """Unmaps every file no live view still exports."""
        for file, (handle, mapped) in list(self.maps.items()):
            try:
                mapped.close()
            except BufferError:
                continue
            handle.close()
            del self.maps[file]


class FP8PackReader:
    """An FP8 pack ("pcketlm-fp8-pack-v1") opened for decode.

    The public calls are those of fp8_pack.py:54-241 (host views, slice and
    span locations, layer experts, telemetry, close), with its error
    messages.  The manifest is parsed once into typed records.  The way into
    HBM is load_to_device: the requested tensors (and scale companions) are
    grouped per pack file and sorted by offset, so each file is read front
    to back by one native transfer that lands every range in its device
    tensor."""

    def __init__(self, model_dir: Path):
        self.model_dir = Path(model_dir).resolve()
        self.pack_dir = default_fp8_pack_dir(self.model_dir)
        self.manifest_path = self.pack_dir / "pack_manifest.json"
        if not self.manifest_path.exists():
            raise FileNotFoundError(f"FP8 pack manifest not found: {self.manifest_path}")
        self.manifest = json.loads(self.manifest_path.read_text(encoding="utf-8"))
        self.tensors: dict[str, dict] = dict(self.manifest.get("tensors") or {})
        self._records = {n: _Record.parse(n, e) for n, e in self.tensors.items()}
        self._files = _PackFiles(self.pack_dir)
        self._reads = 0
        self._returned = 0
        self._device_bytes = 0

    # ----------------------------------------------------------------- into HBM
    def load_to_device(self, names: list[str], device=None, *, with_scales: bool = True) -> dict[str, torch.Tensor]:
        """The named tensors as device tensors of their dtype and shape (FP8
        as uint8 bytes), plus each one's scale companion when with_scales,
        keyed by name."""
        dev = _device(device)
        wanted: dict[str, tuple[str, tuple[int, ...], _Extent]] = {}
        for name in names:
            rec = self._record(name)
            wanted.setdefault(rec.name, (rec.dtype, rec.shape, rec.at))
            if with_scales and rec.scale_at is not None:
                wanted.setdefault(rec.scale_name, (rec.scale_dtype, rec.scale_shape or (), rec.scale_at))
        out = {n: _empty_on(dtype, shape, at.length, dev) for n, (dtype, shape, at) in wanted.items()}
        per_file: dict[int, list[tuple[int, torch.Tensor]]] = {}
        for n, (_dtype, _shape, at) in wanted.items():
            per_file.setdefault(at.file, []).append((at.offset, out[n].view(torch.uint8).reshape(-1)))
        for file in sorted(per_file):
            spans = sorted(per_file[file], key=lambda span: span[0])
            native.file_spans_to_device(self._files.path(file), spans)
            self._device_bytes += sum(t.numel() for _offset, t in spans)
        self._reads += len(per_file)
        return out

    def load_layer_experts(self, layer_idx: int, expert_ids: list[int], device=None) -> dict[int, tuple]:
        """Each expert's (gate, gate_scale_inv, up, up_scale_inv, down,
        down_scale_inv) on the device, as the MoE entry points take them."""
        base = f"model.layers.{int(layer_idx)}.mlp.experts."
        weights = {int(e): [f"{base}{int(e)}.{p}.weight" for p in ("gate_proj", "up_proj", "down_proj")]
                   for e in expert_ids}
        loaded = self.load_to_device([w for ws in weights.values() for w in ws], device)
        experts = {}
        for e, ws in weights.items():
            parts: list[torch.Tensor] = []
            for w in ws:
                scale = self._record(w).scale_name
                if not scale:
                    raise KeyError(f"Tensor {w} has no scale companion in the FP8 pack.")
                parts.extend((loaded[w], loaded[scale]))
            experts[e] = tuple(parts)
        return experts

    # ----------------------------------------------------------------- host views and locations
    def get_tensor(self, name: str) -> PackedTensorView:
        rec = self._record(name)
        raw = self._files.view(rec.at)
        scale = self._files.view(rec.scale_at) if rec.scale_name and rec.scale_at is not None else None
        self._returned_bytes(rec.at.length + (rec.scale_at.length if rec.scale_at is not None else 0))
        return PackedTensorView(name=rec.name, dtype=rec.dtype, shape=list(rec.shape), fp8_bytes=raw,
                                scale_bytes=scale, scale_name=rec.scale_name, scale_dtype=rec.scale_dtype,
                                scale_shape=None if rec.scale_shape is None else list(rec.scale_shape))

    def get_tensor_bytes(self, name: str) -> memoryview:
        return self.get_tensor_slice_bytes(name, 0, self._record(name).at.length)

    def get_tensor_slice_bytes(self, name: str, relative_offset: int, byte_length: int) -> memoryview:
        x = self._sub(name, int(relative_offset), int(byte_length))
        self._returned_bytes(x.length)
        return self._files.view(x)

    def get_tensor_slice_location(self, name: str, relative_offset: int, byte_length: int) -> PackedSliceLocation:
        x = self._sub(name, int(relative_offset), int(byte_length))
        self._files.located.add(x.file)
        self._returned_bytes(x.length)
        return PackedSliceLocation(self._files.path(x.file), x.offset, x.length)

    def get_tensor_span_location(self, names: list[str]) -> PackedSpanLocation:
        x, slices = self._cover(names)
        self._files.located.add(x.file)
        self._returned_bytes(x.length)
        return PackedSpanLocation(self._files.path(x.file), x.offset, x.length, slices)

    def get_tensor_span_bytes(self, names: list[str]) -> PackedSpanView:
        x, slices = self._cover(names)
        self._returned_bytes(x.length)
        return PackedSpanView(bytes=self._files.view(x), tensor_slices=slices)

    def get_layer_experts(self, layer_idx: int, expert_ids: list[int]) -> list[PackedTensorView]:
        """Views of the given experts' weights of one layer (scale companions
        travel inside each view), in pack order."""
        ids = {int(v) for v in expert_ids}
        base = f"model.layers.{int(layer_idx)}.mlp.experts."
        chosen = sorted((r for r in self._records.values()
                         if r.name.startswith(base) and r.expert in ids and not r.companion),
                        key=lambda r: r.order)
        return [self.get_tensor(r.name) for r in chosen]

    # ----------------------------------------------------------------- bookkeeping
    def telemetry(self) -> dict:
        mapped = sum(len(m) for _h, m in self._files.maps.values())
        return {"sequential_reads": self._reads, "scattered_reads": 0, "bytes_returned": self._returned,
                "device_bytes_loaded": self._device_bytes, "pack_files_open": len(self._files.maps),
                "pack_files_accessed": len(self._files.located | set(self._files.maps)),
                "mmap_bytes_mapped": mapped, "mmap_bytes_resident": None if mapped else 0,
                "mmap_residency_measured": False}

    def close(self) -> None:
        """Unmaps every pack file whose views are no longer held."""
        self._files.release()

    def _returned_bytes(self, n: int) -> None:
        self._reads += 1
        self._returned += int(n)

    def _record(self, name: str) -> _Record:
        rec = self._records.get(name)
        if rec is None:
            raise KeyError(f"Tensor {name} is not present in FP8 pack manifest.")
        return rec

    def _sub(self, name: str, offset: int, length: int) -> _Extent:
        """A byte range inside one tensor, checked against its length."""
        at = self._record(name).at
        if offset < 0 or length < 0:
            raise ValueError("Packed tensor slice offset and length must be non-negative.")
        if offset + length > at.length:
            raise ValueError(f"Packed tensor slice exceeds tensor byte length for {name}.")
        return _Extent(at.file, at.offset + offset, length)

    def _cover(self, names: list[str]) -> tuple[_Extent, dict[str, tuple[int, int]]]:
        """The smallest range of one pack file holding every named tensor,
        and each tensor's (offset in it, length)."""
        if not names:
            raise ValueError("Packed tensor span requires at least one tensor name.")
        ats = {str(n): self._record(str(n)).at for n in names}
        if len({x.file for x in ats.values()}) != 1:
            raise ValueError("Packed tensor span crosses pack files.")
        lo = min(x.offset for x in ats.values())
        hi = max(x.end for x in ats.values())
        file = next(iter(ats.values())).file
        return _Extent(file, lo, hi - lo), {n: (x.offset - lo, x.length) for n, x in ats.items()}


def _now() -> str:
    return datetime.now(timezone.utc).isoformat()


def _layer_and_expert(name: str) -> tuple[int | None, int | None]:
    m = _LAYER_EXPERT.search(name)
    if m:
        return int(m.group(1)), int(m.group(2))
    m = _LAYER.search(name)
    return (int(m.group(1)), None) if m else (None, None)


def _base_name(name: str) -> str:
    for suffix in SCALE_SUFFIXES:
        if name.endswith(suffix):
            return name[:-len(suffix)]
    return name


def _order_key(name: str, role: str, layer: int | None, expert: int | None) -> tuple:
    """The writer's tensor order (tools/pack_fp8.py:259-285): by layer, then
    attention / router / routed experts / shared experts / other MLP, expert,
    projection, base name, weight before its scale."""
    low = name.lower()
    if name in {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"} or layer is None:
        group = 0
    elif ".self_attn." in low:
        group = 1
    elif ".mlp.gate." in low:
        group = 2
    elif ".mlp.experts." in low:
        group = 3
    elif ".shared_experts." in low:
        group = 4
    elif ".mlp." in low:
        group = 5
    else:
        group = 6
    projections = ("gate_proj", "up_proj", "down_proj", "q_a_proj", "q_b_proj", "kv_a_proj", "kv_b_proj", "o_proj")
    proj = next((i for i, p in enumerate(projections) if p in low), 0)
    return (-1 if layer is None else layer, group, -1 if expert is None else expert, proj, _base_name(name),
            1 if role == "scale_companion" else 0, name)


def _write_pack(items: list[tuple[str, str, list[int], int, Callable[[], bytes]]], output_dir: Path,
                pack_bytes: int, source: str) -> dict:
    """items: (name, dtype, shape, byte length, read bytes).  Writes the pack
    files and pack_manifest.json the way tools/pack_fp8.py:118-212 does."""
    output_dir = Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=True)
    names = {it[0] for it in items}
    tasks = []
    for name, dtype, shape, length, read in items:
        weight = next((name[:-len(s)] for s in SCALE_SUFFIXES if name.endswith(s) and name[:-len(s)] in names), None)
        scale = None if weight is not None else next((name + s for s in SCALE_SUFFIXES if name + s in names), None)
        layer, expert = _layer_and_expert(name)
        role = "scale_companion" if weight is not None else "weight"
        tasks.append({"name": name, "dtype": dtype, "shape": list(shape), "length": int(length), "read": read,
                      "role": role, "scale": scale, "weight": weight, "layer": layer, "expert": expert})
    tasks.sort(key=lambda t: _order_key(t["name"], t["role"], t["layer"], t["expert"]))
    manifest = {"format": FP8_PACK_FORMAT, "source_model_dir": source, "output_dir": str(output_dir),
                "pack_bytes": int(pack_bytes), "plan": {}, "pack_files": [], "tensors": {},
                "created_at": _now(), "updated_at": _now()}
    index, size, handle = 0, 0, None

    def finish():
        nonlocal handle
        if handle is not None:
            handle.close()
            handle = None
            path = output_dir / f"pack_{index:04d}.bin"
            manifest["pack_files"].append({"index": index, "file_name": path.name,
                                           "byte_length": path.stat().st_size})

    for order, t in enumerate(tasks):
        if size > 0 and size + t["length"] > int(pack_bytes):
            finish()
            index, size = index + 1, 0
        if handle is None:
            handle = (output_dir / f"pack_{index:04d}.bin").open("wb")
        data = t["read"]()
        if len(data) != t["length"]:
            raise OSError(f"{t['name']}: expected {t['length']} bytes, read {len(data)}")
        handle.write(data)
        entry = {"name": t["name"], "dtype": t["dtype"], "shape": t["shape"], "tensor_role": t["role"],
                 "pack_file_index": index, "byte_offset": size, "byte_length": t["length"],
                 "scale_name": t["scale"], "scale_pack_file_index": None, "scale_byte_offset": None,
                 "scale_byte_length": None, "scale_dtype": None, "scale_shape": None, "weight_name": t["weight"],
                 "layer_index": t["layer"], "expert_index": t["expert"], "pack_order": order}
        manifest["tensors"][t["name"]] = entry
        partner = manifest["tensors"].get(t["weight"]) if t["weight"] else None
        if partner is not None:  # a scale after its weight: fill the weight's scale fields
            partner.update(scale_name=t["name"], scale_dtype=t["dtype"], scale_shape=list(t["shape"]),
                           scale_pack_file_index=index, scale_byte_offset=size, scale_byte_length=t["length"])
        scale = manifest["tensors"].get(t["scale"]) if t["scale"] else None
        if scale is not None:  # a weight after its scale
            entry.update(scale_pack_file_index=scale["pack_file_index"], scale_byte_offset=scale["byte_offset"],
                         scale_byte_length=scale["byte_length"], scale_dtype=scale["dtype"],
                         scale_shape=list(scale["shape"]))
        size += t["length"]
    if handle is not None:
        finish()
    manifest["updated_at"] = _now()
    (output_dir / "pack_manifest.json").write_text(json.dumps(manifest, indent=2), encoding="utf-8")
    return manifest


def pack_model_dir_to_fp8(model_dir: Path, output_dir: Path | None = None, *,
                          pack_bytes: int = DEFAULT_PACK_BYTES) -> dict:
    """Pack a safetensors model directory (model.safetensors.index.json and
    its shards) the way tools/pack_fp8.py:62-212 does, without its resume
    state.  Returns the manifest."""
    model_dir = Path(model_dir).resolve()
    output_dir = Path(output_dir) if output_dir is not None else model_dir / "artifacts" / "fp8_pack"
    index = json.loads((model_dir / "model.safetensors.index.json").read_text(encoding="utf-8"))
    headers: dict[str, tuple[dict, int]] = {}
    items = []
    for name, shard in (index.get("weight_map") or {}).items():
        if shard not in headers:
            headers[shard] = read_safetensors_header(model_dir / shard)
        header, base = headers[shard]
        meta = header.get(name)
        if meta is None:
            continue
        start, end = (int(v) for v in meta.get("data_offsets") or [0, 0])

        def read(path=model_dir / shard, off=base + start, n=end - start) -> bytes:
            with path.open("rb") as handle:
                handle.seek(off)
                return handle.read(n)

        items.append((name, str(meta.get("dtype", "")).upper(), [int(v) for v in meta.get("shape", [])], end - start,
                      read))
    return _write_pack(items, output_dir, pack_bytes, str(model_dir))


def write_fp8_pack(tensors: Mapping[str, torch.Tensor], output_dir: Path, *,
                   pack_bytes: int = DEFAULT_PACK_BYTES) -> dict:
    """Pack in-memory tensors (FP8 weights as float8_e4m3fn or uint8 bytes,
    scales fp32, others bf16/fp16) in the same format."""
    items = []
    for name, t in tensors.items():
        t = t.detach().cpu().contiguous()
        if t.dtype not in _NAMES_OF:
            raise TypeError(f"{name}: unsupported dtype {t.dtype}")
        raw = t.view(torch.uint8).reshape(-1) if t.dtype != torch.uint8 else t.reshape(-1)
        items.append((name, _NAMES_OF[t.dtype], list(t.shape), int(raw.numel()),
                      lambda raw=raw: raw.numpy().tobytes()))
    return _write_pack(items, Path(output_dir), pack_bytes, "")


# =========================================================================== row8 artifact

def _row8_manifest(output_dir: Path, source: str) -> dict:
    return {"format": ROW8_FORMAT, "row_block": 8, "source_model_dir": source, "data_file": "row8_packed.bin",
            "tensors": {}, "tensor_count": 0, "total_original_bytes": 0, "total_packed_bytes": 0}


def _row8_write(named: list[tuple[str, str, torch.Tensor]], output_dir: Path, source: str) -> dict:
    output_dir = Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=True)
    manifest = _row8_manifest(output_dir, source)
    offset = 0
    with (output_dir / "row8_packed.bin").open("wb") as out:
        for name, shard, tensor in named:
            if tensor.ndim != 2 or tensor.dtype not in (torch.float16, torch.bfloat16):
                continue
            packed = formats.pack_rows8_tensor(tensor.cpu()).contiguous()
            data = packed.view(torch.uint8).numpy().tobytes()
            out.write(data)
            original = int(tensor.numel() * tensor.element_size())
            manifest["tensors"][name] = {"dtype": "BF16" if tensor.dtype == torch.bfloat16 else "F16",
                                         "shape": [int(v) for v in tensor.shape], "offset": offset,
                                         "nbytes": len(data), "source_shard": shard, "original_nbytes": original}
            manifest["tensor_count"] += 1
            manifest["total_original_bytes"] += original
            manifest["total_packed_bytes"] += len(data)
            offset += len(data)
    total = int(manifest["total_original_bytes"])
    manifest["size_ratio"] = 0.0 if total <= 0 else round(int(manifest["total_packed_bytes"]) / total, 6)
    (output_dir / "row8_manifest.json").write_text(json.dumps(manifest, indent=2), encoding="utf-8")
    return manifest


def build_row8_packed_artifact(model_dir: Path, output_dir: Path, *, include_patterns: list[str] | None = None) -> dict:
    """tools/pack_weights_row8.py:83-121: the 2-D fp16/bf16 tensors of a
    safetensors model directory (names with any include pattern, else every
    *.weight), row8-packed into row8_packed.bin."""
    from safetensors import safe_open

    model_dir = Path(model_dir).resolve()
    weight_map = json.loads((model_dir / "model.safetensors.index.json").read_text(encoding="utf-8"))["weight_map"]
    patterns = list(include_patterns or [])
    if patterns:
        names = [n for n in sorted(weight_map) if any(p in n for p in patterns)]
    else:
        names = sorted(n for n in weight_map if n.endswith(".weight"))
    named = []
    for name in names:
        with safe_open(str(model_dir / weight_map[name]), framework="pt", device="cpu") as shard:
            named.append((name, weight_map[name], shard.get_tensor(name)))
    return _row8_write(named, output_dir, str(model_dir))


def build_row8_artifact_from_tensors(tensors: Mapping[str, torch.Tensor], output_dir: Path) -> dict:
    """The same artifact from tensors in memory."""
    return _row8_write([(n, "", t) for n, t in tensors.items()], output_dir, "")


def load_row8_packed_tensor(artifact_dir: Path, tensor_name: str, device=None) -> tuple[torch.Tensor, dict]:
    """tools/pack_weights_row8.py:124-133, into HBM: the packed uint16
    tensor on the device, and its manifest entry."""
    artifact_dir = Path(artifact_dir)
    manifest = json.loads((artifact_dir / "row8_manifest.json").read_text(encoding="utf-8"))
    entry = manifest["tensors"][tensor_name]
    out = torch.empty(int(entry["nbytes"]) // 2, dtype=torch.uint16, device=_device(device))
    native.file_spans_to_device(artifact_dir / str(manifest["data_file"]), [(int(entry["offset"]), out)])
    return out, entry


def load_row8_unpacked_tensor(artifact_dir: Path, tensor_name: str, device=None) -> torch.Tensor:
    packed, entry = load_row8_packed_tensor(artifact_dir, tensor_name, device)
    dtype = torch.bfloat16 if str(entry["dtype"]).upper() == "BF16" else torch.float16
    return formats.unpack_rows8_tensor(packed, int(entry["shape"][0]), int(entry["shape"][1]), dtype=dtype)


# =========================================================================== Q4 shards

def quantize_tensors_to_q4_artifact(tensors: Mapping[str, torch.Tensor], output_dir: Path,
                                    shard_name: str = "model-00001-of-00001.safetensors") -> dict:
    """q4_quantize.py:92-168 for one shard of in-memory tensors: the packed
    nibbles and fp16 scales of every floating tensor in
    <shard>.q4.safetensors / <shard>.scales.safetensors, and q4_manifest.json."""
    from safetensors.torch import save_file

    output_dir = Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=True)
    q4_shard = shard_name.replace(".safetensors", ".q4.safetensors")
    scale_shard = shard_name.replace(".safetensors", ".scales.safetensors")
    manifest = {"format": Q4_FORMAT, "scheme": Q4_SCHEME, "source_model_dir": "", "tensors": {}, "weight_map": {},
                "scale_map": {}}
    packs, scales = {}, {}
    for name in sorted(tensors):
        t = tensors[name].detach().cpu()
        if not t.dtype.is_floating_point:
            continue
        packed, sc, meta = formats.quantize_tensor_to_q4(t)
        packs[name], scales[name] = packed.contiguous(), sc.contiguous()
        original = int(t.numel() * t.element_size())
        manifest["tensors"][name] = {**meta, "q4_shard": q4_shard, "scale_shard": scale_shard,
                                     "original_nbytes": original,
                                     "q4_nbytes": int(packed.numel() * packed.element_size() + sc.numel() * sc.element_size())}
        manifest["weight_map"][name] = q4_shard
        manifest["scale_map"][name] = scale_shard
    if packs:
        meta = {"format": Q4_FORMAT, "scheme": Q4_SCHEME}
        save_file(packs, str(output_dir / q4_shard), metadata=meta)
        save_file(scales, str(output_dir / scale_shard), metadata=meta)
    orig = sum(int(e["original_nbytes"]) for e in manifest["tensors"].values())
    q4 = sum(int(e["q4_nbytes"]) for e in manifest["tensors"].values())
    manifest.update(total_original_bytes=orig, total_q4_bytes=q4, compression_ratio=0.0 if orig <= 0 else round(q4 / orig, 6))
    (output_dir / "q4_manifest.json").write_text(json.dumps(manifest, indent=2), encoding="utf-8")
    return manifest


def load_q4_tensor(artifact_dir: Path, tensor_name: str, device=None) -> tuple[torch.Tensor, torch.Tensor, dict]:
    """One tensor of a Q4 artifact in HBM: (packed uint8 [ceil(n/2)], scales
    fp16 [channels], manifest entry), read from the shards' byte ranges."""
    artifact_dir = Path(artifact_dir)
    manifest = json.loads((artifact_dir / "q4_manifest.json").read_text(encoding="utf-8"))
    entry = manifest["tensors"][tensor_name]
    dev = _device(device)
    loaded = []
    for shard in (entry["q4_shard"], entry["scale_shard"]):
        header, base = read_safetensors_header(artifact_dir / shard)
        meta = header[tensor_name]
        start, end = (int(v) for v in meta["data_offsets"])
        t = _empty_on(meta["dtype"], meta["shape"], end - start, dev)
        native.file_spans_to_device(artifact_dir / shard, [(base + start, t.view(torch.uint8).reshape(-1))])
        loaded.append(t)
    return loaded[0], loaded[1], entry

"""Drop-in for the hot-path functions of ``pcketlm.native`` on an MI355X.

Same function names, argument meaning, validation messages and exception
types as the reference's ctypes wrappers (src/pcketlm/native/__init__.py,
cited per function), backed by libpocketlm_hip.so.  Differences, all on
purpose:

* Tensors stay on the GPU.  Inputs already on a CUDA device are used in
  place (no ``.cpu()``); results are returned on that device.  CPU inputs are
  copied to the current CUDA device and the result is copied back, so a
  caller written for the CPU reference keeps working (at PCIe cost).
* Calls run on torch's current stream and return without synchronising.
* ``PCKETLM_DISABLE_NATIVE_*`` kill switches make the ``native_*_available``
  predicates return False and the wrappers raise
  ``RuntimeError("... unavailable: disabled")``, as the reference wrappers
  do when their DLL is not loaded.  There is no CPU or torch fallback in this
  package: a missing library raises.
* FP8 weights may be given as ``torch.uint8`` or ``torch.float8_e4m3fn``;
  both are read as raw e4m3 bytes.
* bf16 activations go to the ``*_bf16x_f32`` twin of an FP8 entry point
  where one exists, instead of being widened to fp32 first as the reference
  wrappers do: the twin widens them exactly on the device, so the results
  are the same, and reads half the activation bytes.
"""

from __future__ import annotations

import ctypes
import os
from contextlib import contextmanager
from dataclasses import dataclass
from pathlib import Path
from typing import NamedTuple

import torch

from . import _lib

_TRUE = {"1", "true", "yes", "on"}


def _flag(name: str) -> bool:
    return os.environ.get(name, "").strip().lower() in _TRUE


# --------------------------------------------------------------------------- availability
# Kill switches: src/pcketlm/native/__init__.py:64-138.

def _lib_or_none():
    try:
        return _lib.load()
    except OSError:
        return None


def _available(kill_switch: str) -> bool:
    if _flag(kill_switch):
        return False
    lib = _lib_or_none()
    return bool(lib is not None and torch.cuda.is_available() and lib.pocketlm_device_available() == 1)


def native_fp8_dequant_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_FP8_DEQUANT")


def native_fp8_linear_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_FP8_LINEAR")


native_fp8_dual_linear_available = native_fp8_linear_available
native_fp8_mlp_available = native_fp8_linear_available
native_fp8_mlp_many_available = native_fp8_linear_available
native_fp8_mlp_many_weighted_available = native_fp8_linear_available
native_fp8_mlp_many_row_weighted_available = native_fp8_linear_available
native_fp8_mlp_many_pair_weighted_available = native_fp8_linear_available


def native_fp8_mlp_avx512_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_FP8_AVX512")


native_fp8_mlp_many_weighted_avx512_available = native_fp8_mlp_avx512_available


def native_q4_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_Q4")


def native_fp16_packed_gemv_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_PACKED_GEMV")


def native_ds_moe_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_DS_MOE")


def native_ds_router_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_DS_ROUTER")


def _require(kill_switch: str, what: str):
    if _flag(kill_switch):
        raise RuntimeError(f"{what} is unavailable: disabled")
    try:
        lib = _lib.load()
    except OSError as exc:
        raise RuntimeError(f"{what} is unavailable: {exc}") from exc
    if not torch.cuda.is_available():
        raise RuntimeError(f"{what} is unavailable: no HIP device")
    return lib


# --------------------------------------------------------------------------- plumbing

def _target_device(*tensors: torch.Tensor) -> torch.device:
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.device.type == "cuda":
            return t.device
    return torch.device("cuda", torch.cuda.current_device())


def _on(t: torch.Tensor, device: torch.device, dtype: torch.dtype | None = None) -> torch.Tensor:
    t = t.detach()
    if dtype is not None and t.dtype != dtype:
        if dtype == torch.uint8 and t.dtype == torch.float8_e4m3fn:
            t = t.view(torch.uint8)
        else:
            t = t.to(dtype)
    return t.to(device, non_blocking=False).contiguous()


def _fp8_bytes(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    if t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    if t.dtype != torch.uint8:
        raise TypeError("FP8 weights must be torch.uint8 raw e4m3 bytes or torch.float8_e4m3fn")
    return t.detach().to(device).contiguous()


def _p(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else int(t.data_ptr()))


@contextmanager
def _launch(lib, device: torch.device):
    with torch.cuda.device(device):
        lib.pocketlm_set_stream(ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
        yield


def _check(name: str, code: int) -> None:
    if code != 0:
        detail = _lib.last_error()
        raise RuntimeError(f"{name} failed with code {code}" + (f" ({detail})" if detail else ""))


def _home(result: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """Return the result where the caller's main input lives."""
    if like.device.type == "cuda":
        return result
    return result.to(like.device)


# --------------------------------------------------------------------------- FP8 dequant

def _fp8_dequant(fp8_weight, scale_inv, out_dtype: torch.dtype, symbol: str, what: str) -> torch.Tensor:
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_DEQUANT", what)
    if fp8_weight.ndim != 2:
        raise ValueError("fp8_weight must have shape [rows, cols]")
    if scale_inv.ndim != 2:
        raise ValueError("scale_inv must have shape [scale_rows, scale_cols]")
    dev = _target_device(fp8_weight, scale_inv)
    w = _fp8_bytes(fp8_weight, dev)
    s = _on(scale_inv, dev, torch.float32)
    rows, cols = int(w.shape[0]), int(w.shape[1])
    if tuple(s.shape) != ((rows + 127) // 128, (cols + 127) // 128):
        raise ValueError("scale_inv shape does not match FP8 128x128 block layout")
    out = torch.empty((rows, cols), dtype=out_dtype, device=dev)
    if rows and cols:
        with _launch(lib, dev):
            code = getattr(lib, symbol)(_p(w), _p(s), _p(out), rows, cols, (cols + 127) // 128)
        _check(symbol, code)
    return _home(out, fp8_weight)


def fp8_e4m3_dequant_to_fp16(fp8_weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3378-3407 -> fp8_dequant.cpp:119-164."""
    return _fp8_dequant(fp8_weight, scale_inv, torch.float16, "fp8_e4m3_dequant_to_fp16", "Native FP8 dequant")


def fp8_e4m3_dequant_to_bf16(fp8_weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3410-3439 -> fp8_dequant.cpp:166-204."""
    return _fp8_dequant(fp8_weight, scale_inv, torch.bfloat16, "fp8_e4m3_dequant_to_bf16", "Native FP8 BF16 dequant")


def fp8_e4m3_dequant_to_f32(fp8_weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """The fp32 branch of dequantize_fp8_block_scaled (fp8_source.py:852-858)."""
    return _fp8_dequant(fp8_weight, scale_inv, torch.float32, "fp8_e4m3_dequant_to_f32", "Native FP8 F32 dequant")


def dequantize_fp8_block_scaled(
    fp8_bytes: torch.Tensor,
    scale_inv: torch.Tensor,
    *,
    block_size: int = 128,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """src/pcketlm/core/runtime/fp8_source.py:812-858 on the device.

    fp16 / bf16 / fp32 come straight from the dequant kernels; any other
    dtype is the fp32 result cast with torch, as the reference's torch branch
    does.  Only the 128x128 block layout exists on this path.
    """
    if fp8_bytes.dtype not in (torch.uint8, torch.float8_e4m3fn):
        raise TypeError("fp8_bytes must be a uint8 tensor containing raw E4M3 bytes.")
    if fp8_bytes.ndim != 2:
        raise ValueError("FP8 block dequant currently supports 2D weight tensors only.")
    if scale_inv.ndim != 2:
        raise ValueError("scale_inv must be a 2D block-scale tensor.")
    if int(block_size) != 128:
        raise ValueError("only block_size=128 is supported by the device dequant kernels")
    rows, cols = int(fp8_bytes.shape[0]), int(fp8_bytes.shape[1])
    expected = [(rows + 127) // 128, (cols + 127) // 128]
    if [int(scale_inv.shape[0]), int(scale_inv.shape[1])] != expected:
        raise ValueError(
            "scale_inv shape "
            f"{list(scale_inv.shape)} does not match FP8 weight shape {list(fp8_bytes.shape)} "
            f"with block_size={block_size}; expected {expected}."
        )
    if dtype == torch.float16:
        return fp8_e4m3_dequant_to_fp16(fp8_bytes, scale_inv)
    if dtype == torch.bfloat16:
        return fp8_e4m3_dequant_to_bf16(fp8_bytes, scale_inv)
    out = fp8_e4m3_dequant_to_f32(fp8_bytes, scale_inv)
    return out if dtype == torch.float32 else out.to(dtype).contiguous()


# --------------------------------------------------------------------------- FP8 GEMV family

def _hidden_f32(hidden: torch.Tensor, dev: torch.device) -> torch.Tensor:
    return _on(hidden, dev).reshape(-1, int(hidden.shape[-1])).to(torch.float32).contiguous()


def _hidden_in(hidden: torch.Tensor, dev: torch.device) -> tuple[torch.Tensor, bool]:
    """Activations for an entry point with a bf16 twin: bf16 ones stay bf16
    (the twin widens them on the device, exactly, so the results are those of
    the reference wrapper's cast to fp32), others become fp32."""
    if hidden.dtype == torch.bfloat16:
        return _on(hidden, dev).reshape(-1, int(hidden.shape[-1])).contiguous(), True
    return _hidden_f32(hidden, dev), False


def _twin(name: str, bf16: bool) -> str:
    """The bf16-activation twin of an fp32 entry point name."""
    return name[:-len("_f32")] + "_bf16x_f32" if bf16 else name


def fp8_e4m3_block_linear_f32(fp8_weight: torch.Tensor, scale_inv: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3442-3476 -> fp8_linear.cpp:50-117."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 linear")
    if fp8_weight.ndim != 2:
        raise ValueError("fp8_weight must have shape [out_rows, in_cols]")
    if scale_inv.ndim != 2:
        raise ValueError("scale_inv must have shape [scale_rows, scale_cols]")
    dev = _target_device(fp8_weight, scale_inv, hidden)
    x, bf16 = _hidden_in(hidden, dev)
    w = _fp8_bytes(fp8_weight, dev)
    s = _on(scale_inv, dev, torch.float32)
    out_rows, in_cols = int(w.shape[0]), int(w.shape[1])
    if int(x.shape[1]) != in_cols:
        raise ValueError("hidden input size does not match FP8 weight columns")
    if int(s.shape[0]) != (out_rows + 127) // 128 or int(s.shape[1]) != (in_cols + 127) // 128:
        raise ValueError("scale_inv shape does not match FP8 128x128 block layout")
    out = torch.empty((int(x.shape[0]), out_rows), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_linear_f32", bf16))(_p(w), _p(s), _p(x), _p(out), int(x.shape[0]),
                                                                    out_rows, in_cols, (in_cols + 127) // 128)
    _check("fp8_e4m3_block_linear_f32", code)
    return _home(out, hidden)


class Fp8Tiles8(NamedTuple):
    """A row-major [rows, cols] FP8 e4m3 weight packed in 8-row tiles
    (fp8_e4m3_pack_tiles8): 1 KB tiles of 8 rows x 128 columns, zero-padded.
    No counterpart in the reference."""
    tiles: torch.Tensor  # uint8, fp8_e4m3_tiles8_bytes(rows, cols) bytes
    rows: int
    cols: int


def pack_fp8_tiles8(fp8_weight: torch.Tensor) -> Fp8Tiles8:
    """Packs a row-major FP8 weight into 8-row tiles on its device (no
    counterpart in the reference)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 linear")
    if fp8_weight.ndim != 2:
        raise ValueError("fp8_weight must have shape [out_rows, in_cols]")
    dev = _target_device(fp8_weight)
    w = _fp8_bytes(fp8_weight, dev)
    rows, cols = int(w.shape[0]), int(w.shape[1])
    nbytes = int(lib.fp8_e4m3_tiles8_bytes(rows, cols))
    if nbytes < 0:
        _check("fp8_e4m3_tiles8_bytes", nbytes)
    tiles = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    with _launch(lib, dev):
        code = lib.fp8_e4m3_pack_tiles8(_p(w), _p(tiles), rows, cols)
    _check("fp8_e4m3_pack_tiles8", code)
    return Fp8Tiles8(tiles, rows, cols)


def fp8_e4m3_block_linear_tiles8_f32(packed: Fp8Tiles8, scale_inv: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
    """fp8_e4m3_block_linear_f32 on a weight packed by pack_fp8_tiles8: the
    same values, bit for bit (no counterpart in the reference)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 linear")
    if scale_inv.ndim != 2:
        raise ValueError("scale_inv must have shape [scale_rows, scale_cols]")
    dev = _target_device(packed.tiles, scale_inv, hidden)
    x, bf16 = _hidden_in(hidden, dev)
    s = _on(scale_inv, dev, torch.float32)
    out_rows, in_cols = packed.rows, packed.cols
    if int(x.shape[1]) != in_cols:
        raise ValueError("hidden input size does not match FP8 weight columns")
    if int(s.shape[0]) != (out_rows + 127) // 128 or int(s.shape[1]) != (in_cols + 127) // 128:
        raise ValueError("scale_inv shape does not match FP8 128x128 block layout")
    out = torch.empty((int(x.shape[0]), out_rows), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_linear_tiles8_f32", bf16))(
            _p(packed.tiles), _p(s), _p(x), _p(out), int(x.shape[0]), out_rows, in_cols, (in_cols + 127) // 128)
    _check("fp8_e4m3_block_linear_tiles8_f32", code)
    return _home(out, hidden)


def fp8_e4m3_block_linear_many_f32(weights, hidden: torch.Tensor) -> list[torch.Tensor]:
    """Several fp8_e4m3_block_linear_f32 calls on one hidden (for example
    the q_a and kv_a projections, src/pcketlm/core/runtime/fp8_source.py:
    1943-1945 and 1967-1969) in one launch.  weights: (fp8_weight,
    scale_inv) pairs with the same in_cols.  Returns one fp32 [M, rows_i]
    output per weight, with the single calls' values."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 linear")
    if not 1 <= len(weights) <= 8:
        raise ValueError("1 to 8 weights per call")
    dev = _target_device(hidden, *[w for w, _s in weights])
    x, bf16 = _hidden_in(hidden, dev)
    in_cols = int(x.shape[1])
    ws, ss = [], []
    for fp8_weight, scale_inv in weights:
        if fp8_weight.ndim != 2:
            raise ValueError("fp8_weight must have shape [out_rows, in_cols]")
        w, sc = _fp8_bytes(fp8_weight, dev), _on(scale_inv, dev, torch.float32)
        if int(w.shape[1]) != in_cols:
            raise ValueError("hidden input size does not match FP8 weight columns")
        if tuple(sc.shape) != ((int(w.shape[0]) + 127) // 128, (in_cols + 127) // 128):
            raise ValueError("scale_inv shape does not match FP8 128x128 block layout")
        ws.append(w)
        ss.append(sc)
    batch = int(x.shape[0])
    outs = [torch.empty((batch, int(w.shape[0])), dtype=torch.float32, device=dev) for w in ws]
    n = len(ws)
    wp = (ctypes.c_uint64 * n)(*[int(w.data_ptr()) for w in ws])
    sp = (ctypes.c_uint64 * n)(*[int(t.data_ptr()) for t in ss])
    op = (ctypes.c_uint64 * n)(*[int(o.data_ptr()) for o in outs])
    rp = (ctypes.c_int64 * n)(*[int(w.shape[0]) for w in ws])
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_linear_many_f32", bf16))(
            ctypes.cast(wp, ctypes.c_void_p), ctypes.cast(sp, ctypes.c_void_p), _p(x), ctypes.cast(op, ctypes.c_void_p),
            ctypes.cast(rp, ctypes.c_void_p), n, batch, in_cols, (in_cols + 127) // 128)
    _check("fp8_e4m3_block_linear_many_f32", code)
    return [_home(o, hidden) for o in outs]


def fp8_e4m3_block_dual_linear_f32(
    fp8_weight_a: torch.Tensor,
    scale_inv_a: torch.Tensor,
    fp8_weight_b: torch.Tensor,
    scale_inv_b: torch.Tensor,
    hidden: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """src/pcketlm/native/__init__.py:3479-3530 -> fp8_linear.cpp:119-210."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 dual linear")
    if fp8_weight_a.ndim != 2 or fp8_weight_b.ndim != 2:
        raise ValueError("fp8 weights must have shape [out_rows, in_cols]")
    dev = _target_device(fp8_weight_a, fp8_weight_b, hidden)
    wa, wb = _fp8_bytes(fp8_weight_a, dev), _fp8_bytes(fp8_weight_b, dev)
    if tuple(wa.shape) != tuple(wb.shape):
        raise ValueError("dual FP8 weights must have matching shapes")
    sa, sb = _on(scale_inv_a, dev, torch.float32), _on(scale_inv_b, dev, torch.float32)
    if tuple(sa.shape) != tuple(sb.shape):
        raise ValueError("dual FP8 scales must have matching shapes")
    x, bf16 = _hidden_in(hidden, dev)
    out_rows, in_cols = int(wa.shape[0]), int(wa.shape[1])
    if int(x.shape[1]) != in_cols:
        raise ValueError("hidden input size does not match FP8 weight columns")
    if int(sa.shape[0]) != (out_rows + 127) // 128 or int(sa.shape[1]) != (in_cols + 127) // 128:
        raise ValueError("scale_inv shape does not match FP8 128x128 block layout")
    out_a = torch.empty((int(x.shape[0]), out_rows), dtype=torch.float32, device=dev)
    out_b = torch.empty_like(out_a)
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_dual_linear_f32", bf16))(
            _p(wa), _p(sa), _p(wb), _p(sb), _p(x), _p(out_a), _p(out_b), int(x.shape[0]), out_rows, in_cols,
            (in_cols + 127) // 128)
    _check("fp8_e4m3_block_dual_linear_f32", code)
    return _home(out_a, hidden), _home(out_b, hidden)


def _mlp_common(gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight, down_scale_inv, hidden, dev):
    if gate_weight.ndim != 2 or up_weight.ndim != 2 or down_weight.ndim != 2:
        raise ValueError("FP8 MLP weights must be 2D")
    g, u, d = _fp8_bytes(gate_weight, dev), _fp8_bytes(up_weight, dev), _fp8_bytes(down_weight, dev)
    if tuple(g.shape) != tuple(u.shape):
        raise ValueError("FP8 MLP gate and up weights must have matching shapes")
    inter, hid = int(g.shape[0]), int(g.shape[1])
    if tuple(d.shape) != (hid, inter):
        raise ValueError("FP8 MLP down weight must have shape [hidden, intermediate]")
    gs, us, ds = (_on(t, dev, torch.float32) for t in (gate_scale_inv, up_scale_inv, down_scale_inv))
    if tuple(gs.shape) != tuple(us.shape):
        raise ValueError("FP8 MLP gate and up scales must have matching shapes")
    egs = ((inter + 127) // 128, (hid + 127) // 128)
    eds = ((hid + 127) // 128, (inter + 127) // 128)
    if tuple(gs.shape) != egs:
        raise ValueError("FP8 MLP gate scale shape does not match 128x128 block layout")
    if tuple(ds.shape) != eds:
        raise ValueError("FP8 MLP down scale shape does not match 128x128 block layout")
    x, bf16 = _hidden_in(hidden, dev)
    if int(x.shape[1]) != hid:
        raise ValueError("hidden input size does not match FP8 MLP input size")
    return g, gs, u, us, d, ds, x, bf16, inter, hid, egs[1], eds[1]


def _run_mlp(symbol: str, kill: str, what: str, gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight,
             down_scale_inv, hidden) -> torch.Tensor:
    lib = _require(kill, what)
    dev = _target_device(gate_weight, up_weight, down_weight, hidden)
    g, gs, u, us, d, ds, x, bf16, inter, hid, gsc, dsc = _mlp_common(
        gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight, down_scale_inv, hidden, dev)
    out = torch.empty((int(x.shape[0]), hid), dtype=torch.float32, device=dev)
    entry = "fp8_e4m3_block_mlp_bf16x_f32" if bf16 else symbol  # one kernel behind both MLP names
    with _launch(lib, dev):
        code = getattr(lib, entry)(_p(g), _p(gs), _p(u), _p(us), _p(d), _p(ds), _p(x), _p(out), int(x.shape[0]),
                                   inter, hid, gsc, dsc)
    _check(symbol, code)
    return _home(out, hidden)


def fp8_e4m3_block_mlp_f32(gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight, down_scale_inv,
                           hidden) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3533-3590 -> fp8_linear.cpp:212-362."""
    return _run_mlp("fp8_e4m3_block_mlp_f32", "PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 MLP", gate_weight,
                    gate_scale_inv, up_weight, up_scale_inv, down_weight, down_scale_inv, hidden)


def fp8_e4m3_block_mlp_avx512_f32(gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight,
                                  down_scale_inv, hidden) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3593-3650 (same device kernel as the scalar name)."""
    return _run_mlp("fp8_e4m3_block_mlp_avx512_f32", "PCKETLM_DISABLE_NATIVE_FP8_AVX512", "Native FP8 AVX-512 MLP",
                    gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight, down_scale_inv, hidden)


class _Experts:
    """Validated expert weights on one device plus the six host address tables."""

    def __init__(self, items, hidden, dev: torch.device, bf16_ok: bool = False, check_hidden: bool = True):
        if not items:
            raise ValueError("items must not be empty")
        first = _fp8_bytes(items[0][0], dev)
        self.inter, self.hid = int(first.shape[0]), int(first.shape[1])
        prepared = []
        for gate, gate_scale, up, up_scale, down, down_scale in items:
            g, u, d = _fp8_bytes(gate, dev), _fp8_bytes(up, dev), _fp8_bytes(down, dev)
            gs, us, ds = (_on(t, dev, torch.float32) for t in (gate_scale, up_scale, down_scale))
            if tuple(g.shape) != (self.inter, self.hid):
                raise ValueError("all gate weights must have matching shape")
            if tuple(u.shape) != (self.inter, self.hid):
                raise ValueError("all up weights must have matching shape")
            if tuple(d.shape) != (self.hid, self.inter):
                raise ValueError("all down weights must have matching shape")
            prepared.append((g, gs, u, us, d, ds))
        egs = ((self.inter + 127) // 128, (self.hid + 127) // 128)
        eds = ((self.hid + 127) // 128, (self.inter + 127) // 128)
        for g, gs, u, us, d, ds in prepared:
            if tuple(gs.shape) != egs or tuple(us.shape) != egs:
                raise ValueError("gate/up scale shapes do not match 128x128 block layout")
            if tuple(ds.shape) != eds:
                raise ValueError("down scale shape does not match 128x128 block layout")
        self.gsc, self.dsc = egs[1], eds[1]
        self.prepared = prepared
        self.count = len(prepared)
        self.tables = [(ctypes.c_uint64 * self.count)(*[int(p[i].data_ptr()) for p in prepared]) for i in range(6)]
        if not check_hidden:  # weights only (the device expert table)
            return
        # bf16_ok: the caller has a bf16 twin to send bf16 activations to
        self.x, self.bf16 = _hidden_in(hidden, dev) if bf16_ok else (_hidden_f32(hidden, dev), False)
        if int(self.x.shape[1]) != self.hid:
            raise ValueError("hidden input size does not match FP8 MLP input size")

    def table_args(self):
        return [ctypes.cast(t, ctypes.c_void_p) for t in self.tables]


def fp8_e4m3_block_mlp_many_f32(items, hidden: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3653-3719 -> fp8_linear.cpp:364-473; out [E, M, H]."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 many-MLP")
    dev = _target_device(hidden, *(items[0] if items else ()))
    ex = _Experts(items, hidden, dev)
    out = torch.empty((ex.count, int(ex.x.shape[0]), ex.hid), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = lib.fp8_e4m3_block_mlp_many_f32(*ex.table_args(), _p(ex.x), _p(out), ex.count, int(ex.x.shape[0]),
                                               ex.inter, ex.hid, ex.gsc, ex.dsc)
    _check("fp8_e4m3_block_mlp_many_f32", code)
    return _home(out, hidden)


def _weighted(symbol: str, kill: str, what: str, items, hidden, route_weights, *, per_row: bool) -> torch.Tensor:
    lib = _require(kill, what)
    dev = _target_device(hidden, *(items[0] if items else ()))
    ex = _Experts(items, hidden, dev, bf16_ok=symbol in ("fp8_e4m3_block_mlp_many_row_weighted_f32",
                                                         "fp8_e4m3_block_mlp_many_weighted_f32"))
    batch = int(ex.x.shape[0])
    if per_row:
        route = _on(route_weights, dev, torch.float32)
        if tuple(route.shape) != (ex.count, batch):
            raise ValueError("route_weights must have shape [expert_count, batch]")
    else:
        route = _on(route_weights, dev, torch.float32).reshape(-1)
        if int(route.numel()) != ex.count:
            raise ValueError("route_weights length must match item count")
    out = torch.empty((batch, ex.hid), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = getattr(lib, _twin(symbol, ex.bf16))(*ex.table_args(), _p(ex.x), _p(route), _p(out), ex.count,
                                                    batch, ex.inter, ex.hid, ex.gsc, ex.dsc)
    _check(symbol, code)
    return _home(out, hidden)


def fp8_e4m3_block_mlp_many_weighted_f32(items, hidden, route_weights) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3722-3793 -> fp8_linear.cpp:475-589."""
    return _weighted("fp8_e4m3_block_mlp_many_weighted_f32", "PCKETLM_DISABLE_NATIVE_FP8_LINEAR",
                     "Native FP8 weighted many-MLP", items, hidden, route_weights, per_row=False)


def fp8_e4m3_block_mlp_many_weighted_shared_f32(items, shared, hidden, route_weights):
    """The routed experts (as fp8_e4m3_block_mlp_many_weighted_f32) and the
    shared expert (as fp8_e4m3_block_mlp_f32) in two launches: the pair of
    calls of src/pcketlm/core/runtime/fp8_source.py:1643-1646 and 1849-1859.
    The shared expert has the routed experts' shapes.  Returns (routed,
    shared_out), both fp32 [M, H] with the separate calls' values."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 weighted many-MLP with shared expert")
    dev = _target_device(hidden, *(items[0] if items else ()))
    if not items:
        raise ValueError("items must not be empty")
    ex = _Experts(list(items) + [shared], hidden, dev, bf16_ok=True)
    count = ex.count - 1
    route = _on(route_weights, dev, torch.float32).reshape(-1)
    if int(route.numel()) != count:
        raise ValueError("route_weights length must match item count")
    batch = int(ex.x.shape[0])
    out = torch.empty((batch, ex.hid), dtype=torch.float32, device=dev)
    out_shared = torch.empty((batch, ex.hid), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_mlp_many_weighted_shared_f32", ex.bf16))(
            *ex.table_args(), _p(ex.x), _p(route), _p(out), _p(out_shared), count, batch, ex.inter, ex.hid, ex.gsc,
            ex.dsc)
    _check("fp8_e4m3_block_mlp_many_weighted_shared_f32", code)
    return _home(out, hidden), _home(out_shared, hidden)


class FP8ExpertTable:
    """Every routed expert of one MoE layer resident on one device, and the
    device table [6, num_experts] int64 of their addresses (rows: gate, gate
    scale_inv, up, up scale_inv, down, down scale_inv) that the device-routed
    MoE reads.  ``experts`` maps an expert id to its six tensors (or is a
    sequence indexed by id); ids without weights get null addresses and
    contribute nothing when the router picks them.  The table keeps the
    tensors alive."""

    def __init__(self, experts, num_experts: int, device: torch.device | str | None = None):
        num_experts = int(num_experts)
        if num_experts <= 0:
            raise ValueError("num_experts must be positive")
        items = experts.items() if hasattr(experts, "items") else enumerate(experts)
        chosen = {int(k): v for k, v in items if v is not None}
        if not chosen:
            raise ValueError("experts must not be empty")
        if any(k < 0 or k >= num_experts for k in chosen):
            raise ValueError("expert ids must lie in [0, num_experts)")
        dev = torch.device(device) if device is not None else _target_device(*next(iter(chosen.values())))
        if dev.type != "cuda":
            raise ValueError("the expert table lives on a HIP device")
        ids = sorted(chosen)
        ex = _Experts([chosen[k] for k in ids], torch.zeros((1, 1)), dev, check_hidden=False)
        addr = torch.zeros((6, num_experts), dtype=torch.int64)
        for col, prepared in zip(ids, ex.prepared):
            for role in range(6):
                addr[role, col] = int(prepared[role].data_ptr())
        self.device = dev
        self.num_experts = num_experts
        self.inter, self.hid, self.gsc, self.dsc = ex.inter, ex.hid, ex.gsc, ex.dsc
        self.table = addr.to(dev)
        self._keep = ex.prepared


@dataclass
class DeviceRoutedMoE:
    """Outputs of fp8_e4m3_block_moe_device_routed_f32, all on the device:
    routed (fp32 [M, H], the route-weighted sum), shared (fp32 [M, H] or
    None), output (bf16 [M, H]: routed and shared rounded and added as the
    reference does in bf16, or None) and rejected (int32 [1]: router choices
    out of range, which are left out, plus those of an expert with misaligned
    weights, which contributes nothing)."""

    routed: torch.Tensor
    shared: torch.Tensor | None
    output: torch.Tensor | None
    rejected: torch.Tensor


def fp8_e4m3_block_moe_device_routed_f32(table: FP8ExpertTable, hidden: torch.Tensor, route_indices: torch.Tensor,
                                         route_weights: torch.Tensor, shared=None, *,
                                         bf16_output: bool = True) -> DeviceRoutedMoE:
    """The routed MoE with the experts chosen on the device: the router's
    indices [M, k] and weights [M, k] stay in HBM, and no host read-back sits
    between the router and the experts (run_fp8_moe,
    src/pcketlm/core/runtime/fp8_source.py:1600-1862, reads the indices on
    the host).  Same values as the host-routed calls given the chosen
    experts in ascending order: the weighted kernel at M == 1, the
    row-weighted one above (fp8_linear.cpp:475-589, 591-831), and the
    shared expert as fp8_e4m3_block_mlp_f32.  M <= 8 and M * k <= 64."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 device-routed MoE")
    dev = table.device
    x, bf16 = _hidden_in(hidden, dev)
    if int(x.shape[1]) != table.hid:
        raise ValueError("hidden input size does not match FP8 MLP input size")
    batch = int(x.shape[0])
    idx = _on(route_indices, dev, torch.int64).reshape(batch, -1)
    w = _on(route_weights, dev, torch.float32).reshape(batch, -1)
    if tuple(w.shape) != tuple(idx.shape):
        raise ValueError("route_weights must have the shape of route_indices")
    top_k = int(idx.shape[1])
    shared_arr = None
    keep = []
    if shared is not None:
        sh = _Experts([shared], torch.zeros((1, 1)), dev, check_hidden=False)
        if (sh.inter, sh.hid) != (table.inter, table.hid):
            raise ValueError("the shared expert must have the routed experts' shapes")
        keep.append(sh)
        shared_arr = (ctypes.c_uint64 * 6)(*[int(t.data_ptr()) for t in sh.prepared[0]])
    out = torch.empty((batch, table.hid), dtype=torch.float32, device=dev)
    out_shared = torch.empty_like(out) if shared is not None else None
    out_bf16 = torch.empty((batch, table.hid), dtype=torch.bfloat16, device=dev) if bf16_output else None
    rejected = torch.zeros((1,), dtype=torch.int32, device=dev)
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_moe_device_routed_f32", bf16))(
            _p(table.table), table.num_experts, _p(idx), _p(w), top_k,
            None if shared_arr is None else ctypes.cast(shared_arr, ctypes.c_void_p), _p(x), _p(out),
            _p(out_shared), _p(out_bf16), _p(rejected), batch, table.inter, table.hid, table.gsc, table.dsc)
    _check("fp8_e4m3_block_moe_device_routed_f32", code)
    return DeviceRoutedMoE(out, out_shared, out_bf16, rejected)


@dataclass
class LogitsRoutedMoE(DeviceRoutedMoE):
    """DeviceRoutedMoE plus the router's choices: indices int64 [M, k] and
    weights fp32 [M, k] (bf16 values), as route_deepseek returns them."""
    indices: torch.Tensor | None = None
    weights: torch.Tensor | None = None


def fp8_e4m3_block_moe_from_logits(table: FP8ExpertTable, hidden: torch.Tensor, router_logits: torch.Tensor,
                                   shared=None, *, top_k: int = 8, n_groups: int = 8, topk_groups: int = 4,
                                   scoring_func: str = "sigmoid", route_scale: float = 2.5,
                                   bias: torch.Tensor | None = None) -> LogitsRoutedMoE:
    """One DeepSeek-V3 MoE layer from the router's logits [M, E]: the routing
    of route_deepseek (run_fp8_router, src/pcketlm/core/runtime/
    fp8_source.py:1500-1566) and the plan in one launch, then the gate/up and
    down launches of fp8_e4m3_block_moe_device_routed_f32 (run_fp8_moe,
    1569-1884).  The same values as route_deepseek followed by that call.
    bf16 activations only (the decode path's)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 logits-routed MoE")
    if scoring_func not in ("sigmoid", "softmax"):
        raise ValueError("scoring_func must be 'sigmoid' or 'softmax'")
    dev = table.device
    x = _on(hidden, dev, torch.bfloat16)
    x = x.reshape(-1, int(x.shape[-1])).contiguous()
    if int(x.shape[1]) != table.hid:
        raise ValueError("hidden input size does not match FP8 MLP input size")
    batch = int(x.shape[0])
    lg = _on(router_logits, dev, torch.float32).reshape(batch, -1).contiguous()
    if int(lg.shape[1]) != table.num_experts:
        raise ValueError("router logits must have one column per expert of the table")
    b = None if bias is None else _on(bias, dev, torch.float32).reshape(-1).contiguous()
    k = int(top_k)
    shared_arr = None
    keep = []
    if shared is not None:
        sh = _Experts([shared], torch.zeros((1, 1)), dev, check_hidden=False)
        if (sh.inter, sh.hid) != (table.inter, table.hid):
            raise ValueError("the shared expert must have the routed experts' shapes")
        keep.append(sh)
        shared_arr = (ctypes.c_uint64 * 6)(*[int(t.data_ptr()) for t in sh.prepared[0]])
    out = torch.empty((batch, table.hid), dtype=torch.float32, device=dev)
    out_shared = torch.empty_like(out) if shared is not None else None
    out_bf16 = torch.empty((batch, table.hid), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((batch, k), dtype=torch.int64, device=dev)
    w = torch.empty((batch, k), dtype=torch.float32, device=dev)
    rejected = torch.zeros((1,), dtype=torch.int32, device=dev)
    with _launch(lib, dev):
        code = lib.fp8_e4m3_block_moe_from_logits_bf16x_f32(
            _p(lg), _p(b), int(n_groups), int(topk_groups), 0 if scoring_func == "sigmoid" else 1, float(route_scale),
            _p(table.table), table.num_experts, k, None if shared_arr is None else ctypes.cast(shared_arr, ctypes.c_void_p),
            _p(x), _p(out), _p(out_shared), _p(out_bf16), _p(idx), _p(w), _p(rejected), batch, table.inter, table.hid,
            table.gsc, table.dsc)
    _check("fp8_e4m3_block_moe_from_logits_bf16x_f32", code)
    return LogitsRoutedMoE(out, out_shared, out_bf16, rejected, idx, w)


def fp8_e4m3_block_mlp_many_weighted_avx512_f32(items, hidden, route_weights) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3951-4022 (same device kernel as the scalar name)."""
    return _weighted("fp8_e4m3_block_mlp_many_weighted_avx512_f32", "PCKETLM_DISABLE_NATIVE_FP8_AVX512",
                     "Native FP8 AVX-512 weighted many-MLP", items, hidden, route_weights, per_row=False)


def fp8_e4m3_block_mlp_many_row_weighted_f32(items, hidden, route_weights) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3796-3867 -> fp8_linear.cpp:591-831; route [E, M]."""
    return _weighted("fp8_e4m3_block_mlp_many_row_weighted_f32", "PCKETLM_DISABLE_NATIVE_FP8_LINEAR",
                     "Native FP8 row-weighted many-MLP", items, hidden, route_weights, per_row=True)


def fp8_e4m3_block_mlp_many_pair_weighted_f32(items, hidden, pair_item_indices, pair_row_indices,
                                              pair_weights) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:3870-3948 -> fp8_linear.cpp:833-980."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 pair-weighted many-MLP")
    dev = _target_device(hidden, *(items[0] if items else ()))
    ex = _Experts(items, hidden, dev, bf16_ok=True)
    pi = _on(pair_item_indices, dev, torch.int64).reshape(-1)
    pr = _on(pair_row_indices, dev, torch.int64).reshape(-1)
    pw = _on(pair_weights, dev, torch.float32).reshape(-1)
    if int(pi.numel()) != int(pr.numel()) or int(pi.numel()) != int(pw.numel()):
        raise ValueError("pair index and weight tensors must have matching length")
    batch = int(ex.x.shape[0])
    out = torch.empty((batch, ex.hid), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_mlp_many_pair_weighted_f32", ex.bf16))(
            *ex.table_args(), _p(ex.x), _p(pi), _p(pr), _p(pw), _p(out), ex.count, int(pi.numel()), batch, ex.inter,
            ex.hid, ex.gsc, ex.dsc)
    _check("fp8_e4m3_block_mlp_many_pair_weighted_f32", code)
    return _home(out, hidden)


def fp8_e4m3_block_mlp_many_pair_weighted_nosync(items, hidden, pair_item_indices, pair_row_indices,
                                                pair_weights) -> tuple[torch.Tensor, torch.Tensor]:
    """fp8_e4m3_block_mlp_many_pair_weighted_f32 without the host read-back
    of the pair indices (no stream synchronisation; capturable in a HIP
    graph).  Returns (out fp32 [M, H], bad_pairs int32 [1] on the device):
    pairs with an index out of range are left out and counted instead of
    raising."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "Native FP8 pair-weighted many-MLP")
    dev = _target_device(hidden, *(items[0] if items else ()))
    ex = _Experts(items, hidden, dev, bf16_ok=True)
    pi = _on(pair_item_indices, dev, torch.int64).reshape(-1)
    pr = _on(pair_row_indices, dev, torch.int64).reshape(-1)
    pw = _on(pair_weights, dev, torch.float32).reshape(-1)
    if int(pi.numel()) != int(pr.numel()) or int(pi.numel()) != int(pw.numel()):
        raise ValueError("pair index and weight tensors must have matching length")
    batch = int(ex.x.shape[0])
    out = torch.empty((batch, ex.hid), dtype=torch.float32, device=dev)
    bad = torch.empty((1,), dtype=torch.int32, device=dev)
    with _launch(lib, dev):
        code = getattr(lib, _twin("fp8_e4m3_block_mlp_many_pair_weighted_nosync_f32", ex.bf16))(
            *ex.table_args(), _p(ex.x), _p(pi), _p(pr), _p(pw), _p(out), _p(bad), ex.count, int(pi.numel()), batch,
            ex.inter, ex.hid, ex.gsc, ex.dsc)
    _check("fp8_e4m3_block_mlp_many_pair_weighted_nosync_f32", code)
    return _home(out, hidden), bad


# --------------------------------------------------------------------------- Q4

def q4_dequant_to_fp16(packed: torch.Tensor, scales: torch.Tensor, num_channels: int, channel_size: int) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:4025-4045 -> q4_dequant.cpp:171-208; flat fp16 out."""
    lib = _require("PCKETLM_DISABLE_NATIVE_Q4", "Native Q4 dequant")
    dev = _target_device(packed, scales)
    p = _on(packed, dev, torch.uint8)
    s = _on(scales, dev, torch.float16)
    count = int(num_channels) * int(channel_size)
    if int(p.numel()) < (count + 1) // 2 or int(s.numel()) < int(num_channels):
        raise ValueError("packed / scales are smaller than num_channels * channel_size requires")
    out = torch.empty((count,), dtype=torch.float16, device=dev)
    if count:
        with _launch(lib, dev):
            lib.q4_dequant_to_fp16(_p(p), _p(s), _p(out), int(num_channels), int(channel_size))
        err = _lib.last_error()
        if err:
            raise RuntimeError(f"q4_dequant_to_fp16 failed ({err})")
    return _home(out, packed)


def q4_dequant_many_to_fp16(items) -> list[torch.Tensor]:
    """src/pcketlm/native/__init__.py:4048-4089 -> q4_dequant.cpp:210-286."""
    lib = _require("PCKETLM_DISABLE_NATIVE_Q4", "Native Q4 batch dequant")
    if not items:
        return []
    dev = _target_device(*(t for item in items for t in item[:2]))
    keep, outs = [], []
    n = len(items)
    pp, sp, op = (ctypes.c_void_p * n)(), (ctypes.c_void_p * n)(), (ctypes.c_void_p * n)()
    ch, cs = (ctypes.c_longlong * n)(), (ctypes.c_longlong * n)()
    for i, (packed, scales, num_channels, channel_size) in enumerate(items):
        p = _on(packed, dev, torch.uint8)
        s = _on(scales, dev, torch.float16)
        count = int(num_channels) * int(channel_size)
        if int(p.numel()) < (count + 1) // 2 or int(s.numel()) < int(num_channels):
            raise ValueError("packed / scales are smaller than num_channels * channel_size requires")
        out = torch.empty((count,), dtype=torch.float16, device=dev)
        keep += [p, s]
        outs.append(out)
        pp[i], sp[i], op[i] = p.data_ptr(), s.data_ptr(), out.data_ptr() if count else 0
        ch[i], cs[i] = int(num_channels), int(channel_size)
    with _launch(lib, dev):
        code = lib.q4_dequant_many_to_fp16(ctypes.cast(pp, ctypes.c_void_p), ctypes.cast(sp, ctypes.c_void_p),
                                           ctypes.cast(op, ctypes.c_void_p), ctypes.cast(ch, ctypes.c_void_p),
                                           ctypes.cast(cs, ctypes.c_void_p), n)
    if code != 0:
        raise RuntimeError(f"Native Q4 batch dequant failed with code {code}")
    like = items[0][0]
    return [_home(o, like) for o in outs]


def q4_gemv_f16_f32(packed: torch.Tensor, scales: torch.Tensor, hidden: torch.Tensor, *, rows: int, cols: int) -> torch.Tensor:
    """One Q4 matrix [rows, cols] times an fp16 vector: the row dot of
    q4_moe_selected_forward_u16 (q4_dequant.cpp:314-355) on its own."""
    lib = _require("PCKETLM_DISABLE_NATIVE_Q4", "Native Q4 GEMV")
    dev = _target_device(packed, hidden)
    p = _on(packed, dev, torch.uint8)
    s = _on(scales, dev, torch.float16)
    h = _on(hidden, dev, torch.float16).reshape(-1)
    if int(h.numel()) != int(cols):
        raise ValueError("hidden size mismatch")
    if int(p.numel()) < (int(rows) * int(cols) + 1) // 2 or int(s.numel()) < int(rows):
        raise ValueError("packed / scales are smaller than rows * cols requires")
    out = torch.empty((int(rows),), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = lib.q4_gemv_f16_f32(_p(p), _p(s), _p(h), _p(out), int(rows), int(cols))
    _check("q4_gemv_f16_f32", code)
    return _home(out, hidden)


def q4_moe_selected_forward_u16(hidden: torch.Tensor, experts, route_weights: torch.Tensor, *, hidden_size: int,
                                intermediate_size: int) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:4092-4155 -> q4_dequant.cpp:357-476; fp16 [H] out."""
    lib = _require("PCKETLM_DISABLE_NATIVE_Q4", "Native Q4 MoE selected forward")
    if not experts:
        raise ValueError("experts must not be empty")
    dev = _target_device(hidden, *experts[0])
    h = _on(hidden, dev, torch.float16).reshape(-1)
    if h.numel() != int(hidden_size):
        raise ValueError("hidden size mismatch")
    route = _on(route_weights, dev, torch.float32).reshape(-1)
    if route.numel() != len(experts):
        raise ValueError("route weight count must match selected experts")
    n = len(experts)
    arrays = [(ctypes.c_void_p * n)() for _ in range(6)]
    keep = [h, route]
    H, I = int(hidden_size), int(intermediate_size)
    need = [(I * H + 1) // 2, I, (I * H + 1) // 2, I, (H * I + 1) // 2, H]
    for e, tensors in enumerate(experts):
        for slot, t in enumerate(tensors):
            dt = torch.uint8 if slot % 2 == 0 else torch.float16
            d = _on(t, dev, dt)
            if int(d.numel()) < need[slot]:
                raise ValueError("expert tensor is smaller than hidden_size / intermediate_size require")
            keep.append(d)
            arrays[slot][e] = d.data_ptr()
    out = torch.empty((H,), dtype=torch.float16, device=dev)
    with _launch(lib, dev):
        code = lib.q4_moe_selected_forward_u16(_p(h), *[ctypes.cast(a, ctypes.c_void_p) for a in arrays], _p(route),
                                               _p(out), H, I, n)
    if code != 0:
        raise RuntimeError(f"Native Q4 MoE selected forward failed with code {code}")
    return _home(out, hidden)


# --------------------------------------------------------------------------- row8


class _Row8PackCache:
    """Packed row8 weights kept resident in HBM between calls, keyed by the
    caller's cache key (the reference's cached_pack_weight_rows8,
    src/pcketlm/native/__init__.py:2108-2193: same switches, budget and
    statistics).  The budget, PCKETLM_PACKED_GEMV_CACHE_MB, counts device
    bytes and is read on every call; when a new pack does not fit, the
    entries used longest ago go first.  A pack larger than the whole budget
    is returned without being kept."""

    COUNTERS = ("hits", "misses", "stores", "evictions")

    def __init__(self) -> None:
        self._entries: dict[str, tuple[torch.Tensor, int, int]] = {}  # key -> (pack, bytes, last use)
        self._clock = 0
        self._bytes = 0
        self.counts = dict.fromkeys(self.COUNTERS, 0)

    @staticmethod
    def budget() -> int:
        text = os.environ.get("PCKETLM_PACKED_GEMV_CACHE_MB", "").strip()
        try:
            return max(0, int(text)) << 20 if text else 0
        except ValueError:
            return 0

    def clear(self) -> None:
        self._entries = {}
        self._bytes = 0
        self.counts = dict.fromkeys(self.COUNTERS, 0)

    def stats(self) -> dict[str, int | float]:
        return {**self.counts, "resident_count": len(self._entries), "resident_bytes": self._bytes,
                "resident_mb": round(self._bytes / (1 << 20), 4), "budget_bytes": self.budget()}

    def get(self, key: str, make) -> torch.Tensor:
        self._clock += 1
        limit = 0 if _flag("PCKETLM_DISABLE_PACKED_GEMV_CACHE") else self.budget()
        found = self._entries.get(key) if limit > 0 else None
        if found is not None:
            self._entries[key] = (found[0], found[1], self._clock)
            self.counts["hits"] += 1
            return found[0]
        self.counts["misses"] += 1
        pack = make()
        if limit <= 0:
            return pack
        size = pack.numel() * pack.element_size()
        if size > limit:
            return pack
        while self._entries and self._bytes + size > limit:
            oldest = min(self._entries, key=lambda k: self._entries[k][2])
            self._bytes -= self._entries.pop(oldest)[1]
            self.counts["evictions"] += 1
        self._entries[key] = (pack, size, self._clock)
        self._bytes += size
        self.counts["stores"] += 1
        return pack


_ROW8_PACKS = _Row8PackCache()


def _u16_storage_dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return 0
    if dtype == torch.bfloat16:
        return 1
    raise TypeError("native KV kernels require torch.float16 or torch.bfloat16 tensors")


def reset_packed_gemv_cache() -> None:
    """Drops every resident pack and zeroes the counters."""
    _ROW8_PACKS.clear()


def packed_gemv_cache_stats() -> dict[str, int | float]:
    """hits, misses, stores, evictions, resident_count / _bytes / _mb, budget_bytes."""
    return _ROW8_PACKS.stats()


def pack_weight_rows8(weight: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:2141-2163 -> fp16_packed_gemv.cpp:52-77 (device pack)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_PACKED_GEMV", "Native packed GEMV")
    if weight.dtype not in {torch.float16, torch.bfloat16}:
        raise TypeError("pack_weight_rows8 requires torch.float16 or torch.bfloat16 weight")
    if weight.ndim != 2:
        raise ValueError("weight must have shape [rows, cols]")
    dev = _target_device(weight)
    w = _on(weight, dev)
    rows, cols = int(w.shape[0]), int(w.shape[1])
    packed = torch.empty((((rows + 7) // 8) * cols * 8,), dtype=torch.uint16, device=dev)
    if packed.numel():
        with _launch(lib, dev):
            code = lib.native_pack_u16_rows8(_p(w), _p(packed), rows, cols)
        _check("native_pack_u16_rows8", code)
    return _home(packed, weight)


def cached_pack_weight_rows8(cache_key: str, weight: torch.Tensor) -> torch.Tensor:
    """pack_weight_rows8 through the HBM-resident pack cache (the reference's
    LRU bounded by PCKETLM_PACKED_GEMV_CACHE_MB, src/pcketlm/native/__init__.py:2166-2193)."""
    return _ROW8_PACKS.get(str(cache_key), lambda: pack_weight_rows8(weight))


def packed_gemv_rows8(hidden: torch.Tensor, packed_weight: torch.Tensor, *, rows: int, cols: int) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:2196-2223 -> fp16_packed_gemv.cpp:79-116."""
    lib = _require("PCKETLM_DISABLE_NATIVE_PACKED_GEMV", "Native packed GEMV")
    if hidden.dtype not in {torch.float16, torch.bfloat16}:
        raise TypeError("packed_gemv_rows8 requires torch.float16 or torch.bfloat16 hidden")
    if packed_weight.dtype != torch.uint16:
        raise TypeError("packed_weight must be a torch.uint16 tensor from pack_weight_rows8")
    dev = _target_device(hidden, packed_weight)
    h = _on(hidden, dev).reshape(-1)
    if h.numel() != int(cols):
        raise ValueError("hidden length does not match packed weight column count")
    pw = _on(packed_weight, dev)
    if pw.numel() != ((int(rows) + 7) // 8) * int(cols) * 8:
        raise ValueError("packed weight length does not match rows/cols")
    out = torch.empty((int(rows),), dtype=torch.float32, device=dev)
    if int(rows):
        with _launch(lib, dev):
            code = lib.native_packed_gemv_rows8(_p(h), _p(pw), _p(out), int(rows), int(cols),
                                                _u16_storage_dtype_code(h.dtype))
        _check("native_packed_gemv_rows8", code)
    return _home(out, hidden)


def packed_gemv_rows8_many(hidden: torch.Tensor, packed_weights, rows, *, cols: int, biases=None) -> list[torch.Tensor]:
    """Several row8 GEMVs sharing one hidden vector in one launch (the q/k/v and
    gate/up fusions of fp16_kv_cache.cpp:239-298), with optional biases."""
    lib = _require("PCKETLM_DISABLE_NATIVE_PACKED_GEMV", "Native packed GEMV")
    if hidden.dtype not in {torch.float16, torch.bfloat16}:
        raise TypeError("packed_gemv_rows8 requires torch.float16 or torch.bfloat16 hidden")
    n = len(packed_weights)
    if n == 0 or n != len(rows) or n > 8:
        raise ValueError("packed_weights and rows must have the same length (1..8)")
    dev = _target_device(hidden, *packed_weights)
    h = _on(hidden, dev).reshape(-1)
    if h.numel() != int(cols):
        raise ValueError("hidden length does not match packed weight column count")
    keep, outs = [], []
    pp, bp, op = (ctypes.c_void_p * n)(), (ctypes.c_void_p * n)(), (ctypes.c_void_p * n)()
    rr = (ctypes.c_longlong * n)()
    for i, (pwt, r) in enumerate(zip(packed_weights, rows)):
        if pwt.dtype != torch.uint16:
            raise TypeError("packed_weight must be a torch.uint16 tensor from pack_weight_rows8")
        pw = _on(pwt, dev)
        if pw.numel() != ((int(r) + 7) // 8) * int(cols) * 8:
            raise ValueError("packed weight length does not match rows/cols")
        out = torch.empty((int(r),), dtype=torch.float32, device=dev)
        keep.append(pw)
        outs.append(out)
        pp[i], op[i], rr[i] = pw.data_ptr(), out.data_ptr(), int(r)
        if biases is not None and biases[i] is not None:
            b = _on(biases[i], dev, h.dtype).reshape(-1)
            if b.numel() != int(r):
                raise ValueError("bias length must match rows")
            keep.append(b)
            bp[i] = b.data_ptr()
    with _launch(lib, dev):
        code = lib.native_packed_gemv_rows8_many(_p(h), ctypes.cast(pp, ctypes.c_void_p),
                                                 ctypes.cast(bp, ctypes.c_void_p), ctypes.cast(op, ctypes.c_void_p),
                                                 ctypes.cast(rr, ctypes.c_void_p), n, int(cols),
                                                 _u16_storage_dtype_code(h.dtype))
    _check("native_packed_gemv_rows8_many", code)
    return [_home(o, hidden) for o in outs]


def packed_gemv_rows8_f32_hidden(hidden: torch.Tensor, packed_weight: torch.Tensor, *, rows: int, cols: int,
                                 weight_dtype: torch.dtype) -> torch.Tensor:
    """fp32-activation row8 GEMV of the dense decode's o and down projections
    (packed_rows8_gemv_float_hidden, src/pcketlm/native/fp16_kv_cache.cpp:146-174):
    y = W x with an fp32 x, one fma chain per row, no bias.  weight_dtype is
    the storage type of the packed weight (torch.float16 or torch.bfloat16)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_PACKED_GEMV", "Native packed GEMV")
    if hidden.dtype != torch.float32:
        raise TypeError("packed_gemv_rows8_f32_hidden requires torch.float32 hidden")
    if weight_dtype not in {torch.float16, torch.bfloat16}:
        raise TypeError("weight_dtype must be torch.float16 or torch.bfloat16")
    if packed_weight.dtype != torch.uint16:
        raise TypeError("packed_weight must be a torch.uint16 tensor from pack_weight_rows8")
    dev = _target_device(hidden, packed_weight)
    h = _on(hidden, dev).reshape(-1)
    if h.numel() != int(cols):
        raise ValueError("hidden length does not match packed weight column count")
    pw = _on(packed_weight, dev)
    if pw.numel() != ((int(rows) + 7) // 8) * int(cols) * 8:
        raise ValueError("packed weight length does not match rows/cols")
    out = torch.empty((int(rows),), dtype=torch.float32, device=dev)
    if int(rows):
        with _launch(lib, dev):
            code = lib.native_packed_gemv_rows8_f32_hidden(_p(h), _p(pw), _p(out), int(rows), int(cols),
                                                           _u16_storage_dtype_code(weight_dtype))
        _check("native_packed_gemv_rows8_f32_hidden", code)
    return _home(out, hidden)


# --------------------------------------------------------------------------- DeepSeek session / MoE

class DeepSeekNativeSession:
    """src/pcketlm/native/__init__.py:1411-1519: C-side session with call counters."""

    def __init__(self, *, num_layers: int, hidden_dim: int, num_experts: int, top_k: int,
                 fp8_pack_callback: object | None = None, kv_session_handle: int | None = None):
        lib = _require("PCKETLM_DISABLE_DS_MONOLITHIC", "DeepSeek native session")
        self._lib = lib
        self._callback_keepalive: list[object] = []
        self._tensor_keepalive: list[object] = []
        pack_ptr = 0 if fp8_pack_callback is None else int(ctypes.cast(fp8_pack_callback, ctypes.c_void_p).value or 0)
        kv_ptr = 0 if kv_session_handle is None else int(kv_session_handle)
        handle = lib.ds_session_create(int(num_layers), int(hidden_dim), int(num_experts), int(top_k),
                                       ctypes.c_void_p(pack_ptr), ctypes.c_void_p(kv_ptr))
        if not handle:
            raise RuntimeError("ds_session_create returned a null handle")
        self._handle = ctypes.c_void_p(handle)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            self._lib.ds_session_destroy(self._handle)
            self._handle = None
            self._callback_keepalive.clear()
            self._tensor_keepalive.clear()

    def __enter__(self) -> "DeepSeekNativeSession":
        return self

    def __exit__(self, *_exc: object) -> None:
        self.close()

    @staticmethod
    def tensor_callback(fn):
        return _lib.DS_TENSOR_CALLBACK(fn)

    def register_layer(self, *, layer_idx: int, layer_kind: int, weight_role: int, fp8_callback,
                       scale_callback) -> None:
        cb = _lib.DS_TENSOR_CALLBACK
        fp8_cb = fp8_callback if isinstance(fp8_callback, cb) else cb(fp8_callback)
        scale_cb = scale_callback if isinstance(scale_callback, cb) else cb(scale_callback)
        self._callback_keepalive.extend([fp8_cb, scale_cb])
        code = self._lib.ds_session_register_layer(self._handle, int(layer_idx), int(layer_kind), int(weight_role),
                                                   fp8_cb, scale_cb)
        if code != 0:
            raise RuntimeError(f"ds_session_register_layer failed with code {code}")

    def keep_tensor_alive(self, tensor: object) -> None:
        self._tensor_keepalive.append(tensor)

    def monolithic_call_count(self) -> int:
        return int(self._lib.ds_monolithic_call_counter(self._handle))

    def callback_invocation_count(self) -> int:
        return int(self._lib.ds_callback_invocation_count(self._handle))

    def expert_invocation_count(self) -> int:
        return int(self._lib.ds_expert_invocation_count(self._handle))

    def attention_invocation_count(self) -> int:
        return int(self._lib.ds_attention_invocation_count(self._handle))

    def fused_attention_invocation_count(self) -> int:
        return int(self._lib.ds_fused_attention_invocation_count(self._handle))

    def layers_executed_count(self) -> int:
        return int(self._lib.ds_layers_executed_count(self._handle))

    def registered_layer_count(self) -> int:
        return int(self._lib.ds_registered_layer_count(self._handle))

    def registered_fp8_nbytes(self, index: int) -> int:
        return int(self._lib.ds_registered_fp8_nbytes(self._handle, int(index)))

    def registered_scale_nbytes(self, index: int) -> int:
        return int(self._lib.ds_registered_scale_nbytes(self._handle, int(index)))


def ds_moe_layer_forward(session: DeepSeekNativeSession, expert_outputs: torch.Tensor,
                         route_weights: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:1300-1328 -> ds_forward.cpp:337-367."""
    if not native_ds_moe_available():
        raise RuntimeError("Native DeepSeek MoE combine is unavailable: disabled")
    dev = _target_device(expert_outputs, route_weights)
    outs = _on(expert_outputs, dev, torch.float32)
    if outs.ndim == 2:
        outs = outs.unsqueeze(1)
    if outs.ndim != 3:
        raise ValueError("expert_outputs must be [selected, batch, hidden]")
    w = _on(route_weights, dev, torch.float32).reshape(-1)
    if int(w.numel()) != int(outs.shape[0]):
        raise ValueError("route weight count must match selected expert count")
    out = torch.empty((int(outs.shape[1]), int(outs.shape[2])), dtype=torch.float32, device=dev)
    with _launch(session._lib, dev):
        code = session._lib.ds_moe_layer_forward_f32(session._handle, _p(outs), _p(w), int(outs.shape[0]),
                                                     int(outs.shape[1]), int(outs.shape[2]), _p(out))
    _check("ds_moe_layer_forward_f32", code)
    return _home(out, expert_outputs)


def ds_moe_layer_forward_fp8(session: DeepSeekNativeSession, items, hidden: torch.Tensor,
                             route_weights: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:1331-1400 -> ds_forward.cpp:784-877."""
    if not native_ds_moe_available():
        raise RuntimeError("Native DeepSeek MoE is unavailable: disabled")
    dev = _target_device(hidden, *(items[0] if items else ()))
    ex = _Experts(items, hidden, dev)
    route = _on(route_weights, dev, torch.float32).reshape(-1)
    if int(route.numel()) != ex.count:
        raise ValueError("route weight count must match selected experts")
    batch = int(ex.x.shape[0])
    out = torch.empty((batch, ex.hid), dtype=torch.float32, device=dev)
    with _launch(session._lib, dev):
        code = session._lib.ds_moe_layer_forward_fp8_f32(session._handle, *ex.table_args(), _p(ex.x), _p(route),
                                                         ex.count, batch, ex.inter, ex.hid, ex.gsc, ex.dsc, _p(out))
    _check("ds_moe_layer_forward_fp8_f32", code)
    return _home(out, hidden)


def ds_router_topk(hidden: torch.Tensor, router_weights: torch.Tensor, *, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """src/pcketlm/native/__init__.py:765-801 -> ds_forward.cpp:879-955 (softmax top-k)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_DS_ROUTER", "Native DeepSeek router")
    dtype_code = _u16_storage_dtype_code(router_weights.dtype)
    dev = _target_device(hidden, router_weights)
    r = _on(router_weights, dev)
    h = _on(hidden, dev, r.dtype).reshape(-1)
    if r.ndim != 2 or int(r.shape[1]) != int(h.numel()):
        raise ValueError("router weights must be [num_experts, hidden_dim] matching hidden")
    ids = torch.empty((int(k),), dtype=torch.int64, device=dev)
    weights = torch.empty((int(k),), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = lib.ds_router_topk_u16(_p(h), _p(r), int(r.shape[1]), int(r.shape[0]), int(k), dtype_code, _p(ids),
                                      _p(weights))
    _check("ds_router_topk_u16", code)
    return _home(ids, hidden), _home(weights, hidden)


def ds_router_topk_nosync(hidden: torch.Tensor, router_weights: torch.Tensor, *,
                          k: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """ds_router_topk without waiting on the stream: (ids, weights, status),
    status int32 [1] on the device (0, or 3 / 4 where ds_router_topk would
    raise for a degenerate softmax sum)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_DS_ROUTER", "Native DeepSeek router")
    dtype_code = _u16_storage_dtype_code(router_weights.dtype)
    dev = _target_device(hidden, router_weights)
    r = _on(router_weights, dev)
    h = _on(hidden, dev, r.dtype).reshape(-1)
    if r.ndim != 2 or int(r.shape[1]) != int(h.numel()):
        raise ValueError("router weights must be [num_experts, hidden_dim] matching hidden")
    ids = torch.empty((int(k),), dtype=torch.int64, device=dev)
    weights = torch.empty((int(k),), dtype=torch.float32, device=dev)
    status = torch.empty((1,), dtype=torch.int32, device=dev)
    with _launch(lib, dev):
        code = lib.ds_router_topk_u16_nosync(_p(h), _p(r), int(r.shape[1]), int(r.shape[0]), int(k), dtype_code,
                                             _p(ids), _p(weights), _p(status))
    _check("ds_router_topk_u16_nosync", code)
    return ids, weights, status


def route_deepseek(logits: torch.Tensor, *, top_k: int = 8, n_groups: int = 8, topk_groups: int = 4,
                   scoring_func: str = "sigmoid", route_scale: float = 2.5,
                   bias: torch.Tensor | None = None,
                   weights_dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    """DeepSeek-V3 routing (src/pcketlm/core/runtime/fp8_source.py:1527-1547 with
    _mask_deepseek_route_groups 5125-5140) from router logits [M, E].

    Returns (indices int64 [M, top_k], weights [M, top_k]): bfloat16 as the
    reference returns them, or with weights_dtype=torch.float32 the same
    values as fp32 (what the MoE entry points take, without a conversion
    launch either way).
    """
    if weights_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("weights_dtype must be torch.bfloat16 or torch.float32")
    lib = _require("PCKETLM_DISABLE_NATIVE_DS_ROUTER", "Native DeepSeek router")
    if scoring_func not in ("sigmoid", "softmax"):
        raise ValueError("scoring_func must be 'sigmoid' or 'softmax'")
    dev = _target_device(logits)
    lg = _on(logits, dev, torch.float32)
    lg = lg.reshape(-1, int(lg.shape[-1]))
    m, e = int(lg.shape[0]), int(lg.shape[1])
    k = max(1, min(int(top_k), e))
    b = None if bias is None else _on(bias, dev, torch.float32).reshape(-1)
    idx = torch.empty((m, k), dtype=torch.int64, device=dev)
    w = torch.empty((m, k), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = lib.ds_route_topk_f32(_p(lg), _p(b), m, e, k, int(n_groups), int(topk_groups),
                                     0 if scoring_func == "sigmoid" else 1, float(route_scale), _p(idx), _p(w))
    _check("ds_route_topk_f32", code)
    return _home(idx, logits), _home(w if weights_dtype == torch.float32 else w.to(torch.bfloat16), logits)


# --------------------------------------------------------------------------- lm_head

# --------------------------------------------------------------------------- MLA attention

def native_flash_mla_available() -> bool:
    """src/pcketlm/native/__init__.py:837-842."""
    return _available("PCKETLM_DISABLE_NATIVE_FLASH_MLA")


def native_fused_ds_attention_available() -> bool:
    """src/pcketlm/native/__init__.py:845-850."""
    return _available("PCKETLM_DISABLE_FUSED_DS_ATTENTION")


def ds_mla_attention_flash_forward(q_nope: torch.Tensor, q_pe: torch.Tensor, kv_cache: torch.Tensor,
                                   pe_cache: torch.Tensor, wkv_b: torch.Tensor, *, softmax_scale: float) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:878-939 -> ds_forward.cpp:517-597: MLA
    attention of one token over the latent cache; returns [heads, v_head_dim]
    fp32 where q_nope lives."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FLASH_MLA", "Native flash MLA")
    dev = _target_device(q_nope, q_pe, kv_cache, pe_cache, wkv_b)
    qn, qp, kv, pe, wkv = (_on(t, dev, torch.float32) for t in (q_nope, q_pe, kv_cache, pe_cache, wkv_b))
    if qn.ndim != 2 or qp.ndim != 2:
        raise ValueError("q_nope and q_pe must be [heads, dim]")
    if kv.ndim != 2 or pe.ndim != 2:
        raise ValueError("kv_cache and pe_cache must be [cache_len, dim]")
    if wkv.ndim != 3:
        raise ValueError("wkv_b must be [heads, qk_nope + v_head_dim, kv_lora_rank]")
    heads, nope = int(qn.shape[0]), int(qn.shape[1])
    rope, cache_len, rank = int(qp.shape[1]), int(kv.shape[0]), int(kv.shape[1])
    if int(qp.shape[0]) != heads or int(wkv.shape[0]) != heads:
        raise ValueError("head count mismatch")
    if int(pe.shape[0]) != cache_len or int(pe.shape[1]) != rope:
        raise ValueError("pe_cache shape mismatch")
    if int(wkv.shape[2]) != rank or int(wkv.shape[1]) <= nope:
        raise ValueError("wkv_b shape mismatch")
    v_dim = int(wkv.shape[1]) - nope
    out = torch.empty((heads, v_dim), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = lib.ds_mla_attention_flash_forward(_p(qn), _p(qp), _p(kv), _p(pe), _p(wkv), _p(out), heads, cache_len,
                                                  nope, rope, rank, v_dim, float(softmax_scale))
    _check("ds_mla_attention_flash_forward", code)
    return _home(out, q_nope)


def ds_attention_block_forward(session: "DeepSeekNativeSession", hidden: torch.Tensor, q_a_weight: torch.Tensor,
                               q_b_weight: torch.Tensor, kv_a_weight: torch.Tensor, kv_b_weight: torch.Tensor,
                               o_weight: torch.Tensor, q_norm_weight: torch.Tensor, kv_norm_weight: torch.Tensor, *,
                               previous_kv_cache: torch.Tensor | None, previous_pe_cache: torch.Tensor | None,
                               rope_cos: torch.Tensor, rope_sin: torch.Tensor, q_lora_rank: int, kv_lora_rank: int,
                               num_heads: int, qk_nope_dim: int, qk_rope_dim: int, v_head_dim: int, rms_eps: float,
                               softmax_scale: float):
    """src/pcketlm/native/__init__.py:942-1068 -> ds_forward.cpp:647-782: a
    one-token DeepSeek attention block as one native call.  Returns
    (hidden_out [hidden_dim], (next_kv_cache, next_pe_cache)) where hidden
    lives."""
    lib = _require("PCKETLM_DISABLE_FUSED_DS_ATTENTION", "Native fused DeepSeek attention")
    dev = _target_device(hidden, q_a_weight, q_b_weight, kv_a_weight, kv_b_weight, o_weight)
    x = _on(hidden, dev, torch.float32).reshape(-1)
    if int(x.numel()) <= 0:
        raise ValueError("hidden must not be empty")
    hidden_dim = int(x.numel())
    q_a, q_b, kv_a, kv_b, o = (_on(t, dev, torch.float32) for t in (q_a_weight, q_b_weight, kv_a_weight, kv_b_weight,
                                                                    o_weight))
    q_norm = _on(q_norm_weight, dev, torch.float32).reshape(-1)
    kv_norm = _on(kv_norm_weight, dev, torch.float32).reshape(-1)
    cos = _on(rope_cos, dev, torch.float32).reshape(-1)
    sin = _on(rope_sin, dev, torch.float32).reshape(-1)
    q_rank, kv_rank, heads = int(q_lora_rank), int(kv_lora_rank), int(num_heads)
    nope, rope, v_dim = int(qk_nope_dim), int(qk_rope_dim), int(v_head_dim)
    if tuple(q_a.shape) != (q_rank, hidden_dim):
        raise ValueError("q_a_weight must be [q_lora_rank, hidden_dim]")
    if tuple(q_b.shape) != (heads * (nope + rope), q_rank):
        raise ValueError("q_b_weight shape does not match DeepSeek attention config")
    if tuple(kv_a.shape) != (kv_rank + rope, hidden_dim):
        raise ValueError("kv_a_weight shape does not match DeepSeek attention config")
    if tuple(kv_b.shape) != (heads * (nope + v_dim), kv_rank):
        raise ValueError("kv_b_weight shape does not match DeepSeek attention config")
    if tuple(o.shape) != (hidden_dim, heads * v_dim):
        raise ValueError("o_weight shape does not match DeepSeek attention config")
    if int(q_norm.numel()) != q_rank or int(kv_norm.numel()) != kv_rank:
        raise ValueError("norm weight sizes do not match ranks")
    if int(cos.numel()) != max(0, rope // 2) or int(sin.numel()) != max(0, rope // 2):
        raise ValueError("rope cos/sin sizes must be qk_rope_dim / 2")
    prev_kv = (torch.empty((0, kv_rank), dtype=torch.float32, device=dev) if previous_kv_cache is None
               else _on(previous_kv_cache, dev, torch.float32).reshape(-1, kv_rank))
    prev_pe = (torch.empty((0, rope), dtype=torch.float32, device=dev) if previous_pe_cache is None
               else _on(previous_pe_cache, dev, torch.float32).reshape(-1, rope))
    previous_len = int(prev_kv.shape[0])
    if int(prev_pe.shape[0]) != previous_len:
        raise ValueError("previous KV and PE cache lengths must match")
    next_kv = torch.empty((previous_len + 1, kv_rank), dtype=torch.float32, device=dev)
    next_pe = torch.empty((previous_len + 1, rope), dtype=torch.float32, device=dev)
    out = torch.empty((hidden_dim,), dtype=torch.float32, device=dev)
    prev_kv_p = _p(None) if previous_len == 0 else _p(prev_kv)
    prev_pe_p = _p(None) if previous_len == 0 else _p(prev_pe)
    with _launch(lib, dev):
        code = lib.ds_attention_block_forward_f32(
            session._handle, _p(x), _p(q_a), _p(q_b), _p(kv_a), _p(kv_b), _p(o), _p(q_norm), _p(kv_norm), prev_kv_p,
            prev_pe_p, _p(cos), _p(sin), _p(next_kv), _p(next_pe), _p(out), hidden_dim, q_rank, kv_rank, heads, nope,
            rope, v_dim, previous_len, float(rms_eps), float(softmax_scale))
    _check("ds_attention_block_forward_f32", code)
    # (no keep-alive list: the launches are ordered on torch's stream, so its
    # allocator reuses these buffers only after them)
    return _home(out, hidden), (_home(next_kv, hidden), _home(next_pe, hidden))


def fp8_attention_block_forward(hidden: torch.Tensor, q_a_weight: torch.Tensor, q_a_scale_inv: torch.Tensor,
                                q_b_weight: torch.Tensor, q_b_scale_inv: torch.Tensor, kv_a_weight: torch.Tensor,
                                kv_a_scale_inv: torch.Tensor, kv_b_weight: torch.Tensor, o_weight: torch.Tensor,
                                o_scale_inv: torch.Tensor, q_norm_weight: torch.Tensor, kv_norm_weight: torch.Tensor, *,
                                previous_kv_cache: torch.Tensor | None, previous_pe_cache: torch.Tensor | None,
                                rope_cos: torch.Tensor, rope_sin: torch.Tensor, q_lora_rank: int, kv_lora_rank: int,
                                num_heads: int, qk_nope_dim: int, qk_rope_dim: int, v_head_dim: int, rms_eps: float,
                                softmax_scale: float, dtype: torch.dtype = torch.float32):
    """The FP8 model's one-token attention (src/pcketlm/core/runtime/
    fp8_source.py:6337-6454 at one token) as one native call
    (ds_fp8_attention_block_bf16x_f32): q_a / q_b / kv_a / o are FP8 e4m3
    weights with their 128x128 scale_inv grids, kv_b is the fp32
    dequantized weight (``dequantize_fp8_block_scaled(..., torch.float32)``,
    as the reference loads it).  The hidden state is taken as bf16 (the
    reference widens it to fp32 for its FP8 linears; the widening is exact).
    Returns (hidden_out [hidden_dim] in ``dtype``, (next_kv_cache,
    next_pe_cache)) on the weights' device."""
    lib = _require("PCKETLM_DISABLE_FUSED_DS_ATTENTION", "Native fused DeepSeek attention")
    dev = _target_device(hidden, q_a_weight, q_b_weight, kv_a_weight, kv_b_weight, o_weight)
    x = _on(hidden, dev, torch.bfloat16).reshape(-1)
    hidden_dim = int(x.numel())
    if hidden_dim <= 0:
        raise ValueError("hidden must not be empty")
    q_rank, kv_rank, heads = int(q_lora_rank), int(kv_lora_rank), int(num_heads)
    nope, rope, v_dim = int(qk_nope_dim), int(qk_rope_dim), int(v_head_dim)
    fp8 = {}
    for name, w, s, shape in (("q_a", q_a_weight, q_a_scale_inv, (q_rank, hidden_dim)),
                              ("q_b", q_b_weight, q_b_scale_inv, (heads * (nope + rope), q_rank)),
                              ("kv_a", kv_a_weight, kv_a_scale_inv, (kv_rank + rope, hidden_dim)),
                              ("o", o_weight, o_scale_inv, (hidden_dim, heads * v_dim))):
        wt = _fp8_bytes(w, dev)
        if tuple(wt.shape) != shape:
            raise ValueError(f"{name}_weight shape does not match DeepSeek attention config")
        st = _on(s, dev, torch.float32)
        if st.ndim != 2 or int(st.shape[0]) != -(-shape[0] // 128) or int(st.shape[1]) != -(-shape[1] // 128):
            raise ValueError(f"{name}_scale_inv must be the 128x128 block layout of {name}_weight")
        fp8[name] = (wt, st)
    kv_b = _on(kv_b_weight, dev, torch.float32)
    if tuple(kv_b.shape) != (heads * (nope + v_dim), kv_rank):
        raise ValueError("kv_b_weight shape does not match DeepSeek attention config")
    q_norm = _on(q_norm_weight, dev, torch.float32).reshape(-1)
    kv_norm = _on(kv_norm_weight, dev, torch.float32).reshape(-1)
    if int(q_norm.numel()) != q_rank or int(kv_norm.numel()) != kv_rank:
        raise ValueError("norm weight sizes do not match ranks")
    cos = _on(rope_cos, dev, torch.float32).reshape(-1)
    sin = _on(rope_sin, dev, torch.float32).reshape(-1)
    if int(cos.numel()) != max(0, rope // 2) or int(sin.numel()) != max(0, rope // 2):
        raise ValueError("rope cos/sin sizes must be qk_rope_dim / 2")
    prev_kv = (torch.empty((0, kv_rank), dtype=torch.float32, device=dev) if previous_kv_cache is None
               else _on(previous_kv_cache, dev, torch.float32).reshape(-1, kv_rank))
    prev_pe = (torch.empty((0, rope), dtype=torch.float32, device=dev) if previous_pe_cache is None
               else _on(previous_pe_cache, dev, torch.float32).reshape(-1, rope))
    previous_len = int(prev_kv.shape[0])
    if int(prev_pe.shape[0]) != previous_len:
        raise ValueError("previous KV and PE cache lengths must match")
    next_kv = torch.empty((previous_len + 1, kv_rank), dtype=torch.float32, device=dev)
    next_pe = torch.empty((previous_len + 1, rope), dtype=torch.float32, device=dev)
    out = torch.empty((hidden_dim,), dtype=torch.float32, device=dev)
    prev_kv_p = _p(None) if previous_len == 0 else _p(prev_kv)
    prev_pe_p = _p(None) if previous_len == 0 else _p(prev_pe)
    with _launch(lib, dev):
        code = lib.ds_fp8_attention_block_bf16x_f32(
            _p(x), *[_p(t) for name in ("q_a", "q_b", "kv_a") for t in fp8[name]], _p(kv_b), *[_p(t) for t in fp8["o"]],
            _p(q_norm), _p(kv_norm), prev_kv_p, prev_pe_p, _p(cos), _p(sin), _p(next_kv), _p(next_pe), _p(out),
            hidden_dim, q_rank, kv_rank, heads, nope, rope, v_dim, previous_len, float(rms_eps), float(softmax_scale))
    _check("ds_fp8_attention_block_bf16x_f32", code)
    return _home(out.to(dtype), hidden), (_home(next_kv, hidden), _home(next_pe, hidden))


def native_lm_head_topk_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_MATMUL")


native_fp16_matmul_available = native_lm_head_topk_available


def fp16_matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """src/pcketlm/native/__init__.py:2226-2249 -> fp16_matmul.cpp:344-396:
    a [m, k] @ b [k, n] in fp16 with fp32 accumulation, rounded to fp16."""
    lib = _require("PCKETLM_DISABLE_NATIVE_MATMUL", "Native fp16 matmul")
    if a.dtype != torch.float16 or b.dtype != torch.float16:
        raise TypeError("fp16_matmul requires torch.float16 inputs")
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("fp16_matmul requires 2D matrices")
    if int(a.shape[1]) != int(b.shape[0]):
        raise ValueError("fp16_matmul input shapes are incompatible")
    dev = _target_device(a, b)
    ad, bd = _on(a, dev), _on(b, dev)
    m, k, n = int(ad.shape[0]), int(ad.shape[1]), int(bd.shape[1])
    out = torch.empty((m, n), dtype=torch.float16, device=dev)
    with _launch(lib, dev):
        code = lib.native_fp16_matmul(_p(ad), _p(bd), _p(out), m, n, k)
    _check("native_fp16_matmul", code)
    return _home(out, a)


def lm_head_topk_u16(hidden: torch.Tensor, weight: torch.Tensor, *, top_k: int,
                     token_offset: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """src/pcketlm/native/__init__.py:2283-2323 -> fp16_matmul.cpp:155-204:
    the top_k logits of weight [rows, hidden] @ hidden and their token ids
    (row + token_offset), sorted by logit, descending."""
    lib = _require("PCKETLM_DISABLE_NATIVE_MATMUL", "Native lm_head top-k")
    if hidden.dtype != weight.dtype:
        raise TypeError("lm_head_topk_u16 requires hidden and weight to share dtype")
    if hidden.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("lm_head_topk_u16 requires torch.float16 or torch.bfloat16 tensors")
    dev = _target_device(weight, hidden)
    w = _on(weight, dev)
    if w.ndim != 2:
        raise ValueError("weight must have shape [rows, hidden_size]")
    rows, hidden_size = int(w.shape[0]), int(w.shape[1])
    h = _on(hidden, dev).reshape(-1).contiguous()
    if int(h.numel()) != hidden_size:
        raise ValueError("hidden size does not match lm_head weight")
    ids = torch.empty((int(top_k),), dtype=torch.int64, device=dev)
    logits = torch.empty((int(top_k),), dtype=torch.float32, device=dev)
    with _launch(lib, dev):
        code = lib.native_lm_head_topk_u16(_p(h), _p(w), _p(ids), _p(logits), rows, hidden_size, int(top_k),
                                           1 if hidden.dtype == torch.bfloat16 else 0, int(token_offset))
    _check("native_lm_head_topk_u16", code)
    return _home(logits, hidden), _home(ids, hidden)


# --------------------------------------------------------------------------- weight files to HBM

def native_row8_artifact_available() -> bool:
    return _available("PCKETLM_DISABLE_NATIVE_ROW8_ARTIFACT")


def file_spans_to_device(path: str | Path, spans) -> None:
    """Copy file byte ranges straight into device tensors: spans is a list of
    (file_offset, tensor) pairs, each tensor a contiguous device tensor that
    receives tensor.nbytes bytes from file_offset.  Returns when the bytes
    are in device memory (pocketlm_file_spans_to_device)."""
    lib = _require("PCKETLM_DISABLE_NATIVE_FILE_IO", "Native file transfer")
    spans = [(int(off), t) for off, t in spans if int(t.numel()) > 0]
    if not spans:
        return
    dev = spans[0][1].device
    for _off, t in spans:
        if t.device != dev or t.device.type != "cuda" or not t.is_contiguous():
            raise ValueError("span destinations must be contiguous tensors on one HIP device")
    n = len(spans)
    offs = (ctypes.c_uint64 * n)(*[off for off, _t in spans])
    lens = (ctypes.c_uint64 * n)(*[t.numel() * t.element_size() for _off, t in spans])
    dsts = (ctypes.c_uint64 * n)(*[t.data_ptr() for _off, t in spans])
    with _launch(lib, dev):
        code = lib.pocketlm_file_spans_to_device(str(path).encode("utf-8"), ctypes.cast(offs, ctypes.c_void_p),
                                                 ctypes.cast(lens, ctypes.c_void_p), ctypes.cast(dsts, ctypes.c_void_p),
                                                 n)
    _check("pocketlm_file_spans_to_device", code)


class NativeRow8Tensor:
    """src/pcketlm/native/__init__.py:2017-2049: nbytes at offset of a row8
    artifact file, loaded by the library.  ptr is a device pointer here."""

    def __init__(self, path: str | Path, offset: int, nbytes: int):
        lib = _require("PCKETLM_DISABLE_NATIVE_ROW8_ARTIFACT", "Native row8 artifact cache")
        with _launch(lib, torch.device("cuda", torch.cuda.current_device())):
            handle = lib.row8_artifact_load_tensor(str(Path(path)).encode("utf-8"), ctypes.c_ulonglong(int(offset)),
                                                   ctypes.c_ulonglong(int(nbytes)))
        if not handle:
            raise OSError(f"row8_artifact_load_tensor failed for {path}")
        self._lib = lib
        self._handle = ctypes.c_void_p(handle)
        self.nbytes = int(lib.row8_artifact_tensor_nbytes(self._handle))
        ptr = lib.row8_artifact_tensor_data(self._handle)
        if not ptr or self.nbytes != int(nbytes):
            self.close()
            raise OSError(f"row8_artifact_tensor_data failed for {path}")
        self.ptr = int(ptr)
        self.path = str(path)
        self.offset = int(offset)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            self._lib.row8_artifact_free_tensor(self._handle)
            self._handle = None
            self.ptr = 0

    def __del__(self):  # pragma: no cover - GC safety net
        try:
            self.close()
        except Exception:
            pass


def load_native_row8_tensor(path: str | Path, offset: int, nbytes: int) -> NativeRow8Tensor:
    return NativeRow8Tensor(path, offset, nbytes)


class NativeRow8MappedFile:
    """src/pcketlm/native/__init__.py:2056-2090: a read-only host mapping
    (host memory: needs the library but no device)."""

    def __init__(self, path: str | Path):
        if _flag("PCKETLM_DISABLE_NATIVE_ROW8_ARTIFACT"):
            raise RuntimeError("Native row8 artifact cache is unavailable: disabled")
        try:
            lib = _lib.load()
        except OSError as exc:
            raise RuntimeError(f"Native row8 artifact cache is unavailable: {exc}") from exc
        handle = lib.row8_artifact_map_file(str(Path(path)).encode("utf-8"))
        if not handle:
            raise OSError(f"row8_artifact_map_file failed for {path}")
        self._lib = lib
        self._handle = ctypes.c_void_p(handle)
        self.nbytes = int(lib.row8_artifact_mapped_nbytes(self._handle))
        self.path = str(path)

    def data_ptr(self, offset: int, nbytes: int) -> int:
        ptr = self._lib.row8_artifact_mapped_data(self._handle, ctypes.c_ulonglong(int(offset)),
                                                  ctypes.c_ulonglong(int(nbytes)))
        if not ptr:
            raise ValueError("row8 mapped tensor range is invalid")
        return int(ptr)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            self._lib.row8_artifact_unmap_file(self._handle)
            self._handle = None

    def __del__(self):  # pragma: no cover - GC safety net
        try:
            self.close()
        except Exception:
            pass


class NativeRow8MappedTensor:
    def __init__(self, mapped_file: NativeRow8MappedFile, offset: int, nbytes: int):
        self._mapped_file = mapped_file
        self.offset = int(offset)
        self.nbytes = int(nbytes)
        self.ptr = mapped_file.data_ptr(offset, nbytes)


def map_native_row8_file(path: str | Path) -> NativeRow8MappedFile:
    return NativeRow8MappedFile(path)


# --------------------------------------------------------------------------- KV session, dense layer decode

def native_fp16_kv_available() -> bool:
    """src/pcketlm/native/__init__.py native_fp16_kv_available, kill switch
    PCKETLM_DISABLE_NATIVE_KV."""
    if _flag("PCKETLM_DISABLE_NATIVE_KV"):
        return False
    try:
        _lib.load()
    except OSError:
        return False
    return torch.cuda.is_available()


class NativeKvSession:
    """src/pcketlm/native/__init__.py:2796-3260 over a device-resident cache
    (fp16_kv_cache.cpp's session, kv_cache.hip here).  Rows and results are
    device tensors on the session's device; host tensors passed in are moved
    there.  Lengths are host-side, so commit/rollback never touch the GPU."""

    def __init__(self, layer_count: int, max_seq_len: int, kv_width: int, dtype: torch.dtype = torch.float16,
                 device: torch.device | str | None = None):
        lib = _require("PCKETLM_DISABLE_NATIVE_KV", "Native fp16 KV cache")
        dtype_code = _u16_storage_dtype_code(dtype)
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        with torch.cuda.device(self.device):
            handle = lib.kv_prefill_init_typed(int(layer_count), int(max_seq_len), int(kv_width), dtype_code)
        if not handle:
            detail = _lib.last_error()
            raise RuntimeError("kv_prefill_init failed" + (f" ({detail})" if detail else ""))
        self._lib = lib
        self._handle = ctypes.c_void_p(handle)
        self.layer_count = int(layer_count)
        self.max_seq_len = int(max_seq_len)
        self.kv_width = int(kv_width)
        self.dtype = dtype

    @property
    def handle(self) -> int:
        if not self._handle:
            raise RuntimeError("NativeKvSession is closed")
        return int(self._handle.value)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            self._lib.kv_free(self._handle)
            self._handle = None

    def __del__(self):  # pragma: no cover - GC safety net
        try:
            self.close()
        except Exception:
            pass

    def _append(self, fn_name: str, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, count: int) -> None:
        if k_new.dtype != self.dtype or v_new.dtype != self.dtype:
            raise TypeError(f"KV cache append requires {self.dtype} tensors")
        k = _on(k_new, self.device).reshape(-1)
        v = _on(v_new, self.device).reshape(-1)
        expected = int(count) * self.kv_width
        if k.numel() != expected or v.numel() != expected:
            raise ValueError("KV tensor size does not match count * kv_width")
        with _launch(self._lib, self.device):
            code = getattr(self._lib, fn_name)(self._handle, int(layer), _p(k), _p(v), int(count))
        _check(fn_name, code)

    def append_committed(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, count: int) -> None:
        self._append("kv_append_committed", layer, k_new, v_new, count)

    def append_tentative(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, count: int) -> None:
        self._append("kv_append_tentative", layer, k_new, v_new, count)

    def commit(self, count: int) -> None:
        _check("kv_commit", self._lib.kv_commit(self._handle, int(count)))

    def rollback(self) -> None:
        _check("kv_rollback", self._lib.kv_rollback(self._handle))

    def committed_length(self, layer: int) -> int:
        return int(self._lib.kv_committed_length(self._handle, int(layer)))

    def tentative_length(self, layer: int) -> int:
        return int(self._lib.kv_tentative_length(self._handle, int(layer)))

    def copy_layer(self, layer: int, *, include_tentative: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
        count = self.committed_length(layer) + (self.tentative_length(layer) if include_tentative else 0)
        k_out = torch.empty((count, self.kv_width), dtype=self.dtype, device=self.device)
        v_out = torch.empty((count, self.kv_width), dtype=self.dtype, device=self.device)
        with _launch(self._lib, self.device):
            code = self._lib.kv_copy_layer(self._handle, int(layer), _p(k_out), _p(v_out), count,
                                           1 if include_tentative else 0)
        _check("kv_copy_layer", code)
        return k_out, v_out

    def dense_layer_decode_packed_rows8(self, layer: int, hidden: torch.Tensor, input_norm_weight: torch.Tensor,
                                        post_norm_weight: torch.Tensor, q_weight_packed: torch.Tensor,
                                        k_weight_packed: torch.Tensor, v_weight_packed: torch.Tensor,
                                        o_weight_packed: torch.Tensor, gate_weight_packed: torch.Tensor,
                                        up_weight_packed: torch.Tensor, down_weight_packed: torch.Tensor, *,
                                        hidden_size: int, intermediate_size: int, num_heads: int, num_kv_heads: int,
                                        head_dim: int | None = None, rms_eps: float, rope_theta: float,
                                        q_bias: torch.Tensor | None = None, k_bias: torch.Tensor | None = None,
                                        v_bias: torch.Tensor | None = None,
                                        q_norm_weight: torch.Tensor | None = None,
                                        k_norm_weight: torch.Tensor | None = None) -> torch.Tensor:
        """src/pcketlm/native/__init__.py:3041-3120 ->
        kv_dense_layer_decode_u16_ext_packed_rows8 (fp16_kv_cache.cpp:1533).
        The new k/v row is appended as a tentative row of `layer`."""
        raw = [hidden, input_norm_weight, post_norm_weight]
        if any(t.dtype != self.dtype for t in raw):
            raise TypeError(f"dense_layer_decode_packed_rows8 requires {self.dtype} raw tensors")
        packed = [q_weight_packed, k_weight_packed, v_weight_packed, o_weight_packed, gate_weight_packed,
                  up_weight_packed, down_weight_packed]
        if any(t.dtype != torch.uint16 for t in packed):
            raise TypeError("packed dense layer weights must be torch.uint16")
        if head_dim is not None and int(head_dim) * int(num_heads) != int(hidden_size):
            raise ValueError("head_dim must equal hidden_size // num_heads for this entry point")
        dev = self.device
        raw_d = [_on(t, dev).reshape(-1) for t in raw]
        if raw_d[0].numel() != int(hidden_size):
            raise ValueError("hidden length does not match hidden_size")
        H, inter, kvw = int(hidden_size), int(intermediate_size), self.kv_width
        if int(num_heads) <= 0 or H % int(num_heads) != 0:
            raise ValueError("hidden_size must be a multiple of num_heads")
        hd = H // int(num_heads)
        if any(t.numel() != H for t in raw_d):
            raise ValueError("hidden and norm weights must hold hidden_size values")
        packed_d = [_on(t, dev) for t in packed]
        blocks = lambda rows: (rows + 7) // 8 * 8  # noqa: E731
        want = [blocks(H) * H, blocks(kvw) * H, blocks(kvw) * H, blocks(H) * H, blocks(inter) * H,
                blocks(inter) * H, blocks(H) * inter]
        if [t.numel() for t in packed_d] != want:
            raise ValueError("packed weight sizes do not match the layer shape")
        opt = [None if t is None else _on(t, dev).reshape(-1)
               for t in (q_bias, k_bias, v_bias, q_norm_weight, k_norm_weight)]
        for t, n in zip(opt, (H, kvw, kvw, hd, hd)):
            if t is not None and (t.numel() != n or t.dtype != self.dtype):
                raise ValueError(f"biases and q/k norm weights must be {self.dtype} of the layer's sizes")
        out = torch.empty((int(hidden_size),), dtype=self.dtype, device=dev)
        with _launch(self._lib, dev):
            code = self._lib.kv_dense_layer_decode_u16_ext_packed_rows8(
                self._handle, int(layer), *[_p(t) for t in raw_d], *[_p(t) for t in packed_d],
                *[_p(t) for t in opt], _p(out), int(hidden_size), int(intermediate_size), int(num_heads),
                int(num_kv_heads), float(rms_eps), float(rope_theta))
        _check("kv_dense_layer_decode_u16_ext_packed_rows8", code)
        return out

    def dense_layer_prefill_packed_rows8(self, layer: int, hidden: torch.Tensor, *weights: torch.Tensor,
                                         **kwargs) -> torch.Tensor:
        """kv_dense_layer_prefill_u16_ext's loop (fp16_kv_cache.cpp:1591-1673)
        over the packed decode: each row is decoded, then committed."""
        rows = hidden.reshape(-1, int(kwargs["hidden_size"]))
        if self.committed_length(layer) + self.tentative_length(layer) + rows.shape[0] > self.max_seq_len:
            raise RuntimeError("kv_dense_layer_prefill failed with code 4 (cache full)")
        outs = []
        for row in rows:
            outs.append(self.dense_layer_decode_packed_rows8(layer, row, *weights, **kwargs))
            self.commit(1)
        return torch.stack(outs)

"""CPU oracle for the PocketLM quantized-decode hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import this package, and only as the
checker: the product (``pocketlm_amd``) never calls into it.

``oracle.c`` restates the reference kernels in C with their loop nests and
fp32 accumulation order (each function cites the reference file:line it
follows).  This module wraps it for numpy arrays.  ``ref`` exposes the
reference's own ``fp8_linear.cpp`` and ``fp16_packed_gemv.cpp`` compiled
from source into ``oracle/_ref`` (``make -C oracle ref``) when that build is
present; the tests use it to pin the restatement bit for bit.

The pure-numpy helpers at the bottom restate the torch-level parts of the
path (Q4 quantizer, row8 pack, DeepSeek-V3 router) for small inputs.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboracle.so"
_REF_DIR = _DIR / "_ref"

_c_i64 = ctypes.c_longlong
_vp = ctypes.c_void_p


def build(force: bool = False) -> Path:
    """Compile liboracle.so (and the reference build when its sources exist)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_DIR), "liboracle.so"], check=True)
    if Path("/root/reference/src/pcketlm/native/fp8_linear.cpp").exists():
        subprocess.run(["make", "-s", "-C", str(_DIR), "ref"], check=True)
    return _LIB_PATH


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(_LIB_PATH))
        handle.orc_e4m3_linear.restype = ctypes.c_float
        handle.orc_e4m3_linear.argtypes = [ctypes.c_uint8]
        handle.orc_e4m3_dequant.restype = ctypes.c_float
        handle.orc_e4m3_dequant.argtypes = [ctypes.c_uint8]
        handle.orc_f16_to_f32.restype = ctypes.c_float
        handle.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        for name in ("orc_f32_to_f16_sw", "orc_f32_to_f16_hw", "orc_f32_to_bf16"):
            getattr(handle, name).restype = ctypes.c_uint16
            getattr(handle, name).argtypes = [ctypes.c_float]
        handle.orc_q4_dequant_f16.restype = None
        handle.orc_num_threads.restype = ctypes.c_int
        _LIB = handle
    return _LIB


def num_threads() -> int:
    return int(lib().orc_num_threads())


def _ptr(a: np.ndarray) -> _vp:
    return _vp(a.ctypes.data)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _check(name: str, code: int) -> None:
    if code != 0:
        raise RuntimeError(f"{name} failed with code {code}")


# --------------------------------------------------------------------------- scalars

def e4m3_linear(byte: int) -> float:
    return float(lib().orc_e4m3_linear(int(byte)))


def e4m3_dequant_bits(byte: int) -> int:
    v = np.array([lib().orc_e4m3_dequant(int(byte))], dtype=np.float32)
    return int(v.view(np.uint32)[0])


def f32_to_f16_hw(values: np.ndarray) -> np.ndarray:
    f = lib().orc_f32_to_f16_hw
    flat = _c(values, np.float32).reshape(-1)
    return np.array([f(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(values))


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    f = lib().orc_f32_to_bf16
    flat = _c(values, np.float32).reshape(-1)
    return np.array([f(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(values))


# --------------------------------------------------------------------------- FP8

def scale_cols(cols: int) -> int:
    return (int(cols) + 127) // 128


def fp8_linear(w: np.ndarray, s: np.ndarray, x: np.ndarray, *, batch_reuse: bool = False) -> np.ndarray:
    w = _c(w, np.uint8)
    s = _c(s, np.float32)
    x = _c(x, np.float32).reshape(-1, w.shape[1])
    out = np.empty((x.shape[0], w.shape[0]), dtype=np.float32)
    code = lib().orc_fp8_linear(_ptr(w), _ptr(s), _ptr(x), _ptr(out), _c_i64(x.shape[0]),
                                _c_i64(w.shape[0]), _c_i64(w.shape[1]), _c_i64(scale_cols(w.shape[1])),
                                ctypes.c_int(1 if batch_reuse else 0))
    _check("orc_fp8_linear", code)
    return out


def fp8_dual_linear(wa, sa, wb, sb, x):
    wa, wb = _c(wa, np.uint8), _c(wb, np.uint8)
    sa, sb = _c(sa, np.float32), _c(sb, np.float32)
    x = _c(x, np.float32).reshape(-1, wa.shape[1])
    oa = np.empty((x.shape[0], wa.shape[0]), dtype=np.float32)
    ob = np.empty_like(oa)
    code = lib().orc_fp8_dual_linear(_ptr(wa), _ptr(sa), _ptr(wb), _ptr(sb), _ptr(x), _ptr(oa), _ptr(ob),
                                     _c_i64(x.shape[0]), _c_i64(wa.shape[0]), _c_i64(wa.shape[1]),
                                     _c_i64(scale_cols(wa.shape[1])))
    _check("orc_fp8_dual_linear", code)
    return oa, ob


def fp8_mlp(g, gs, u, us, d, ds, x):
    g, u, d = _c(g, np.uint8), _c(u, np.uint8), _c(d, np.uint8)
    gs, us, ds = _c(gs, np.float32), _c(us, np.float32), _c(ds, np.float32)
    inter, hid = g.shape
    x = _c(x, np.float32).reshape(-1, hid)
    out = np.empty((x.shape[0], hid), dtype=np.float32)
    code = lib().orc_fp8_mlp(_ptr(g), _ptr(gs), _ptr(u), _ptr(us), _ptr(d), _ptr(ds), _ptr(x), _ptr(out),
                             _c_i64(x.shape[0]), _c_i64(inter), _c_i64(hid), _c_i64(scale_cols(hid)),
                             _c_i64(scale_cols(inter)))
    _check("orc_fp8_mlp", code)
    return out


def _ptr_table(items):
    """Six uint64 address arrays (gate, gate_scale, up, up_scale, down, down_scale)."""
    prepared = [tuple(_c(t, np.uint8 if i % 2 == 0 else np.float32) for i, t in enumerate(item)) for item in items]
    tables = [np.array([p[i].ctypes.data for p in prepared], dtype=np.uint64) for i in range(6)]
    return prepared, tables


def fp8_mlp_many(items, x):
    prepared, t = _ptr_table(items)
    inter, hid = prepared[0][0].shape
    x = _c(x, np.float32).reshape(-1, hid)
    out = np.empty((len(items), x.shape[0], hid), dtype=np.float32)
    code = lib().orc_fp8_mlp_many(*[_ptr(a) for a in t], _ptr(x), _ptr(out), _c_i64(len(items)),
                                  _c_i64(x.shape[0]), _c_i64(inter), _c_i64(hid), _c_i64(scale_cols(hid)),
                                  _c_i64(scale_cols(inter)))
    _check("orc_fp8_mlp_many", code)
    del prepared
    return out


def fp8_mlp_many_weighted(items, x, route):
    prepared, t = _ptr_table(items)
    inter, hid = prepared[0][0].shape
    x = _c(x, np.float32).reshape(-1, hid)
    route = _c(route, np.float32).reshape(-1)
    out = np.empty((x.shape[0], hid), dtype=np.float32)
    code = lib().orc_fp8_mlp_many_weighted(*[_ptr(a) for a in t], _ptr(x), _ptr(route), _ptr(out),
                                           _c_i64(len(items)), _c_i64(x.shape[0]), _c_i64(inter), _c_i64(hid),
                                           _c_i64(scale_cols(hid)), _c_i64(scale_cols(inter)))
    _check("orc_fp8_mlp_many_weighted", code)
    del prepared
    return out


def fp8_mlp_many_row_weighted(items, x, route):
    prepared, t = _ptr_table(items)
    inter, hid = prepared[0][0].shape
    x = _c(x, np.float32).reshape(-1, hid)
    route = _c(route, np.float32).reshape(len(items), x.shape[0])
    out = np.empty((x.shape[0], hid), dtype=np.float32)
    code = lib().orc_fp8_mlp_many_row_weighted(*[_ptr(a) for a in t], _ptr(x), _ptr(route), _ptr(out),
                                               _c_i64(len(items)), _c_i64(x.shape[0]), _c_i64(inter),
                                               _c_i64(hid), _c_i64(scale_cols(hid)), _c_i64(scale_cols(inter)))
    _check("orc_fp8_mlp_many_row_weighted", code)
    del prepared
    return out


def fp8_mlp_many_pair_weighted(items, x, pair_items, pair_rows, pair_weights):
    prepared, t = _ptr_table(items)
    inter, hid = prepared[0][0].shape
    x = _c(x, np.float32).reshape(-1, hid)
    pi = _c(pair_items, np.int64).reshape(-1)
    pr = _c(pair_rows, np.int64).reshape(-1)
    pw = _c(pair_weights, np.float32).reshape(-1)
    out = np.empty((x.shape[0], hid), dtype=np.float32)
    code = lib().orc_fp8_mlp_many_pair_weighted(*[_ptr(a) for a in t], _ptr(x), _ptr(pi), _ptr(pr), _ptr(pw),
                                                _ptr(out), _c_i64(len(items)), _c_i64(pi.size),
                                                _c_i64(x.shape[0]), _c_i64(inter), _c_i64(hid),
                                                _c_i64(scale_cols(hid)), _c_i64(scale_cols(inter)))
    _check("orc_fp8_mlp_many_pair_weighted", code)
    del prepared
    return out


def ds_moe_combine(outputs: np.ndarray, route: np.ndarray) -> np.ndarray:
    outputs = _c(outputs, np.float32)
    if outputs.ndim == 2:
        outputs = outputs[:, None, :]
    route = _c(route, np.float32).reshape(-1)
    out = np.empty(outputs.shape[1:], dtype=np.float32)
    code = lib().orc_ds_moe_combine(_ptr(outputs), _ptr(route), _c_i64(outputs.shape[0]),
                                    _c_i64(outputs.shape[1]), _c_i64(outputs.shape[2]), _ptr(out))
    _check("orc_ds_moe_combine", code)
    return out


def fp8_dequant(w: np.ndarray, s: np.ndarray, out_dtype: str) -> np.ndarray:
    """out_dtype: 'f16' / 'bf16' (uint16 bit patterns returned) or 'f32'."""
    w = _c(w, np.uint8)
    s = _c(s, np.float32)
    code_of = {"f16": 0, "bf16": 1, "f32": 2}[out_dtype]
    out = np.empty(w.shape, dtype=np.float32 if code_of == 2 else np.uint16)
    code = lib().orc_fp8_dequant(_ptr(w), _ptr(s), _ptr(out), _c_i64(w.shape[0]), _c_i64(w.shape[1]),
                                 _c_i64(scale_cols(w.shape[1])), ctypes.c_int(code_of))
    _check("orc_fp8_dequant", code)
    return out


# --------------------------------------------------------------------------- Q4

def q4_dequant_f16(packed: np.ndarray, scales_f16_bits: np.ndarray, channels: int, channel_size: int) -> np.ndarray:
    packed = _c(packed, np.uint8).reshape(-1)
    scales = _c(scales_f16_bits, np.uint16).reshape(-1)
    out = np.empty((int(channels) * int(channel_size),), dtype=np.uint16)
    if out.size:
        lib().orc_q4_dequant_f16(_ptr(packed), _ptr(scales), _ptr(out), _c_i64(channels), _c_i64(channel_size))
    return out


def q4_gemv(packed, scales_f16_bits, x, rows, cols) -> np.ndarray:
    packed = _c(packed, np.uint8).reshape(-1)
    scales = _c(scales_f16_bits, np.uint16).reshape(-1)
    x = _c(x, np.float32).reshape(-1)
    y = np.empty((int(rows),), dtype=np.float32)
    _check("orc_q4_gemv", lib().orc_q4_gemv(_ptr(packed), _ptr(scales), _ptr(x), _ptr(y), _c_i64(rows), _c_i64(cols)))
    return y


def q4_moe_selected(hidden_f16_bits, experts, route, hidden_size, intermediate_size) -> np.ndarray:
    """experts: list of (gate_packed, gate_scales_bits, up_packed, up_scales_bits, down_packed, down_scales_bits)."""
    hidden = _c(hidden_f16_bits, np.uint16).reshape(-1)
    keep = []
    arrays = []
    for slot in range(6):
        dtype = np.uint8 if slot % 2 == 0 else np.uint16
        tensors = [_c(e[slot], dtype).reshape(-1) for e in experts]
        keep.append(tensors)
        arr = (ctypes.c_void_p * len(experts))(*[t.ctypes.data for t in tensors])
        arrays.append(arr)
    route = _c(route, np.float32).reshape(-1)
    out = np.empty((int(hidden_size),), dtype=np.uint16)
    code = lib().orc_q4_moe_selected(_ptr(hidden), *arrays, _ptr(route), _ptr(out), _c_i64(hidden_size),
                                     _c_i64(intermediate_size), _c_i64(len(experts)))
    _check("orc_q4_moe_selected", code)
    del keep
    return out


# --------------------------------------------------------------------------- row8

def pack_rows8(w_bits: np.ndarray) -> np.ndarray:
    w = _c(w_bits, np.uint16)
    rows, cols = w.shape
    out = np.empty((((rows + 7) // 8) * cols * 8,), dtype=np.uint16)
    _check("orc_pack_rows8", lib().orc_pack_rows8(_ptr(w), _ptr(out), _c_i64(rows), _c_i64(cols)))
    return out


def packed_gemv_rows8(hidden_bits, packed, rows, cols, dtype_code, bias_bits=None) -> np.ndarray:
    h = _c(hidden_bits, np.uint16).reshape(-1)
    p = _c(packed, np.uint16).reshape(-1)
    out = np.empty((int(rows),), dtype=np.float32)
    b = None if bias_bits is None else _c(bias_bits, np.uint16).reshape(-1)
    code = lib().orc_packed_gemv_rows8(_ptr(h), _ptr(p), _ptr(out), _c_i64(rows), _c_i64(cols),
                                       ctypes.c_int(dtype_code), _vp(0) if b is None else _ptr(b))
    _check("orc_packed_gemv_rows8", code)
    return out


def packed_gemv_rows8_f32_hidden(hidden, packed, rows, cols, dtype_code) -> np.ndarray:
    """fp16_kv_cache.cpp:146-174 (fp32 activations, no bias)."""
    h = _c(hidden, np.float32).reshape(-1)
    p = _c(packed, np.uint16).reshape(-1)
    out = np.empty((int(rows),), dtype=np.float32)
    code = lib().orc_packed_gemv_rows8_f32_hidden(_ptr(h), _ptr(p), _ptr(out), _c_i64(rows), _c_i64(cols),
                                                  ctypes.c_int(dtype_code))
    _check("orc_packed_gemv_rows8_f32_hidden", code)
    return out


def router_topk_u16(hidden_bits, router_bits, k: int, dtype_code: int):
    h = _c(hidden_bits, np.uint16).reshape(-1)
    r = _c(router_bits, np.uint16)
    ids = np.empty((int(k),), dtype=np.int64)
    wts = np.empty((int(k),), dtype=np.float32)
    code = lib().orc_router_topk_u16(_ptr(h), _ptr(r), _c_i64(r.shape[1]), _c_i64(r.shape[0]), _c_i64(k),
                                     _c_i64(dtype_code), _ptr(ids), _ptr(wts))
    _check("orc_router_topk_u16", code)
    return ids, wts


# --------------------------------------------------------------------------- numpy restatements

def q4_quantize(tensor_f32: np.ndarray):
    """Per-row symmetric Q4 (src/pcketlm/core/model_import/q4_quantize.py:48-71).

    Returns (packed uint8, scale fp16 bit patterns, shape).  Rows are
    shape[0] (a 0-D tensor is one row of one value, a 1-D tensor of n
    values is n rows of one value); scale = max|row| / 7 in fp32 (1 for an
    all-zero row), stored as fp16; q = clamp(round-half-even(v / scale),
    -7, 7); element 2i goes in the low nibble of byte i.
    """
    t = np.asarray(tensor_f32, dtype=np.float32)
    shape = list(t.shape)
    if t.ndim == 0:
        m = t.reshape(1, 1)
    elif t.ndim == 1:
        m = t.reshape(t.shape[0], 1)
    else:
        m = t.reshape(t.shape[0], -1)
    max_abs = np.abs(m).max(axis=1) if m.size else np.zeros((m.shape[0],), np.float32)
    scales = np.where(max_abs > 0, max_abs / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(m / scales[:, None]), -7, 7).astype(np.int8)
    return pack_int4(q.reshape(-1)), scales.astype(np.float16).view(np.uint16), shape


def pack_int4(values: np.ndarray) -> np.ndarray:
    """q4_quantize.py:21-33: two's-complement nibbles, element 2i low."""
    v = np.asarray(values, dtype=np.int16).reshape(-1)
    if v.size == 0:
        return np.zeros((0,), dtype=np.uint8)
    enc = (v & 0x0F).astype(np.uint8)
    if enc.size % 2:
        enc = np.concatenate([enc, np.zeros((1,), np.uint8)])
    return (enc[0::2] | (enc[1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray, count: int) -> np.ndarray:
    """q4_quantize.py:36-45."""
    b = np.asarray(packed, dtype=np.uint8).reshape(-1)
    u = np.empty((b.size * 2,), dtype=np.int16)
    u[0::2] = b & 0x0F
    u[1::2] = (b >> 4) & 0x0F
    return np.where(u >= 8, u - 16, u)[: int(count)].astype(np.int8)


def q4_shape_params(shape) -> tuple[int, int]:
    """tensor_loader.py:598-605 (_q4_dequant_shape_params)."""
    if not shape:
        return 1, 1
    count = int(np.prod(shape))
    if len(shape) == 1:
        return int(shape[0]), 1
    return int(shape[0]), max(1, count // int(shape[0]))


def unpack_rows8(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Inverse of pack_rows8 (tools/pack_weights_row8.py:37-48)."""
    blocks = (int(rows) + 7) // 8
    view = np.asarray(packed, dtype=np.uint16).reshape(blocks, int(cols), 8)
    return view.transpose(0, 2, 1).reshape(blocks * 8, int(cols))[: int(rows)].copy()


def _topk_desc(values: np.ndarray, k: int) -> np.ndarray:
    # Stable descending order: larger first, lower index on ties.
    order = np.argsort(-values, kind="stable")
    return order[:k]


def deepseek_route(logits: np.ndarray, *, top_k: int = 8, n_groups: int = 8, topk_groups: int = 4,
                   route_scale: float = 2.5, bias: np.ndarray | None = None, scoring: str = "sigmoid"):
    """DeepSeek-V3 routing from router logits (fp8_source.py:1527-1547 with
    _mask_deepseek_route_groups 5125-5140), in fp32.

    Returns (indices int64 [M, top_k], weights fp32 [M, top_k]) with the
    weights already rounded to bf16 (fp8_source.py:1547) and widened back.
    Ties between exactly equal scores resolve to the lower expert id.
    """
    logits = np.asarray(logits, dtype=np.float32)
    if scoring == "softmax":
        z = logits - logits.max(axis=-1, keepdims=True)
        e = np.exp(z).astype(np.float32)
        scores = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    else:
        scores = (np.float32(1.0) / (np.float32(1.0) + np.exp(-logits))).astype(np.float32)
    choice = scores + bias.astype(np.float32) if bias is not None else scores.copy()
    m, n = choice.shape
    if n_groups > 1:
        grouped = choice.reshape(m, n_groups, -1)
        if bias is not None:
            top2 = -np.sort(-grouped, axis=-1)[..., :2]
            gscore = top2.sum(axis=-1)
        else:
            gscore = grouped.max(axis=-1)
        keep = max(1, min(int(topk_groups), int(n_groups)))
        masked = np.full_like(grouped, -np.inf)
        for row in range(m):
            for g in _topk_desc(gscore[row], keep):
                masked[row, g] = grouped[row, g]
        choice = masked.reshape(m, n)
    k = max(1, min(int(top_k), n))
    idx = np.stack([_topk_desc(choice[row], k) for row in range(m)]).astype(np.int64)
    w = np.take_along_axis(scores, idx, axis=1).astype(np.float32)
    if scoring == "sigmoid":
        w = w / np.maximum(w.sum(axis=-1, keepdims=True), np.float32(1e-12))
    w = (w * np.float32(route_scale)).astype(np.float32)
    w_bf16 = f32_to_bf16(w)
    return idx, (w_bf16.astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------- MoE layer orchestration

def _bf16_values(f32: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned widened to fp32."""
    return (f32_to_bf16(np.asarray(f32, np.float32)).astype(np.uint32) << 16).view(np.float32)


def run_fp8_moe(x_bf16: np.ndarray, route_idx: np.ndarray, route_w: np.ndarray, experts: dict, shared,
                *, mode: str = "auto") -> tuple[np.ndarray, list[int], str]:
    """DeepSeek MoE layer orchestration of run_fp8_moe
    (src/pcketlm/core/runtime/fp8_source.py:1569-1884) on the oracle's kernels.

    x_bf16: [M, H] activations as bf16 values (fp32 array); route_idx [M, k]
    int64; route_w [M, k] fp32 holding bf16 values (the router's output);
    experts: {expert id: (gate, gate_s, up, up_s, down, down_s)}; shared: the
    shared expert's six arrays or None.  mode "auto" picks the path the
    reference picks with its default flags: the route-weighted many-expert
    kernel at M == 1 (1643-1646, 1736-1764), per-expert MLPs on each expert's
    rows otherwise (1806-1836); "row" and "pair" force the row- and
    pair-weighted kernels (1647-1734).  Every add into the output is a bf16
    add (torch bf16 arithmetic: fp32 operation, round to nearest even).
    Returns (output bf16 values [M, H] as fp32, selected experts, path).
    """
    x = np.asarray(x_bf16, np.float32)
    m = x.shape[0]
    selected = sorted({int(v) for v in np.asarray(route_idx).reshape(-1)})
    jobs = []
    for e in selected:
        rows, tops = np.nonzero(np.asarray(route_idx) == e)
        jobs.append((e, rows, tops))
    out = np.zeros_like(x)
    items = [experts[e] for e, _r, _t in jobs]
    if mode == "pair" and m > 1:
        pi, pr, pw = [], [], []
        for item, (_e, rows, tops) in enumerate(jobs):
            for r, t in zip(rows.tolist(), tops.tolist()):
                pi.append(item)
                pr.append(r)
                pw.append(float(route_w[r, t]))
        y = fp8_mlp_many_pair_weighted(items, x, np.array(pi, np.int64), np.array(pr, np.int64),
                                       np.array(pw, np.float32))
        out = _bf16_values(out + _bf16_values(y))
        path = "pair_weighted"
    elif mode == "row" and m > 1:
        route = np.zeros((len(jobs), m), np.float32)
        for item, (_e, rows, tops) in enumerate(jobs):
            route[item, rows] = route_w[rows, tops]
        y = fp8_mlp_many_row_weighted(items, x, route)
        out = _bf16_values(out + _bf16_values(y))
        path = "row_weighted"
    elif m == 1:
        route = np.array([route_w[rows[0], tops[0]] for _e, rows, tops in jobs], np.float32)
        y = fp8_mlp_many_weighted(items, x, route)
        out = _bf16_values(out + _bf16_values(y))
        path = "weighted"
    else:
        for e, rows, tops in jobs:
            y = _bf16_values(fp8_mlp(*experts[e], x[rows]))
            r = route_w[rows, tops].astype(np.float32).reshape(-1, 1)
            out[rows] = _bf16_values(out[rows] + _bf16_values(y * r))
        path = "per_expert"
    if shared is not None:
        out = _bf16_values(out + _bf16_values(fp8_mlp(*shared, x)))
    return out, selected, path

"""Write the golden vectors under tests/golden/ (run in the build container).

    python tests/golden/make_golden.py

Inputs are the reference's own test fixtures (re-created from the recipes
in its tests: linspace grids, seeded torch.randn, the all-bytes table) plus a
few seeded larger cases.  Expected outputs come from two independent
sources, never from this repository's oracle:

* the reference's C++ compiled from its own sources into oracle/_ref
  (``make -C oracle ref``): fp8_linear.cpp for every FP8 GEMV / MLP / MoE
  kernel, fp16_packed_gemv.cpp for the row8 pack and GEMV;
* torch, the library the reference itself uses as the oracle of its
  dequant tests (``view(float8_e4m3fn).to(float32) * scale``, ``.to(float16)``,
  ``.to(bfloat16)``) and of its Q4 quantizer / dequant tests.

Every file is small data (a few hundred KB in total).  Nothing here is
shipped or imported by the product.
"""

from __future__ import annotations

import ctypes
import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
REF = REPO / "oracle" / "_ref"


def _load_ref():
    lin = ctypes.CDLL(str(REF / "libref_fp8_linear.so"))
    row8 = ctypes.CDLL(str(REF / "libref_fp16_packed_gemv.so"))
    return lin, row8


def fp8_bytes(values: torch.Tensor) -> np.ndarray:
    return values.to(torch.float8_e4m3fn).view(torch.uint8).contiguous().numpy()


def vp(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


I64 = ctypes.c_longlong


# --------------------------------------------------------------------------- reference calls

def ref_linear(lin, w, s, x, reuse=False):
    w, s, x = np.ascontiguousarray(w, np.uint8), np.ascontiguousarray(s, np.float32), np.ascontiguousarray(x, np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    _env(reuse)
    code = lin.fp8_e4m3_block_linear_f32(vp(w), vp(s), vp(x), vp(out), I64(x.shape[0]), I64(w.shape[0]),
                                         I64(w.shape[1]), I64((w.shape[1] + 127) // 128))
    assert code == 0, code
    return out


def ref_dual(lin, wa, sa, wb, sb, x, reuse=False):
    oa = np.empty((x.shape[0], wa.shape[0]), np.float32)
    ob = np.empty_like(oa)
    _env(reuse)
    code = lin.fp8_e4m3_block_dual_linear_f32(vp(wa), vp(sa), vp(wb), vp(sb), vp(x), vp(oa), vp(ob),
                                              I64(x.shape[0]), I64(wa.shape[0]), I64(wa.shape[1]),
                                              I64((wa.shape[1] + 127) // 128))
    assert code == 0, code
    return oa, ob


def ref_mlp(lin, g, gs, u, us, d, ds, x, reuse=False):
    inter, hid = g.shape
    out = np.empty((x.shape[0], hid), np.float32)
    _env(reuse)
    code = lin.fp8_e4m3_block_mlp_f32(vp(g), vp(gs), vp(u), vp(us), vp(d), vp(ds), vp(x), vp(out), I64(x.shape[0]),
                                      I64(inter), I64(hid), I64((hid + 127) // 128), I64((inter + 127) // 128))
    assert code == 0, code
    return out


def _tables(items):
    return [np.array([it[i].ctypes.data for it in items], np.uint64) for i in range(6)]


def ref_many(lin, items, x):
    inter, hid = items[0][0].shape
    t = _tables(items)
    out = np.empty((len(items), x.shape[0], hid), np.float32)
    code = lin.fp8_e4m3_block_mlp_many_f32(*[vp(a) for a in t], vp(x), vp(out), I64(len(items)), I64(x.shape[0]),
                                           I64(inter), I64(hid), I64((hid + 127) // 128), I64((inter + 127) // 128))
    assert code == 0, code
    return out


def ref_weighted(lin, items, x, route, symbol, reuse=False):
    inter, hid = items[0][0].shape
    t = _tables(items)
    out = np.empty((x.shape[0], hid), np.float32)
    _env(reuse)
    code = getattr(lin, symbol)(*[vp(a) for a in t], vp(x), vp(route), vp(out), I64(len(items)), I64(x.shape[0]),
                                I64(inter), I64(hid), I64((hid + 127) // 128), I64((inter + 127) // 128))
    assert code == 0, code
    return out


def ref_pair(lin, items, x, pi, pr, pw):
    inter, hid = items[0][0].shape
    t = _tables(items)
    out = np.empty((x.shape[0], hid), np.float32)
    code = lin.fp8_e4m3_block_mlp_many_pair_weighted_f32(*[vp(a) for a in t], vp(x), vp(pi), vp(pr), vp(pw), vp(out),
                                                         I64(len(items)), I64(pi.size), I64(x.shape[0]), I64(inter),
                                                         I64(hid), I64((hid + 127) // 128), I64((inter + 127) // 128))
    assert code == 0, code
    return out


def _env(reuse: bool) -> None:
    if reuse:
        os.environ["PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE"] = "1"
    else:
        os.environ.pop("PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE", None)


def mlp_item(seed, inter, hid, scale=0.25, gsv=1.0, usv=1.0, dsv=1.0):
    g = torch.Generator().manual_seed(seed)
    gate = fp8_bytes(torch.randn((inter, hid), generator=g) * scale)
    up = fp8_bytes(torch.randn((inter, hid), generator=g) * scale)
    down = fp8_bytes(torch.randn((hid, inter), generator=g) * scale)
    gs = np.full(((inter + 127) // 128, (hid + 127) // 128), gsv, np.float32)
    us = np.full_like(gs, usv)
    ds = np.full(((hid + 127) // 128, (inter + 127) // 128), dsv, np.float32)
    return (gate, gs, up, us, down, ds)


def pack_items(prefix: str, items, store: dict) -> None:
    for e, it in enumerate(items):
        for slot, name in enumerate(("g", "gs", "u", "us", "d", "ds")):
            store[f"{prefix}_{name}{e}"] = it[slot]
    store[f"{prefix}_count"] = np.array(len(items))


# --------------------------------------------------------------------------- FP8 dequant (torch closed form)

def torch_dequant(w: np.ndarray, s: np.ndarray):
    wt = torch.from_numpy(w)
    st = torch.from_numpy(s)
    rows, cols = w.shape
    vals = wt.view(torch.float8_e4m3fn).to(torch.float32)
    exp = st.repeat_interleave(128, 0).repeat_interleave(128, 1)[:rows, :cols]
    f32 = (vals * exp).contiguous()
    return (f32.view(torch.int32).numpy().view(np.uint32),
            f32.to(torch.float16).view(torch.int16).numpy().view(np.uint16),
            f32.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


def make_fp8_dequant() -> None:
    out: dict[str, np.ndarray] = {}
    cases = {
        # tests/test_native_fp8_dequant.py:13-28
        "lin16": (fp8_bytes(torch.linspace(-4.0, 4.0, steps=256).reshape(16, 16)), np.array([[0.75]], np.float32)),
        # tests/test_native_fp8_dequant.py:31-46
        "lin8x32": (fp8_bytes(torch.linspace(-8.0, 8.0, steps=256).reshape(8, 32)), np.array([[1.25]], np.float32)),
        # tests/test_native_fp8_dequant.py:49-63 (all 256 bytes, NaN included)
        "allbytes": (np.arange(256, dtype=np.uint8).reshape(16, 16), np.array([[1.0]], np.float32)),
        # tests/test_runtime_fp8_source.py:736-743
        "runtime": (fp8_bytes(torch.tensor([[0.5, 1.0, 2.0, -1.0], [3.0, 4.0, -2.0, -0.5]])), np.array([[2.0]], np.float32)),
    }
    g = torch.Generator().manual_seed(20261201)
    # Multi-block grids with partial last blocks and distinct per-block scales.
    for name, (r, c) in {"blocks300x260": (300, 260), "blocks136x1024": (136, 1024), "blocks20x4112": (20, 4112)}.items():
        w = fp8_bytes(torch.randn((r, c), generator=g) * 0.5)
        s = (torch.rand(((r + 127) // 128, (c + 127) // 128), generator=g) * 9e-3 + 1e-3).numpy().astype(np.float32)
        cases[name] = (w, s)
    # The all-bytes table tiled across several scale blocks.
    tile = np.tile(np.arange(256, dtype=np.uint8), 4 * 33).reshape(132, 256)
    cases["allbytes_blocks"] = (tile, (torch.rand((2, 2), generator=g) * 4 + 0.1).numpy().astype(np.float32))
    for name, (w, s) in cases.items():
        f32, f16, bf16 = torch_dequant(w, s)
        out[f"{name}_w"] = w
        out[f"{name}_s"] = s
        out[f"{name}_f32"] = f32
        out[f"{name}_f16"] = f16
        out[f"{name}_bf16"] = bf16
    out["cases"] = np.array(list(cases))
    # e4m3 decode of every byte (torch's float8_e4m3fn -> float32), bits
    all_bytes = torch.arange(256, dtype=torch.uint8)
    out["e4m3_f32_bits"] = all_bytes.view(torch.float8_e4m3fn).to(torch.float32).view(torch.int32).numpy().view(np.uint32)
    np.savez_compressed(HERE / "fp8_dequant.npz", **out)


# --------------------------------------------------------------------------- FP8 GEMV family (reference C++)

def make_fp8_gemv(lin) -> None:
    out: dict[str, np.ndarray] = {}
    # tests/test_native_fp8_linear.py:15-30
    w = fp8_bytes(torch.linspace(-1.5, 1.5, steps=32 * 64).reshape(32, 64))
    s = np.array([[0.875]], np.float32)
    x = torch.linspace(-0.5, 0.5, steps=2 * 64).reshape(2, 64).numpy()
    out.update(lin_w=w, lin_s=s, lin_x=x, lin_y=ref_linear(lin, w, s, x))
    # tests/test_native_fp8_linear.py:33-52 (batch reuse == per-row)
    w = fp8_bytes(torch.linspace(-1.5, 1.5, steps=64 * 128).reshape(64, 128))
    x = torch.linspace(-0.5, 0.5, steps=5 * 128).reshape(5, 128).numpy()
    out.update(reuse_w=w, reuse_s=s, reuse_x=x, reuse_y=ref_linear(lin, w, s, x, reuse=True),
               reuse_y_rows=np.concatenate([ref_linear(lin, w, s, x[i:i + 1]) for i in range(5)]))
    # tests/test_native_fp8_linear.py:55-77 (dual)
    gate = fp8_bytes(torch.linspace(-1.0, 1.0, steps=64 * 128).reshape(64, 128))
    up = fp8_bytes(torch.linspace(1.0, -1.0, steps=64 * 128).reshape(64, 128))
    gs, us = np.full((1, 1), 0.75, np.float32), np.full((1, 1), 1.25, np.float32)
    x = torch.linspace(-0.5, 0.5, steps=4 * 128).reshape(4, 128).numpy()
    ya, yb = ref_dual(lin, gate, gs, up, us, x, reuse=True)
    out.update(dual_a=gate, dual_sa=gs, dual_b=up, dual_sb=us, dual_x=x, dual_ya=ya, dual_yb=yb)
    # tests/test_native_fp8_linear.py:80-103 (MLP)
    hid, inter = 64, 32
    x = torch.linspace(-0.5, 0.5, steps=hid).reshape(1, hid).numpy()
    g = fp8_bytes(torch.linspace(-1.0, 1.0, steps=inter * hid).reshape(inter, hid))
    u = fp8_bytes(torch.linspace(1.0, -1.0, steps=inter * hid).reshape(inter, hid))
    d = fp8_bytes(torch.linspace(-0.75, 0.75, steps=hid * inter).reshape(hid, inter))
    gs, us, ds = np.array([[1.0]], np.float32), np.array([[0.75]], np.float32), np.array([[1.25]], np.float32)
    out.update(mlp_g=g, mlp_gs=gs, mlp_u=u, mlp_us=us, mlp_d=d, mlp_ds=ds, mlp_x=x,
               mlp_y=ref_mlp(lin, g, gs, u, us, d, ds, x))
    # tests/test_native_fp8_linear.py:106-139 (MLP batch reuse)
    gen = torch.Generator().manual_seed(777)
    x = (torch.randn((4, 128), generator=gen) * 0.25).numpy()
    g = fp8_bytes(torch.randn((128, 128), generator=gen) * 0.25)
    u = fp8_bytes(torch.randn((128, 128), generator=gen) * 0.25)
    d = fp8_bytes(torch.randn((128, 128), generator=gen) * 0.25)
    gs, us, ds = np.full((1, 1), 0.875, np.float32), np.full((1, 1), 1.125, np.float32), np.full((1, 1), 0.75, np.float32)
    out.update(mlpr_g=g, mlpr_gs=gs, mlpr_u=u, mlpr_us=us, mlpr_d=d, mlpr_ds=ds, mlpr_x=x,
               mlpr_y=ref_mlp(lin, g, gs, u, us, d, ds, x, reuse=True))
    # tests/test_native_fp8_linear.py:250-291 AVX-512 MLP inputs (scalar result = reference)
    gen = torch.Generator().manual_seed(555)
    x = (torch.randn((2, 256), generator=gen) * 0.25).numpy()
    g = fp8_bytes(torch.randn((384, 256), generator=gen) * 0.25)
    u = fp8_bytes(torch.randn((384, 256), generator=gen) * 0.25)
    d = fp8_bytes(torch.randn((256, 384), generator=gen) * 0.25)
    gs, us, ds = np.full((3, 2), 0.875, np.float32), np.full((3, 2), 1.125, np.float32), np.full((2, 3), 0.75, np.float32)
    out.update(mlpa_g=g, mlpa_gs=gs, mlpa_u=u, mlpa_us=us, mlpa_d=d, mlpa_ds=ds, mlpa_x=x,
               mlpa_y=ref_mlp(lin, g, gs, u, us, d, ds, x))
    # tests/test_native_fp8_linear.py:142-162 (weighted == sum route * many)
    hid, inter = 64, 32
    x = torch.linspace(-0.5, 0.5, steps=hid).reshape(1, hid).numpy()
    items = [mlp_item(seed, inter, hid) for seed in (1, 2, 3)]
    route = np.array([0.5, 0.3, 0.2], np.float32)
    pack_items("wt", items, out)
    out.update(wt_x=x, wt_route=route, wt_y=ref_weighted(lin, items, x, route, "fp8_e4m3_block_mlp_many_weighted_f32"),
               wt_many=ref_many(lin, items, x))
    # tests/test_native_fp8_linear.py:165-247 (row-weighted, pair-weighted)
    x = torch.linspace(-0.5, 0.5, steps=3 * hid).reshape(3, hid).numpy()
    items = [mlp_item(seed, inter, hid) for seed in (5, 6, 7, 8)]
    route = np.array([[0.6, 0.0, 0.4], [0.4, 0.5, 0.0], [0.0, 0.5, 0.35], [0.0, 0.0, 0.25]], np.float32)
    pack_items("rw", items, out)
    pi, pr, pw = [], [], []
    for it in range(route.shape[0]):
        for row in range(route.shape[1]):
            if route[it, row] != 0.0:
                pi.append(it)
                pr.append(row)
                pw.append(route[it, row])
    pi, pr, pw = np.array(pi, np.int64), np.array(pr, np.int64), np.array(pw, np.float32)
    out.update(rw_x=x, rw_route=route,
               rw_y=ref_weighted(lin, items, x, route, "fp8_e4m3_block_mlp_many_row_weighted_f32", reuse=True),
               rw_y_default=ref_weighted(lin, items, x, route, "fp8_e4m3_block_mlp_many_row_weighted_f32"),
               rw_many=ref_many(lin, items, x), rw_pi=pi, rw_pr=pr, rw_pw=pw,
               rw_pair=ref_pair(lin, items, x, pi, pr, pw))
    # tests/test_native_fp8_linear.py:250-270 (AVX-512 weighted inputs, 4 experts 128x128)
    x = torch.linspace(-0.5, 0.5, steps=128).reshape(1, 128).numpy()
    items = [mlp_item(seed, 128, 128, gsv=0.875, usv=1.125, dsv=0.75) for seed in (11, 22, 33, 44)]
    route = np.array([0.31, 0.17, 0.29, 0.23], np.float32)
    pack_items("wa", items, out)
    out.update(wa_x=x, wa_route=route, wa_y=ref_weighted(lin, items, x, route, "fp8_e4m3_block_mlp_many_weighted_f32"))
    # tests/test_native_ds_moe.py:19-32 (H=4, I=2, seeds 1, 2)
    x = np.array([[0.5, -0.25, 0.75, 1.0]], np.float32)
    items = [mlp_item(seed, 2, 4) for seed in (1, 2)]
    pack_items("ds", items, out)
    out.update(ds_x=x, ds_route=np.array([0.6, 0.4], np.float32), ds_many=ref_many(lin, items, x))
    # Seeded DeepSeek-shaped blocks: N(0, 0.02) weights, scales U(1e-3, 1e-2),
    # including partial 128-blocks and K not a multiple of 16.
    gen = torch.Generator().manual_seed(20261202)
    for name, (n, k, m) in {"big_a": (256, 2048, 3), "big_b": (300, 1040, 2), "big_c": (130, 520, 4),
                            "big_d": (128, 7168, 8)}.items():
        w = fp8_bytes(torch.randn((n, k), generator=gen) * 0.02)
        s = (torch.rand(((n + 127) // 128, (k + 127) // 128), generator=gen) * 9e-3 + 1e-3).numpy().astype(np.float32)
        x = torch.randn((m, k), generator=gen).to(torch.bfloat16).float().numpy()
        out.update({f"{name}_w": w, f"{name}_s": s, f"{name}_x": x, f"{name}_y": ref_linear(lin, w, s, x)})
    # A small MoE with DeepSeek-like scales: 6 experts, inter 256, hidden 256, M = 3.
    items = []
    for e in range(6):
        g = fp8_bytes(torch.randn((256, 256), generator=gen) * 0.02)
        u = fp8_bytes(torch.randn((256, 256), generator=gen) * 0.02)
        d = fp8_bytes(torch.randn((256, 256), generator=gen) * 0.02)
        gs = (torch.rand((2, 2), generator=gen) * 9e-3 + 1e-3).numpy().astype(np.float32) * 400
        us = (torch.rand((2, 2), generator=gen) * 9e-3 + 1e-3).numpy().astype(np.float32) * 400
        ds = (torch.rand((2, 2), generator=gen) * 9e-3 + 1e-3).numpy().astype(np.float32) * 400
        items.append((g, gs, u, us, d, ds))
    x = torch.randn((3, 256), generator=gen).to(torch.bfloat16).float().numpy()
    route = (torch.rand((6, 3), generator=gen) * (torch.rand((6, 3), generator=gen) > 0.4)).numpy().astype(np.float32)
    pack_items("moe", items, out)
    out.update(moe_x=x, moe_route=route,
               moe_y=ref_weighted(lin, items, x, route, "fp8_e4m3_block_mlp_many_row_weighted_f32"),
               moe_y1=ref_weighted(lin, items, x[:1], np.ascontiguousarray(route[:, 0]),
                                   "fp8_e4m3_block_mlp_many_weighted_f32"))
    _env(False)
    np.savez_compressed(HERE / "fp8_gemv.npz", **out)


# --------------------------------------------------------------------------- Q4 (torch closed forms)

def torch_quantize_q4(t: torch.Tensor):
    """The torch arithmetic of quantize_tensor_to_q4 (q4_quantize.py:48-71)."""
    work = t.detach().float()
    if work.ndim == 0:
        m = work.reshape(1, 1)
    elif work.ndim == 1:
        m = work.reshape(work.shape[0], 1)
    else:
        m = work.reshape(work.shape[0], -1)
    max_abs = m.abs().amax(dim=1)
    scales = torch.where(max_abs > 0, max_abs / 7.0, torch.ones_like(max_abs))
    q = torch.round(m / scales[:, None]).clamp(-7, 7).to(torch.int8).flatten()
    enc = torch.bitwise_and(q.to(torch.int16), 0x0F).to(torch.uint8)
    if enc.numel() % 2:
        enc = torch.cat([enc, torch.zeros((1,), dtype=torch.uint8)])
    packed = torch.bitwise_or(enc[0::2], torch.bitwise_left_shift(enc[1::2], 4))
    return packed.numpy(), scales.to(torch.float16).view(torch.int16).numpy().view(np.uint16), q.numpy()


def torch_q4_dequant(q: np.ndarray, scales_bits: np.ndarray, shape) -> np.ndarray:
    qt = torch.from_numpy(q.astype(np.int8)).to(torch.float32)
    s = torch.from_numpy(scales_bits.view(np.int16)).view(torch.float16).float()
    if not shape:
        m = qt.reshape(1, 1)
    elif len(shape) == 1:
        m = qt.reshape(shape[0], 1)
    else:
        m = qt.reshape(shape[0], -1)
    return (m * s.reshape(-1, 1)).to(torch.float16).reshape(-1).view(torch.int16).numpy().view(np.uint16)


def make_q4() -> None:
    out: dict[str, np.ndarray] = {}
    # tests/test_native_q4_dequant.py:16-44: 10 listed shapes + 90 seeded 2-D shapes, seed 1234
    shapes = [(), (1,), (7,), (1, 1), (1, 17), (2, 5), (3, 4), (8, 8), (5, 3, 2), (4, 7, 3)]
    gen = torch.Generator().manual_seed(1234)
    tensors = [torch.randn(s, generator=gen, dtype=torch.float16) for s in shapes]
    for i in range(90):
        tensors.append(torch.randn((1 + (i % 9), 1 + ((i * 7) % 37)), generator=gen, dtype=torch.float16))
    # Plus Qwen-like rows (K a multiple of 32) and an odd-K wide case.
    tensors.append(torch.randn((48, 3584), generator=gen, dtype=torch.float16) * 0.02)
    tensors.append(torch.randn((20, 1001), generator=gen, dtype=torch.float16))
    for i, t in enumerate(tensors):
        packed, scales, q = torch_quantize_q4(t)
        out[f"t{i}_in"] = t.view(torch.int16).numpy().view(np.uint16)
        out[f"t{i}_shape"] = np.array(list(t.shape), np.int64)
        out[f"t{i}_packed"] = packed
        out[f"t{i}_scales"] = scales
        out[f"t{i}_deq"] = torch_q4_dequant(q, scales, list(t.shape))
    out["count"] = np.array(len(tensors))
    # tests/test_q4_quantizer.py:28-34 pack/unpack KAT
    out["kat_values"] = np.array([-7, -6, -1, 0, 1, 6, 7], np.int8)
    # tests/test_q4_quantizer.py:53-93: Q4 SwiGLU MoE, seed 123, H=16, I=12, S=2
    torch.manual_seed(123)
    H, I, S = 16, 12, 2
    hidden = torch.randn((1, H), dtype=torch.float16)
    route = torch.tensor([0.7, 0.3], dtype=torch.float32)
    expected = torch.zeros((1, H), dtype=torch.float32)
    for e in range(S):
        gate = torch.randn((I, H), dtype=torch.float16)
        up = torch.randn((I, H), dtype=torch.float16)
        down = torch.randn((H, I), dtype=torch.float16)
        deq = []
        for name, w in (("g", gate), ("u", up), ("d", down)):
            packed, scales, q = torch_quantize_q4(w)
            out[f"moe_{name}{e}_packed"] = packed
            out[f"moe_{name}{e}_scales"] = scales
            deq.append(torch.from_numpy(torch_q4_dequant(q, scales, list(w.shape)).view(np.int16)).view(torch.float16)
                       .reshape(w.shape))
        act = torch.nn.functional.silu(hidden.float() @ deq[0].float().T) * (hidden.float() @ deq[1].float().T)
        expected = expected + (act @ deq[2].float().T) * route[e]
    out["moe_hidden"] = hidden.view(torch.int16).numpy().view(np.uint16)
    out["moe_route"] = route.numpy()
    out["moe_expected_f32"] = expected.numpy()
    np.savez_compressed(HERE / "q4.npz", **out)


# --------------------------------------------------------------------------- row8 (reference C++ + torch.mv)

def make_row8(row8) -> None:
    out: dict[str, np.ndarray] = {}
    # tests/test_packed_weight_artifact.py:16-21 (arange(130) as 10 x 13)
    for dt_name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        t = torch.arange(130, dtype=torch.float32).reshape(10, 13).to(dt).view(torch.int16).numpy().view(np.uint16)
        packed = np.empty((2 * 13 * 8,), np.uint16)
        assert row8.native_pack_u16_rows8(vp(t), vp(packed), I64(10), I64(13)) == 0
        out[f"pack_{dt_name}_w"] = t
        out[f"pack_{dt_name}_packed"] = packed
    # tests/test_native_fp16_packed_gemv.py:7-19, seed 20260504
    torch.manual_seed(20260504)
    cases = []
    for code, dt in ((0, torch.float16), (1, torch.bfloat16)):
        for rows, cols in ((1, 7), (8, 16), (17, 31), (32, 64)):
            hidden = (torch.randn((cols,), dtype=torch.float32) * 0.2).to(dt)
            weight = (torch.randn((rows, cols), dtype=torch.float32) * 0.2).to(dt)
            h = hidden.view(torch.int16).numpy().view(np.uint16)
            w = weight.view(torch.int16).numpy().view(np.uint16)
            packed = np.empty((((rows + 7) // 8) * cols * 8,), np.uint16)
            assert row8.native_pack_u16_rows8(vp(w), vp(packed), I64(rows), I64(cols)) == 0
            y = np.empty((rows,), np.float32)
            assert row8.native_packed_gemv_rows8(vp(h), vp(packed), vp(y), I64(rows), I64(cols), ctypes.c_int(code)) == 0
            key = f"g{len(cases)}"
            out.update({f"{key}_h": h, f"{key}_w": w, f"{key}_packed": packed, f"{key}_y": y,
                        f"{key}_mv": torch.mv(weight.float(), hidden.float()).numpy(), f"{key}_code": np.array(code)})
            cases.append(key)
    # Larger seeded cases (Qwen-like widths) through the reference C++.
    gen = torch.Generator().manual_seed(20261203)
    for code, dt in ((0, torch.float16), (1, torch.bfloat16)):
        for rows, cols in ((77, 3584), (64, 1024)):
            hidden = torch.randn((cols,), generator=gen).to(dt)
            weight = (torch.randn((rows, cols), generator=gen) * 0.02).to(dt)
            h = hidden.view(torch.int16).numpy().view(np.uint16)
            w = weight.view(torch.int16).numpy().view(np.uint16)
            packed = np.empty((((rows + 7) // 8) * cols * 8,), np.uint16)
            assert row8.native_pack_u16_rows8(vp(w), vp(packed), I64(rows), I64(cols)) == 0
            y = np.empty((rows,), np.float32)
            assert row8.native_packed_gemv_rows8(vp(h), vp(packed), vp(y), I64(rows), I64(cols), ctypes.c_int(code)) == 0
            key = f"g{len(cases)}"
            out.update({f"{key}_h": h, f"{key}_w": w, f"{key}_y": y,
                        f"{key}_mv": torch.mv(weight.float(), hidden.float()).numpy(), f"{key}_code": np.array(code)})
            cases.append(key)
    out["cases"] = np.array(cases)
    np.savez_compressed(HERE / "row8.npz", **out)


# --------------------------------------------------------------------------- routers

def make_router() -> None:
    out: dict[str, np.ndarray] = {}
    # tests/test_native_ds_router.py:8-18: seed 20260519, router 11 x 16, 5 hidden rows, k=4.
    gen = torch.Generator().manual_seed(20260519)
    router = torch.randn((11, 16), generator=gen, dtype=torch.float32).mul(0.25).to(torch.float16)
    hidden = torch.randn((5, 16), generator=gen, dtype=torch.float32).mul(0.5).to(torch.float16)
    out["softmax_router"] = router.view(torch.int16).numpy().view(np.uint16)
    out["softmax_hidden"] = hidden.view(torch.int16).numpy().view(np.uint16)
    # Closed form in float64: softmax over fp32 scores, top-4, renormalised.
    ids, wts = [], []
    for row in hidden:
        scores = (router.double() @ row.double())
        p = torch.softmax(scores, dim=0)
        top = torch.topk(p, 4)
        ids.append(top.indices.numpy())
        wts.append((top.values / top.values.sum()).numpy())
    out["softmax_ids"] = np.stack(ids).astype(np.int64)
    out["softmax_weights"] = np.stack(wts).astype(np.float64)
    # tests/test_runtime_fp8_source.py:772-784 with the fixture of 1740-1800:
    # hidden ones(1,4), gate rows [4,4,4,4] and [0,0,0,0], bias [-20, 0],
    # sigmoid, n_group 1, top-1, routed_scaling_factor 2.5 -> expert 1, 2.5.
    out["ds_kat_logits"] = np.array([[16.0, 0.0]], np.float32)
    out["ds_kat_bias"] = np.array([-20.0, 0.0], np.float32)
    out["ds_kat_ids"] = np.array([[1]], np.int64)
    out["ds_kat_weights"] = np.array([[2.5]], np.float32)
    np.savez_compressed(HERE / "router.npz", **out)


def main() -> int:
    if not (REF / "libref_fp8_linear.so").exists():
        print("oracle/_ref is not built: run `make -C oracle ref` (needs the reference sources)", file=sys.stderr)
        return 1
    lin, row8 = _load_ref()
    make_fp8_dequant()
    make_fp8_gemv(lin)
    make_q4()
    make_row8(row8)
    make_router()
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")
    return 0


if __name__ == "__main__":
    sys.exit(main())

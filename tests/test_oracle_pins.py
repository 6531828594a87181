"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against something it was not derived
from: the golden vectors (the reference's own C++ compiled from source, or
torch closed forms the reference's tests themselves use), the live
reference build in oracle/_ref when present, closed forms and invariants.
The last tests plant plausible mistakes in copies of the oracle's numpy-level
arithmetic and show the pins catch them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import items_from, rel_l2


# --------------------------------------------------------------------------- e4m3 and conversions

def test_e4m3_dequant_decode_matches_torch_for_all_bytes(oracle_mod, golden):
    expected = golden("fp8_dequant")["e4m3_f32_bits"]
    got = np.array([oracle_mod.e4m3_dequant_bits(b) for b in range(256)], dtype=np.uint32)
    assert np.array_equal(got, expected)
    assert got[0x7F] == 0x7FF00000 and got[0xFF] == 0xFFF00000


def test_e4m3_linear_decode_closed_form(oracle_mod):
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e, m = (b >> 3) & 0xF, b & 7
        if e == 0xF and m == 7:
            want = 0.0  # NaN bytes contribute zero in the GEMV kernels
        elif e == 0:
            want = s * m * 2.0 ** -9
        else:
            want = s * (1 + m / 8) * 2.0 ** (e - 7)
        got = oracle_mod.e4m3_linear(b)
        assert got == want and math.copysign(1, got) == math.copysign(1, want) or (want == 0 and got == 0)
    assert oracle_mod.e4m3_linear(0x7E) == 448.0 and oracle_mod.e4m3_linear(0x01) == 2.0 ** -9


def test_f16_conversion_matches_numpy_rne_and_f16c_nan(oracle_mod):
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 4000),
        np.array([65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0, -0.0,
                  np.inf, -np.inf, 5.960464477539063e-08, 6.097555160522461e-05], np.float32),
    ])
    got = oracle_mod.f32_to_f16_hw(vals)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    nan_bits = np.array([0x7FF00000, 0xFFF00000, 0x7FC00000, 0x7F800001], np.uint32).view(np.float32)
    torch_bits = torch.from_numpy(nan_bits.copy()).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle_mod.f32_to_f16_hw(nan_bits)[:2], torch_bits[:2])


def test_bf16_conversion_matches_torch(oracle_mod):
    rng = np.random.default_rng(6)
    vals = rng.standard_normal(5000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 5000)
    vals = np.concatenate([vals, np.array([np.inf, -np.inf, 3.3895313892515355e38, 0.0, -0.0], np.float32)])
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle_mod.f32_to_bf16(vals), want)


# --------------------------------------------------------------------------- FP8 dequant

@pytest.mark.parametrize("out", ["f32", "f16", "bf16"])
def test_fp8_dequant_matches_torch_golden(oracle_mod, golden, out):
    g = golden("fp8_dequant")
    for case in g["cases"]:
        w, s = g[f"{case}_w"], g[f"{case}_s"]
        got = oracle_mod.fp8_dequant(w, s, out)
        if out == "f32":
            got = got.view(np.uint32)
        assert np.array_equal(got, g[f"{case}_{out}"]), case


# --------------------------------------------------------------------------- FP8 GEMV family vs reference C++

def test_fp8_linear_matches_reference_build(oracle_mod, golden):
    g = golden("fp8_gemv")
    assert np.array_equal(oracle_mod.fp8_linear(g["lin_w"], g["lin_s"], g["lin_x"]), g["lin_y"])
    for name in ("big_a", "big_b", "big_c", "big_d"):
        assert np.array_equal(oracle_mod.fp8_linear(g[f"{name}_w"], g[f"{name}_s"], g[f"{name}_x"]), g[f"{name}_y"]), name


def test_fp8_linear_matches_fp64_closed_form(oracle_mod, golden):
    g = golden("fp8_gemv")
    for name in ("lin", "big_a", "big_b", "big_c", "big_d"):
        w, s, x = g[f"{name}_w"], g[f"{name}_s"], g[f"{name}_x"]
        deq = torch.from_numpy(w).view(torch.float8_e4m3fn).double()
        sc = torch.from_numpy(s).double().repeat_interleave(128, 0).repeat_interleave(128, 1)[: w.shape[0], : w.shape[1]]
        want = (torch.from_numpy(x).double() @ (deq * sc).T).numpy()
        assert rel_l2(oracle_mod.fp8_linear(w, s, x), want) < 1e-6, name


def test_fp8_batch_reuse_is_bit_exact_to_rows(oracle_mod, golden):
    g = golden("fp8_gemv")
    w, s, x = g["reuse_w"], g["reuse_s"], g["reuse_x"]
    batch = oracle_mod.fp8_linear(w, s, x, batch_reuse=True)
    assert np.array_equal(batch, g["reuse_y"])
    assert np.array_equal(batch, g["reuse_y_rows"])
    assert np.array_equal(batch, oracle_mod.fp8_linear(w, s, x, batch_reuse=False))


def test_fp8_dual_and_mlp_match_reference_build(oracle_mod, golden):
    g = golden("fp8_gemv")
    ya, yb = oracle_mod.fp8_dual_linear(g["dual_a"], g["dual_sa"], g["dual_b"], g["dual_sb"], g["dual_x"])
    assert np.array_equal(ya, g["dual_ya"]) and np.array_equal(yb, g["dual_yb"])
    for p in ("mlp", "mlpr", "mlpa"):
        got = oracle_mod.fp8_mlp(*(g[f"{p}_{k}"] for k in ("g", "gs", "u", "us", "d", "ds", "x")))
        assert np.array_equal(got, g[f"{p}_y"]), p


def test_fp8_moe_family_matches_reference_build(oracle_mod, golden):
    g = golden("fp8_gemv")
    wt = items_from(g, "wt")
    assert np.array_equal(oracle_mod.fp8_mlp_many(wt, g["wt_x"]), g["wt_many"])
    assert np.array_equal(oracle_mod.fp8_mlp_many_weighted(wt, g["wt_x"], g["wt_route"]), g["wt_y"])
    rw = items_from(g, "rw")
    assert np.array_equal(oracle_mod.fp8_mlp_many(rw, g["rw_x"]), g["rw_many"])
    row = oracle_mod.fp8_mlp_many_row_weighted(rw, g["rw_x"], g["rw_route"])
    assert np.array_equal(row, g["rw_y"]) and np.array_equal(row, g["rw_y_default"])
    pair = oracle_mod.fp8_mlp_many_pair_weighted(rw, g["rw_x"], g["rw_pi"], g["rw_pr"], g["rw_pw"])
    assert np.array_equal(pair, g["rw_pair"])
    assert np.array_equal(pair, row)  # pair == row-weighted, bit for bit
    wa = items_from(g, "wa")
    assert np.array_equal(oracle_mod.fp8_mlp_many_weighted(wa, g["wa_x"], g["wa_route"]), g["wa_y"])
    moe = items_from(g, "moe")
    assert np.array_equal(oracle_mod.fp8_mlp_many_row_weighted(moe, g["moe_x"], g["moe_route"]), g["moe_y"])
    assert np.array_equal(oracle_mod.fp8_mlp_many_weighted(moe, g["moe_x"][:1], g["moe_route"][:, 0]), g["moe_y1"])


def test_weighted_equals_route_sum_of_many(oracle_mod, golden):
    g = golden("fp8_gemv")
    wt = items_from(g, "wt")
    many = oracle_mod.fp8_mlp_many(wt, g["wt_x"])
    want = (many.astype(np.float64) * g["wt_route"].astype(np.float64)[:, None, None]).sum(0)
    assert np.allclose(oracle_mod.fp8_mlp_many_weighted(wt, g["wt_x"], g["wt_route"]), want, atol=1e-5, rtol=1e-5)
    # ds_moe KAT (tests/test_native_ds_moe.py:6-16)
    outs = np.array([[[1, 2, 3, 4]], [[10, 20, 30, 40]]], np.float32)
    got = oracle_mod.ds_moe_combine(outs, np.array([0.75, 0.25], np.float32))
    assert np.array_equal(got, np.array([[3.25, 6.5, 9.75, 13.0]], np.float32))


def test_mlp_matches_fp64_swiglu_closed_form(oracle_mod, golden):
    g = golden("fp8_gemv")

    def deq(w, s):
        d = torch.from_numpy(w).view(torch.float8_e4m3fn).double()
        sc = torch.from_numpy(s).double().repeat_interleave(128, 0).repeat_interleave(128, 1)[: w.shape[0], : w.shape[1]]
        return d * sc

    for p in ("mlp", "mlpr", "mlpa"):
        x = torch.from_numpy(g[f"{p}_x"]).double()
        gate = x @ deq(g[f"{p}_g"], g[f"{p}_gs"]).T
        up = x @ deq(g[f"{p}_u"], g[f"{p}_us"]).T
        want = ((gate * torch.sigmoid(gate)) * up) @ deq(g[f"{p}_d"], g[f"{p}_ds"]).T
        assert rel_l2(g[f"{p}_y"], want.numpy()) < 1e-5, p


def test_live_reference_build_agrees(oracle_mod, golden):
    from pathlib import Path
    import ctypes

    so = Path(oracle_mod.__file__).parent / "_ref" / "libref_fp8_linear.so"
    if not so.exists():
        pytest.skip("oracle/_ref not built")
    ref = ctypes.CDLL(str(so))
    g = golden("fp8_gemv")
    w, s, x = g["big_b_w"], g["big_b_s"], g["big_b_x"]
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    code = ref.fp8_e4m3_block_linear_f32(ctypes.c_void_p(w.ctypes.data), ctypes.c_void_p(s.ctypes.data),
                                         ctypes.c_void_p(x.ctypes.data), ctypes.c_void_p(out.ctypes.data),
                                         ctypes.c_longlong(x.shape[0]), ctypes.c_longlong(w.shape[0]),
                                         ctypes.c_longlong(w.shape[1]), ctypes.c_longlong((w.shape[1] + 127) // 128))
    assert code == 0
    assert np.array_equal(out, oracle_mod.fp8_linear(w, s, x))


# --------------------------------------------------------------------------- Q4

def test_q4_quantizer_and_dequant_match_torch(oracle_mod, golden):
    g = golden("q4")
    for i in range(int(g["count"])):
        t = g[f"t{i}_in"].view(np.float16).astype(np.float32).reshape(tuple(g[f"t{i}_shape"]))
        packed, scales, shape = oracle_mod.q4_quantize(t)
        assert np.array_equal(packed, g[f"t{i}_packed"]), i
        assert np.array_equal(scales, g[f"t{i}_scales"]), i
        ch, cs = oracle_mod.q4_shape_params(shape)
        deq = oracle_mod.q4_dequant_f16(packed, scales, ch, cs)
        assert np.array_equal(deq, g[f"t{i}_deq"]), i


def test_q4_pack_unpack_kat(oracle_mod, golden):
    v = golden("q4")["kat_values"]
    packed = oracle_mod.pack_int4(v)
    assert packed.tolist() == [0xA9, 0x0F, 0x61, 0x07]
    assert oracle_mod.unpack_int4(packed, v.size).tolist() == v.tolist()


def test_q4_grid_round_trip(oracle_mod):
    t = np.array([[-7.0, -3.0, 0.0, 3.0, 7.0], [-14.0, -6.0, 0.0, 6.0, 14.0]], np.float32)
    packed, scales, shape = oracle_mod.q4_quantize(t)
    deq = oracle_mod.q4_dequant_f16(packed, scales, 2, 5).view(np.float16).astype(np.float32).reshape(2, 5)
    rel = np.abs(deq - t) / np.maximum(np.abs(t), 1e-6)
    assert rel.max() < 0.02


def _q4_moe_inputs(g):
    experts = []
    for e in range(2):
        experts.append(tuple(g[f"moe_{n}{e}_{k}"] for n in ("g", "u", "d") for k in ("packed", "scales")))
    return experts


def test_q4_moe_matches_dequant_closed_form(oracle_mod, golden):
    g = golden("q4")
    out = oracle_mod.q4_moe_selected(g["moe_hidden"], _q4_moe_inputs(g), g["moe_route"], 16, 12)
    got = out.view(np.float16).astype(np.float32)
    want = g["moe_expected_f32"].reshape(-1)
    assert np.allclose(got, want.astype(np.float16).astype(np.float32), atol=1e-2, rtol=1e-2)
    assert rel_l2(got, want) < 2e-3  # fp16 output rounding


def test_q4_gemv_matches_fp64(oracle_mod, golden):
    g = golden("q4")
    i = int(g["count"]) - 2  # the 48 x 3584 case
    shape = tuple(g[f"t{i}_shape"])
    q = oracle_mod.unpack_int4(g[f"t{i}_packed"], int(np.prod(shape))).astype(np.float64).reshape(shape)
    s = g[f"t{i}_scales"].view(np.float16).astype(np.float64)
    x = np.random.default_rng(3).standard_normal(shape[1]).astype(np.float32)
    want = (q * s[:, None]) @ x.astype(np.float64)
    got = oracle_mod.q4_gemv(g[f"t{i}_packed"], g[f"t{i}_scales"], x, shape[0], shape[1])
    assert rel_l2(got, want) < 1e-6


# --------------------------------------------------------------------------- row8

def test_row8_pack_matches_reference_and_round_trips(oracle_mod, golden):
    g = golden("row8")
    for dt in ("f16", "bf16"):
        w = g[f"pack_{dt}_w"]
        packed = oracle_mod.pack_rows8(w)
        assert np.array_equal(packed, g[f"pack_{dt}_packed"])
        assert np.array_equal(oracle_mod.unpack_rows8(packed, 10, 13), w)


def test_row8_gemv_matches_reference_build_and_torch_mv(oracle_mod, golden):
    g = golden("row8")
    for key in g["cases"]:
        w, h, code = g[f"{key}_w"], g[f"{key}_h"], int(g[f"{key}_code"])
        rows, cols = w.shape
        y = oracle_mod.packed_gemv_rows8(h, oracle_mod.pack_rows8(w), rows, cols, code)
        assert np.array_equal(y, g[f"{key}_y"]), key
        assert np.allclose(y, g[f"{key}_mv"], atol=1e-4, rtol=1e-4), key


def test_row8_f32_hidden_pinned_to_reference_build_and_fp64(oracle_mod, golden):
    # With x holding exactly the fp16 / bf16 values of the reference build's
    # cases, the fp32-activation chain is the same fma chain: bit-exact to
    # the reference's outputs.
    g = golden("row8")
    for key in g["cases"]:
        w, h, code = g[f"{key}_w"], g[f"{key}_h"], int(g[f"{key}_code"])
        rows, cols = w.shape
        hf = (h.astype(np.uint32) << 16).view(np.float32) if code else h.view(np.float16).astype(np.float32)
        y = oracle_mod.packed_gemv_rows8_f32_hidden(hf, oracle_mod.pack_rows8(w), rows, cols, code)
        assert np.array_equal(y, g[f"{key}_y"]), key
    # Arbitrary fp32 activations against the fp64 product.
    rng = np.random.default_rng(31)
    w = (rng.standard_normal((37, 300)) * 0.05).astype(np.float16)
    x = rng.standard_normal(300).astype(np.float32)
    y = oracle_mod.packed_gemv_rows8_f32_hidden(x, oracle_mod.pack_rows8(w.view(np.uint16)), 37, 300, 0)
    want = w.astype(np.float64) @ x.astype(np.float64)
    assert np.abs(y - want).max() < 1e-5 * np.abs(want).max()
    # A planted transposed block order must fail the closed form.
    bad = oracle_mod.pack_rows8(w.view(np.uint16)).reshape(-1, 300, 8)[::-1].reshape(-1)
    y_bad = oracle_mod.packed_gemv_rows8_f32_hidden(x, bad, 37, 300, 0)
    assert np.abs(y_bad - want).max() > 1e-2 * np.abs(want).max()


# --------------------------------------------------------------------------- routers

def test_softmax_router_matches_fp64_closed_form(oracle_mod, golden):
    g = golden("router")
    for i, h in enumerate(g["softmax_hidden"]):
        ids, w = oracle_mod.router_topk_u16(h, g["softmax_router"], 4, 0)
        assert ids.tolist() == g["softmax_ids"][i].tolist()
        assert np.allclose(w, g["softmax_weights"][i], atol=1e-6, rtol=1e-6)


def test_deepseek_route_kat_and_invariants(oracle_mod, golden):
    g = golden("router")
    idx, w = oracle_mod.deepseek_route(g["ds_kat_logits"], top_k=1, n_groups=1, topk_groups=1, route_scale=2.5,
                                       bias=g["ds_kat_bias"])
    assert idx.tolist() == g["ds_kat_ids"].tolist() and np.array_equal(w, g["ds_kat_weights"])
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((6, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    idx, w = oracle_mod.deepseek_route(logits, bias=bias)
    scores = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    for r in range(6):
        choice = scores[r] + bias
        groups = choice.reshape(8, 32)
        gsc = np.sort(groups, axis=1)[:, -2:].sum(1)
        kept = set(np.argsort(-gsc, kind="stable")[:4].tolist())
        assert {int(i) // 32 for i in idx[r]} <= kept
        allowed = np.concatenate([np.arange(gi * 32, gi * 32 + 32) for gi in sorted(kept)])
        best = allowed[np.argsort(-choice[allowed], kind="stable")[:8]]
        assert sorted(best.tolist()) == sorted(idx[r].tolist())
        want = scores[r][idx[r]] / scores[r][idx[r]].sum() * 2.5
        assert np.allclose(w[r], want, rtol=8e-3)  # bf16 rounding
        assert abs(float(w[r].sum()) - 2.5) < 0.05


# --------------------------------------------------------------------------- planted mistakes

def _numpy_linear(w, s, x, *, transpose_scale=False, drop_scale=False, nan_as_nan=False):
    deq = torch.from_numpy(w).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    if not nan_as_nan:
        deq = np.nan_to_num(deq, nan=0.0)
    sg = s.T if transpose_scale else s
    sc = np.repeat(np.repeat(sg, 128, 0), 128, 1)[: w.shape[0], : w.shape[1]]
    if drop_scale:
        sc = np.ones_like(sc)
    return x.astype(np.float64) @ (deq * sc).T


def test_pins_catch_planted_mistakes(golden):
    g = golden("fp8_gemv")
    w, s, x, y = g["big_a_w"], g["big_a_s"], g["big_a_x"], g["big_a_y"]
    assert rel_l2(_numpy_linear(w, s, x), y) < 1e-6
    assert rel_l2(_numpy_linear(w, s, x, drop_scale=True), y) > 1e-3
    # a transposed scale grid (the 256 x 2048 case has a 2 x 16 grid)
    s_sq = np.ascontiguousarray(np.tile(s, (8, 1))[:16, :16])
    w_sq = np.ascontiguousarray(np.tile(w, (8, 1))[:2048, :2048])
    good = _numpy_linear(w_sq, s_sq, x[:, :2048])
    assert rel_l2(_numpy_linear(w_sq, s_sq, x[:, :2048], transpose_scale=True), good) > 1e-3
    # NaN bytes must contribute zero, not NaN
    w_nan = w.copy()
    w_nan[3, 17] = 0x7F
    assert np.isnan(_numpy_linear(w_nan, s, x, nan_as_nan=True)[:, 3]).all()
    assert np.isfinite(_numpy_linear(w_nan, s, x)).all()

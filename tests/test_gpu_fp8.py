"""FP8 block-scaled dequant / GEMV / MLP / MoE on the GPU against the oracle
and the golden vectors (reference C++ outputs, torch closed forms).

Bars: dequant bit-exact; GEMV / MLP / MoE outputs within rel-L2 1e-5 (the
north-star bar is 1e-3); batched calls bit-exact to per-row calls; pair ==
row-weighted bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import items_from, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_fp8_linear_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def host(t):
    """Device tensor -> numpy; bf16 / uint16 come back as their 16-bit patterns."""
    torch.cuda.synchronize()
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.uint16):
        t = t.view(torch.int16)
    return t.numpy()


def cuda_items(items):
    return [tuple(dev(a) for a in it) for it in items]


def synth_fp8(rows, cols, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn((rows, cols), generator=g) * std).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    s = (torch.rand(((rows + 127) // 128, (cols + 127) // 128), generator=g) * 9e-3 + 1e-3).numpy().astype(np.float32)
    return w, s


def synth_x(m, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((m, k), generator=g).to(torch.bfloat16).float().numpy()


# --------------------------------------------------------------------------- dequant

@pytest.mark.parametrize("out", ["f32", "f16", "bf16"])
def test_dequant_golden_bit_exact(nat, golden, out):
    g = golden("fp8_dequant")
    fn = {"f32": nat.fp8_e4m3_dequant_to_f32, "f16": nat.fp8_e4m3_dequant_to_fp16,
          "bf16": nat.fp8_e4m3_dequant_to_bf16}[out]
    for case in g["cases"]:
        print("dequant", out, case, flush=True)
        got = host(fn(dev(g[f"{case}_w"]), dev(g[f"{case}_s"])))
        bits = got.view(np.uint32) if out == "f32" else got.view(np.uint16)
        assert np.array_equal(bits, g[f"{case}_{out}"]), case


def test_dequant_full_size_bit_exact(nat, oracle_mod):
    w, s = synth_fp8(2048, 7168, 101, std=0.3)
    w[::97, ::89] = 0x7F  # NaN bytes across many blocks
    w[5, :256] = np.arange(256, dtype=np.uint8)
    dw, ds = dev(w), dev(s)
    for out, fn in (("f32", nat.fp8_e4m3_dequant_to_f32), ("f16", nat.fp8_e4m3_dequant_to_fp16),
                    ("bf16", nat.fp8_e4m3_dequant_to_bf16)):
        got = host(fn(dw, ds))
        want = oracle_mod.fp8_dequant(w, s, out)
        width = np.uint32 if out == "f32" else np.uint16
        assert np.array_equal(got.view(width), want.view(width)), out


def test_dequant_dispatcher_and_errors(nat):
    w, s = synth_fp8(256, 384, 7)
    out = nat.dequantize_fp8_block_scaled(dev(w), dev(s), dtype=torch.float32)
    assert out.dtype == torch.float32 and out.is_cuda
    half = nat.dequantize_fp8_block_scaled(dev(w).view(torch.float8_e4m3fn), dev(s), dtype=torch.float16)
    assert torch.equal(half, out.to(torch.float16))
    with pytest.raises(ValueError, match="128x128 block layout"):
        nat.fp8_e4m3_dequant_to_fp16(torch.zeros((256, 256), dtype=torch.uint8, device="cuda"),
                                     torch.ones((1, 1), device="cuda"))
    # CPU inputs still work (copied through) and come back on the CPU
    cpu = nat.fp8_e4m3_dequant_to_fp16(torch.from_numpy(w), torch.from_numpy(s))
    assert cpu.device.type == "cpu" and torch.equal(cpu, half.cpu())


# --------------------------------------------------------------------------- linear / dual

def test_linear_golden(nat, golden):
    g = golden("fp8_gemv")
    for name in ("lin", "big_a", "big_b", "big_c", "big_d"):
        print("linear", name, flush=True)
        y = host(nat.fp8_e4m3_block_linear_f32(dev(g[f"{name}_w"]), dev(g[f"{name}_s"]), dev(g[f"{name}_x"])))
        assert rel_l2(y, g[f"{name}_y"]) < TOL, name
        assert np.allclose(y, g[f"{name}_y"], atol=1e-5, rtol=1e-5), name


def test_linear_batch_is_bit_exact_to_rows(nat, golden):
    g = golden("fp8_gemv")
    for name in ("reuse", "big_a", "big_b", "big_d"):
        w, s, x = dev(g[f"{name}_w"]), dev(g[f"{name}_s"]), dev(g[f"{name}_x"])
        batch = nat.fp8_e4m3_block_linear_f32(w, s, x)
        rows = torch.cat([nat.fp8_e4m3_block_linear_f32(w, s, x[i:i + 1]) for i in range(x.shape[0])])
        assert torch.equal(batch, rows), name
    assert rel_l2(host(batch), g["big_d_y"]) < TOL


def test_linear_nan_bytes_contribute_zero(nat, oracle_mod):
    w, s = synth_fp8(256, 2048, 9)
    w[7, 100] = 0x7F
    w[40, 1500] = 0xFF
    w[200, :16] = 0x7F
    x = synth_x(3, 2048, 10)
    y = host(nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), dev(x)))
    assert np.isfinite(y).all()
    assert rel_l2(y, oracle_mod.fp8_linear(w, s, x)) < TOL


def test_dual_golden_and_equal_to_two_linears(nat, golden):
    g = golden("fp8_gemv")
    a, sa, b, sb, x = (dev(g[k]) for k in ("dual_a", "dual_sa", "dual_b", "dual_sb", "dual_x"))
    ya, yb = nat.fp8_e4m3_block_dual_linear_f32(a, sa, b, sb, x)
    assert rel_l2(host(ya), g["dual_ya"]) < TOL and rel_l2(host(yb), g["dual_yb"]) < TOL
    assert torch.equal(ya, nat.fp8_e4m3_block_linear_f32(a, sa, x))
    assert torch.equal(yb, nat.fp8_e4m3_block_linear_f32(b, sb, x))


@pytest.mark.parametrize("shape", [(2048, 7168), (1536, 7168), (576, 7168), (7168, 16384), (7168, 2048)])
@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_deepseek_shapes_vs_oracle(nat, oracle_mod, shape, m):
    n, k = shape
    print("deepseek shape", shape, "M", m, flush=True)
    w, s = synth_fp8(n, k, 1000 + n + k)
    x = synth_x(m, k, 77 + m)
    dw, ds, dx = dev(w), dev(s), dev(x)
    y = nat.fp8_e4m3_block_linear_f32(dw, ds, dx)
    assert rel_l2(host(y), oracle_mod.fp8_linear(w, s, x)) < TOL
    if m > 1:
        rows = torch.cat([nat.fp8_e4m3_block_linear_f32(dw, ds, dx[i:i + 1]) for i in range(m)])
        assert torch.equal(y, rows)


def test_linear_batch_above_eight_rows(nat, oracle_mod):
    w, s = synth_fp8(384, 1024, 21)
    x = synth_x(11, 1024, 22)
    y = nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), dev(x))
    assert rel_l2(host(y), oracle_mod.fp8_linear(w, s, x)) < TOL
    assert torch.equal(y[9:10], nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), dev(x[9:10])))


# --------------------------------------------------------------------------- MLP

def test_mlp_golden_and_batch_rows(nat, golden):
    g = golden("fp8_gemv")
    for p in ("mlp", "mlpr", "mlpa"):
        args = [dev(g[f"{p}_{k}"]) for k in ("g", "gs", "u", "us", "d", "ds", "x")]
        y = nat.fp8_e4m3_block_mlp_f32(*args)
        assert rel_l2(host(y), g[f"{p}_y"]) < TOL, p
        y512 = nat.fp8_e4m3_block_mlp_avx512_f32(*args)
        assert torch.equal(y, y512)
        if args[-1].shape[0] > 1:
            rows = torch.cat([nat.fp8_e4m3_block_mlp_f32(*args[:-1], args[-1][i:i + 1])
                              for i in range(args[-1].shape[0])])
            assert torch.equal(y, rows), p


def test_shared_expert_shape_vs_oracle(nat, oracle_mod):
    g, gs = synth_fp8(2048, 7168, 31)
    u, us = synth_fp8(2048, 7168, 32)
    d, ds = synth_fp8(7168, 2048, 33)
    x = synth_x(2, 7168, 34)
    y = nat.fp8_e4m3_block_mlp_f32(*(dev(a) for a in (g, gs, u, us, d, ds, x)))
    assert rel_l2(host(y), oracle_mod.fp8_mlp(g, gs, u, us, d, ds, x)) < TOL


# --------------------------------------------------------------------------- many-expert MoE

def test_moe_family_golden(nat, golden):
    g = golden("fp8_gemv")
    wt = cuda_items(items_from(g, "wt"))
    many = nat.fp8_e4m3_block_mlp_many_f32(wt, dev(g["wt_x"]))
    assert rel_l2(host(many), g["wt_many"]) < TOL
    y = nat.fp8_e4m3_block_mlp_many_weighted_f32(wt, dev(g["wt_x"]), dev(g["wt_route"]))
    assert rel_l2(host(y), g["wt_y"]) < TOL
    want = (host(many).astype(np.float64) * g["wt_route"][:, None, None]).sum(0)
    assert np.allclose(host(y), want, atol=1e-5, rtol=1e-5)
    rw = cuda_items(items_from(g, "rw"))
    row = nat.fp8_e4m3_block_mlp_many_row_weighted_f32(rw, dev(g["rw_x"]), dev(g["rw_route"]))
    assert rel_l2(host(row), g["rw_y"]) < TOL
    pair = nat.fp8_e4m3_block_mlp_many_pair_weighted_f32(rw, dev(g["rw_x"]), dev(g["rw_pi"]), dev(g["rw_pr"]),
                                                         dev(g["rw_pw"]))
    assert torch.equal(pair, row)
    assert rel_l2(host(pair), g["rw_pair"]) < TOL
    wa = cuda_items(items_from(g, "wa"))
    ya = nat.fp8_e4m3_block_mlp_many_weighted_avx512_f32(wa, dev(g["wa_x"]), dev(g["wa_route"]))
    assert rel_l2(host(ya), g["wa_y"]) < TOL
    assert torch.equal(ya, nat.fp8_e4m3_block_mlp_many_weighted_f32(wa, dev(g["wa_x"]), dev(g["wa_route"])))
    moe = cuda_items(items_from(g, "moe"))
    ym = nat.fp8_e4m3_block_mlp_many_row_weighted_f32(moe, dev(g["moe_x"]), dev(g["moe_route"]))
    assert rel_l2(host(ym), g["moe_y"]) < TOL
    y1 = nat.fp8_e4m3_block_mlp_many_weighted_f32(moe, dev(g["moe_x"][:1]), dev(g["moe_route"][:, 0]))
    assert rel_l2(host(y1), g["moe_y1"]) < TOL


def test_pair_weighted_rejects_bad_index(nat, golden):
    g = golden("fp8_gemv")
    rw = cuda_items(items_from(g, "rw"))
    bad = torch.tensor([0, 9], dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="code -4"):
        nat.fp8_e4m3_block_mlp_many_pair_weighted_f32(rw, dev(g["rw_x"]), bad, torch.tensor([0, 1], device="cuda"),
                                                      torch.tensor([0.5, 0.5], device="cuda"))


def test_null_expert_pointers_are_skipped(oracle_mod, golden):
    import ctypes

    from pocketlm_amd import _lib

    lib = _lib.load()
    g = golden("fp8_gemv")
    items = items_from(g, "wt")
    di = cuda_items(items)
    x = dev(g["wt_x"])
    route = dev(g["wt_route"])
    out = torch.empty((1, 64), device="cuda")
    tables = [(ctypes.c_uint64 * 3)(*[int(t[i].data_ptr()) for t in di]) for i in range(6)]
    for i in range(6):
        tables[i][1] = 0  # expert 1 has no weights at all
    lib.pocketlm_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    code = lib.fp8_e4m3_block_mlp_many_weighted_f32(*[ctypes.cast(t, ctypes.c_void_p) for t in tables],
                                                    ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(route.data_ptr()),
                                                    ctypes.c_void_p(out.data_ptr()), 3, 1, 32, 64, 1, 1)
    assert code == 0
    keep = [items[0], items[2]]
    want = oracle_mod.fp8_mlp_many_weighted(keep, g["wt_x"], g["wt_route"][[0, 2]])
    assert rel_l2(host(out), want) < TOL


def test_deepseek_moe_layer_shapes_vs_oracle(nat, oracle_mod):
    """8 routed experts (2048 x 7168 / 7168 x 2048) at M=1 and M=4."""
    items = []
    for e in range(8):
        g, gs = synth_fp8(2048, 7168, 500 + 3 * e)
        u, us = synth_fp8(2048, 7168, 501 + 3 * e)
        d, ds = synth_fp8(7168, 2048, 502 + 3 * e)
        items.append((g, gs, u, us, d, ds))
    di = cuda_items(items)
    x = synth_x(4, 7168, 600)
    route = np.random.default_rng(1).uniform(0.05, 0.4, 8).astype(np.float32)
    y = nat.fp8_e4m3_block_mlp_many_weighted_f32(di, dev(x[:1]), dev(route))
    assert rel_l2(host(y), oracle_mod.fp8_mlp_many_weighted(items, x[:1], route)) < TOL
    rroute = (np.random.default_rng(2).uniform(0.0, 0.4, (8, 4)) *
              (np.random.default_rng(3).uniform(size=(8, 4)) > 0.3)).astype(np.float32)
    yr = nat.fp8_e4m3_block_mlp_many_row_weighted_f32(di, dev(x), dev(rroute))
    assert rel_l2(host(yr), oracle_mod.fp8_mlp_many_row_weighted(items, x, rroute)) < TOL


def test_weighted_with_shared_expert_equals_separate_calls(nat, oracle_mod, golden):
    """Routed + shared experts in two launches give the separate calls'
    values: the DeepSeek-V3 layer (8 routed + shared, M=1) and the small
    golden experts at one and two activation rows."""
    items = []
    for e in range(9):
        g, gs = synth_fp8(2048, 7168, 700 + 3 * e)
        u, us = synth_fp8(2048, 7168, 701 + 3 * e)
        d, ds = synth_fp8(7168, 2048, 702 + 3 * e)
        items.append((g, gs, u, us, d, ds))
    di = cuda_items(items)
    xh = synth_x(1, 7168, 610)
    x = dev(xh)
    route_h = np.random.default_rng(4).uniform(0.05, 0.4, 8).astype(np.float32)
    route = dev(route_h)
    y, ys = nat.fp8_e4m3_block_mlp_many_weighted_shared_f32(di[:8], di[8], x, route)
    assert torch.equal(y, nat.fp8_e4m3_block_mlp_many_weighted_f32(di[:8], x, route))
    assert torch.equal(ys, nat.fp8_e4m3_block_mlp_f32(*di[8], x))
    assert rel_l2(host(y), oracle_mod.fp8_mlp_many_weighted(items[:8], xh, route_h)) < TOL
    assert rel_l2(host(ys), oracle_mod.fp8_mlp(*items[8], xh)) < TOL
    gd = golden("fp8_gemv")
    wt = cuda_items(items_from(gd, "wt"))
    for m in (1, 2):
        xs = dev(np.repeat(gd["wt_x"], m, axis=0) * np.arange(1, m + 1, dtype=np.float32)[:, None])
        r = dev(gd["wt_route"][:2])
        y2, ys2 = nat.fp8_e4m3_block_mlp_many_weighted_shared_f32(wt[:2], wt[2], xs, r)
        assert torch.equal(y2, nat.fp8_e4m3_block_mlp_many_weighted_f32(wt[:2], xs, r))
        assert torch.equal(ys2, nat.fp8_e4m3_block_mlp_f32(*wt[2], xs))
    # K not a multiple of 16: both phases take the one-thread-per-output kernels
    odd = []
    for e in range(4):
        g, gs = synth_fp8(40, 72, 800 + 3 * e)
        u, us = synth_fp8(40, 72, 801 + 3 * e)
        d, ds = synth_fp8(72, 40, 802 + 3 * e)
        odd.append((g, gs, u, us, d, ds))
    do = cuda_items(odd)
    xo_h = synth_x(2, 72, 620)
    xo = dev(xo_h)
    ro_h = np.array([0.5, 0.25, 0.125], dtype=np.float32)
    ro = dev(ro_h)
    y3, ys3 = nat.fp8_e4m3_block_mlp_many_weighted_shared_f32(do[:3], do[3], xo, ro)
    assert torch.equal(y3, nat.fp8_e4m3_block_mlp_many_weighted_f32(do[:3], xo, ro))
    assert torch.equal(ys3, nat.fp8_e4m3_block_mlp_f32(*do[3], xo))
    assert rel_l2(host(y3), oracle_mod.fp8_mlp_many_weighted(odd[:3], xo_h, ro_h)) < TOL
    assert rel_l2(host(ys3), oracle_mod.fp8_mlp(*odd[3], xo_h)) < TOL


def test_bf16_activation_twins_equal_fp32_calls(nat):
    """bf16 activations go to the *_bf16x_f32 twins, which widen them on the
    device: every twin returns exactly what its fp32 entry point returns for
    the widened activations (the reference wrappers' cast), at 1..8 rows,
    batch rows equal single-row calls, and the odd-K scalar path agrees."""
    w, s = synth_fp8(1536, 7168, 900)
    x16 = dev(synth_x(8, 7168, 901)).to(torch.bfloat16)
    for m in (1, 2, 3, 4, 8):
        y16 = nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), x16[:m])
        assert torch.equal(y16, nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), x16[:m].float()))
    rows = torch.cat([nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), x16[i:i + 1]) for i in range(5)])
    assert torch.equal(rows, nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), x16[:5]))
    wb, sb = synth_fp8(1536, 7168, 902)
    a16, b16 = nat.fp8_e4m3_block_dual_linear_f32(dev(w), dev(s), dev(wb), dev(sb), x16[:4])
    a32, b32 = nat.fp8_e4m3_block_dual_linear_f32(dev(w), dev(s), dev(wb), dev(sb), x16[:4].float())
    assert torch.equal(a16, a32) and torch.equal(b16, b32)
    items = []
    for e in range(3):
        g, gs = synth_fp8(256, 7168, 910 + 3 * e)
        u, us = synth_fp8(256, 7168, 911 + 3 * e)
        d, ds = synth_fp8(7168, 256, 912 + 3 * e)
        items.append((g, gs, u, us, d, ds))
    di = cuda_items(items)
    assert torch.equal(nat.fp8_e4m3_block_mlp_f32(*di[0], x16[:3]), nat.fp8_e4m3_block_mlp_f32(*di[0], x16[:3].float()))
    route = dev((np.random.default_rng(5).uniform(0.0, 0.5, (3, 4)) *
                 (np.random.default_rng(6).uniform(size=(3, 4)) > 0.3)).astype(np.float32))
    assert torch.equal(nat.fp8_e4m3_block_mlp_many_row_weighted_f32(di, x16[:4], route),
                       nat.fp8_e4m3_block_mlp_many_row_weighted_f32(di, x16[:4].float(), route))
    rw = dev(np.array([0.5, 0.25], dtype=np.float32))
    assert torch.equal(nat.fp8_e4m3_block_mlp_many_weighted_f32(di[:2], x16[:1], rw),
                       nat.fp8_e4m3_block_mlp_many_weighted_f32(di[:2], x16[:1].float(), rw))
    ya, ysa = nat.fp8_e4m3_block_mlp_many_weighted_shared_f32(di[:2], di[2], x16[:1], rw)
    yb, ysb = nat.fp8_e4m3_block_mlp_many_weighted_shared_f32(di[:2], di[2], x16[:1].float(), rw)
    assert torch.equal(ya, yb) and torch.equal(ysa, ysb)
    pi = torch.tensor([0, 0, 1, 2, 2], dtype=torch.int64, device="cuda")
    pr = torch.tensor([0, 3, 1, 0, 2], dtype=torch.int64, device="cuda")
    pw = torch.tensor([0.25, 0.5, 0.125, 0.75, 0.375], device="cuda")
    assert torch.equal(nat.fp8_e4m3_block_mlp_many_pair_weighted_f32(di, x16[:4], pi, pr, pw),
                       nat.fp8_e4m3_block_mlp_many_pair_weighted_f32(di, x16[:4].float(), pi, pr, pw))
    # K not a multiple of 16: the one-thread-per-output kernel reads bf16 too
    wo, so = synth_fp8(40, 72, 920)
    xo = dev(synth_x(3, 72, 921)).to(torch.bfloat16)
    assert torch.equal(nat.fp8_e4m3_block_linear_f32(dev(wo), dev(so), xo),
                       nat.fp8_e4m3_block_linear_f32(dev(wo), dev(so), xo.float()))


def test_linear_many_equals_single_linears(nat):
    """q_a and kv_a (and a third, odd-sized weight) from one hidden in one
    launch: every output equals its single linear call, fp32 and bf16
    activations, 1..8 and 11 rows; an odd K falls back to single calls."""
    mats = [synth_fp8(1536, 7168, 930), synth_fp8(576, 7168, 931), synth_fp8(200, 7168, 932)]
    dm = [(dev(w), dev(s)) for w, s in mats]
    x32 = dev(synth_x(11, 7168, 933))
    for m in (1, 2, 3, 8, 11):
        for xx in (x32[:m], x32[:m].to(torch.bfloat16)):
            outs = nat.fp8_e4m3_block_linear_many_f32(dm, xx)
            for (w, s), y in zip(dm, outs):
                assert torch.equal(y, nat.fp8_e4m3_block_linear_f32(w, s, xx)), m
    odd = [synth_fp8(40, 72, 934), synth_fp8(24, 72, 935)]
    do = [(dev(w), dev(s)) for w, s in odd]
    xo = dev(synth_x(2, 72, 936))
    for (w, s), y in zip(do, nat.fp8_e4m3_block_linear_many_f32(do, xo)):
        assert torch.equal(y, nat.fp8_e4m3_block_linear_f32(w, s, xo))
    with pytest.raises(ValueError, match="1 to 8 weights"):
        nat.fp8_e4m3_block_linear_many_f32(dm * 3, x32[:1])


# --------------------------------------------------------------------------- DeepSeek session

def test_ds_session_combine_kat_and_counters(nat):
    outs = torch.tensor([[[1.0, 2.0, 3.0, 4.0]], [[10.0, 20.0, 30.0, 40.0]]], device="cuda")
    route = torch.tensor([0.75, 0.25], device="cuda")
    with nat.DeepSeekNativeSession(num_layers=2, hidden_dim=4, num_experts=4, top_k=2) as session:
        got = nat.ds_moe_layer_forward(session, outs, route)
        assert torch.equal(got.cpu(), torch.tensor([[3.25, 6.5, 9.75, 13.0]]))
        assert session.monolithic_call_count() == 1 and session.expert_invocation_count() == 2


def test_ds_moe_fp8_matches_many_plus_combine(nat, golden):
    g = golden("fp8_gemv")
    items = cuda_items(items_from(g, "ds"))
    x, route = dev(g["ds_x"]), dev(g["ds_route"])
    many = nat.fp8_e4m3_block_mlp_many_f32(items, x)
    assert rel_l2(host(many), g["ds_many"]) < TOL
    expected = (many * route.view(-1, 1, 1)).sum(0)
    with nat.DeepSeekNativeSession(num_layers=2, hidden_dim=4, num_experts=4, top_k=2) as session:
        got = nat.ds_moe_layer_forward_fp8(session, items, x, route)
        assert torch.allclose(got, expected, atol=1e-6, rtol=1e-6)
        assert session.monolithic_call_count() == 1 and session.expert_invocation_count() == 2

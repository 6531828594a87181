"""Q4, row8 and router kernels on the GPU against the oracle and the golden
vectors.  Dequant and pack are bit-exact; dot products within rel-L2 1e-5
(fp32 outputs) or one fp16 ulp (fp16 outputs)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_q4_available(), "libpocketlm_hip.so must load on the GPU box"
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


def q4_matrix(oracle_mod, rows, cols, seed, std=0.02):
    w = (np.random.default_rng(seed).standard_normal((rows, cols)) * std).astype(np.float16).astype(np.float32)
    packed, scales, _ = oracle_mod.q4_quantize(w)
    return packed, scales


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x.astype(np.float16)).view(np.uint16)


# --------------------------------------------------------------------------- Q4

def test_q4_dequant_golden_bit_exact(nat, golden, oracle_mod):
    g = golden("q4")
    for i in range(int(g["count"])):
        ch, cs = oracle_mod.q4_shape_params(list(g[f"t{i}_shape"]))
        got = host(nat.q4_dequant_to_fp16(dev(g[f"t{i}_packed"]), dev(g[f"t{i}_scales"]).view(torch.float16), ch, cs))
        assert np.array_equal(got.view(np.uint16), g[f"t{i}_deq"]), i


def test_q4_dequant_full_size_and_many(nat, oracle_mod):
    packed, scales = q4_matrix(oracle_mod, 18944, 3584, 1)
    got = host(nat.q4_dequant_to_fp16(dev(packed), dev(scales).view(torch.float16), 18944, 3584))
    assert np.array_equal(got.view(np.uint16), oracle_mod.q4_dequant_f16(packed, scales, 18944, 3584))
    items, wants = [], []
    for j, (r, c) in enumerate(((64, 3584), (7, 33), (5, 17), (3, 1))):
        p, s = q4_matrix(oracle_mod, r, c, 10 + j, std=1.0)
        items.append((dev(p), dev(s).view(torch.float16), r, c))
        wants.append(oracle_mod.q4_dequant_f16(p, s, r, c))
    outs = nat.q4_dequant_many_to_fp16(items)
    for o, w in zip(outs, wants):
        assert np.array_equal(host(o).view(np.uint16), w)


@pytest.mark.parametrize("shape", [(18944, 3584), (3584, 18944), (64, 96), (33, 1001)])
def test_q4_gemv_vs_oracle(nat, oracle_mod, shape):
    rows, cols = shape
    packed, scales = q4_matrix(oracle_mod, rows, cols, rows + cols)
    x16 = np.random.default_rng(cols).standard_normal(cols).astype(np.float16)
    y = host(nat.q4_gemv_f16_f32(dev(packed), dev(scales).view(torch.float16), dev(x16), rows=rows, cols=cols))
    want = oracle_mod.q4_gemv(packed, scales, x16.astype(np.float32), rows, cols)
    # fp16 activations run on the matrix cores: exact products, sums rounded
    # inside the MFMA (about 1e-5 relative at K = 18944); the bar for the
    # path is 1e-3.
    assert rel_l2(y, want) < 1e-4


def _moe_experts(g):
    out = []
    for e in range(2):
        out.append(tuple(g[f"moe_{n}{e}_{k}"] for n in ("g", "u", "d") for k in ("packed", "scales")))
    return out


def test_q4_moe_kat(nat, golden, oracle_mod):
    g = golden("q4")
    experts = _moe_experts(g)
    dexp = [tuple(dev(a) if i % 2 == 0 else dev(a).view(torch.float16) for i, a in enumerate(e)) for e in experts]
    out = nat.q4_moe_selected_forward_u16(dev(g["moe_hidden"]).view(torch.float16), dexp, dev(g["moe_route"]),
                                          hidden_size=16, intermediate_size=12)
    got = host(out).astype(np.float32)
    want = g["moe_expected_f32"].reshape(-1)
    assert np.allclose(got, want.astype(np.float16).astype(np.float32), atol=1e-2, rtol=1e-2)
    orc = oracle_mod.q4_moe_selected(g["moe_hidden"], experts, g["moe_route"], 16, 12).view(np.float16)
    assert np.allclose(got, orc.astype(np.float32), rtol=2e-3, atol=1e-3)


def test_q4_mlp_qwen_shape_vs_oracle(nat, oracle_mod):
    H, I = 3584, 18944
    g = q4_matrix(oracle_mod, I, H, 41)
    u = q4_matrix(oracle_mod, I, H, 42)
    d = q4_matrix(oracle_mod, H, I, 43)
    x16 = np.random.default_rng(44).standard_normal(H).astype(np.float16)
    expert = (g[0], g[1], u[0], u[1], d[0], d[1])
    dexp = [tuple(dev(a) if i % 2 == 0 else dev(a).view(torch.float16) for i, a in enumerate(expert))]
    out = nat.q4_moe_selected_forward_u16(dev(x16), dexp, torch.ones(1, device="cuda"), hidden_size=H,
                                          intermediate_size=I)
    want = oracle_mod.q4_moe_selected(x16.view(np.uint16), [expert], np.ones(1, np.float32), H, I)
    assert rel_l2(host(out).astype(np.float32), want.view(np.float16).astype(np.float32)) < 1e-3


def _q4_moe_case(oracle_mod, H, I, S, seed, gate_std=0.02, down_std=0.02):
    experts = []
    for e in range(S):
        g = q4_matrix(oracle_mod, I, H, seed + 3 * e, std=gate_std)
        u = q4_matrix(oracle_mod, I, H, seed + 3 * e + 1, std=gate_std)
        d = q4_matrix(oracle_mod, H, I, seed + 3 * e + 2, std=down_std)
        experts.append((g[0], g[1], u[0], u[1], d[0], d[1]))
    x16 = np.random.default_rng(seed).standard_normal(H).astype(np.float16)
    route = np.random.default_rng(seed + 1).random(S).astype(np.float32) + 0.1
    return experts, x16, route


def _run_q4_moe(nat, experts, x16, route, H, I):
    dexp = [tuple(dev(a) if i % 2 == 0 else dev(a).view(torch.float16) for i, a in enumerate(e)) for e in experts]
    out = nat.q4_moe_selected_forward_u16(dev(x16), dexp, dev(route), hidden_size=H, intermediate_size=I)
    return host(out).astype(np.float32)


def test_q4_moe_multi_expert_partial_step(nat, oracle_mod):
    # three experts (the down phase folds each expert's sum with its scale and
    # route weight) and I = 1568, whose last 512-value step is one 32-value piece
    H, I, S = 1024, 1568, 3
    experts, x16, route = _q4_moe_case(oracle_mod, H, I, S, 61)
    got = _run_q4_moe(nat, experts, x16, route, H, I)
    want = oracle_mod.q4_moe_selected(x16.view(np.uint16), experts, route, H, I).view(np.float16).astype(np.float32)
    assert rel_l2(got, want) < 1e-3


def test_q4_moe_intermediate_beyond_fp16_takes_exact_path(nat, oracle_mod):
    # Large gate/up weights push silu(gate) * up past the fp16 range (the
    # matrix-core down phase reads the intermediate as fp16 planes); tiny down
    # weights keep the fp16 output finite.  The call must fall back to the fp32
    # intermediate, and the next ordinary call must still be right.
    H, I, S = 512, 1024, 2
    experts, x16, route = _q4_moe_case(oracle_mod, H, I, S, 71, gate_std=50.0, down_std=1e-5)
    acts = []
    for g_p, g_s, u_p, u_s, _d, _ds in experts:
        gate = oracle_mod.q4_gemv(g_p, g_s, x16.astype(np.float32), I, H)
        up = oracle_mod.q4_gemv(u_p, u_s, x16.astype(np.float32), I, H)
        with np.errstate(over="ignore"):
            acts.append(gate / (1.0 + np.exp(-gate.astype(np.float64))) * up)
    assert max(np.abs(a).max() for a in acts) > 65504.0
    want = oracle_mod.q4_moe_selected(x16.view(np.uint16), experts, route, H, I).view(np.float16).astype(np.float32)
    assert np.isfinite(want).all()
    got = _run_q4_moe(nat, experts, x16, route, H, I)
    assert rel_l2(got, want) < 1e-3
    experts2, x2, route2 = _q4_moe_case(oracle_mod, H, I, S, 81)
    got2 = _run_q4_moe(nat, experts2, x2, route2, H, I)
    want2 = oracle_mod.q4_moe_selected(x2.view(np.uint16), experts2, route2, H, I).view(np.float16).astype(np.float32)
    assert rel_l2(got2, want2) < 1e-3


# --------------------------------------------------------------------------- row8

def test_row8_pack_golden_and_full(nat, golden, oracle_mod):
    g = golden("row8")
    for dt, tdt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        w = dev(g[f"pack_{dt}_w"]).view(tdt)
        assert np.array_equal(host(nat.pack_weight_rows8(w)).view(np.uint16), g[f"pack_{dt}_packed"])
    w = np.random.default_rng(5).standard_normal((3589, 515)).astype(np.float16)
    got = host(nat.pack_weight_rows8(dev(w))).view(np.uint16)
    assert np.array_equal(got, oracle_mod.pack_rows8(w.view(np.uint16)))


def test_row8_gemv_golden(nat, golden):
    g = golden("row8")
    for key in g["cases"]:
        code = int(g[f"{key}_code"])
        tdt = torch.float16 if code == 0 else torch.bfloat16
        w = dev(g[f"{key}_w"]).view(tdt)
        h = dev(g[f"{key}_h"]).view(tdt)
        rows, cols = g[f"{key}_w"].shape
        y = host(nat.packed_gemv_rows8(h, nat.pack_weight_rows8(w), rows=rows, cols=cols))
        assert np.allclose(y, g[f"{key}_mv"], atol=1e-5, rtol=1e-5), key
        assert rel_l2(y, g[f"{key}_y"]) < 1e-5, key


@pytest.mark.parametrize("shape", [(3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_row8_qwen_shapes_vs_oracle(nat, oracle_mod, shape, dt):
    rows, cols = shape
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    rng = np.random.default_rng(rows + cols)
    w = torch.from_numpy((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)).to(tdt)
    h = torch.from_numpy(rng.standard_normal(cols).astype(np.float32)).to(tdt)
    packed = nat.pack_weight_rows8(w.cuda())
    y = host(nat.packed_gemv_rows8(h.cuda(), packed, rows=rows, cols=cols))
    want = oracle_mod.packed_gemv_rows8(h.view(torch.int16).numpy().view(np.uint16),
                                        host(packed).view(np.uint16), rows, cols, 0 if dt == "f16" else 1)
    assert rel_l2(y, want) < 1e-5


def test_row8_many_with_bias(nat, oracle_mod):
    cols = 3584
    rng = np.random.default_rng(8)
    h = rng.standard_normal(cols).astype(np.float16)
    mats, packs, biases, rows = [], [], [], (3584, 512, 512)
    for r in rows:
        w = (rng.standard_normal((r, cols)) * 0.02).astype(np.float16)
        mats.append(w)
        packs.append(nat.pack_weight_rows8(dev(w)))
        biases.append(dev(rng.standard_normal(r).astype(np.float16)))
    outs = nat.packed_gemv_rows8_many(dev(h), packs, rows, cols=cols, biases=biases)
    for w, p, b, o, r in zip(mats, packs, biases, outs, rows):
        want = oracle_mod.packed_gemv_rows8(h.view(np.uint16), host(p).view(np.uint16), r, cols, 0,
                                            host(b).view(np.uint16))
        assert rel_l2(host(o), want) < 1e-5


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_row8_f32_hidden_vs_oracle(nat, oracle_mod, dt):
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    rng = np.random.default_rng(77)
    for rows, cols in ((3584, 3584), (3584, 18944), (13, 40)):
        w = torch.from_numpy((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)).to(tdt)
        x = rng.standard_normal(cols).astype(np.float32)
        packed = nat.pack_weight_rows8(w.cuda())
        y = host(nat.packed_gemv_rows8_f32_hidden(dev(x), packed, rows=rows, cols=cols, weight_dtype=tdt))
        want = oracle_mod.packed_gemv_rows8_f32_hidden(x, host(packed).view(np.uint16), rows, cols,
                                                       0 if dt == "f16" else 1)
        assert rel_l2(y, want) < 1e-5, (rows, cols)


# --------------------------------------------------------------------------- routers

def test_softmax_router_golden(nat, golden):
    g = golden("router")
    router = dev(g["softmax_router"]).view(torch.float16)
    for i, h in enumerate(g["softmax_hidden"]):
        ids, w = nat.ds_router_topk(dev(h).view(torch.float16), router, k=4)
        assert host(ids).tolist() == g["softmax_ids"][i].tolist()
        assert np.allclose(host(w), g["softmax_weights"][i], atol=1e-6, rtol=1e-6)


def test_softmax_router_nosync_equals_checked_call(nat, golden):
    """ds_router_topk_u16_nosync: the same ids and weights, the status in
    device memory (0 here; 3 for a softmax whose sum is not positive, where
    the checked call raises)."""
    g = golden("router")
    router = dev(g["softmax_router"]).view(torch.float16)
    for h in g["softmax_hidden"]:
        hx = dev(h).view(torch.float16)
        ids, w = nat.ds_router_topk(hx, router, k=4)
        ids2, w2, status = nat.ds_router_topk_nosync(hx, router, k=4)
        assert torch.equal(ids, ids2) and torch.equal(w, w2) and int(status.item()) == 0
    bad = torch.full_like(hx, float("nan"))
    _ids, _w, status = nat.ds_router_topk_nosync(bad, router, k=4)
    assert int(status.item()) == 3
    with pytest.raises(RuntimeError):
        nat.ds_router_topk(bad, router, k=4)


def test_deepseek_route_kat_and_random(nat, golden, oracle_mod):
    g = golden("router")
    idx, w = nat.route_deepseek(dev(g["ds_kat_logits"]), top_k=1, n_groups=1, topk_groups=1, route_scale=2.5,
                                bias=dev(g["ds_kat_bias"]))
    assert host(idx).tolist() == [[1]] and host(w.float()).tolist() == [[2.5]]
    rng = np.random.default_rng(12)
    logits = rng.standard_normal((8, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    for b in (bias, None):
        idx, w = nat.route_deepseek(dev(logits), bias=None if b is None else dev(b))
        oi, ow = oracle_mod.deepseek_route(logits, bias=b)
        assert host(idx).tolist() == oi.tolist()
        assert np.allclose(host(w.float()), ow, rtol=8e-3)


@pytest.mark.parametrize("experts,groups,kept,top_k", [
    (16, 8, 4, 8),       # two experts per group
    (90, 3, 2, 6),       # a count that is not a multiple of 4 (scalar loads)
    (160, 1, 1, 6),      # DeepSeek-V2 width, flat top-k
    (384, 8, 4, 8),      # 16 experts per lane
    (1024, 16, 8, 12),
    (2048, 8, 4, 8),     # 64 experts per lane
    (4096, 64, 16, 32),
])
def test_deepseek_route_widths_against_oracle(nat, oracle_mod, experts, groups, kept, top_k):
    """Every lane width of the one-wave router (4, 16, 64 experts per lane),
    with and without a correction bias, sigmoid and softmax scoring, batches
    of 1 and 5 rows: the oracle's indices, its weights to bf16 rounding."""
    rng = np.random.default_rng(experts)
    for rows in (1, 5):
        logits = rng.standard_normal((rows, experts)).astype(np.float32)
        bias = (rng.standard_normal(experts) * 0.1).astype(np.float32)
        for b in (None, bias):
            for scoring in ("sigmoid", "softmax"):
                idx, w = nat.route_deepseek(dev(logits), top_k=top_k, n_groups=groups, topk_groups=kept,
                                            scoring_func=scoring, bias=None if b is None else dev(b))
                oi, ow = oracle_mod.deepseek_route(logits, top_k=top_k, n_groups=groups, topk_groups=kept, bias=b,
                                                   scoring=scoring)
                assert host(idx).tolist() == oi.tolist(), (rows, b is None, scoring)
                assert np.allclose(host(w.float()), ow, rtol=8e-3), (rows, b is None, scoring)


@pytest.mark.parametrize("experts,groups,kept,top_k", [
    (256, 8, 4, 8), (256, 4, 2, 8), (256, 1, 1, 8), (64, 8, 2, 6), (64, 16, 5, 7), (32, 2, 1, 4),
])
def test_register_router_equals_general_router(nat, experts, groups, kept, top_k):
    """The register version of the 4-experts-per-lane router (16-byte
    aligned logits) and the general version (the same logits one float off
    that alignment) give the same indices and weight bits, with ties,
    infinite logits, a bias and batches."""
    rng = np.random.default_rng(experts * 100 + groups)
    for rows in (1, 7):
        logits = (rng.standard_normal((rows, experts)) * 3).astype(np.float32)
        logits[:, 5::9] = logits[:, 2:3]  # ties
        logits[0, 3] = np.inf
        logits[-1, 7] = -np.inf
        bias = (rng.standard_normal(experts) * 0.1).astype(np.float32)
        for b in (None, bias):
            aligned = dev(logits)
            buf = torch.zeros(rows * experts + 1, device="cuda")
            buf[1:] = aligned.reshape(-1)
            shifted = buf[1:].view(rows, experts)
            assert aligned.data_ptr() % 16 == 0 and shifted.data_ptr() % 16 != 0
            kw = dict(top_k=top_k, n_groups=groups, topk_groups=kept, bias=None if b is None else dev(b),
                      weights_dtype=torch.float32)
            ia, wa = nat.route_deepseek(aligned, **kw)
            ib, wb = nat.route_deepseek(shifted, **kw)
            assert torch.equal(ia, ib), (rows, b is None)
            assert torch.equal(wa.view(torch.int32), wb.view(torch.int32)), (rows, b is None)


def _route_in_order(logits, top_k, n_groups, topk_groups, bias, scale):
    """The routing as one in-order scan per step (strict > keeps the first
    of equal values; a NaN is kept only when it is where a scan starts)."""
    out_i, out_w = [], []
    for lg in logits.astype(np.float32):
        with np.errstate(all="ignore"):
            score = (np.float32(1) / (np.float32(1) + np.exp(-lg))).astype(np.float32)
        choice = (score + bias).astype(np.float32) if bias is not None else score.copy()
        e_n = len(choice)
        if n_groups > 1:
            gsz = e_n // n_groups
            gs = []
            for g in range(n_groups):
                b1 = b2 = np.float32(-np.inf)
                for v in choice[g * gsz:(g + 1) * gsz]:
                    if v > b1:
                        b1, b2 = v, b1
                    elif v > b2:
                        b2 = v
                gs.append(np.float32(b1 + b2) if bias is not None else b1)
            keep = set()
            for _ in range(max(1, min(topk_groups, n_groups))):
                best = -1
                for g in range(n_groups):
                    if g not in keep and (best < 0 or gs[g] > gs[best]):
                        best = g
                keep.add(best)
            for g in range(n_groups):
                if g not in keep:
                    choice[g * gsz:(g + 1) * gsz] = -np.inf
        taken, sel = set(), []
        for _ in range(top_k):
            best = -1
            for e in range(e_n):
                if e not in taken and (best < 0 or choice[e] > choice[best]):
                    best = e
            taken.add(best)
            sel.append(best)
        out_i.append(sel)
    return np.array(out_i, dtype=np.int64)


def test_deepseek_route_ties_nans_and_masked_experts(nat):
    """The block-wide arg max of the router picks what the in-order scan
    picks: exact ties (lowest id), NaN logits, and more choices than the
    kept groups hold (the rest from the masked -inf experts, lowest ids)."""
    rng = np.random.default_rng(5)
    tied = rng.choice(np.array([-1.0, 0.0, 0.5, 1.0], dtype=np.float32), size=(6, 256))
    nans = rng.standard_normal((4, 256)).astype(np.float32)
    nans[0, 0] = np.nan          # the first expert: a scan starts on it
    nans[1, [3, 77, 200]] = np.nan
    nans[2, :] = np.nan
    nans[3, 5:40] = np.nan
    bias = (rng.choice(np.array([0.0, 0.25], dtype=np.float32), size=256))
    for logits in (tied, nans):
        for b in (None, bias):
            for top_k, groups, kept in ((8, 8, 4), (40, 8, 1), (8, 1, 1), (16, 4, 2)):
                idx, _w = nat.route_deepseek(dev(logits), top_k=top_k, n_groups=groups, topk_groups=kept,
                                             bias=None if b is None else dev(b))
                want = _route_in_order(logits, top_k, groups, kept, b, 2.5)
                assert host(idx).tolist() == want.tolist(), (top_k, groups, kept, b is None)

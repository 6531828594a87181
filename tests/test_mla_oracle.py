"""Pins of the MLA oracle (oracle/mla.py) on the CPU.

ds_forward.cpp cannot be built here (it includes <windows.h>), so the
restatement of ds_mla_attention_flash_forward (online softmax, float32) is
pinned against:
  * the reference's own Python formulation of the attention
    (native/__init__.py:857-876: einsum / softmax / einsum, here in float64),
    on the inputs of the reference tests (tests/test_native_flash_mla.py:8-24,
    the same generator and seed);
  * closed forms: one cache row (softmax = 1, out = Wv . kv), a zero query
    (uniform weights, out = Wv . mean(kv)), invariance under a permutation of
    the cache rows;
  * planted mistakes (a dropped rope term, the key and value halves of kv_b
    swapped, a missing scale) that move the result well past the tolerance.
The block restatement (ds_forward.cpp:647-782) is pinned against the
reference test's torch formulation (tests/test_native_ds_fused_attention.py:
12-68, restated with torch ops).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mla


def make_inputs(heads, cache_len, qk_nope, qk_rope, rank, v_head_dim, seed=1234):
    """tests/test_native_flash_mla.py:8-24 (the reference test's generator)."""
    g = torch.Generator().manual_seed(seed)
    q_nope = torch.randn((heads, qk_nope), generator=g, dtype=torch.float32) * 0.05
    q_pe = torch.randn((heads, qk_rope), generator=g, dtype=torch.float32) * 0.05
    kv = torch.randn((cache_len, rank), generator=g, dtype=torch.float32) * 0.05
    pe = torch.randn((cache_len, qk_rope), generator=g, dtype=torch.float32) * 0.05
    wkv_b = torch.randn((heads, qk_nope + v_head_dim, rank), generator=g, dtype=torch.float32) * 0.05
    return [t.numpy() for t in (q_nope, q_pe, kv, pe, wkv_b)]


REF_CASES = [  # (dims, softmax_scale) of the reference tests
    ((4, 7, 3, 2, 5, 3), 0.25),
    ((2, 4, 2, 1, 4, 2), 0.5),
    ((16, 64, 32, 16, 64, 32), 0.125),
]


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("dims,scale", REF_CASES)
def test_online_matches_the_reference_python_formulation(dims, scale):
    args = make_inputs(*dims)
    got = mla.mla_flash_online(*args, scale)
    want = mla.mla_flash_closed_form(*args, scale)
    assert np.allclose(got, want, atol=1e-6, rtol=1e-6)  # the reference test's bar
    assert rel(got, want) < 1e-5


def test_larger_scores_exercise_the_running_max():
    rng = np.random.default_rng(3)
    q_nope = rng.standard_normal((8, 16)).astype(np.float32)
    q_pe = rng.standard_normal((8, 8)).astype(np.float32)
    kv = rng.standard_normal((200, 32)).astype(np.float32)
    pe = rng.standard_normal((200, 8)).astype(np.float32)
    w = (rng.standard_normal((8, 24, 32)) * 0.3).astype(np.float32)
    got = mla.mla_flash_online(q_nope, q_pe, kv, pe, w, 0.3)
    assert rel(got, mla.mla_flash_closed_form(q_nope, q_pe, kv, pe, w, 0.3)) < 1e-5


def test_single_row_is_the_value_projection_of_that_row():
    q_nope, q_pe, kv, pe, w = make_inputs(4, 1, 3, 2, 5, 3, seed=7)
    want = np.einsum("hdc,c->hd", w[:, 3:].astype(np.float64), kv[0].astype(np.float64))
    assert rel(mla.mla_flash_closed_form(q_nope, q_pe, kv, pe, w, 0.25), want) < 1e-12
    assert rel(mla.mla_flash_online(q_nope, q_pe, kv, pe, w, 0.25), want) < 1e-6


def test_zero_query_averages_the_rows():
    q_nope, q_pe, kv, pe, w = make_inputs(4, 9, 3, 2, 5, 3, seed=8)
    q_nope[:] = 0
    q_pe[:] = 0
    want = np.einsum("hdc,c->hd", w[:, 3:].astype(np.float64), kv.astype(np.float64).mean(axis=0))
    assert rel(mla.mla_flash_closed_form(q_nope, q_pe, kv, pe, w, 0.25), want) < 1e-12
    assert rel(mla.mla_flash_online(q_nope, q_pe, kv, pe, w, 0.25), want) < 1e-6


def test_row_order_does_not_matter():
    q_nope, q_pe, kv, pe, w = make_inputs(4, 23, 3, 2, 5, 3, seed=9)
    perm = np.random.default_rng(0).permutation(23)
    a = mla.mla_flash_online(q_nope, q_pe, kv, pe, w, 0.25)
    b = mla.mla_flash_online(q_nope, q_pe, kv[perm], pe[perm], w, 0.25)
    assert rel(a, b) < 1e-6


def test_planted_mistakes_are_caught():
    q_nope, q_pe, kv, pe, w = make_inputs(16, 64, 32, 16, 64, 32)
    q_nope, q_pe, kv, pe = (a * 20 for a in (q_nope, q_pe, kv, pe))  # scores of order one
    good = mla.mla_flash_closed_form(q_nope, q_pe, kv, pe, w, 0.125)
    no_rope = mla.mla_flash_closed_form(q_nope, np.zeros_like(q_pe), kv, np.zeros_like(pe), w, 0.125)
    swapped = mla.mla_flash_closed_form(q_nope, q_pe, kv, pe, np.concatenate([w[:, 32:], w[:, :32]], axis=1), 0.125)
    unscaled = mla.mla_flash_closed_form(q_nope, q_pe, kv, pe, w, 1.0)
    for bad in (no_rope, swapped, unscaled):
        assert rel(bad, good) > 1e-3
    assert rel(mla.mla_flash_online(q_nope, q_pe, kv, pe, w, 0.125), good) < 1e-5


def _torch_block(hidden, q_a, q_b, kv_a, kv_b, o, q_norm, kv_norm, prev_kv, prev_pe, cos, sin, *, heads, nope, rope,
                 v, rank, eps, scale):
    """tests/test_native_ds_fused_attention.py:12-68 restated in torch."""

    def rms(x, w):
        return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w

    def rot(x):
        pair = x.reshape(*x.shape[:-1], x.shape[-1] // 2, 2)
        return torch.stack((pair[..., 0] * cos - pair[..., 1] * sin, pair[..., 0] * sin + pair[..., 1] * cos),
                           dim=-1).flatten(-2)

    q_low = rms(F.linear(hidden.reshape(1, -1), q_a), q_norm)
    q = F.linear(q_low, q_b).view(heads, nope + rope)
    q_nope, q_pe = torch.split(q, [nope, rope], dim=-1)
    q_pe = rot(q_pe)
    kv = F.linear(hidden.reshape(1, -1), kv_a).reshape(-1)
    latent = rms(kv[:rank], kv_norm)
    k_pe = rot(kv[rank:].reshape(1, rope)).reshape(-1)
    kv_cache = torch.cat([prev_kv, latent.reshape(1, rank)], dim=0)
    pe_cache = torch.cat([prev_pe, k_pe.reshape(1, rope)], dim=0)
    w = kv_b.view(heads, nope + v, rank)
    q_abs = torch.einsum("hd,hdc->hc", q_nope, w[:, :nope])
    s = (torch.einsum("hc,tc->ht", q_abs, kv_cache) + torch.einsum("hr,tr->ht", q_pe, pe_cache)) * scale
    lat = torch.einsum("ht,tc->hc", s.softmax(dim=-1), kv_cache)
    heads_out = torch.einsum("hc,hdc->hd", lat, w[:, nope:])
    return F.linear(heads_out.reshape(1, -1), o).reshape(-1), kv_cache, pe_cache


def block_inputs(hidden_dim, q_rank, kv_rank, heads, nope, rope, v, prev, seed=12):
    """tests/test_native_ds_fused_attention.py:71-95 (the reference test's shapes and scales)."""
    torch.manual_seed(seed)
    t = dict(
        hidden=torch.randn(hidden_dim),
        q_a=torch.randn(q_rank, hidden_dim) * 0.02,
        q_b=torch.randn(heads * (nope + rope), q_rank) * 0.02,
        kv_a=torch.randn(kv_rank + rope, hidden_dim) * 0.02,
        kv_b=torch.randn(heads * (nope + v), kv_rank) * 0.02,
        o=torch.randn(hidden_dim, heads * v) * 0.02,
        q_norm=torch.ones(q_rank),
        kv_norm=torch.ones(kv_rank),
        prev_kv=torch.randn(prev, kv_rank) * 0.02,
        prev_pe=torch.randn(prev, rope) * 0.02,
    )
    angles = torch.arange(rope // 2, dtype=torch.float32) * 0.1
    t["cos"], t["sin"] = angles.cos(), angles.sin()
    return t


@pytest.mark.parametrize("dims", [(16, 6, 5, 4, 3, 4, 2, 3), (64, 16, 16, 4, 8, 8, 8, 32), (48, 8, 12, 2, 4, 6, 4, 0)])
def test_block_matches_the_reference_test_formulation(dims):
    hidden_dim, q_rank, kv_rank, heads, nope, rope, v, prev = dims
    t = block_inputs(*dims)
    want, want_kv, want_pe = _torch_block(t["hidden"], t["q_a"], t["q_b"], t["kv_a"], t["kv_b"], t["o"], t["q_norm"],
                                          t["kv_norm"], t["prev_kv"], t["prev_pe"], t["cos"], t["sin"], heads=heads,
                                          nope=nope, rope=rope, v=v, rank=kv_rank, eps=1e-6, scale=0.25)
    n = {k: a.numpy() for k, a in t.items()}
    got, got_kv, got_pe = mla.attention_block(
        n["hidden"], n["q_a"], n["q_b"], n["kv_a"], n["kv_b"], n["o"], n["q_norm"], n["kv_norm"],
        n["prev_kv"] if prev else None, n["prev_pe"] if prev else None, n["cos"], n["sin"], num_heads=heads,
        qk_nope_dim=nope, qk_rope_dim=rope, v_head_dim=v, kv_lora_rank=kv_rank, rms_eps=1e-6, softmax_scale=0.25)
    assert np.allclose(got, want.numpy(), atol=1e-5, rtol=1e-5)  # the reference test's bar
    assert np.allclose(got_kv, want_kv.numpy(), atol=1e-6, rtol=1e-6)
    assert np.allclose(got_pe, want_pe.numpy(), atol=1e-6, rtol=1e-6)
    assert got_kv.shape == (prev + 1, kv_rank)


def test_rope_leaves_an_odd_width_alone():
    x = np.arange(5, dtype=np.float32)
    assert np.array_equal(mla.rope(x, np.ones(2, np.float32), np.zeros(2, np.float32)), x)
    y = mla.rope(np.array([1.0, 0.0], np.float32), np.array([0.0], np.float32), np.array([1.0], np.float32))
    assert np.allclose(y, [0.0, 1.0])  # a quarter turn


def fp8_attention_inputs(hidden_dim, q_rank, kv_rank, heads, nope, rope, v, prev, seed=31):
    """FP8 e4m3 weights (N(0, 0.05), cast as torch casts), scale_inv grids
    ~U(0.5, 1.5), bf16-valued hidden state, fp32 norms, caches and rotations."""
    g = torch.Generator().manual_seed(seed)

    def fp8(rows, cols):
        w = (torch.randn((rows, cols), generator=g) * 0.05).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        s = (torch.rand((-(-rows // 128), -(-cols // 128)), generator=g) + 0.5).numpy()
        return w, s

    weights = {"q_a": fp8(q_rank, hidden_dim), "q_b": fp8(heads * (nope + rope), q_rank),
               "kv_a": fp8(kv_rank + rope, hidden_dim), "o": fp8(hidden_dim, heads * v)}
    kv_b = fp8(heads * (nope + v), kv_rank)
    hidden = torch.randn(hidden_dim, generator=g).to(torch.bfloat16).float().numpy()
    q_norm = (1 + 0.1 * torch.randn(q_rank, generator=g)).numpy()
    kv_norm = (1 + 0.1 * torch.randn(kv_rank, generator=g)).numpy()
    prev_kv = torch.randn((prev, kv_rank), generator=g).numpy()
    prev_pe = torch.randn((prev, rope), generator=g).numpy()
    ang = np.arange(rope // 2, dtype=np.float32) * 0.37
    return dict(hidden=hidden, fp8=weights, kv_b=kv_b, q_norm=q_norm, kv_norm=kv_norm, prev_kv=prev_kv,
                prev_pe=prev_pe, cos=np.cos(ang).astype(np.float32), sin=np.sin(ang).astype(np.float32))


FP8_DIMS = (256, 128, 64, 4, 16, 8, 16, 20)  # hidden, q rank, latent rank, heads, nope, rope, v, previous rows


def _fp8_block(t, dims, fp8=None, flash=mla.mla_flash_online):
    hidden_dim, q_rank, kv_rank, heads, nope, rope, v, prev = dims
    import oracle

    kv_b = oracle.fp8_dequant(*t["kv_b"], "f32")
    return mla.fp8_attention_block(t["hidden"], fp8 or t["fp8"], kv_b, t["q_norm"], t["kv_norm"], t["prev_kv"],
                                   t["prev_pe"], t["cos"], t["sin"], num_heads=heads, qk_nope_dim=nope,
                                   qk_rope_dim=rope, v_head_dim=v, kv_lora_rank=kv_rank, rms_eps=1e-6,
                                   softmax_scale=float(1 / np.sqrt(nope + rope)), flash=flash)


def test_fp8_attention_matches_the_reference_formulation_on_dequantized_weights():
    """fp8_source.py:6337-6454 restated with torch on the dequantized
    weights (F.linear, _rms_norm_any, _apply_rope_real, the einsums): the
    FP8 linears' block-sum-then-scale order differs only by rounding."""
    import oracle

    hidden_dim, q_rank, kv_rank, heads, nope, rope, v, prev = FP8_DIMS
    t = fp8_attention_inputs(*FP8_DIMS)
    got, got_kv, got_pe = _fp8_block(t, FP8_DIMS)
    deq = {k: torch.from_numpy(oracle.fp8_dequant(*t["fp8"][k], "f32")) for k in t["fp8"]}
    want, want_kv, want_pe = _torch_block(
        torch.from_numpy(t["hidden"]), deq["q_a"], deq["q_b"], deq["kv_a"],
        torch.from_numpy(oracle.fp8_dequant(*t["kv_b"], "f32")), deq["o"], torch.from_numpy(t["q_norm"]),
        torch.from_numpy(t["kv_norm"]), torch.from_numpy(t["prev_kv"]), torch.from_numpy(t["prev_pe"]),
        torch.from_numpy(t["cos"]), torch.from_numpy(t["sin"]), heads=heads, nope=nope, rope=rope, v=v, rank=kv_rank,
        eps=1e-6, scale=float(1 / np.sqrt(nope + rope)))
    assert rel(got, want.numpy()) < 1e-5
    assert rel(got_kv, want_kv.numpy()) < 1e-6 and rel(got_pe, want_pe.numpy()) < 1e-6
    assert got_kv.shape == (prev + 1, kv_rank)


def test_fp8_attention_planted_mistakes_are_caught():
    t = fp8_attention_inputs(*FP8_DIMS)
    good = _fp8_block(t, FP8_DIMS)[0]
    w, s = t["fp8"]["q_b"]
    bad_scale = dict(t["fp8"], q_b=(w, s * np.float32(1.25)))
    w, s = t["fp8"]["kv_a"]
    swapped_rows = dict(t["fp8"], kv_a=(np.ascontiguousarray(w[::-1]), s))
    for fp8 in (bad_scale, swapped_rows):
        assert rel(_fp8_block(t, FP8_DIMS, fp8=fp8)[0], good) > 1e-3

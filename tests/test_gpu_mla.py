"""MLA attention on the GPU (ds_mla_attention_flash_forward and
ds_attention_block_forward_f32, mla.hip) against the oracle (oracle/mla.py).

Bars: the reference tests' own (atol = rtol = 1e-6 for the attention on
their fixtures, 1e-5 for the block) and rel-L2 1e-5 against the float64
closed form at DeepSeek-V3 dimensions (128 heads, nope 128, rope 64, latent
rank 512, v 128) from 1 to 4100 cached rows, which covers one and many
splits, ragged last tiles and tiles of one row.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import mla
from test_mla_oracle import FP8_DIMS, REF_CASES, _fp8_block, block_inputs, fp8_attention_inputs, make_inputs, rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_flash_mla_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("dims,scale", REF_CASES)
def test_reference_fixtures(nat, dims, scale):
    args = make_inputs(*dims)
    got = host(nat.ds_mla_attention_flash_forward(*(dev(a) for a in args), softmax_scale=scale))
    want = mla.mla_flash_closed_form(*args, scale)
    assert np.allclose(got, want, atol=1e-6, rtol=1e-6)


def ds_inputs(cache_len, seed, scale_q=1.0):
    rng = np.random.default_rng(seed)
    q_nope = (rng.standard_normal((128, 128)) * scale_q).astype(np.float32)
    q_pe = (rng.standard_normal((128, 64)) * scale_q).astype(np.float32)
    kv = rng.standard_normal((cache_len, 512)).astype(np.float32)
    pe = rng.standard_normal((cache_len, 64)).astype(np.float32)
    wkv_b = (rng.standard_normal((128, 256, 512)) * 0.02).astype(np.float32)
    return q_nope, q_pe, kv, pe, wkv_b


@pytest.mark.parametrize("cache_len", [1, 16, 17, 1000, 4100])
def test_deepseek_v3_dimensions(nat, cache_len):
    print("mla cache_len", cache_len, flush=True)
    args = ds_inputs(cache_len, 100 + cache_len, scale_q=0.05)
    scale = 1.0 / np.sqrt(192.0)
    got = host(nat.ds_mla_attention_flash_forward(*(dev(a) for a in args), softmax_scale=scale))
    assert rel(got, mla.mla_flash_closed_form(*args, scale)) < 1e-5


@pytest.mark.parametrize("heads,cache_len,nope,rope,rank,v", [
    (20, 100, 32, 256, 1024, 48),  # the largest instance, 4 heads of a second group
    (17, 45, 24, 62, 510, 40),     # rank and rope not multiples of 4 (element loads)
    (3, 33, 8, 6, 200, 8),         # one chunk of rope columns
])
def test_kernel_instances(nat, heads, cache_len, nope, rope, rank, v):
    print("mla instance", heads, cache_len, nope, rope, rank, v, flush=True)
    rng = np.random.default_rng(heads * 1000 + rank)
    args = [rng.standard_normal(s).astype(np.float32) * 0.1 for s in
            ((heads, nope), (heads, rope), (cache_len, rank), (cache_len, rope), (heads, nope + v, rank))]
    scale = 1.0 / np.sqrt(nope + rope)
    got = host(nat.ds_mla_attention_flash_forward(*(dev(a) for a in args), softmax_scale=scale))
    assert rel(got, mla.mla_flash_closed_form(*args, scale)) < 1e-5


def test_peaked_scores(nat):
    """Large scores: a few rows dominate each head, so the running max moves
    across tiles and splits."""
    args = ds_inputs(777, 5, scale_q=1.0)
    got = host(nat.ds_mla_attention_flash_forward(*(dev(a) for a in args), softmax_scale=0.2))
    assert np.isfinite(got).all()
    assert rel(got, mla.mla_flash_closed_form(*args, 0.2)) < 1e-5


def test_rope_width_zero_and_no_nope(nat):
    """nope = rope = 0 through the C ABI (the arrays of width 0 are stand-in
    buffers, not read): every score is 0, so the weights are uniform."""
    from pocketlm_amd import _lib

    lib = _lib.load()
    _, _, kv, _, w = make_inputs(6, 40, 0, 0, 24, 8, seed=3)
    dkv, dw = dev(kv), dev(w)
    stand_in = torch.zeros(16, device="cuda")
    out = torch.empty((6, 8), device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    lib.pocketlm_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    code = lib.ds_mla_attention_flash_forward(P(stand_in), P(stand_in), P(dkv), P(stand_in), P(dw), P(out), 6, 40, 0,
                                              0, 24, 8, 0.3)
    assert code == 0
    want = np.einsum("hdc,c->hd", w.astype(np.float64), kv.astype(np.float64).mean(axis=0))  # uniform weights
    assert rel(host(out), want) < 1e-6


def test_error_codes(nat):
    from pocketlm_amd import _lib

    lib = _lib.load()
    a = torch.zeros(4096, device="cuda")
    p = ctypes.c_void_p(a.data_ptr())
    n = ctypes.c_void_p(0)
    assert lib.ds_mla_attention_flash_forward(n, p, p, p, p, p, 1, 1, 1, 1, 1, 1, 1.0) == 1
    assert lib.ds_mla_attention_flash_forward(p, p, p, p, p, p, 0, 1, 1, 1, 1, 1, 1.0) == 2
    assert lib.ds_mla_attention_flash_forward(p, p, p, p, p, p, 1, 1, 1, 1, 1, 0, 1.0) == 2
    assert lib.ds_mla_attention_flash_forward(p, p, p, p, p, p, 1, 1, 1, 1, 2048, 1, 1.0) == 2  # rank limit
    assert lib.ds_mla_attention_flash_forward(p, p, p, p, p, p, 1, 1, 1, 512, 8, 1, 1.0) == 2  # rope limit
    handle = lib.ds_session_create(1, 8, 0, 0, None, None)
    try:
        args = [p] * 15
        assert lib.ds_attention_block_forward_f32(None, *args, 8, 4, 4, 1, 2, 2, 2, 0, 1e-6, 1.0) == 1
        assert lib.ds_attention_block_forward_f32(handle, *args, 0, 4, 4, 1, 2, 2, 2, 0, 1e-6, 1.0) == 2
        with_null_prev = [p] * 8 + [n, n] + [p] * 5
        assert lib.ds_attention_block_forward_f32(handle, *with_null_prev, 8, 4, 4, 1, 2, 2, 2, 3, 1e-6, 1.0) == 3
    finally:
        lib.ds_session_destroy(handle)


@pytest.mark.parametrize("dims", [(16, 6, 5, 4, 3, 4, 2, 3), (64, 16, 16, 4, 8, 8, 8, 32), (48, 8, 12, 2, 4, 6, 4, 0),
                                  (32, 8, 16, 3, 4, 5, 4, 7),  # odd rope width: the pe part stays unrotated
                                  # rows of 4104 values (q_a, kv_a: the row-group GEMV) with row
                                  # counts that are not multiples of 4, and unaligned q_b rows
                                  (4104, 386, 64, 4, 16, 14, 16, 5)])
def test_block_matches_the_oracle(nat, dims):
    hidden_dim, q_rank, kv_rank, heads, nope, rope, v, prev = dims
    t = block_inputs(*dims)
    n = {k: a.numpy() for k, a in t.items()}
    want, want_kv, want_pe = mla.attention_block(
        n["hidden"], n["q_a"], n["q_b"], n["kv_a"], n["kv_b"], n["o"], n["q_norm"], n["kv_norm"],
        n["prev_kv"] if prev else None, n["prev_pe"] if prev else None, n["cos"], n["sin"], num_heads=heads,
        qk_nope_dim=nope, qk_rope_dim=rope, v_head_dim=v, kv_lora_rank=kv_rank, rms_eps=1e-6, softmax_scale=0.25)
    with nat.DeepSeekNativeSession(num_layers=3, hidden_dim=hidden_dim, num_experts=0, top_k=0) as session:
        got, (got_kv, got_pe) = nat.ds_attention_block_forward(
            session, *(t[k].cuda() for k in ("hidden", "q_a", "q_b", "kv_a", "kv_b", "o", "q_norm", "kv_norm")),
            previous_kv_cache=t["prev_kv"].cuda() if prev else None,
            previous_pe_cache=t["prev_pe"].cuda() if prev else None, rope_cos=t["cos"].cuda(),
            rope_sin=t["sin"].cuda(), q_lora_rank=q_rank, kv_lora_rank=kv_rank, num_heads=heads, qk_nope_dim=nope,
            qk_rope_dim=rope, v_head_dim=v, rms_eps=1e-6, softmax_scale=0.25)
        assert session.fused_attention_invocation_count() == 1
        assert session.attention_invocation_count() == 1
        assert session.monolithic_call_count() == 1
    assert np.allclose(host(got), want, atol=1e-5, rtol=1e-5)
    assert np.allclose(host(got_kv), want_kv, atol=1e-6, rtol=1e-6)
    assert np.allclose(host(got_pe), want_pe, atol=1e-6, rtol=1e-6)
    if prev:
        assert torch.equal(got_kv[:prev].cpu(), t["prev_kv"]) and torch.equal(got_pe[:prev].cpu(), t["prev_pe"])


def test_block_deepseek_like_dimensions_in_place_cache(nat):
    """hidden 1024, q rank 384, latent 512, 16 heads of 128 + 64 (v 128) over
    300 cached rows; the new row is written after them in the same buffers."""
    hid, q_rank, rank, heads, nope, rope, v, prev = 1024, 384, 512, 16, 128, 64, 128, 300
    rng = np.random.default_rng(21)
    w = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)  # noqa: E731
    hidden = rng.standard_normal(hid).astype(np.float32)
    q_a, q_b, kv_a, kv_b, o = w(q_rank, hid), w(heads * (nope + rope), q_rank), w(rank + rope, hid), \
        w(heads * (nope + v), rank), w(hid, heads * v)
    q_norm = (1 + rng.standard_normal(q_rank) * 0.1).astype(np.float32)
    kv_norm = (1 + rng.standard_normal(rank) * 0.1).astype(np.float32)
    prev_kv = rng.standard_normal((prev, rank)).astype(np.float32)
    prev_pe = rng.standard_normal((prev, rope)).astype(np.float32)
    ang = (np.arange(rope // 2) * 0.37).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    scale = float(1.0 / np.sqrt(nope + rope))
    want, want_kv, want_pe = mla.attention_block(hidden, q_a, q_b, kv_a, kv_b, o, q_norm, kv_norm, prev_kv, prev_pe,
                                                 cos, sin, num_heads=heads, qk_nope_dim=nope, qk_rope_dim=rope,
                                                 v_head_dim=v, kv_lora_rank=rank, rms_eps=1e-6, softmax_scale=scale,
                                                 flash=mla.mla_flash_closed_form)
    from pocketlm_amd import _lib

    lib = _lib.load()
    kv_buf = torch.zeros((prev + 1, rank), device="cuda")
    pe_buf = torch.zeros((prev + 1, rope), device="cuda")
    kv_buf[:prev] = dev(prev_kv)
    pe_buf[:prev] = dev(prev_pe)
    out = torch.empty(hid, device="cuda")
    ins = [dev(a) for a in (hidden, q_a, q_b, kv_a, kv_b, o, q_norm, kv_norm)]
    cs = [dev(cos), dev(sin)]
    handle = lib.ds_session_create(1, hid, 0, 0, None, None)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    try:
        lib.pocketlm_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        code = lib.ds_attention_block_forward_f32(handle, *[P(t) for t in ins], P(kv_buf), P(pe_buf),
                                                  *[P(t) for t in cs], P(kv_buf), P(pe_buf), P(out), hid, q_rank,
                                                  rank, heads, nope, rope, v, prev, 1e-6, scale)
        assert code == 0
        assert lib.ds_fused_attention_invocation_count(handle) == 1
    finally:
        lib.ds_session_destroy(handle)
    assert rel(host(out), want) < 1e-5
    assert np.array_equal(host(kv_buf)[:prev], prev_kv) and np.array_equal(host(pe_buf)[:prev], prev_pe)
    assert rel(host(kv_buf)[prev], want_kv[prev]) < 1e-6 and rel(host(pe_buf)[prev], want_pe[prev]) < 1e-6


@pytest.mark.parametrize("dims", [FP8_DIMS, (7168, 1536, 512, 16, 128, 64, 128, 300),
                                  (256, 128, 64, 3, 16, 5, 16, 7)])  # odd rope width: pe unrotated
def test_fp8_attention_block_matches_the_oracle(nat, dims):
    """The FP8 model's one-token attention (fp8_source.py:6337-6454) through
    ds_fp8_attention_block_bf16x_f32 against the oracle's restatement (C
    oracle FP8 linears, float32 attention); the second case has DeepSeek-V3's
    projection widths with 16 heads."""
    print("fp8 attention", dims, flush=True)
    hidden_dim, q_rank, kv_rank, heads, nope, rope, v, prev = dims
    t = fp8_attention_inputs(*dims)
    want, want_kv, want_pe = _fp8_block(t, dims)
    import oracle

    d = {k: (torch.from_numpy(w).cuda(), torch.from_numpy(s).cuda()) for k, (w, s) in t["fp8"].items()}
    kv_b = torch.from_numpy(oracle.fp8_dequant(*t["kv_b"], "f32")).cuda()
    hidden = torch.from_numpy(t["hidden"]).to(torch.bfloat16).cuda()
    kw = dict(previous_kv_cache=dev(t["prev_kv"]), previous_pe_cache=dev(t["prev_pe"]), rope_cos=dev(t["cos"]),
              rope_sin=dev(t["sin"]), q_lora_rank=q_rank, kv_lora_rank=kv_rank, num_heads=heads, qk_nope_dim=nope,
              qk_rope_dim=rope, v_head_dim=v, rms_eps=1e-6, softmax_scale=float(1 / np.sqrt(nope + rope)))
    got, (got_kv, got_pe) = nat.fp8_attention_block_forward(
        hidden, *d["q_a"], *d["q_b"], *d["kv_a"], kv_b, *d["o"], dev(t["q_norm"]), dev(t["kv_norm"]), **kw)
    assert rel(host(got), want) < 1e-5
    assert rel(host(got_kv), want_kv) < 1e-6 and rel(host(got_pe), want_pe) < 1e-6
    assert np.array_equal(host(got_kv)[:prev], t["prev_kv"]) and np.array_equal(host(got_pe)[:prev], t["prev_pe"])
    got16, _ = nat.fp8_attention_block_forward(
        hidden, *d["q_a"], *d["q_b"], *d["kv_a"], kv_b, *d["o"], dev(t["q_norm"]), dev(t["kv_norm"]),
        dtype=torch.bfloat16, **kw)
    assert got16.dtype == torch.bfloat16 and torch.equal(got16, got.to(torch.bfloat16))


def test_fp8_attention_block_error_codes(nat):
    from pocketlm_amd import _lib

    lib = _lib.load()
    a = torch.zeros(4096, device="cuda")
    p = ctypes.c_void_p(a.data_ptr())
    n = ctypes.c_void_p(0)
    args = [p] * 19
    assert lib.ds_fp8_attention_block_bf16x_f32(n, *args[1:], 128, 128, 4, 1, 2, 2, 2, 0, 1e-6, 1.0) == 1
    assert lib.ds_fp8_attention_block_bf16x_f32(*args, 0, 128, 4, 1, 2, 2, 2, 0, 1e-6, 1.0) == 2
    assert lib.ds_fp8_attention_block_bf16x_f32(*args, 128, 128, 2048, 1, 2, 2, 2, 0, 1e-6, 1.0) == 102
    with_null_prev = [p] * 12 + [n, n] + [p] * 5
    assert lib.ds_fp8_attention_block_bf16x_f32(*with_null_prev, 128, 128, 4, 1, 2, 2, 2, 3, 1e-6, 1.0) == 3

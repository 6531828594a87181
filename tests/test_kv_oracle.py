"""Pins for the KV session / dense layer oracle (oracle/kv_dense.py): the
reference test's session fixtures (tests/test_native_fp16_kv_cache.py:
82-131), an independent torch formulation of one decode (F.linear and
torch.softmax, as that test's _reference_decode, 20-68), RoPE invariants,
and the reference's fp16_kv_cache.cpp built from source (oracle/_ref)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import kv_dense as kvo


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint16).numpy().copy()


def test_session_commit_and_rollback_roundtrip():
    s = kvo.KvSessionOracle(2, 16, 4)
    ck = _bits(torch.arange(12, dtype=torch.float16).reshape(3, 4))
    tk = _bits(torch.arange(8, dtype=torch.float16).reshape(2, 4) + 1000)
    s.append(0, ck, ck + 1, tentative=False)
    s.append(0, tk, tk + 1, tentative=True)
    assert (s.committed_length(0), s.tentative_length(0)) == (3, 2)
    s.commit(1)
    assert (s.committed_length(0), s.tentative_length(0)) == (4, 1)
    assert np.array_equal(s.copy_layer(0)[0], np.concatenate([ck, tk]))
    s.rollback()
    k, v = s.copy_layer(0)
    assert np.array_equal(k, np.concatenate([ck, tk[:1]])) and np.array_equal(v, np.concatenate([ck, tk[:1]]) + 1)
    assert s.append(1, np.zeros((17, 4), np.uint16), np.zeros((17, 4), np.uint16), tentative=True) == 2


def test_u16_conversions_match_torch_and_the_reference_rounding():
    x = np.array([1.0, -2.5, 3.14159, 65504.0, 1e-8, 0.1, 1.00390625, 1.01171875], np.float32)
    assert np.array_equal(kvo.f32_to_u16(x, 0), _bits(torch.from_numpy(x).to(torch.float16)))
    assert np.array_equal(kvo.f32_to_u16(x, 1), _bits(torch.from_numpy(x).to(torch.bfloat16)))
    assert np.array_equal(kvo.u16_to_f32(kvo.f32_to_u16(x, 1), 1), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_rope_invariants():
    rng = np.random.default_rng(0)
    v = rng.standard_normal((3, 8)).astype(np.float32)
    assert np.array_equal(kvo.rope(v, 0, 10000.0), v)  # position 0: identity
    r = kvo.rope(v, 37, 10000.0)
    pairs = lambda a: a[:, :4] ** 2 + a[:, 4:] ** 2  # noqa: E731
    assert np.allclose(pairs(r), pairs(v), rtol=1e-5)  # rotation keeps each pair's length
    # dim 0 rotates by angle = position exactly
    c, s = np.cos(np.float32(37)), np.sin(np.float32(37))
    assert np.allclose(r[:, 0], v[:, 0] * c - v[:, 4] * s, rtol=1e-6)


def _torch_decode(h, w, prefix_k, prefix_v, position, nh, nkv, theta, eps, biases, norms):
    """One decode of the whole layer written with torch primitives."""
    hidden_size = h.numel()
    hd = hidden_size // nh
    xn = (h * torch.rsqrt(h.pow(2).mean() + eps) * w["in"]).half().float()
    q = F.linear(xn, w["q"], biases[0]).reshape(nh, hd)
    k = F.linear(xn, w["k"], biases[1]).reshape(nkv, hd)
    v = F.linear(xn, w["v"], biases[2]).reshape(nkv, hd)
    if norms is not None:
        q = q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + eps) * norms[0]
        k = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + eps) * norms[1]
    q = torch.from_numpy(kvo.rope(q.numpy(), position, theta))
    k = torch.from_numpy(kvo.rope(k.numpy(), position, theta)).half().float()
    v = v.half().float()
    keys = torch.cat([prefix_k.reshape(-1, nkv, hd), k[None]])
    vals = torch.cat([prefix_v.reshape(-1, nkv, hd), v[None]])
    ctx = torch.stack([torch.softmax(keys[:, hh // (nh // nkv)] @ q[hh] / hd ** 0.5, -1) @ vals[:, hh // (nh // nkv)]
                       for hh in range(nh)])
    resid = h + F.linear(ctx.reshape(-1), w["o"]).half().float()
    post = (resid.half().float() * torch.rsqrt(resid.half().float().pow(2).mean() + eps) * w["post"]).half().float()
    mlp = F.linear(F.silu(F.linear(post, w["gate"])) * F.linear(post, w["up"]), w["down"])
    return (resid + mlp).half()


@pytest.mark.parametrize("with_extras", [False, True])
def test_oracle_decode_matches_a_torch_formulation(with_extras):
    g = torch.Generator().manual_seed(5)
    H, I, nh, nkv, theta, eps = 32, 48, 4, 2, 10000.0, 1e-6
    kvw = H // nh * nkv
    w = {n: (torch.randn(shape, generator=g) * 0.2).half().float() for n, shape in
         [("q", (H, H)), ("k", (kvw, H)), ("v", (kvw, H)), ("o", (H, H)), ("gate", (I, H)), ("up", (I, H)),
          ("down", (H, I))]}
    w["in"] = (torch.rand(H, generator=g) + 0.5).half().float()
    w["post"] = (torch.rand(H, generator=g) + 0.5).half().float()
    biases = [(torch.randn(n, generator=g) * 0.1).half().float() if with_extras else None for n in (H, kvw, kvw)]
    norms = [(torch.rand(H // nh, generator=g) + 0.5).half().float() for _ in range(2)] if with_extras else None
    s = kvo.KvSessionOracle(1, 16, kvw, 0)
    prefix_k = (torch.randn((5, kvw), generator=g)).half()
    prefix_v = (torch.randn((5, kvw), generator=g)).half()
    s.append(0, _bits(prefix_k), _bits(prefix_v), tentative=False)
    h = torch.randn(H, generator=g).half()
    b = lambda t: None if t is None else _bits(t.half())  # noqa: E731
    got = s.dense_layer_decode(0, _bits(h), b(w["in"]), b(w["post"]), *[b(w[n]) for n in
                               ("q", "k", "v", "o", "gate", "up", "down")], num_heads=nh, num_kv_heads=nkv,
                               rms_eps=eps, rope_theta=theta, q_bias=b(biases[0]), k_bias=b(biases[1]),
                               v_bias=b(biases[2]), q_norm=None if norms is None else b(norms[0]),
                               k_norm=None if norms is None else b(norms[1]))
    want = _torch_decode(h.float(), w, prefix_k.float(), prefix_v.float(), 5, nh, nkv, theta, eps, biases, norms)
    got_f = kvo.u16_to_f32(got, 0)
    assert np.linalg.norm(got_f - want.float().numpy()) <= 2e-3 * np.linalg.norm(want.float().numpy())
    assert s.tentative_length(0) == 1


def _layer(seed, H, I, nh, nkv, dc, extras):
    rng = np.random.default_rng(seed)
    kvw = H // nh * nkv
    f = lambda *shape, sc=0.1: kvo.f32_to_u16((rng.standard_normal(shape) * sc).astype(np.float32), dc)  # noqa: E731
    w = {"q": f(H, H), "k": f(kvw, H), "v": f(kvw, H), "o": f(H, H), "gate": f(I, H), "up": f(I, H),
         "down": f(H, I)}
    norms = {n: kvo.f32_to_u16((rng.random(H) + 0.5).astype(np.float32), dc) for n in ("in", "post")}
    extra = {}
    if extras:
        extra = {"q_bias": f(H), "k_bias": f(kvw), "v_bias": f(kvw),
                 "q_norm": kvo.f32_to_u16((rng.random(H // nh) + 0.5).astype(np.float32), dc),
                 "k_norm": kvo.f32_to_u16((rng.random(H // nh) + 0.5).astype(np.float32), dc)}
    return w, norms, extra, rng


@pytest.mark.skipif(not kvo.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("dc,extras", [(0, False), (1, True)])
def test_oracle_matches_the_reference_build(dc, extras):
    H, I, nh, nkv, theta, eps = 64, 96, 8, 2, 1e6, 1e-6
    w, norms, extra, rng = _layer(7, H, I, nh, nkv, dc, extras)
    kvw = H // nh * nkv
    ours, ref = kvo.KvSessionOracle(2, 64, kvw, dc), kvo.RefKvSession(2, 64, kvw, dc)
    pre = kvo.f32_to_u16(rng.standard_normal((2, 20, kvw)).astype(np.float32), dc)
    for sess in (ours, ref):
        assert sess.append(1, pre[0], pre[1], tentative=False) == 0
    packed = [oracle.pack_rows8(w[n]) for n in ("q", "k", "v", "o", "gate", "up", "down")]
    worst = 0.0
    for step in range(6):
        if step == 3:
            ours.rollback()
            ref.rollback()
        h = kvo.f32_to_u16(rng.standard_normal(H).astype(np.float32), dc)
        kw = dict(num_heads=nh, num_kv_heads=nkv, rms_eps=eps, rope_theta=theta)
        a = ours.dense_layer_decode(1, h, norms["in"], norms["post"], *[w[n] for n in
                                    ("q", "k", "v", "o", "gate", "up", "down")], **kw, **extra)
        b = ref.dense_layer_decode_packed_rows8(1, h, norms["in"], norms["post"], packed, hidden_size=H,
                                                intermediate_size=I, **kw, **extra)
        fa, fb = kvo.u16_to_f32(a, dc), kvo.u16_to_f32(b, dc)
        worst = max(worst, float(np.linalg.norm(fa - fb) / np.linalg.norm(fb)))
        if step == 1:
            ours.commit(1)
            ref.commit(1)
    assert worst <= 1e-3
    ka, va = ours.copy_layer(1)
    kb, vb = ref.copy_layer(1)
    assert ka.shape == kb.shape == (20 + 4, kvw)
    ulp = np.abs(ka.astype(np.int32) - kb.astype(np.int32))
    assert ulp.max() <= 1 and np.array_equal(va.shape, vb.shape)
    assert ref.lengths(1) == (ours.committed_length(1), ours.tentative_length(1)) == (21, 3)
    ref.close()

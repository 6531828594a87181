"""KV session and dense layer decode on the GPU (kv_cache.hip) against the
oracle (oracle/kv_dense.py) and, where oracle/_ref is built, the reference's
own fp16_kv_cache.cpp: session fixtures of the reference's tests
(tests/test_native_fp16_kv_cache.py:82-165), decode steps with tentative
rows, commit and rollback, prefill == sequential decode + commit (466-541),
a Qwen2.5-7B-shaped layer over a 1000-row context, and the error codes.
Floating-point results within 1e-3 relative L2; cache rows within one unit
of the 16-bit type."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import kv_dense as kvo

pytestmark = pytest.mark.gpu

NAMES = ("q", "k", "v", "o", "gate", "up", "down")


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_fp16_kv_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


def _t(bits: np.ndarray, dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(dtype).cuda()


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_session_roundtrip_on_device(nat):
    for dtype in (torch.float16, torch.bfloat16):
        s = nat.NativeKvSession(layer_count=2, max_seq_len=16, kv_width=4, dtype=dtype)
        ck = torch.arange(12, dtype=torch.float32).reshape(3, 4).to(dtype)
        tk = (torch.arange(8, dtype=torch.float32).reshape(2, 4) + 1000).to(dtype)
        s.append_committed(0, ck, (ck.float() + 100).to(dtype), count=3)
        s.append_tentative(0, tk, (tk.float() + 100).to(dtype), count=2)
        k, v = s.copy_layer(0)
        assert k.is_cuda and torch.equal(k.cpu(), torch.cat([ck, tk]))
        s.commit(1)
        assert (s.committed_length(0), s.tentative_length(0)) == (4, 1)
        s.rollback()
        k, v = s.copy_layer(0)
        assert torch.equal(k.cpu(), torch.cat([ck, tk[:1]]))
        assert torch.equal(v.cpu(), (torch.cat([ck, tk[:1]]).float() + 100).to(dtype))
        # rollback replaces the tentative suffix (82-131)
        s.append_tentative(0, tk, tk, count=2)
        s.rollback()
        s.append_tentative(0, ck[:2], ck[:2], count=2)
        assert torch.equal(s.copy_layer(0)[0].cpu(), torch.cat([ck, tk[:1], ck[:2]]))
        # committed rows go in front of tentative ones
        s.append_committed(0, tk, tk, count=2)
        k, _ = s.copy_layer(0)
        assert torch.equal(k.cpu(), torch.cat([ck, tk[:1], tk, ck[:2]]))
        assert torch.equal(s.copy_layer(0, include_tentative=False)[0].cpu(), torch.cat([ck, tk[:1], tk]))
        assert s.committed_length(5) == -1
        with pytest.raises(RuntimeError, match="code 2"):
            s.append_tentative(1, torch.zeros((17, 4), dtype=dtype), torch.zeros((17, 4), dtype=dtype), count=17)
        s.close()


def _layer(seed, H, I, nh, nkv, dc, extras, scale=0.1):
    rng = np.random.default_rng(seed)
    kvw = H // nh * nkv
    f = lambda *shape: kvo.f32_to_u16((rng.standard_normal(shape) * scale).astype(np.float32), dc)  # noqa: E731
    w = {"q": f(H, H), "k": f(kvw, H), "v": f(kvw, H), "o": f(H, H), "gate": f(I, H), "up": f(I, H),
         "down": f(H, I)}
    norms = {n: kvo.f32_to_u16((rng.random(H) + 0.5).astype(np.float32), dc) for n in ("in", "post")}
    extra = {}
    if extras:
        extra = {"q_bias": f(H), "k_bias": f(kvw), "v_bias": f(kvw),
                 "q_norm": kvo.f32_to_u16((rng.random(H // nh) + 0.5).astype(np.float32), dc),
                 "k_norm": kvo.f32_to_u16((rng.random(H // nh) + 0.5).astype(np.float32), dc)}
    return w, norms, extra, rng


def _device_layer(nat, w, norms, extra, dtype):
    packed = [nat.pack_weight_rows8(_t(w[n], dtype)) for n in NAMES]
    kw = {"q_bias": "q_bias", "k_bias": "k_bias", "v_bias": "v_bias", "q_norm_weight": "q_norm",
          "k_norm_weight": "k_norm"}
    opt = {k: _t(extra[v], dtype) for k, v in kw.items() if v in extra}
    return [_t(norms["in"], dtype), _t(norms["post"], dtype), *packed], opt


def _rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("dtype,extras,shape,ctx", [
    (torch.float16, False, (8, 16, 2, 1), 30),        # the reference test's layer
    (torch.bfloat16, True, (256, 512, 8, 2), 30),     # biases, q/k norm, head_dim 32
    (torch.float16, True, (512, 384, 4, 4), 30),      # head_dim 128, no grouping
    (torch.bfloat16, False, (960, 640, 15, 5), 30),   # 3 query heads per kv head, head_dim 64
    (torch.float16, False, (480, 256, 12, 4), 200),   # head_dim 40: some lanes without a K piece
    (torch.bfloat16, False, (432, 256, 12, 4), 200),  # head_dim 36: scalar K reads
    (torch.bfloat16, False, (1728, 512, 9, 1), 150),  # 9 query heads per kv head, head_dim 192
    (torch.float16, True, (4096, 512, 16, 1), 300),   # 16 query heads per kv head, head_dim 256: two sum slots
    (torch.bfloat16, False, (960, 640, 15, 5), 1700),  # 32-token splits
    (torch.float16, False, (1024, 256, 32, 8), 2040),  # 64-token splits with 4 query heads per kv head
])
def test_decode_steps_match_the_oracle(nat, dtype, extras, shape, ctx):
    H, I, nh, nkv = shape
    dc = 1 if dtype == torch.bfloat16 else 0
    kvw = H // nh * nkv
    # N(0, 0.02) weights as in the Qwen2.5-7B workload (the reference test's
    # 0.1 for its 8-wide layer): with 0.1 at width 960 the layer is so
    # sensitive that the reference's own build and the float32 oracle differ
    # by 4.9e-3 in bf16.
    w, norms, extra, rng = _layer(H + I, H, I, nh, nkv, dc, extras, scale=0.1 if H <= 8 else 0.02)
    dev_w, opt = _device_layer(nat, w, norms, extra, dtype)
    ours = nat.NativeKvSession(layer_count=2, max_seq_len=ctx + 34, kv_width=kvw, dtype=dtype)
    ora = kvo.KvSessionOracle(2, ctx + 34, kvw, dc)
    pre = kvo.f32_to_u16(rng.standard_normal((2, ctx, kvw)).astype(np.float32), dc)
    ours.append_committed(1, _t(pre[0], dtype), _t(pre[1], dtype), count=ctx)
    ora.append(1, pre[0], pre[1], tentative=False)
    kw = dict(num_heads=nh, num_kv_heads=nkv, rms_eps=1e-6, rope_theta=10000.0)
    for step in range(7):
        if step == 4:
            ours.rollback()
            ora.rollback()
        h = kvo.f32_to_u16(rng.standard_normal(H).astype(np.float32), dc)
        got = ours.dense_layer_decode_packed_rows8(1, _t(h, dtype), *dev_w, hidden_size=H, intermediate_size=I,
                                                   **kw, **opt)
        want = ora.dense_layer_decode(1, h, norms["in"], norms["post"], *[w[n] for n in NAMES], **kw, **extra)
        rel = _rel(kvo.u16_to_f32(_bits(got), dc), kvo.u16_to_f32(want, dc))
        assert rel <= 1e-3, (step, rel)
        if step == 2:
            ours.commit(2)
            ora.commit(2)
    assert (ours.committed_length(1), ours.tentative_length(1)) == (ora.committed_length(1), ora.tentative_length(1))
    k, v = ours.copy_layer(1)
    kw_, vw_ = ora.copy_layer(1)
    for a, b in ((k, kw_), (v, vw_)):
        a = _bits(a)
        assert a.shape == b.shape
        # within one unit in the last place, or (where RoPE cancels, leaving a
        # value far below the row's scale) within 1e-3 of the cache's largest value
        close_bits = np.abs(a.astype(np.int32) - b.astype(np.int32)) <= 1
        af, bf = kvo.u16_to_f32(a, dc), kvo.u16_to_f32(b, dc)
        close_abs = np.abs(af - bf) <= 1e-3 * np.abs(bf).max()
        assert np.all(close_bits | close_abs)
    assert ours.committed_length(0) == 0
    ours.close()


def test_prefill_equals_sequential_decode_and_commit(nat):
    H, I, nh, nkv = 128, 256, 4, 2
    kvw = H // nh * nkv
    w, norms, extra, rng = _layer(3, H, I, nh, nkv, 0, True)
    dev_w, opt = _device_layer(nat, w, norms, extra, torch.float16)
    hidden = _t(kvo.f32_to_u16(rng.standard_normal((5, H)).astype(np.float32), 0), torch.float16).reshape(5, H)
    kw = dict(hidden_size=H, intermediate_size=I, num_heads=nh, num_kv_heads=nkv, rms_eps=1e-6, rope_theta=1e4)
    a = nat.NativeKvSession(layer_count=1, max_seq_len=16, kv_width=kvw)
    out_a = a.dense_layer_prefill_packed_rows8(0, hidden, *dev_w, **kw, **opt)
    b = nat.NativeKvSession(layer_count=1, max_seq_len=16, kv_width=kvw)
    rows = []
    for r in range(5):
        rows.append(b.dense_layer_decode_packed_rows8(0, hidden[r], *dev_w, **kw, **opt))
        b.commit(1)
    assert torch.equal(out_a, torch.stack(rows))
    assert a.committed_length(0) == 5 and a.tentative_length(0) == 0
    for x, y in zip(a.copy_layer(0, include_tentative=False), b.copy_layer(0, include_tentative=False)):
        assert torch.equal(x, y)
    with pytest.raises(RuntimeError, match="code 4"):
        a.dense_layer_prefill_packed_rows8(0, torch.cat([hidden, hidden, hidden]), *dev_w, **kw, **opt)  # 5 + 15 > 16


def test_qwen25_7b_layer_over_a_long_context(nat):
    """hidden 3584, intermediate 18944, 28 query / 4 kv heads of 128, q/k/v
    biases, rope theta 1e6, 1000 committed rows: two decode steps, fp16 as
    the Qwen2.5-7B row8 workload.  (In bf16 the layer's 16-bit roundings of
    the normed input, attention output and residual alone move the result by
    about 1.2e-3 relative, so bf16 is covered at the smaller shapes.)"""
    H, I, nh, nkv = 3584, 18944, 28, 4
    kvw = H // nh * nkv
    w, norms, extra, rng = _layer(11, H, I, nh, nkv, 0, False, scale=0.02)
    extra = {k: kvo.f32_to_u16((rng.standard_normal(n) * 0.1).astype(np.float32), 0)
             for k, n in (("q_bias", H), ("k_bias", kvw), ("v_bias", kvw))}
    dev_w, opt = _device_layer(nat, w, norms, extra, torch.float16)
    ours = nat.NativeKvSession(layer_count=1, max_seq_len=4096, kv_width=kvw, dtype=torch.float16)
    ora = kvo.KvSessionOracle(1, 4096, kvw, 0)
    pre = kvo.f32_to_u16(rng.standard_normal((2, 1000, kvw)).astype(np.float32), 0)
    ours.append_committed(0, _t(pre[0], torch.float16), _t(pre[1], torch.float16), count=1000)
    ora.append(0, pre[0], pre[1], tentative=False)
    kw = dict(num_heads=nh, num_kv_heads=nkv, rms_eps=1e-6, rope_theta=1e6)
    for _ in range(2):
        h = kvo.f32_to_u16(rng.standard_normal(H).astype(np.float32), 0)
        got = ours.dense_layer_decode_packed_rows8(0, _t(h, torch.float16), *dev_w, hidden_size=H,
                                                   intermediate_size=I, **kw, **opt)
        want = ora.dense_layer_decode(0, h, norms["in"], norms["post"], *[w[n] for n in NAMES], **kw, **extra)
        assert _rel(kvo.u16_to_f32(_bits(got), 0), kvo.u16_to_f32(want, 0)) <= 1e-3
    if kvo.ref_available():
        ref = kvo.RefKvSession(1, 4096, kvw, 0)
        ref.append(0, pre[0], pre[1], tentative=False)
        ora2 = kvo.KvSessionOracle(1, 4096, kvw, 0)
        ora2.append(0, pre[0], pre[1], tentative=False)
        packed_host = [_bits(t) for t in dev_w[2:]]
        h = kvo.f32_to_u16(rng.standard_normal(H).astype(np.float32), 0)
        ours.rollback()
        got = ours.dense_layer_decode_packed_rows8(0, _t(h, torch.float16), *dev_w, hidden_size=H,
                                                   intermediate_size=I, **kw, **opt)
        want = ref.dense_layer_decode_packed_rows8(0, h, norms["in"], norms["post"], packed_host, hidden_size=H,
                                                   intermediate_size=I, **kw, **extra)
        assert _rel(kvo.u16_to_f32(_bits(got), 0), kvo.u16_to_f32(want, 0)) <= 1e-3
        ref.close()
    ours.close()


def test_error_codes(nat):
    H, I, nh, nkv = 64, 64, 4, 2
    kvw = H // nh * nkv
    w, norms, extra, _rng = _layer(1, H, I, nh, nkv, 0, False)
    dev_w, _ = _device_layer(nat, w, norms, extra, torch.float16)
    h = torch.zeros(H, dtype=torch.float16, device="cuda")
    s = nat.NativeKvSession(layer_count=1, max_seq_len=2, kv_width=kvw)
    kw = dict(hidden_size=H, intermediate_size=I, rms_eps=1e-6, rope_theta=1e4)
    with pytest.raises(RuntimeError, match="code 101"):
        s.dense_layer_decode_packed_rows8(3, h, *dev_w, num_heads=nh, num_kv_heads=nkv, **kw)
    with pytest.raises(RuntimeError, match="code 103"):
        s.dense_layer_decode_packed_rows8(0, h, *dev_w, num_heads=nh, num_kv_heads=3, **kw)
    with pytest.raises(RuntimeError, match="code 104"):
        s.dense_layer_decode_packed_rows8(0, h, *dev_w, num_heads=nh, num_kv_heads=1, **kw)
    s.dense_layer_decode_packed_rows8(0, h, *dev_w, num_heads=nh, num_kv_heads=nkv, **kw)
    s.dense_layer_decode_packed_rows8(0, h, *dev_w, num_heads=nh, num_kv_heads=nkv, **kw)
    with pytest.raises(RuntimeError, match="code 105"):
        s.dense_layer_decode_packed_rows8(0, h, *dev_w, num_heads=nh, num_kv_heads=nkv, **kw)
    s.close()
    w32, norms32, _e, _r = _layer(2, H, I, 32, 1, 0, False)  # 32 query heads of 2 on one kv head
    dev_w32, _ = _device_layer(nat, w32, norms32, {}, torch.float16)
    big = nat.NativeKvSession(layer_count=1, max_seq_len=4, kv_width=H // 32)
    with pytest.raises(RuntimeError, match="code 106"):
        big.dense_layer_decode_packed_rows8(0, h, *dev_w32, num_heads=32, num_kv_heads=1, **kw)
    with pytest.raises(ValueError):  # weights of another layer shape never reach the kernels
        big.dense_layer_decode_packed_rows8(0, h, *dev_w, num_heads=32, num_kv_heads=1, **kw)
    big.close()

"""CPU oracle for DeepSeek multi-head latent attention (MLA) decode.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline
leg as the checker, never by the product.

src/pcketlm/native/ds_forward.cpp does not build here (it includes
<windows.h>), so nothing of the reference runs.  Two restatements, pinned
against each other and against closed forms in tests/test_mla_oracle.py:

``mla_flash_online`` follows ds_mla_attention_flash_forward
(ds_forward.cpp:517-597) step by step in numpy float32: per head, the
absorbed query q_abs = q_nope . Wk (552-560), then one cache position at a
time the score (q_abs . kv + q_pe . pe) * scale (563-568), the running max
with the rescale of the accumulator (569-577), inv_sum = 1 / sum or 0
(580-583), and the value rows of kv_b (588-594).  The dot products use
numpy's float32 summation, not the reference's 8-lane AVX2 order.

``mla_flash_closed_form`` is the reference's own Python formulation of the
same attention (native/__init__.py:857-876: einsum, softmax, einsum) in
float64: the value the float32 computations approximate.

``fp8_attention_block`` follows the FP8 model's one-token attention
(core/runtime/fp8_source.py:6337-6454): the native FP8 linear (the C
oracle's ``fp8_linear``, pinned to the reference's fp8_linear.cpp) for q_a
(6373), q_b (6384) and kv_a (6393) on fp32 activations, RMSNorm
(``_rms_norm_any``, 5311-5317: x * rsqrt(mean(x^2) + eps) * w), RoPE on
pairs (``_apply_rope_real``, 5191-5209), the latent and pe rows appended
after the previous rows (6422-6428), kv_b as fp32 (dequantized, 6399-6402),
the absorbed-query attention (6429-6451: one query row, so no causal mask)
and o as an FP8 linear (6452-6458).

``attention_block`` follows ds_attention_block_forward_f32
(ds_forward.cpp:647-782): q_a (698), RMSNorm (699; 610-619), q_b split into
nope / pe (701-713), RoPE on the pe parts (714-716; 621-645: an odd rope
width is left unrotated), the previous rows copied and the new latent row
(kv_a, RMSNorm) and pe row (kv_a, RoPE) appended (718-744), the MLA above
over previous_len + 1 rows (746-763), then o (769).
"""

from __future__ import annotations

import numpy as np

f32 = np.float32


def mla_flash_online(q_nope, q_pe, kv, pe, wkv_b, scale):
    """ds_forward.cpp:517-597 in float32; returns out [H, v]."""
    q_nope = np.asarray(q_nope, f32)
    q_pe = np.asarray(q_pe, f32)
    kv = np.asarray(kv, f32)
    pe = np.asarray(pe, f32)
    wkv_b = np.asarray(wkv_b, f32)
    H, nope = q_nope.shape
    rope = q_pe.shape[1]
    L, R = kv.shape
    v = wkv_b.shape[1] - nope
    out = np.empty((H, v), dtype=f32)
    scale = f32(scale)
    for h in range(H):
        wk = wkv_b[h, :nope]            # [nope, R]
        q_abs = (q_nope[h][:, None] * wk).sum(axis=0, dtype=f32) if nope else np.zeros(R, f32)
        acc = np.zeros(R, dtype=f32)
        run_max = f32(-np.inf)
        run_sum = f32(0.0)
        for t in range(L):
            score = f32(np.dot(q_abs, kv[t]))
            if rope > 0:
                score = f32(score + f32(np.dot(q_pe[h], pe[t])))
            score = f32(score * scale)
            new_max = run_max if run_max > score else score
            old_scale = f32(np.exp(f32(run_max - new_max))) if np.isfinite(run_max) else f32(0.0)
            s_scale = f32(np.exp(f32(score - new_max)))
            acc = (acc * old_scale + kv[t] * s_scale).astype(f32)
            run_sum = f32(run_sum * old_scale + s_scale)
            run_max = new_max
        inv = f32(1.0) / run_sum if run_sum > 0 else f32(0.0)
        acc = (acc * inv).astype(f32)
        out[h] = (wkv_b[h, nope:nope + v] @ acc).astype(f32)
    return out


def mla_flash_closed_form(q_nope, q_pe, kv, pe, wkv_b, scale):
    """native/__init__.py:857-876 (einsum / softmax / einsum) in float64."""
    q_nope = np.asarray(q_nope, np.float64)
    q_pe = np.asarray(q_pe, np.float64)
    kv = np.asarray(kv, np.float64)
    pe = np.asarray(pe, np.float64)
    w = np.asarray(wkv_b, np.float64)
    nope = q_nope.shape[1]
    v = w.shape[1] - nope
    q_abs = np.einsum("hd,hdc->hc", q_nope, w[:, :nope])
    scores = (np.einsum("hc,tc->ht", q_abs, kv) + np.einsum("hr,tr->ht", q_pe, pe)) * float(scale)
    scores -= scores.max(axis=1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=1, keepdims=True)
    latent = p @ kv
    return np.einsum("hc,hdc->hd", latent, w[:, nope:nope + v])


def rms_norm(x, w, eps):
    """ds_forward.cpp:610-619: x * (1 / sqrt(mean(x^2) + eps)) * w."""
    x = np.asarray(x, f32)
    ss = f32((x.astype(np.float64) ** 2).sum())
    inv = f32(1.0) / f32(np.sqrt(f32(ss / f32(x.size) + f32(eps))))
    return (x * inv * np.asarray(w, f32)).astype(f32)


def rope(x, cos, sin):
    """ds_forward.cpp:621-645 on one group: pairs (x0, x1) rotated; an odd
    width is returned unchanged."""
    x = np.asarray(x, f32).copy()
    if x.size == 0 or x.size % 2:
        return x
    x0, x1 = x[0::2].copy(), x[1::2].copy()
    c, s = np.asarray(cos, f32), np.asarray(sin, f32)
    x[0::2] = x0 * c - x1 * s
    x[1::2] = x0 * s + x1 * c
    return x


def attention_block(hidden, q_a, q_b, kv_a, kv_b, o, q_norm, kv_norm, prev_kv, prev_pe, cos, sin, *, num_heads,
                    qk_nope_dim, qk_rope_dim, v_head_dim, kv_lora_rank, rms_eps, softmax_scale,
                    flash=mla_flash_online):
    """ds_forward.cpp:647-782; returns (hidden_out, next_kv, next_pe)."""
    H, nope, rp, v, R = num_heads, qk_nope_dim, qk_rope_dim, v_head_dim, kv_lora_rank
    hidden = np.asarray(hidden, f32).reshape(-1)
    q_low = rms_norm((np.asarray(q_a, f32) @ hidden).astype(f32), q_norm, rms_eps)
    q = (np.asarray(q_b, f32) @ q_low).astype(f32).reshape(H, nope + rp)
    q_nope = q[:, :nope]
    q_pe = np.stack([rope(q[h, nope:], cos, sin) for h in range(H)]) if rp else np.zeros((H, 0), f32)
    kv_raw = (np.asarray(kv_a, f32) @ hidden).astype(f32)
    new_kv = rms_norm(kv_raw[:R], kv_norm, rms_eps)
    new_pe = rope(kv_raw[R:], cos, sin)
    prev_kv = np.zeros((0, R), f32) if prev_kv is None else np.asarray(prev_kv, f32).reshape(-1, R)
    prev_pe = np.zeros((0, rp), f32) if prev_pe is None else np.asarray(prev_pe, f32).reshape(-1, rp)
    next_kv = np.concatenate([prev_kv, new_kv[None]], axis=0)
    next_pe = np.concatenate([prev_pe, new_pe[None]], axis=0)
    heads = np.asarray(flash(q_nope, q_pe, next_kv, next_pe, np.asarray(kv_b, f32).reshape(H, nope + v, R),
                             softmax_scale), f32).reshape(-1)
    return (np.asarray(o, f32) @ heads).astype(f32), next_kv, next_pe


def rms_norm_rsqrt(x, w, eps):
    """fp8_source.py:5311-5317 in float32: x * rsqrt(mean(x^2) + eps) * w."""
    x = np.asarray(x, f32)
    var = f32(np.mean(x.astype(np.float64) ** 2))
    return (x * f32(1.0 / np.sqrt(np.float64(var) + np.float64(eps))) * np.asarray(w, f32)).astype(f32)


def fp8_attention_block(hidden, fp8, kv_b, q_norm, kv_norm, prev_kv, prev_pe, cos, sin, *, num_heads, qk_nope_dim,
                        qk_rope_dim, v_head_dim, kv_lora_rank, rms_eps, softmax_scale, flash=mla_flash_online):
    """fp8_source.py:6337-6454 at one token.  fp8: {"q_a"|"q_b"|"kv_a"|"o":
    (e4m3 bytes [N, K], scale_inv [ceil(N/128), ceil(K/128)])}; kv_b fp32
    [H (nope + v), R].  Returns (hidden_out fp32, next_kv, next_pe)."""
    import oracle  # the C oracle (fp8_linear pinned to the reference build)

    H, nope, rp, v, R = num_heads, qk_nope_dim, qk_rope_dim, v_head_dim, kv_lora_rank
    x = np.asarray(hidden, f32).reshape(1, -1)
    q_low = rms_norm_rsqrt(oracle.fp8_linear(*fp8["q_a"], x).reshape(-1), q_norm, rms_eps)
    q = oracle.fp8_linear(*fp8["q_b"], q_low.reshape(1, -1)).reshape(H, nope + rp)
    kv_raw = oracle.fp8_linear(*fp8["kv_a"], x).reshape(-1)
    q_nope = q[:, :nope]
    q_pe = np.stack([rope(q[h, nope:], cos, sin) for h in range(H)]) if rp else np.zeros((H, 0), f32)
    new_kv = rms_norm_rsqrt(kv_raw[:R], kv_norm, rms_eps)
    new_pe = rope(kv_raw[R:], cos, sin)
    prev_kv = np.zeros((0, R), f32) if prev_kv is None else np.asarray(prev_kv, f32).reshape(-1, R)
    prev_pe = np.zeros((0, rp), f32) if prev_pe is None else np.asarray(prev_pe, f32).reshape(-1, rp)
    next_kv = np.concatenate([prev_kv, new_kv[None]], axis=0)
    next_pe = np.concatenate([prev_pe, new_pe[None]], axis=0)
    heads = np.asarray(flash(q_nope, q_pe, next_kv, next_pe, np.asarray(kv_b, f32).reshape(H, nope + v, R),
                             softmax_scale), f32).reshape(1, -1)
    return oracle.fp8_linear(*fp8["o"], heads).reshape(-1), next_kv, next_pe


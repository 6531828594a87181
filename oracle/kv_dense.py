"""CPU oracle for the KV session and the dense decoder layer decode.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline
leg as the checker, never by the product.

``KvSessionOracle`` restates src/pcketlm/native/fp16_kv_cache.cpp in numpy
float32, step by step in the reference's order:
  - the session (12-46, 594-778): committed and tentative rows per layer,
    append / commit / rollback / copy;
  - ``dense_layer_decode`` (1398-1531, with the attention decode 920-1060):
    rms_norm_one (541-559), q/k/v with biases, rms_norm_heads_inplace
    (561-584), apply_rope_one (518-539), the new k/v rounded and appended as
    a tentative row, softmax attention over every row, o projection,
    residual, post norm, SiLU MLP (1493-1529).
The matrix-vector products use numpy's float32 matmul (a different summation
order from the reference's AVX2 loops), so results agree to float32 rounding
and to one unit of the 16-bit type where a rounding boundary falls between.

``RefKvSession`` drives the reference's own fp16_kv_cache.cpp compiled from
source into oracle/_ref (``make -C oracle ref``) through its C ABI, for the
tests that pin this restatement.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_REF_SO = Path(__file__).resolve().parent / "_ref" / "libref_fp16_kv_cache.so"


def u16_to_f32(bits: np.ndarray, dtype_code: int) -> np.ndarray:
    """read_u16 (fp16_kv_cache.cpp:50-79)."""
    bits = np.asarray(bits, dtype=np.uint16)
    if dtype_code == 1:
        return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def f32_to_u16(values: np.ndarray, dtype_code: int) -> np.ndarray:
    """write_u16 (fp16_kv_cache.cpp:56-83): fp16 round-to-nearest-even; bf16
    by adding 0x7FFF + lsb and truncating (no NaN special case)."""
    values = np.asarray(values, dtype=np.float32)
    if dtype_code == 1:
        bits = values.view(np.uint32)
        return ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    return values.astype(np.float16).view(np.uint16)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x * (1 / sqrt(mean(x^2) + eps)) * w over the last axis, float32."""
    x = x.astype(np.float32)
    ms = np.float32(np.sum(x * x, axis=-1, keepdims=True, dtype=np.float32) / np.float32(x.shape[-1]))
    scale = np.float32(1.0) / np.sqrt(ms + np.float32(eps))
    return (x * scale) * w.astype(np.float32)


def rope(values: np.ndarray, position: int, theta: float) -> np.ndarray:
    """apply_rope_one (518-539) on [heads, head_dim] float32."""
    heads, hd = values.shape
    half = hd // 2
    dims = np.arange(half, dtype=np.float32)
    inv_freq = np.power(np.float32(theta), -(np.float32(2.0) * dims) / np.float32(hd)).astype(np.float32)
    angle = np.float32(position) * inv_freq
    c, s = np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)
    out = values.astype(np.float32).copy()
    x0, x1 = values[:, :half].astype(np.float32), values[:, half:2 * half].astype(np.float32)
    out[:, :half] = x0 * c - x1 * s
    out[:, half:2 * half] = x1 * c + x0 * s
    return out


class KvSessionOracle:
    def __init__(self, layer_count: int, max_seq_len: int, kv_width: int, dtype_code: int = 0):
        self.max_seq_len = int(max_seq_len)
        self.kv_width = int(kv_width)
        self.dtype_code = int(dtype_code)
        empty = np.zeros((0, kv_width), np.uint16)
        self.committed = [[empty, empty] for _ in range(layer_count)]
        self.tentative = [[empty, empty] for _ in range(layer_count)]

    def committed_length(self, layer: int) -> int:
        return self.committed[layer][0].shape[0]

    def tentative_length(self, layer: int) -> int:
        return self.tentative[layer][0].shape[0]

    def append(self, layer: int, k: np.ndarray, v: np.ndarray, *, tentative: bool) -> int:
        """append_to_region (626-659)."""
        k = np.asarray(k, np.uint16).reshape(-1, self.kv_width)
        v = np.asarray(v, np.uint16).reshape(-1, self.kv_width)
        if self.committed_length(layer) + self.tentative_length(layer) + k.shape[0] > self.max_seq_len:
            return 2
        region = self.tentative if tentative else self.committed
        region[layer] = [np.concatenate([region[layer][0], k]), np.concatenate([region[layer][1], v])]
        return 0

    def commit(self, count: int) -> None:
        """kv_commit (681-715)."""
        for layer in range(len(self.committed)):
            take = min(count, self.tentative_length(layer))
            for i in range(2):
                self.committed[layer][i] = np.concatenate([self.committed[layer][i], self.tentative[layer][i][:take]])
                self.tentative[layer][i] = self.tentative[layer][i][take:]

    def rollback(self) -> None:
        """kv_rollback (717-728)."""
        for layer in range(len(self.tentative)):
            self.tentative[layer] = [self.tentative[layer][0][:0], self.tentative[layer][1][:0]]

    def copy_layer(self, layer: int, include_tentative: bool = True) -> tuple[np.ndarray, np.ndarray]:
        """kv_copy_layer (746-778)."""
        if not include_tentative:
            return self.committed[layer][0].copy(), self.committed[layer][1].copy()
        return (np.concatenate([self.committed[layer][0], self.tentative[layer][0]]),
                np.concatenate([self.committed[layer][1], self.tentative[layer][1]]))

    def dense_layer_decode(self, layer: int, hidden, input_norm, post_norm, q_w, k_w, v_w, o_w, gate_w, up_w,
                           down_w, *, num_heads: int, num_kv_heads: int, rms_eps: float, rope_theta: float,
                           q_bias=None, k_bias=None, v_bias=None, q_norm=None, k_norm=None) -> np.ndarray:
        """kv_dense_layer_decode_u16_ext (1398-1531).  Weights are row-major
        [out, in] 16-bit bit patterns (the packed entry point computes the
        same products from the row8 layout); returns the output bits."""
        dc = self.dtype_code
        rd = lambda a: u16_to_f32(a, dc)  # noqa: E731
        wr = lambda a: f32_to_u16(a, dc)  # noqa: E731
        h = rd(hidden)
        hidden_size = h.shape[0]
        hd = hidden_size // num_heads
        group = num_heads // num_kv_heads
        xn = rd(wr(rms_norm(h, rd(input_norm), rms_eps)))

        def linear(w, x, bias=None):
            y = rd(w).astype(np.float32) @ x.astype(np.float32)
            return y if bias is None else y + rd(bias)

        q = linear(q_w, xn, q_bias).reshape(num_heads, hd)
        k = linear(k_w, xn, k_bias).reshape(num_kv_heads, hd)
        v = linear(v_w, xn, v_bias).reshape(num_kv_heads, hd)
        if q_norm is not None:
            q = rms_norm(q, rd(q_norm), rms_eps)
        if k_norm is not None:
            k = rms_norm(k, rd(k_norm), rms_eps)
        position = self.committed_length(layer) + self.tentative_length(layer)
        q = rope(q, position, rope_theta)
        k = rope(k, position, rope_theta)
        code = self.append(layer, wr(k).reshape(1, -1), wr(v).reshape(1, -1), tentative=True)
        if code:
            raise RuntimeError(f"cache full (code {code})")
        keys, values = self.copy_layer(layer)
        keys = rd(keys).reshape(-1, num_kv_heads, hd)
        values = rd(values).reshape(-1, num_kv_heads, hd)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        context = np.zeros((num_heads, hd), np.float32)
        for head in range(num_heads):
            kvh = head // group
            scores = (keys[:, kvh] @ q[head]) * scale
            e = np.exp(scores - scores.max()).astype(np.float32)
            context[head] = (e / e.sum(dtype=np.float32)) @ values[:, kvh]
        attention_out = wr(linear(o_w, context.reshape(-1)))
        resid = h + rd(attention_out)
        post = rd(wr(rms_norm(rd(wr(resid)), rd(post_norm), rms_eps)))
        g = linear(gate_w, post)
        act = (g / (np.float32(1.0) + np.exp(-g))) * linear(up_w, post)
        return wr(resid + linear(down_w, act.astype(np.float32)))


# --------------------------------------------------------------------------- the reference, built from source

def ref_available() -> bool:
    return _REF_SO.exists()


def _ref_lib() -> ctypes.CDLL:
    lib = ctypes.CDLL(str(_REF_SO))
    i64, vp = ctypes.c_longlong, ctypes.c_void_p
    lib.kv_prefill_init_typed.argtypes = [i64, i64, i64, ctypes.c_int]
    lib.kv_prefill_init_typed.restype = vp
    lib.kv_free.argtypes = [vp]
    lib.kv_append_committed.argtypes = [vp, i64, vp, vp, i64]
    lib.kv_append_tentative.argtypes = [vp, i64, vp, vp, i64]
    lib.kv_commit.argtypes = [vp, i64]
    lib.kv_rollback.argtypes = [vp]
    lib.kv_copy_layer.argtypes = [vp, i64, vp, vp, i64, ctypes.c_int]
    for name in ("kv_committed_length", "kv_tentative_length"):
        getattr(lib, name).argtypes = [vp, i64]
        getattr(lib, name).restype = i64
    lib.kv_dense_layer_decode_u16_ext_packed_rows8.argtypes = [vp, i64] + [vp] * 16 + [i64] * 4 + [
        ctypes.c_float, ctypes.c_float]
    return lib


def _ptr(a):
    return ctypes.c_void_p(0 if a is None else a.ctypes.data)


class RefKvSession:
    """The reference's session (host memory) through its own C ABI."""

    def __init__(self, layer_count: int, max_seq_len: int, kv_width: int, dtype_code: int = 0):
        self.lib = _ref_lib()
        self.kv_width = kv_width
        self.h = self.lib.kv_prefill_init_typed(layer_count, max_seq_len, kv_width, dtype_code)
        assert self.h

    def close(self):
        if self.h:
            self.lib.kv_free(self.h)
            self.h = None

    def append(self, layer, k, v, *, tentative: bool) -> int:
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        fn = self.lib.kv_append_tentative if tentative else self.lib.kv_append_committed
        return fn(self.h, layer, _ptr(k), _ptr(v), k.size // self.kv_width)

    def commit(self, count):
        return self.lib.kv_commit(self.h, count)

    def rollback(self):
        return self.lib.kv_rollback(self.h)

    def lengths(self, layer):
        return self.lib.kv_committed_length(self.h, layer), self.lib.kv_tentative_length(self.h, layer)

    def copy_layer(self, layer, include_tentative=True):
        c, t = self.lengths(layer)
        n = c + (t if include_tentative else 0)
        k = np.zeros((n, self.kv_width), np.uint16)
        v = np.zeros((n, self.kv_width), np.uint16)
        assert self.lib.kv_copy_layer(self.h, layer, _ptr(k), _ptr(v), n, 1 if include_tentative else 0) == 0
        return k, v

    def dense_layer_decode_packed_rows8(self, layer, hidden, input_norm, post_norm, packed, *, hidden_size,
                                        intermediate_size, num_heads, num_kv_heads, rms_eps, rope_theta,
                                        q_bias=None, k_bias=None, v_bias=None, q_norm=None, k_norm=None):
        """packed: the seven row8-packed weights (q, k, v, o, gate, up, down)."""
        arrs = [np.ascontiguousarray(a, np.uint16) if a is not None else None
                for a in [hidden, input_norm, post_norm, *packed, q_bias, k_bias, v_bias, q_norm, k_norm]]
        out = np.zeros(hidden_size, np.uint16)
        code = self.lib.kv_dense_layer_decode_u16_ext_packed_rows8(
            self.h, layer, *[_ptr(a) for a in arrs], _ptr(out), hidden_size, intermediate_size, num_heads,
            num_kv_heads, ctypes.c_float(rms_eps), ctypes.c_float(rope_theta))
        if code:
            raise RuntimeError(f"reference dense layer decode failed with code {code}")
        return out

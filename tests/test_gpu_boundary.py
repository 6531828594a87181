"""The loader-required entry points on the device: the DeepSeek session's
callback bridges copy the callback's fp32 output from device or host
memory into device or host buffers (ds_forward.cpp:369-512), and the
row-major KV entry points return their documented code 90.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from pocketlm_amd import _lib

    lib = _lib.load()
    assert lib.pocketlm_device_available() == 1, "libpocketlm_hip.so must find the gfx950 device"
    lib.pocketlm_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return lib


def _cb_source(where: str, n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(n, generator=g)
    return t.cuda() if where == "device" else t


@pytest.mark.parametrize("src_where,dst_where", [("device", "device"), ("host", "device"), ("device", "host")])
def test_ds_bridges_copy_callback_output(lib, src_where, dst_where):
    from pocketlm_amd import _lib

    layers, hidden, vocab = 4, 32, 100
    h = lib.ds_session_create(layers, hidden, 8, 2, None, None)
    assert h
    seen = []
    srcs = {}

    def dst(n):
        t = torch.full((n,), -7.0)
        return t.cuda() if dst_where == "device" else t

    @_lib.DS_ATTENTION_CALLBACK
    def attn(layer, hidden_in, batch, hidden_dim, out_pp, out_count):
        seen.append(("attn", layer, batch, hidden_dim, hidden_in))
        t = srcs.setdefault("attn", _cb_source(src_where, batch * hidden_dim, 1))
        out_pp[0] = t.data_ptr()
        out_count[0] = t.numel()
        return 0

    @_lib.DS_DECODE_CALLBACK
    def dec(token, out_pp, out_count):
        seen.append(("decode", token))
        t = srcs.setdefault("decode", _cb_source(src_where, vocab, 2))
        out_pp[0] = t.data_ptr()
        out_count[0] = vocab
        return 0

    @_lib.DS_PREFILL_CALLBACK
    def pre(ids, n, out_pp, out_count):
        seen.append(("prefill", [ctypes.cast(ids, ctypes.POINTER(ctypes.c_longlong))[i] for i in range(n)]))
        t = srcs.setdefault("prefill", _cb_source(src_where, vocab, 3))
        out_pp[0] = t.data_ptr()
        out_count[0] = vocab
        return 0

    @_lib.DS_VERIFY_CALLBACK
    def ver(ids, k, out_pp, out_count):
        seen.append(("verify", k))
        t = srcs.setdefault("verify", _cb_source(src_where, k * vocab, 4))
        out_pp[0] = t.data_ptr()
        out_count[0] = k * vocab
        return 0

    x = torch.randn(2 * hidden).cuda()
    out = dst(2 * hidden)
    assert lib.ds_attention_layer_forward_f32(h, 3, ctypes.c_void_p(x.data_ptr()), 2, hidden, attn,
                                              ctypes.c_void_p(out.data_ptr())) == 0
    assert torch.equal(out.cpu(), srcs["attn"].cpu())
    assert seen[-1][:4] == ("attn", 3, 2, hidden) and seen[-1][4] == x.data_ptr()

    logits = dst(vocab)
    assert lib.ds_forward_decode_f32(h, 42, dec, ctypes.c_void_p(logits.data_ptr()), vocab) == 0
    assert torch.equal(logits.cpu(), srcs["decode"].cpu()) and seen[-1] == ("decode", 42)

    toks = (ctypes.c_longlong * 3)(5, 6, 7)
    logits2 = dst(vocab)
    assert lib.ds_forward_prefill_f32(h, ctypes.cast(toks, ctypes.c_void_p), 3, pre,
                                      ctypes.c_void_p(logits2.data_ptr()), vocab) == 0
    assert torch.equal(logits2.cpu(), srcs["prefill"].cpu()) and seen[-1] == ("prefill", [5, 6, 7])

    per_pos = dst(2 * vocab)
    assert lib.ds_forward_verify_f32(h, ctypes.cast(toks, ctypes.c_void_p), 2, ver,
                                     ctypes.c_void_p(per_pos.data_ptr()), vocab) == 0
    assert torch.equal(per_pos.cpu(), srcs["verify"].cpu())

    assert lib.ds_callback_invocation_count(h) == 4
    assert lib.ds_monolithic_call_counter(h) == 4
    assert lib.ds_attention_invocation_count(h) == 1
    assert lib.ds_layers_executed_count(h) == layers * (1 + 3 + 2)
    lib.ds_session_destroy(h)


def test_rowmajor_kv_entry_points_return_90(lib):
    from pocketlm_amd import _lib

    sess = lib.kv_prefill_init_typed(1, 4, 8, 0)
    assert sess
    t = torch.zeros(64, dtype=torch.float16, device="cuda")
    p = ctypes.c_void_p(t.data_ptr())
    assert lib.kv_attention_decode_fp16(sess, 0, *([p] * 6), 8, 1, 1, 1e4) == 90
    assert "native_pack_u16_rows8" in _lib.last_error()
    assert lib.kv_attention_decode_u16_ext(sess, 0, *([p] * 11), 8, 1, 1, 1e4, 1e-6) == 90
    assert lib.kv_dense_layer_decode_fp16(sess, 0, *([p] * 11), 8, 16, 1, 1, 1e-6, 1e4) == 90
    assert lib.kv_dense_layer_decode_u16_ext(sess, 0, *([p] * 16), 8, 16, 1, 1, 1e-6, 1e4) == 90
    assert lib.kv_attention_decode_fp16(sess, 1, *([p] * 6), 8, 1, 1, 1e4) == 1
    assert lib.kv_committed_length(sess, 0) == 0 and lib.kv_tentative_length(sess, 0) == 0
    lib.kv_free(sess)

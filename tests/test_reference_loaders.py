"""The reference's own ctypes loaders accept this library.

Each reference loader in src/pcketlm/native/__init__.py binds some symbols
unconditionally (a missing one raises inside the loader, which then returns
None and disables the whole family) and probes others with ``hasattr``.
The lists below are those unconditional bindings with the number of
arguments each argtypes list declares, transcribed per loader with the
line of each binding.  The tests check that the built library exports every
one of them and that the header and the Python binding declare the same
argument count.  The DeepSeek session's callback bridges are then called
through the C ABI on the CPU for their argument and callback checks.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from pocketlm_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "pocketlm_hip.h"

# (symbol, argument count, native/__init__.py line of the binding)
REFERENCE_LOADERS = {
    "_load_q4_lib (160-195)": [
        ("q4_dequant_to_fp16", 5, 160),
        ("q4_cpu_has_avx2_f16c", 0, 194),
    ],
    "_load_fp8_dequant_lib (270-290)": [
        ("fp8_dequant_cpu_has_avx2_f16c", 0, 270),
        ("fp8_e4m3_dequant_to_fp16", 6, 272),
    ],
    "_load_fp8_linear_lib (322-442)": [
        ("fp8_e4m3_block_linear_f32", 8, 322),
    ],
    "_load_fp8_linear_avx512_lib (462-501)": [
        ("fp8_linear_avx512_cpu_has_avx512", 0, 462),
        ("fp8_e4m3_block_mlp_many_weighted_avx512_f32", 15, 484),
    ],
    "_load_ds_forward_lib (563-737)": [
        ("ds_cpu_has_avx2", 0, 574),
        ("ds_session_create", 6, 576),
        ("ds_session_destroy", 1, 585),
        ("ds_session_register_layer", 6, 587),
        ("ds_monolithic_call_counter", 1, 596),
        ("ds_callback_invocation_count", 1, 598),
        ("ds_expert_invocation_count", 1, 600),
        ("ds_attention_invocation_count", 1, 602),
        ("ds_layers_executed_count", 1, 607),
        ("ds_registered_layer_count", 1, 609),
        ("ds_registered_fp8_nbytes", 2, 611),
        ("ds_registered_scale_nbytes", 2, 613),
        ("ds_router_topk_u16", 8, 615),
        ("ds_moe_layer_forward_f32", 7, 626),
        ("ds_attention_layer_forward_f32", 7, 636),
        ("ds_forward_decode_f32", 5, 646),
        ("ds_forward_prefill_f32", 6, 654),
        ("ds_forward_verify_f32", 6, 663),
        ("ds_moe_layer_forward_fp8_f32", 16, 719),
    ],
    "_load_fp16_matmul_lib (1573-1581)": [
        ("native_fp16_matmul", 6, 1573),
    ],
    "_load_fp16_packed_gemv_lib (1634-1649)": [
        ("native_pack_u16_rows8", 4, 1634),
        ("native_packed_gemv_rows8", 6, 1641),
    ],
    "_load_row8_artifact_lib (1678-1701)": [
        ("row8_artifact_load_tensor", 3, 1678),
        ("row8_artifact_free_tensor", 1, 1684),
        ("row8_artifact_tensor_data", 1, 1686),
        ("row8_artifact_tensor_nbytes", 1, 1688),
        ("row8_artifact_map_file", 1, 1690),
        ("row8_artifact_unmap_file", 1, 1692),
        ("row8_artifact_mapped_data", 3, 1694),
        ("row8_artifact_mapped_nbytes", 1, 1700),
    ],
    "_load_fp16_kv_lib (2588-2745)": [
        ("kv_prefill_init", 3, 2588),
        ("kv_prefill_init_typed", 4, 2590),
        ("kv_free", 1, 2592),
        ("kv_append_committed", 5, 2594),
        ("kv_append_tentative", 5, 2594),
        ("kv_commit", 2, 2598),
        ("kv_rollback", 1, 2600),
        ("kv_committed_length", 2, 2602),
        ("kv_tentative_length", 2, 2604),
        ("kv_copy_layer", 6, 2606),
        ("kv_attention_decode_fp16", 12, 2615),
        ("kv_attention_decode_u16_ext", 18, 2630),
        ("kv_dense_layer_decode_fp16", 19, 2674),
        ("kv_dense_layer_decode_u16_ext", 24, 2720),
    ],
}

# Bound by the same loaders behind hasattr: optional for the reference, but
# exported here with the same argument count where the header declares them.
REFERENCE_OPTIONAL = [
    ("q4_dequant_many_to_fp16", 6), ("q4_moe_selected_forward_u16", 12), ("fp8_e4m3_dequant_to_bf16", 6),
    ("fp8_e4m3_block_dual_linear_f32", 11), ("fp8_e4m3_block_mlp_f32", 13), ("fp8_e4m3_block_mlp_many_f32", 14),
    ("fp8_e4m3_block_mlp_many_weighted_f32", 15), ("fp8_e4m3_block_mlp_many_row_weighted_f32", 15),
    ("fp8_e4m3_block_mlp_many_pair_weighted_f32", 18), ("fp8_e4m3_block_mlp_avx512_f32", 13),
    ("ds_fused_attention_invocation_count", 1), ("kv_dense_layer_decode_u16_ext_packed_rows8", 24),
    # bound behind hasattr by _load_ds_forward_lib (native/__init__.py:672-718)
    ("ds_mla_attention_flash_forward", 13), ("ds_attention_block_forward_f32", 26),
]


def header_arg_counts() -> dict[str, int]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"typedef[^;]*;", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from pocketlm_amd import build

        build.build()
    return _lib.load()


@pytest.fixture(scope="module")
def raw():
    """A plain CDLL of the library, as the reference's loaders open it."""
    if not _lib.LIB_PATH.exists():
        from pocketlm_amd import build

        build.build()
    return ctypes.CDLL(str(_lib.LIB_PATH))


@pytest.mark.parametrize("loader", sorted(REFERENCE_LOADERS))
def test_every_unguarded_binding_is_exported(raw, loader):
    counts = header_arg_counts()
    for name, nargs, line in REFERENCE_LOADERS[loader]:
        assert hasattr(raw, name), f"{loader}: {name} (native/__init__.py:{line}) is not exported"
        assert counts.get(name) == nargs, f"{name}: header declares {counts.get(name)} arguments, reference {nargs}"
        assert len(_lib._SIGNATURES[name][1]) == nargs, f"{name}: binding argument count"


def test_optional_bindings_keep_the_reference_argument_counts(raw):
    counts = header_arg_counts()
    for name, nargs in REFERENCE_OPTIONAL:
        assert hasattr(raw, name), name
        assert counts.get(name) == nargs, name
        assert len(_lib._SIGNATURES[name][1]) == nargs, name


def test_feature_probes_do_not_fail_the_loaders_without_a_device(raw):
    # The reference loaders reject the library when a probe returns != 1.  On
    # a machine without a gfx950 device the probes return 0, so the reference
    # families are (correctly) unavailable rather than silently wrong.
    for probe in ("fp8_dequant_cpu_has_avx2_f16c", "fp8_linear_avx512_cpu_has_avx512", "q4_cpu_has_avx2_f16c",
                  "ds_cpu_has_avx2"):
        fn = getattr(raw, probe)
        fn.restype = ctypes.c_int
        assert fn() in (0, 1)


def _session(lib, layers=3):
    handle = lib.ds_session_create(layers, 8, 4, 2, None, None)
    assert handle
    return handle


def test_ds_callback_bridges_argument_and_callback_codes(lib):
    """Codes of ds_forward.cpp:369-512 that return before any copy: null
    handle / pointer / callback -> 1, bad sizes or layer -> 2, callback
    failure k -> 10 + k, null buffer -> 10, wrong count -> 20; the callback
    count goes up on every callback, the others only on success."""
    h = _session(lib)
    buf = (ctypes.c_float * 64)()
    hid = ctypes.cast(buf, ctypes.c_void_p)
    toks = (ctypes.c_longlong * 4)(1, 2, 3, 4)
    tok_p = ctypes.cast(toks, ctypes.c_void_p)
    keep = []

    def attn(code, count):
        @_lib.DS_ATTENTION_CALLBACK
        def cb(layer, hidden_in, batch, hidden_dim, out_pp, out_count):
            out_pp[0] = ctypes.cast(buf, ctypes.c_void_p).value if code >= 0 else None
            out_count[0] = count
            return max(code, 0)
        keep.append(cb)
        return cb

    assert lib.ds_attention_layer_forward_f32(None, 0, hid, 1, 8, attn(0, 8), hid) == 1
    assert lib.ds_attention_layer_forward_f32(h, 0, hid, 1, 8, _lib.DS_ATTENTION_CALLBACK(), hid) == 1
    assert lib.ds_attention_layer_forward_f32(h, 3, hid, 1, 8, attn(0, 8), hid) == 2
    assert lib.ds_attention_layer_forward_f32(h, 0, hid, 0, 8, attn(0, 8), hid) == 2
    assert lib.ds_callback_invocation_count(h) == 0
    assert lib.ds_attention_layer_forward_f32(h, 0, hid, 1, 8, attn(4, 8), hid) == 14
    assert lib.ds_attention_layer_forward_f32(h, 0, hid, 1, 8, attn(-1, 8), hid) == 10  # null buffer
    assert lib.ds_attention_layer_forward_f32(h, 0, hid, 2, 8, attn(0, 8), hid) == 20  # 8 != 2 * 8
    assert lib.ds_callback_invocation_count(h) == 3
    assert lib.ds_monolithic_call_counter(h) == 0 and lib.ds_attention_invocation_count(h) == 0

    def dec(code, count):
        @_lib.DS_DECODE_CALLBACK
        def cb(token, out_pp, out_count):
            out_pp[0] = ctypes.cast(buf, ctypes.c_void_p).value
            out_count[0] = count
            return code
        keep.append(cb)
        return cb

    assert lib.ds_forward_decode_f32(h, 5, dec(0, 16), None, 16) == 1
    assert lib.ds_forward_decode_f32(h, 5, dec(0, 16), hid, 0) == 2
    assert lib.ds_forward_decode_f32(h, 5, dec(2, 16), hid, 16) == 12
    assert lib.ds_forward_decode_f32(h, 5, dec(0, 15), hid, 16) == 20

    def seq(cbtype, code, count):
        @cbtype
        def cb(ids, n, out_pp, out_count):
            out_pp[0] = ctypes.cast(buf, ctypes.c_void_p).value
            out_count[0] = count
            return code
        keep.append(cb)
        return cb

    assert lib.ds_forward_prefill_f32(h, None, 4, seq(_lib.DS_PREFILL_CALLBACK, 0, 16), hid, 16) == 1
    assert lib.ds_forward_prefill_f32(h, tok_p, 0, seq(_lib.DS_PREFILL_CALLBACK, 0, 16), hid, 16) == 2
    assert lib.ds_forward_prefill_f32(h, tok_p, 4, seq(_lib.DS_PREFILL_CALLBACK, 3, 16), hid, 16) == 13
    assert lib.ds_forward_prefill_f32(h, tok_p, 4, seq(_lib.DS_PREFILL_CALLBACK, 0, 64), hid, 16) == 20
    assert lib.ds_forward_verify_f32(h, tok_p, 4, seq(_lib.DS_VERIFY_CALLBACK, 0, 16), hid, 16) == 20  # 4 * 16
    assert lib.ds_forward_verify_f32(h, tok_p, 0, seq(_lib.DS_VERIFY_CALLBACK, 0, 16), hid, 16) == 2
    assert lib.ds_forward_verify_f32(h, tok_p, 4, seq(_lib.DS_VERIFY_CALLBACK, 1, 64), hid, 16) == 11
    assert lib.ds_layers_executed_count(h) == 0 and lib.ds_monolithic_call_counter(h) == 0
    lib.ds_session_destroy(h)


@pytest.mark.gpu
def test_rowmajor_kv_entry_points_are_documented_not_implemented(lib):
    """kv_attention_decode_* / kv_dense_layer_decode_{fp16,u16_ext}: the
    reference's argument codes, then 90 with the reason."""
    sess = lib.kv_prefill_init_typed(1, 4, 8, 0)
    if not sess:
        pytest.skip("no device to hold a KV session")
    one = ctypes.c_void_p(16)
    assert lib.kv_attention_decode_fp16(sess, 0, None, one, one, one, one, one, 8, 1, 1, 1e4) == 1
    assert lib.kv_attention_decode_fp16(sess, 5, one, one, one, one, one, one, 8, 1, 1, 1e4) == 1
    assert lib.kv_attention_decode_fp16(sess, 0, one, one, one, one, one, one, 0, 1, 1, 1e4) == 2
    assert lib.kv_attention_decode_fp16(sess, 0, one, one, one, one, one, one, 8, 1, 1, 1e4) == 90
    assert "native_pack_u16_rows8" in _lib.last_error()
    assert lib.kv_attention_decode_u16_ext(sess, 0, *([one] * 11), 8, 1, 1, 1e4, 1e-6) == 90
    assert lib.kv_dense_layer_decode_fp16(sess, 0, *([one] * 11), 8, 16, 1, 1, 1e-6, 1e4) == 90
    assert lib.kv_dense_layer_decode_u16_ext(sess, 0, *([one] * 16), 8, 16, 1, 1, 1e-6, 1e4) == 90
    assert lib.kv_dense_layer_decode_u16_ext(sess, 0, *([one] * 15), None, 8, 16, 1, 1, 1e-6, 1e4) == 1
    lib.kv_free(sess)

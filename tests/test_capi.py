"""The C ABI library on the CPU: it loads, exports every symbol the header
declares, the Python binding covers them, and the host-only logic (argument
checks that return before any device work, the session object and its
counters, kill switches) behaves as the reference's.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from pocketlm_amd import _lib, native

HEADER = Path(__file__).resolve().parent.parent / "include" / "pocketlm_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"typedef[^;]*;", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted({n for n in names if n not in {"typedef"}})


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from pocketlm_amd import build

        build.build()
    return _lib.load()


def test_header_declares_the_reference_entry_points():
    names = set(declared_functions())
    for required in (
        "fp8_e4m3_dequant_to_fp16", "fp8_e4m3_dequant_to_bf16", "fp8_e4m3_block_linear_f32",
        "fp8_e4m3_block_dual_linear_f32", "fp8_e4m3_block_mlp_f32", "fp8_e4m3_block_mlp_many_f32",
        "fp8_e4m3_block_mlp_many_weighted_f32", "fp8_e4m3_block_mlp_many_row_weighted_f32",
        "fp8_e4m3_block_mlp_many_pair_weighted_f32", "fp8_e4m3_block_mlp_avx512_f32",
        "fp8_e4m3_block_mlp_many_weighted_avx512_f32", "q4_dequant_to_fp16", "q4_dequant_many_to_fp16",
        "q4_moe_selected_forward_u16", "native_pack_u16_rows8", "native_packed_gemv_rows8",
        "ds_session_create", "ds_moe_layer_forward_f32", "ds_moe_layer_forward_fp8_f32", "ds_router_topk_u16",
    ):
        assert required in names, required


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_binding_covers_every_declared_symbol():
    assert sorted(declared_functions()) == sorted(_lib.exported_names())


def test_argument_checks_return_reference_codes_without_device_work(lib):
    null = ctypes.c_void_p(0)
    one = ctypes.c_void_p(16)
    assert lib.fp8_e4m3_block_linear_f32(null, one, one, one, 1, 1, 1, 1) == -1
    assert lib.fp8_e4m3_block_linear_f32(one, one, one, one, 0, 1, 1, 1) == -2
    assert lib.fp8_e4m3_block_linear_f32(one, one, one, one, 1, 1, 300, 2) == -2  # scale grid too narrow
    assert lib.fp8_e4m3_dequant_to_fp16(null, one, one, 1, 1, 1) == -1
    assert lib.fp8_e4m3_dequant_to_bf16(one, one, one, 0, 1, 1) == -2
    assert lib.fp8_e4m3_dequant_to_fp16(one, one, one, 4, 300, 2) == -3
    assert lib.fp8_e4m3_block_mlp_many_pair_weighted_f32(*([one] * 11), 1, -1, 1, 1, 1, 1, 1) == -2
    assert lib.q4_dequant_many_to_fp16(null, one, one, one, one, 1) == 1
    assert lib.q4_dequant_many_to_fp16(one, one, one, one, one, 0) == 2
    assert lib.q4_moe_selected_forward_u16(*([null] * 9), 1, 1, 1) == 1
    assert lib.native_pack_u16_rows8(null, one, 1, 1) == 1
    assert lib.native_pack_u16_rows8(one, one, -1, 1) == 2
    assert lib.native_packed_gemv_rows8(one, one, one, 1, 1, 7) == 2
    assert lib.ds_router_topk_u16(one, one, 4, 3, 4, 0, one, one) == 2  # k > experts
    assert "bad dimensions" in _lib.last_error() or _lib.last_error()


def test_session_counters_and_callbacks(lib):
    h = lib.ds_session_create(2, 4, 4, 2, None, None)
    assert h
    h = ctypes.c_void_p(h)
    assert lib.ds_monolithic_call_counter(h) == 0
    assert lib.ds_registered_layer_count(h) == 0
    blob = (ctypes.c_uint8 * 64)()
    calls = []

    def good(layer, kind, role, out_ptr, out_nbytes):
        calls.append((layer, kind, role))
        out_ptr[0] = ctypes.cast(blob, ctypes.c_void_p).value
        out_nbytes[0] = 64 if role == 0 else 8
        return 0

    def bad(layer, kind, role, out_ptr, out_nbytes):
        return 5

    cb_good, cb_bad = _lib.DS_TENSOR_CALLBACK(good), _lib.DS_TENSOR_CALLBACK(bad)
    assert lib.ds_session_register_layer(h, 1, 2, 0, cb_good, cb_good) == 0
    assert lib.ds_registered_layer_count(h) == 1
    assert lib.ds_registered_fp8_nbytes(h, 0) == 64 and lib.ds_registered_scale_nbytes(h, 0) == 64
    assert lib.ds_callback_invocation_count(h) == 2
    assert lib.ds_session_register_layer(h, 1, 2, 0, cb_bad, cb_good) == 15
    assert lib.ds_session_register_layer(h, 1, 2, 0, cb_good, cb_bad) == 25
    assert lib.ds_session_register_layer(h, 9, 2, 0, cb_good, cb_good) == 1
    assert lib.ds_registered_fp8_nbytes(h, 5) == -1
    assert lib.ds_monolithic_call_counter(ctypes.c_void_p(0)) == -1
    assert len(calls) == 3 and lib.ds_callback_invocation_count(h) == 5
    lib.ds_session_destroy(h)
    assert not lib.ds_session_create(0, 4, 4, 2, None, None)


def test_kill_switches(monkeypatch):
    monkeypatch.setenv("PCKETLM_DISABLE_NATIVE_FP8_LINEAR", "1")
    assert native.native_fp8_linear_available() is False
    with pytest.raises(RuntimeError, match="unavailable: disabled"):
        native.fp8_e4m3_block_linear_f32(torch.zeros((8, 8), dtype=torch.uint8), torch.ones((1, 1)), torch.ones((1, 8)))
    monkeypatch.setenv("PCKETLM_DISABLE_NATIVE_PACKED_GEMV", "1")
    with pytest.raises(RuntimeError, match="unavailable"):
        native.pack_weight_rows8(torch.ones((8, 8), dtype=torch.float16))
    monkeypatch.setenv("PCKETLM_DISABLE_NATIVE_Q4", "yes")
    assert native.native_q4_available() is False
    monkeypatch.setenv("PCKETLM_DISABLE_NATIVE_FP8_DEQUANT", "on")
    with pytest.raises(RuntimeError, match="unavailable: disabled"):
        native.fp8_e4m3_dequant_to_fp16(torch.zeros((4, 4), dtype=torch.uint8), torch.ones((1, 1)))
    # tests/test_native_fp16_matmul.py:30-39
    monkeypatch.setenv("PCKETLM_DISABLE_NATIVE_MATMUL", "1")
    assert native.native_fp16_matmul_available() is False
    with pytest.raises(RuntimeError, match="unavailable"):
        native.fp16_matmul(torch.ones((1, 1), dtype=torch.float16), torch.ones((1, 1), dtype=torch.float16))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the behaviour without a device")
def test_no_device_means_unavailable_not_fallback(lib):
    assert lib.pocketlm_device_available() == 0
    assert native.native_fp8_linear_available() is False
    with pytest.raises(RuntimeError, match="unavailable"):
        native.fp8_e4m3_block_linear_f32(torch.zeros((8, 8), dtype=torch.uint8), torch.ones((1, 1)), torch.ones((1, 8)))


def test_packed_gemv_cache_lru(monkeypatch):
    calls = []
    monkeypatch.setattr(native, "pack_weight_rows8", lambda w: calls.append(1) or torch.zeros(64, dtype=torch.uint16))
    native.reset_packed_gemv_cache()
    monkeypatch.setenv("PCKETLM_PACKED_GEMV_CACHE_MB", "1")
    w = torch.ones((8, 8), dtype=torch.float16)
    native.cached_pack_weight_rows8("a", w)
    native.cached_pack_weight_rows8("a", w)
    stats = native.packed_gemv_cache_stats()
    assert stats["hits"] == 1 and stats["misses"] == 1 and stats["stores"] == 1 and len(calls) == 1
    monkeypatch.setenv("PCKETLM_DISABLE_PACKED_GEMV_CACHE", "1")
    native.cached_pack_weight_rows8("a", w)
    assert len(calls) == 2
    native.reset_packed_gemv_cache()


def test_packed_gemv_cache_evicts_least_recently_used(monkeypatch):
    """A 1 MiB budget holds two 400 KiB packs: a third evicts the one used
    longest ago (a hit refreshes), and a pack above the budget is returned
    without being kept."""
    sizes = {"a": 200 << 10, "b": 200 << 10, "c": 200 << 10, "big": 600 << 10}  # uint16 elements
    monkeypatch.setattr(native, "pack_weight_rows8", lambda w: torch.zeros(int(w.item()), dtype=torch.uint16))
    monkeypatch.setenv("PCKETLM_PACKED_GEMV_CACHE_MB", "1")
    native.reset_packed_gemv_cache()
    pack = {k: native.cached_pack_weight_rows8(k, torch.tensor(n)) for k, n in (("a", sizes["a"]), ("b", sizes["b"]))}
    assert native.cached_pack_weight_rows8("a", torch.tensor(1)) is pack["a"]  # hit: "a" is now the newest
    native.cached_pack_weight_rows8("c", torch.tensor(sizes["c"]))                # evicts "b"
    st = native.packed_gemv_cache_stats()
    assert (st["hits"], st["misses"], st["stores"], st["evictions"]) == (1, 3, 3, 1)
    assert st["resident_count"] == 2 and st["resident_bytes"] == 800 << 10 and st["budget_bytes"] == 1 << 20
    assert native.cached_pack_weight_rows8("a", torch.tensor(1)) is pack["a"]
    assert native.cached_pack_weight_rows8("b", torch.tensor(sizes["b"])) is not pack["b"]  # was evicted
    native.cached_pack_weight_rows8("big", torch.tensor(sizes["big"]))
    st = native.packed_gemv_cache_stats()
    assert (st["stores"], st["evictions"], st["resident_count"], st["resident_bytes"]) == (4, 2, 2, 800 << 10)
    native.reset_packed_gemv_cache()
    assert native.packed_gemv_cache_stats()["resident_count"] == 0

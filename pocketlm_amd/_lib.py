"""ctypes binding of libpocketlm_hip.so (declarations: include/pocketlm_hip.h).

The library is loaded once, after ``import torch`` so that it binds to the
HIP runtime torch already loaded (both are libamdhip64.so.7).  There is no
fallback: a missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library)

LIB_PATH = Path(__file__).resolve().parent / "libpocketlm_hip.so"

_i64 = ctypes.c_longlong
_i32 = ctypes.c_int
_vp = ctypes.c_void_p
_f32 = ctypes.c_float

DS_TENSOR_CALLBACK = ctypes.CFUNCTYPE(
    ctypes.c_int,
    ctypes.c_longlong,
    ctypes.c_longlong,
    ctypes.c_longlong,
    ctypes.POINTER(ctypes.c_void_p),
    ctypes.POINTER(ctypes.c_longlong),
)

DS_ATTENTION_CALLBACK = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_longlong,
                                         ctypes.c_longlong, ctypes.POINTER(ctypes.c_void_p),
                                         ctypes.POINTER(ctypes.c_longlong))
DS_DECODE_CALLBACK = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_longlong, ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.POINTER(ctypes.c_longlong))
DS_PREFILL_CALLBACK = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_longlong,
                                       ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_longlong))
DS_VERIFY_CALLBACK = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_longlong,
                                      ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_longlong))

# name: (restype, argtypes)
_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "pocketlm_set_stream": (_i32, [_vp]),
    "pocketlm_last_error": (ctypes.c_char_p, []),
    "pocketlm_scratch_bytes": (_i64, []),
    "pocketlm_release_scratch": (_i32, []),
    "pocketlm_device_available": (_i32, []),
    "fp8_dequant_cpu_has_avx2_f16c": (_i32, []),
    "fp8_linear_avx512_cpu_has_avx512": (_i32, []),
    "q4_cpu_has_avx2_f16c": (_i32, []),
    "ds_cpu_has_avx2": (_i32, []),
    "fp8_e4m3_dequant_to_fp16": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64]),
    "fp8_e4m3_dequant_to_bf16": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64]),
    "fp8_e4m3_dequant_to_f32": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64]),
    "fp8_e4m3_block_linear_f32": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64]),
    "fp8_e4m3_block_dual_linear_f32": (_i32, [_vp] * 7 + [_i64] * 4),
    "fp8_e4m3_block_mlp_f32": (_i32, [_vp] * 8 + [_i64] * 5),
    "fp8_e4m3_block_mlp_avx512_f32": (_i32, [_vp] * 8 + [_i64] * 5),
    "fp8_e4m3_block_mlp_many_f32": (_i32, [_vp] * 8 + [_i64] * 6),
    "fp8_e4m3_block_mlp_many_weighted_f32": (_i32, [_vp] * 9 + [_i64] * 6),
    "fp8_e4m3_block_mlp_many_weighted_shared_f32": (_i32, [_vp] * 10 + [_i64] * 6),
    "fp8_e4m3_block_linear_bf16x_f32": (_i32, [_vp] * 4 + [_i64] * 4),
    "fp8_e4m3_tiles8_bytes": (_i64, [_i64, _i64]),
    "fp8_e4m3_pack_tiles8": (_i32, [_vp] * 2 + [_i64] * 2),
    "fp8_e4m3_block_linear_tiles8_f32": (_i32, [_vp] * 4 + [_i64] * 4),
    "fp8_e4m3_block_linear_tiles8_bf16x_f32": (_i32, [_vp] * 4 + [_i64] * 4),
    "fp8_e4m3_block_linear_many_f32": (_i32, [_vp] * 5 + [_i64] * 4),
    "fp8_e4m3_block_linear_many_bf16x_f32": (_i32, [_vp] * 5 + [_i64] * 4),
    "fp8_e4m3_block_dual_linear_bf16x_f32": (_i32, [_vp] * 7 + [_i64] * 4),
    "fp8_e4m3_block_mlp_bf16x_f32": (_i32, [_vp] * 8 + [_i64] * 5),
    "fp8_e4m3_block_mlp_many_weighted_bf16x_f32": (_i32, [_vp] * 9 + [_i64] * 6),
    "fp8_e4m3_block_mlp_many_weighted_shared_bf16x_f32": (_i32, [_vp] * 10 + [_i64] * 6),
    "native_lm_head_topk_u16": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i64]),
    "native_fp16_matmul": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64]),
    "pocketlm_file_spans_to_device": (_i32, [ctypes.c_char_p, _vp, _vp, _vp, _i64]),
    "row8_artifact_load_tensor": (_vp, [ctypes.c_char_p, ctypes.c_ulonglong, ctypes.c_ulonglong]),
    "row8_artifact_free_tensor": (None, [_vp]),
    "row8_artifact_tensor_data": (_vp, [_vp]),
    "row8_artifact_tensor_nbytes": (ctypes.c_ulonglong, [_vp]),
    "row8_artifact_map_file": (_vp, [ctypes.c_char_p]),
    "row8_artifact_unmap_file": (None, [_vp]),
    "row8_artifact_mapped_data": (_vp, [_vp, ctypes.c_ulonglong, ctypes.c_ulonglong]),
    "row8_artifact_mapped_nbytes": (ctypes.c_ulonglong, [_vp]),
    "kv_prefill_init_typed": (_vp, [_i64, _i64, _i64, _i32]),
    "kv_prefill_init": (_vp, [_i64, _i64, _i64]),
    "kv_free": (None, [_vp]),
    "kv_append_committed": (_i32, [_vp, _i64, _vp, _vp, _i64]),
    "kv_append_tentative": (_i32, [_vp, _i64, _vp, _vp, _i64]),
    "kv_commit": (_i32, [_vp, _i64]),
    "kv_rollback": (_i32, [_vp]),
    "kv_committed_length": (_i64, [_vp, _i64]),
    "kv_tentative_length": (_i64, [_vp, _i64]),
    "kv_copy_layer": (_i32, [_vp, _i64, _vp, _vp, _i64, _i32]),
    "kv_dense_layer_decode_u16_ext_packed_rows8": (_i32, [_vp, _i64] + [_vp] * 16 + [_i64] * 4 + [_f32, _f32]),
    "fp8_e4m3_block_moe_device_routed_f32": (_i32, [_vp, _i64, _vp, _vp, _i64] + [_vp] * 6 + [_i64] * 5),
    "fp8_e4m3_block_moe_device_routed_bf16x_f32": (_i32, [_vp, _i64, _vp, _vp, _i64] + [_vp] * 6 + [_i64] * 5),
    "fp8_e4m3_block_moe_from_logits_bf16x_f32": (_i32, [_vp, _vp, _i64, _i64, _i32, _f32, _vp, _i64, _i64] + [_vp] * 8
                                                 + [_i64] * 5),
    "fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc": (_i32, [_vp, _i64, _vp, _vp, _i64] + [_vp] * 6 + [_i64] * 5),
    "fp8_e4m3_block_mlp_many_row_weighted_bf16x_f32": (_i32, [_vp] * 9 + [_i64] * 6),
    "fp8_e4m3_block_mlp_many_pair_weighted_bf16x_f32": (_i32, [_vp] * 11 + [_i64] * 7),
    "fp8_e4m3_block_mlp_many_weighted_avx512_f32": (_i32, [_vp] * 9 + [_i64] * 6),
    "fp8_e4m3_block_mlp_many_row_weighted_f32": (_i32, [_vp] * 9 + [_i64] * 6),
    "fp8_e4m3_block_mlp_many_pair_weighted_f32": (_i32, [_vp] * 11 + [_i64] * 7),
    "fp8_e4m3_block_mlp_many_pair_weighted_nosync_f32": (_i32, [_vp] * 12 + [_i64] * 7),
    "fp8_e4m3_block_mlp_many_pair_weighted_nosync_bf16x_f32": (_i32, [_vp] * 12 + [_i64] * 7),
    "q4_dequant_to_fp16": (None, [_vp, _vp, _vp, _i64, _i64]),
    "q4_dequant_many_to_fp16": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64]),
    "q4_moe_selected_forward_u16": (_i32, [_vp] * 9 + [_i64] * 3),
    "q4_gemv_f16_f32": (_i32, [_vp] * 4 + [_i64] * 2),
    "native_pack_u16_rows8": (_i32, [_vp, _vp, _i64, _i64]),
    "native_packed_gemv_rows8": (_i32, [_vp, _vp, _vp, _i64, _i64, _i32]),
    "native_packed_gemv_rows8_many": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32]),
    "native_packed_gemv_rows8_f32_hidden": (_i32, [_vp, _vp, _vp, _i64, _i64, _i32]),
    "ds_session_create": (_vp, [_i64, _i64, _i64, _i64, _vp, _vp]),
    "ds_session_destroy": (None, [_vp]),
    "ds_session_register_layer": (_i32, [_vp, _i64, _i64, _i64, DS_TENSOR_CALLBACK, DS_TENSOR_CALLBACK]),
    "ds_monolithic_call_counter": (_i64, [_vp]),
    "ds_callback_invocation_count": (_i64, [_vp]),
    "ds_expert_invocation_count": (_i64, [_vp]),
    "ds_attention_invocation_count": (_i64, [_vp]),
    "ds_fused_attention_invocation_count": (_i64, [_vp]),
    "ds_layers_executed_count": (_i64, [_vp]),
    "ds_registered_layer_count": (_i64, [_vp]),
    "ds_registered_fp8_nbytes": (_i64, [_vp, _i64]),
    "ds_registered_scale_nbytes": (_i64, [_vp, _i64]),
    "ds_moe_layer_forward_f32": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "ds_moe_layer_forward_fp8_f32": (_i32, [_vp] * 9 + [_i64] * 6 + [_vp]),
    "ds_router_topk_u16": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "ds_router_topk_u16_nosync": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "ds_route_topk_f32": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _f32, _vp, _vp]),
    "ds_attention_layer_forward_f32": (_i32, [_vp, _i64, _vp, _i64, _i64, DS_ATTENTION_CALLBACK, _vp]),
    "ds_forward_decode_f32": (_i32, [_vp, _i64, DS_DECODE_CALLBACK, _vp, _i64]),
    "ds_forward_prefill_f32": (_i32, [_vp, _vp, _i64, DS_PREFILL_CALLBACK, _vp, _i64]),
    "ds_forward_verify_f32": (_i32, [_vp, _vp, _i64, DS_VERIFY_CALLBACK, _vp, _i64]),
    "ds_mla_attention_flash_forward": (_i32, [_vp] * 6 + [_i64] * 6 + [_f32]),
    "ds_attention_block_forward_f32": (_i32, [_vp] * 16 + [_i64] * 8 + [_f32, _f32]),
    "ds_fp8_attention_block_bf16x_f32": (_i32, [_vp] * 19 + [_i64] * 8 + [_f32, _f32]),
    "kv_attention_decode_fp16": (_i32, [_vp, _i64] + [_vp] * 6 + [_i64] * 3 + [_f32]),
    "kv_attention_decode_u16_ext": (_i32, [_vp, _i64] + [_vp] * 11 + [_i64] * 3 + [_f32, _f32]),
    "kv_dense_layer_decode_fp16": (_i32, [_vp, _i64] + [_vp] * 11 + [_i64] * 4 + [_f32, _f32]),
    "kv_dense_layer_decode_u16_ext": (_i32, [_vp, _i64] + [_vp] * 16 + [_i64] * 4 + [_f32, _f32]),
}

_LIB: ctypes.CDLL | None = None
_LOCK = threading.Lock()


def load() -> ctypes.CDLL:
    """Load and bind the library (raises OSError when it is missing)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not LIB_PATH.exists():
                raise OSError(
                    f"{LIB_PATH} is not built; run `python -m pocketlm_amd.build` (ROCm hipcc, gfx950)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _LIB = lib
    return _LIB


def exported_names() -> list[str]:
    return list(_SIGNATURES)


def last_error() -> str:
    raw = load().pocketlm_last_error()
    return raw.decode("utf-8", "replace") if raw else ""

"""Loads libameva_hip.so (the HIP kernels behind the C ABI of include/ameva_hip.h) and declares its signatures.

There is no fallback: if the library is missing or fails to load, every operator raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libameva_hip.so")

P, I32, I64, F32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# name -> (restype, argtypes); every symbol include/ameva_hip.h declares
SIGNATURES = {
    "amv_last_error": (ctypes.c_char_p, []),
    "amv_version": (I32, []),
    "amv_weight_bytes": (I64, [I32, I64, I64]),
    "amv_repack": (I32, [I32, P, P, I64, I64, P]),
    "amv_unrepack": (I32, [I32, P, P, I64, I64, P]),
    "amv_act_bytes": (I64, [I32, I64, I64]),
    "amv_quantize_act": (I32, [I32, P, I64, I64, I32, P, P, P]),
    "amv_quantize_q4_0": (I32, [P, I64, I64, P, P]),
    "amv_mul_mat_vec": (I32, [I32, P, I64, I64, P, I64, P, I64, P]),
    "amv_debug_gemv_generic": (I32, [I32]),
    "amv_mul_mat_vec_raw": (I32, [I32, P, I64, I64, I64, P, I64, P, I64, P, P]),
    "amv_debug_gemv_read_probe": (I32, [P, I64, I64, P, I32, P]),
    "amv_mul_mat_vec_ep": (I32, [I32, P, I64, I64, P, P, I32, P, P, P]),
    "amv_mul_mat_block_sums": (I32, [I32, P, I64, I64, P, I64, P, P]),
    "amv_quantize_k": (I32, [I32, P, I64, I64, P, P]),
    "amv_mul_mat_q": (I32, [I32, P, I64, I64, P, I64, P, I64, P]),
    "amv_mul_mat_q_block_sums": (I32, [I32, P, I64, I64, P, I64, P, P]),
    "amv_mul_mat_q_act": (I32, [I32, P, I64, I64, P, I32, I64, P, I64, P]),
    "amv_mul_mat_q_act_add": (I32, [I32, P, I64, I64, P, I32, I64, P, I64, P, P]),
    "amv_mul_mat_q_act_block_sums": (I32, [I32, P, I64, I64, P, I32, I64, P, P]),
    "amv_i2s_act_bytes": (I64, [I64, I64]),
    "amv_i2s_quantize_act": (I32, [P, I64, I64, P, P]),
    "amv_i2s_gemv": (I32, [P, I64, I64, P, I64, F32, P, I64, P]),
    "amv_i2s_gemv_sums": (I32, [P, I64, I64, P, I64, P, P]),
    "amv_i2s_gemv_f32": (I32, [P, I64, I64, P, F32, P, P]),
    "amv_rms_norm_act": (I32, [P, I64, I64, F32, P, P, P, P, I32, I32, P]),
    "amv_rms_norm": (I32, [P, I64, I64, F32, P, P, P, P, I32, P]),
    "amv_rope": (I32, [P, P, P, I64, I64, I64, I32, I32, F32, F32, F32, P]),
    "amv_gemv_rope_kv": (I32, [I32, P, I64, I64, P, P, I64, I64, I64, P, F32, F32, F32, P, P, I64, P, I64, P, P]),
    "amv_gemv_add_rms_norm": (I32, [I32, P, I64, I64, P, P, P, P, F32, P, P, P, P, I32, I32, P, P]),
    "amv_gemv_swiglu_q8": (I32, [I32, P, I64, I64, P, P, P, P, I32, I32, P, P]),
    "amv_gemv_rope_kv_seg": (I32, [I32, P, P, P, I64, P, P, P, P, I64, I64, I64, P, F32, F32, F32, P, P, I64, P, I64,
                                   P, P]),
    "amv_gemv_swiglu_q8_seg": (I32, [I32, P, P, I64, I64, P, P, P, I32, I32, P, P]),
    "amv_rms_norm_gemv_rope_kv": (I32, [P, P, F32, I32, I32, P, I64, I64, P, I64, I64, I64, P, F32, F32, F32, P, P,
                                        I64, P, I64, P, P]),
    "amv_rms_norm_gemv_swiglu_q8": (I32, [P, P, F32, I32, I32, P, I64, I64, P, P, P, P, P]),
    "amv_rms_norm_gemv_rope_kv_seg": (I32, [P, P, F32, I32, I32, P, P, P, I64, P, P, P, I64, I64, I64, P, F32, F32,
                                            F32, P, P, I64, P, I64, P, P]),
    "amv_rms_norm_gemv_swiglu_q8_seg": (I32, [P, P, F32, I32, I32, P, P, I64, I64, P, P, P, P]),
    "amv_debug_norm_gemv_threads": (None, [I32]),
    "amv_flash_attn_decode_ex": (I32, [P, P, P, P, P, I64, I64, I64, P, I64, I64, I64, I64, I64, F32, P, I64, P, P,
                                          I32, I32, P]),
    "amv_rope_kv_store": (I32, [P, P, I64, I64, I64, I64, I32, I32, F32, F32, F32, P, P, I64, P, I64, P, P]),
    "amv_swiglu": (I32, [P, P, P, I64, P]),
    "amv_swiglu_rows": (I32, [P, I64, P, I64, P, I64, I64, I64, P, I32, P]),
    "amv_swiglu_rows_act": (I32, [P, I64, P, I64, P, I64, I64, I64, P, I32, I32, P]),
    "amv_flash_attn_workspace_bytes": (I64, [I64, I64, I64, I64]),
    "amv_flash_attn_decode": (I32, [P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, I64, F32, P, I64, P, I32, P]),
    "amv_flash_attn_prefill": (I32, [P, I64, I64, P, P, P, I64, P, I64, I64, I64, I64, I64, I64, I64, I64, I64, F32,
                                     I64, P]),
    "amv_binary": (I32, [I32, P, P, P, I64, I64, I64, P]),
    "amv_set_rows_f16": (I32, [P, I64, P, I64, I64, I64, P, I32, I64, P, P]),
    "amv_i2s_gemv_acc": (I32, [P, I64, I64, P, F32, P, P]),
    "amv_bitnet_norm_q8": (I32, [P, P, P, I64, F32, I32, I32, P, P, P]),
    "amv_bitnet_rope_kv": (I32, [P, P, P, P, P, P, P, I64, I64, I64, I64, P]),
    "amv_gemv_f16": (I32, [P, I64, I64, P, P, P]),
    "amv_bitnet_gemv_fused": (I32, [P, P, P, I64, F32, I32, I32, I32, P, P, P, P, I32, P, P, I64, P]),
    "amv_bitnet_gemv_fa_merge": (I32, [P, I32, I32, I64, P, P, I64, F32, I32, P, I64, F32, P, I32, P]),
    "amv_set_rows_q": (I32, [I32, P, I64, P, I64, I64, I64, P, I32, I64, I32, P, P]),
    "amv_flash_attn_split_kv": (I32, [I32, P, P, P, P, I64, I64, I64, P, I64, I64, I64, I64, I64, F32, P, I64, I32, P,
                                      P, P]),
    "amv_flash_attn_decode_kv": (I32, [I32, P, P, P, P, P, I64, I64, I64, P, I64, I64, I64, I64, I64, F32, P, I64, P,
                                       P, I32, I32, P]),
    "amv_flash_attn_noalloc_max_bytes": (I64, []),
    "amv_flash_attn_decode_noalloc": (I32, [I32, P, P, P, P, P, I64, I64, I64, P, I64, I64, I64, I64, I64, F32, P,
                                            I32, I32, P]),
    "amv_get_rows": (I32, [I32, P, I64, I64, P, I64, P, P, P]),
    "amv_argmax": (I32, [P, I64, P, P, P, I64, P]),
    "amv_argmax_ex": (I32, [P, I64, P, P, P, I64, P, P, P, P, P]),
}

_lib = None


class AmevaError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AmevaError(f"{LIB_PATH} is not built: run __graft_entry__.build() (no CPU fallback exists)")
        _lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().amv_last_error().decode(errors="replace")
        raise AmevaError(f"{what} failed ({rc}): {msg} (FAIL-FAST)")

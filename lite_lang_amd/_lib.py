"""ctypes binding of liblitelang_amd.so (the C ABI in include/litelang_amd.h).

The library is mandatory: importing an op module without it raises, there is
no CPU or torch fallback for any op.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblitelang_amd.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "litelang_amd.h")

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float

# name -> (restype, argtypes), mirroring include/litelang_amd.h
SIGNATURES = {
    "ll_version": (I32, []),
    "ll_last_error": (ctypes.c_char_p, []),
    "ll_decode_attention_workspace_size": (I64, [I64, I64, I64, I64, I64]),
    "ll_decode_attention_xcc_probe": (I32, [I64, I64, I64, I64, I64, P, I64, P]),
    "ll_decode_attention_noalloc_max_bytes": (I64, []),
    "ll_decode_attention_noalloc_init": (I32, []),
    "ll_decode_attention_set_same_launch_merge": (I32, [I32]),
    "ll_decode_attention_noalloc": (I32, [P, I64, I64, P, I64, I64, P, I64, I64, P, I64, P, I32,
                                          P, I32, P, I64, I64, I64, I64, I64, I64, I64, F32, I32,
                                          P]),
    "ll_decode_attention": (I32, [P, I64, I64, P, I64, I64, P, I64, I64, P, I64, P, I32, P, I32,
                                  P, I64, I64, I64, I64, I64, I64, I64, F32, I32, P, I64, P]),
    "ll_prefill_attention": (I32, [P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I64,
                                   P, I32, P, I32, P, I32, P, I32, I64, I64, I64, I64, I64, F32,
                                   I32, P]),
    "ll_rmsnorm": (I32, [P, I64, P, I64, P, P, I64, I64, I64, F32, I32, P]),
    "ll_rotary_emb": (I32, [P, I64, I64, I64, P, I64, I64, I64, P, I64, P, I64, I64, I64, I32,
                            I32, P]),
    "ll_rope_kv_scatter": (I32, [P, I64, I64, I64, I64, I64, P, I32, P, P, I64, I32, P, P, I64,
                                 I64, I32, P]),
    "ll_kv_store": (I32, [P, I64, I64, I64, I64, P, P, I64, I64, I64, I32, P]),
    "ll_silu_and_mul": (I32, [P, I64, P, I64, I64, I64, I32, P]),
    "ll_embedding_rmsnorm": (I32, [P, I64, I64, P, I32, P, I64, P, P, I64, I64, I64, F32, I32, P]),
    "ll_embedding_rmsnorm_epoch": (I32, [P, I64, I64, P, I32, P, I64, P, P, I64, I64, I64, F32,
                                         I32, P, P, I64, P, P, P, P]),
    "ll_embedding": (I32, [P, I64, I64, P, I32, P, I64, I64, I64, I32, P]),
    "ll_argmax_workspace_size": (I64, [I64, I64]),
    "ll_argmax": (I32, [P, I64, I64, I64, P, P, I64, I32, P]),
    "ll_argmax_status": (I32, [P, I64, I64, I64, P, P, I64, I32, P, P]),
    "ll_assign_slots": (I32, [P, I64, P, P, P, I64, P]),
    "ll_gemm_tiled_supported": (I32, [I64, I64, I64, I32]),
    "ll_gemm_tiled": (I32, [P, I64, P, I64, P, P, I64, I64, I64, I64, I32, P]),
    "ll_gemm_interleave_gate_up": (I32, [P, I64, I64, I64, I64, P, P]),
    "ll_gemm_gate_up_silu_tiled": (I32, [P, I64, P, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_i8_tiled": (I32, [P, I64, P, P, I64, P, I32, P, P, I64, I64, I64, I64, I32, P]),
    "ll_gemm_i8_i32_tiled": (I32, [P, I64, P, I64, P, I64, I64, I64, I64, P]),
    "ll_gemm_i8_i32": (I32, [P, I64, P, I64, P, I64, I64, I64, I64, P]),
    "ll_gemm_i8_gate_up_silu_tiled": (I32, [P, I64, P, P, P, I32, I64, I64, I64, I32, P, I64,
                                            P]),
    "ll_gemm_workspace_size": (I64, [I64, I64, I64]),
    "ll_gemm": (I32, [P, I64, P, I64, P, P, I64, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_splitk_count": (I32, [I64, I64, I64]),
    "ll_gemm_splitk": (I32, [P, I64, P, I64, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_packed_bytes": (I64, [I64, I64]),
    "ll_gemm_pack": (I32, [P, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_splitk_packed": (I32, [P, I64, P, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_packed": (I32, [P, I64, P, P, P, I64, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_packed_f32": (I32, [P, I64, P, P, P, I64, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_packed_f32_argmax_workspace_size": (I64, [I64, I64, I64]),
    "ll_gemm_packed_f32_argmax": (I32, [P, I64, P, P, P, I64, I64, I64, I64, I32, P, P, P, I64, P]),
    "ll_gemm_packed_gate_up_bytes": (I64, [I64, I64]),
    "ll_gemm_pack_gate_up": (I32, [P, I64, I64, I64, I32, P, I64, P]),
    "ll_gemm_packed_tile_rows": (I32, [I64, I64]),
    "ll_gemm_packed_gate_up_tile_rows": (I32, [I64]),
    "ll_gemm_gate_up_silu_packed": (I32, [P, I64, P, I64, I64, I64, I32, P, I64, P]),
    "ll_quant_weight_per_channel": (I32, [P, I64, I64, I64, I32, P, I64, P, P]),
    "ll_quant_per_token": (I32, [P, I64, I64, I64, I32, P, I64, P, P]),
    "ll_gemm_i8_packed_bytes": (I64, [I64, I64]),
    "ll_gemm_i8_pack": (I32, [P, I64, I64, I64, P, I64, P]),
    "ll_gemm_i8_packed_gate_up_bytes": (I64, [I64, I64]),
    "ll_gemm_i8_pack_gate_up": (I32, [P, I64, I64, I64, P, I64, P]),
    "ll_gemm_i8_gate_up_silu_packed": (I32, [P, I64, P, I64, I64, I64, P, P, I32, P, I64, I32, P]),
    "ll_gemm_i8_splitk_count": (I32, [I64, I64, I64]),
    "ll_gemm_i8_splitk_packed": (I32, [P, I64, P, I64, I64, I64, P, I64, P]),
    "ll_quant_static": (I32, [P, I64, I64, I64, I32, P, P, I64, P, P]),
    "ll_dequant_splitk": (I32, [P, I32, P, P, I32, P, I64, I64, P]),
    "ll_add_rmsnorm_splitk": (I32, [P, I64, P, I32, P, P, I64, I64, I64, F32, I32, P]),
    "ll_silu_and_mul_splitk": (I32, [P, I32, P, I64, I64, I64, I32, P]),
    "ll_add_rmsnorm_qkv_splits": (I32, [I64, I64, I64]),
    "ll_add_rmsnorm_qkv_splitk": (I32, [P, I64, P, I32, P, F32, P, P, P, I64, I64, I64, I64, I32,
                                        P, P, ctypes.c_uint32, P]),
    "ll_decode_sync_bytes": (I64, []),
    "ll_decode_sync_error_offset": (I64, []),
    "ll_decode_sync_set_spin_limit": (I32, [I32]),
    "ll_decode_sync_status": (I32, [P, I32, P]),
    "ll_decode_attention_rope_splitk": (I32, [P, I32, P, P, I32, P, P, I64, I32, P, P, I64, I64,
                                              P, I64, I64, P, I64, P, I32, P, I32, P, I64, I64,
                                              I64, I64, I64, I64, I64, F32, I32, P, I64, P, P]),
    "ll_decode_attention_rope_splitk_i32": (I32, [P, I32, P, P, I32, P, P, I32, P, P, I64, I32, P,
                                                  P, I64, I64, P, I64, I64, P, I64, P, I32, P,
                                                  I32, P, I64, I64, I64, I64, I64, I64, I64, F32,
                                                  I32, P, I64, P, P, I64, P, P, P]),
    "ll_add_rmsnorm_splitk_i32": (I32, [P, I64, P, I32, P, P, I32, P, P, I64, I64, I64, F32, I32,
                                        P, I64, P, P]),
    "ll_silu_and_mul_splitk_i32": (I32, [P, I32, P, P, I32, P, I64, I64, I64, I32, P]),
    "ll_rope_kv_scatter_splitk": (I32, [P, I32, P, P, I64, I64, I64, I64, I64, P, I32, P, P, I64,
                                        I32, P, P, I64, I64, I32, P]),
    "ll_probe_stream_read": (I32, [P, I64, I64, P, P]),
    "ll_probe_kv_gather": (I32, [P, I64, I64, P, I64, I64, P, I64, P, I32, P, I32, I64, I64, I64,
                                 I64, I64, I64, I32, P, P]),
    "ll_decode_attention_split_count": (I32, [I64, I64, I64, I64]),
    "ll_probe_launch": (I32, [P, I64, I64, P]),
}


class LiteLangError(RuntimeError):
    pass


def header_symbols() -> list[str]:
    """Every function name declared in include/litelang_amd.h."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\*]+\s+\**(ll_\w+)\s*\(", text, re.M)))


_lib = None


def load(path: str = LIB_PATH):
    """Load the shared library (once) and bind every declared symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise LiteLangError(
            f"{path} is missing: build it with `python -m lite_lang_amd.build` "
            "(there is no fallback implementation)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.ll_last_error().decode(errors="replace") if _lib is not None else ""
        raise LiteLangError(f"{what} failed (code {rc}): {msg}")

"""ctypes binding of libtenzo_hip.so (the C ABI in include/tenzo_hip.h and
include/tenzo.h). Loading fails loudly when the library is missing: there is
no CPU fallback."""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtenzo_hip.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_S = ctypes.c_char_p

# name: (restype, argtypes)
SIGNATURES = {
    "tenzo_hip_version": (_S, []),
    "tenzo_hip_last_error": (_S, []),
    "tenzo_hip_device_count": (_I, []),
    "tenzo_hip_release_scratch": (_I, []),
    "tenzo_hip_tl1_packed_bytes": (_SZ, [_I64, _I64]),
    "tenzo_hip_tl1_repack": (_I, [_P, _P, _I64, _I64, _P]),
    "tenzo_hip_tl1_repack_raw": (_I, [_P, _P, _I64, _I64, _P]),
    "tenzo_hip_rmsnorm_quant31": (_I, [_P, _P, _I, _F, _I64, _I64, _P, _P, _P, _P]),
    "tenzo_hip_bitlinear_tl1": (_I, [_P, _P, _P, _F, _I64, _I64, _I64, _P, _P, _P]),
    "tenzo_hip_bitlinear_tl1_lut": (_I, [_P, _P, _P, _F, _I64, _I64, _I64, _P, _P, _P]),
    "tenzo_hip_bitlinear_tl1_f32": (_I, [_P, _P, _F, _I64, _I64, _I64, _P, _P]),
    "tenzo_hip_bitlinear_tl1_batch": (_I, [_P, _P, _P, _F, _I64, _I64, _I64, _P, _P, _I, _P]),
    "tenzo_hip_rmsnorm": (_I, [_P, _P, _P, _I64, _F, _P]),
    "tenzo_hip_attn_int8_decode": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                        _P, _P, _P, _P]),
    "tenzo_hip_attn_int8_decode_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                                _I, _P, _P, _P, _P]),
    "tenzo_hip_attn_tern_decode": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                        _I, _P, _P, _P, _P]),
    "tenzo_hip_attn_paged_int8_decode": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _I,
                                              _I, _I, _P, _P]),
    "tenzo_hip_engine_block_table": (_I, [_P, _P, _I]),
    "tenzo_hip_rope_table": (None, [_F, _I, _I, _I, _P]),
    "tenzo_hip_gemv_q4_0": (_I, [_P, _I, _P, _P, _I, _I, _I, _P]),
    "tenzo_hip_gemv_q8_0": (_I, [_P, _I, _P, _P, _I, _I, _I, _P]),
    "tenzo_hip_gemv_q4_0_q8_0": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "tenzo_hip_gemv_gptq": (_I, [_P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P]),
    "tenzo_hip_gemv_awq": (_I, [_P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P]),
    "tenzo_hip_i8_packed_bytes": (_SZ, [_I64, _I64]),
    "tenzo_hip_i8_rows_repack": (_I, [_P, _P, _I64, _I64, _P]),
    "tenzo_hip_lm_head_i8": (_I, [_P, _P, _F, _P, _P, _P, _I64, _I64, _P]),
    "tenzo_hip_argmax": (_I, [_P, _I64, _P, _P]),
    "tenzo_hip_sample_top_k_top_p": (_I, [_P, _I64, _I, _F, _F, _F, _P, _P]),
    "tenzo_hip_quant_rows_i8": (_I, [_P, _I64, _I64, _P, _P, _P]),
    "tenzo_hip_parse_model_mlir": (_I, [_S, _P, _I, _P, _I, _P, _P]),
    "tenzo_hip_rmsnorm_quant127": (_I, [_P, _P, _I, _F, _I64, _I64, _P, _P, _P]),
    "tenzo_hip_lm_head_i8_codes": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _P, _P]),
    "tenzo_hip_embed_i8": (_I, [_P, _P, _P, _I64, _I64, _P, _P]),
    "tenzo_hip_execute_bitlinear_tl1": (_I, [_P, _P, _P, _SZ, _SZ, _SZ, _F]),
    "tenzo_hip_execute_rmsnorm": (_I, [_P, _P, _P, _SZ, _F]),
    "tenzo_hip_engine_set_kv": (_I, [_P, _P, _P, _P, _P, _I, _I]),
    "tenzo_hip_engine_get_kv": (_I, [_P, _P, _P, _P, _P, _I]),
    "tenzo_hip_engine_set_seq_len": (_I, [_P, _I]),
    "tenzo_hip_engine_set_rope_theta": (_I, [_P, _F]),
    "tenzo_hip_engine_get_logits": (_I, [_P, _P]),
    "tenzo_hip_engine_get_buffer": (_I, [_P, _S, _P, _I64]),
    "tenzo_hip_engine_get_layer_state": (_I, [_P, _I, _I, _P, _I64]),
    "tenzo_hip_engine_use_graph": (_I, [_P, _I]),
    "tenzo_hip_engine_set_mode": (_I, [_P, _I]),
    "tenzo_hip_engine_get_mode": (_I, [_P]),
    "tenzo_hip_engine_trace": (_I, [_P, _I]),
    "tenzo_hip_engine_decode": (_I, [_P, _I, _I, _P, _P]),
    "tenzo_hip_engine_prefill": (_I, [_P, _P, _I, _I]),
    "tenzo_hip_engine_get_trace": (_I64, [_P, _P, _I64]),
    "tenzo_hip_engine_stream": (_P, [_P]),
    # include/tenzo.h
    "tenzo_get_version": (_S, []),
    # struct returns: restype set by tenzo_amd.engine
    "tenzo_default_config": (None, []),
    "tenzo_default_sampling_params": (None, []),
    "tenzo_create_engine": (_P, [_P]),
    "tenzo_destroy_engine": (None, [_P]),
    "tenzo_reset": (None, [_P]),
    "tenzo_get_seq_len": (_I, [_P]),
    "tenzo_set_layer_weights": (_I, [_P, _I, _P]),
    "tenzo_set_final_norm": (_I, [_P, _P]),
    "tenzo_set_lm_head_f32": (_I, [_P, _P, _I, _I]),
    "tenzo_set_lm_head_i8": (_I, [_P, _P, _P, _I, _I]),
    "tenzo_load_model": (_I, [_P, _S, _S]),
    "tenzo_prefill_token": (_I, [_P, _I]),
    "tenzo_generate_step": (_I, [_P, _I, _P, _P, _I]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads libtenzo_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m tenzo_amd.build` "
                "(there is no CPU fallback for the decode path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(L, name)
            except AttributeError:
                continue  # reported by missing_symbols(); calling it raises
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> list:
    return list(SIGNATURES)


def missing_symbols() -> list:
    L = load()
    out = []
    for name in SIGNATURES:
        try:
            getattr(L, name)
        except AttributeError:
            out.append(name)
    return out


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = load().tenzo_hip_last_error().decode(errors="replace")
        raise RuntimeError(f"{what or 'tenzo_hip call'} failed ({rc}): {msg}")

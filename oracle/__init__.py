"""CPU checker for the Tenzo decode hot path: test infrastructure only.

Two libraries, both loaded with ctypes:

* ``liboracle.so`` - the C restatement in ``tenzo_oracle.c`` (each function
  cites the reference line it follows; ``tenzo_oracle.h`` lists how each one is
  pinned).
* ``_ref/libtenzo_ref.so`` - the reference's own CPU engine compiled in place
  from the reference checkout by ``Makefile`` (target ``ref``). Optional: it
  exists only where it was built.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline
legs (the reference engine step and the per-config reference functions) may
import this package, and only to check or time the CPU path. The
product (``tenzo_amd``) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_HERE, "liboracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libtenzo_ref.so")
REFERENCE_DIR = "/root/reference"

_lib = None
_ref = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float


def build(ref: bool | None = None) -> None:
    """Compile liboracle.so and, when the reference checkout is present, _ref/."""
    subprocess.run(["make", "-s", "-C", _HERE, "oracle"], check=True)
    if ref is None:
        ref = os.path.isdir(os.path.join(REFERENCE_DIR, "src", "runtime"))
    if ref:
        subprocess.run(["make", "-s", "-C", _HERE, "ref", f"REF={REFERENCE_DIR}"], check=True)


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the oracle must be C-contiguous"
    return a.ctypes.data_as(_P)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build(ref=False)
        L = ctypes.CDLL(ORACLE_SO)
        sig = {
            "orc_f16_to_f32": (_F, [ctypes.c_uint16]),
            "orc_f32_to_f16": (ctypes.c_uint16, [_F]),
            "orc_tl1_pack": (None, [_P, _I64, _I64, _P]),
            "orc_tl1_pack_raw": (None, [_P, _I64, _I64, _P]),
            "orc_tl1_unpack": (None, [_P, _I64, _I64, _P]),
            "orc_quant31": (_F, [_P, _I64, _P]),
            "orc_build_lut": (None, [_P, _I64, _P]),
            "orc_tl1_gemv_i32": (None, [_P, _P, _I64, _I64, _P]),
            "orc_tl1_gemv": (_F, [_P, _P, _I64, _I64, _F, _P, _P]),
            "orc_sumsq": (_F, [_P, _I64]),
            "orc_rsqrt_est": (_F, [_F]),
            "orc_inv_rms": (_F, [_F, _I64, _F]),
            "orc_rms_norm": (None, [_P, _P, _P, _I64, _F]),
            "orc_kv_quant": (_F, [_P, _I, _P]),
            "orc_rope_table": (None, [_F, _I, _I, _P]),
            "orc_rope_apply": (None, [_P, _I, _I, _P]),
            "orc_attn_int8": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
            "orc_attention_step": (None, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P]),
            "orc_lm_head": (_F, [_P, _P, _P, _I64, _I64, _P, _P]),
            "orc_argmax": (_I, [_P, _I64]),
            "orc_rep_penalty": (None, [_P, _I64, _P, _I, _F]),
            "orc_sample_top_k_top_p": (_I, [_P, _I64, _I, _F, _F, _F]),
            "orc_quant_rows_i8": (None, [_P, _I64, _I64, _P, _P]),
            "orc_embed_i8": (None, [_P, _P, _I64, _I, _P]),
            "orc_q4_0": (None, [_P, _P, _P, _I, _I]),
            "orc_q8_0": (None, [_P, _P, _P, _I, _I]),
            "orc_gptq": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
            "orc_awq": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
            "orc_quantize_q8_0": (None, [_P, _I, _P]),
            "orc_q4_0_q8act": (None, [_P, _P, _P, _I, _I]),
            "orc_decode_step": (_I, [_P, _I, _I, _P, _P, _P]),
            "orc_tern_stats": (None, [_P, _I, _P, _P]),
            "orc_tern_pack": (None, [_P, _I, _F, _P]),
            "orc_tern_bitplanes": (None, [_P, _F, _P]),
            "orc_attn_tern": (None, [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
            "orc_attention_step_paged": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                                _I, _P, _P]),
            "orc_attention_step_tern": (None, [_I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                               _P, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref() -> ctypes.CDLL:
    """The compiled reference (raises if it was not built here)."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_SO):
            raise FileNotFoundError(f"{REF_SO} not built (make -C oracle ref)")
        R = ctypes.CDLL(REF_SO)
        sig = {
            "ref_build_lut": (_F, [_P, _I64, _P]),
            "ref_tl1_gemv": (None, [_P, _P, _I64, _I64, _F, _P]),
            "ref_tl1_gemv_acc": (_F, [_P, _P, _I64, _I64, _P]),
            "ref_rms_norm": (None, [_P, _P, _P, _I, _F]),
            "ref_pack_raw": (None, [_P, _I64, _I64, _P]),
            "ref_attention_int8": (None, [_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
            "ref_attention_tern": (None, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
            "ref_engine_create_mode": (_P, [_I, _I, _I, _I, _I, _I, _I, _I]),
            "ref_engine_get_kv_tern": (None, [_P, _I, _P, _P, _P, _P]),
            "ref_engine_set_kv_tern": (None, [_P, _I, _P, _P, _P, _P, _I]),
            "ref_attention_paged": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                                         _I, _P]),
            "ref_engine_get_kv_paged": (_I, [_P, _P, _P, _P, _P, _P]),
            "ref_q4_0": (None, [_P, _P, _P, _I, _I]),
            "ref_q8_0": (None, [_P, _P, _P, _I, _I]),
            "ref_gptq": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
            "ref_awq": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
            "ref_engine_create": (_P, [_I, _I, _I, _I, _I, _I, _I]),
            "ref_engine_destroy": (None, [_P]),
            "ref_engine_set_layer": (_I, [_P, _I, _P]),
            "ref_engine_set_head": (_I, [_P, _P, _P, _P, _I, _I]),
            "ref_engine_set_kv": (None, [_P, _P, _P, _P, _P, _I]),
            "ref_engine_get_kv": (None, [_P, _P, _P, _P, _P]),
            "ref_engine_seq_len": (_I, [_P]),
            "ref_engine_step": (_I, [_P, _I, _P]),
            "ref_engine_sample": (_I, [_P, _P, _F, _F, _I, _F, _P, _I]),
            "ref_engine_load": (_I, [_P, ctypes.c_char_p, ctypes.c_char_p]),
            "ref_engine_layer_data": (ctypes.c_long, [_P, _I, _I, _P, _P]),
            "ref_engine_head_data": (None, [_P, _P, _P, _P]),
            "ref_engine_prefill": (_I, [_P, _I]),
            "ref_engine_hidden": (None, [_P, _P]),
            "ref_num_threads": (_I, []),
            "ref_attention_int8_time": (ctypes.c_double, [_I, _I, _I, _I, _I, _P, _P, _P, _P,
                                                          _P, _P, _P, _I]),
            "ref_engine_embed": (None, [_P, _I]),
            "ref_engine_layer": (None, [_P, _I]),
            "ref_engine_finish": (None, [_P]),
            "ref_engine_buf": (_I, [_P, _I, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(R, name)
            fn.restype = res
            fn.argtypes = args
        _ref = R
    return _ref


# --------------------------------------------------------------------------
# numpy conveniences over liboracle.so
# --------------------------------------------------------------------------

def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def tl1_pack(tern: np.ndarray) -> np.ndarray:
    tern = np.ascontiguousarray(tern, dtype=np.int8)
    N, K = tern.shape
    out = np.empty(N * K // 4, np.uint8)
    lib().orc_tl1_pack(_ptr(tern), N, K, _ptr(out))
    return out


def tl1_pack_raw(raw: np.ndarray, N: int, K: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(N * K // 4, np.uint8)
    lib().orc_tl1_pack_raw(_ptr(raw), N, K, _ptr(out))
    return out


def tl1_unpack(w: np.ndarray, N: int, K: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty((N, K), np.int8)
    lib().orc_tl1_unpack(_ptr(w), N, K, _ptr(out))
    return out


def quant31(x: np.ndarray):
    x = f32(x)
    codes = np.empty(x.size, np.int8)
    inv = lib().orc_quant31(_ptr(x), x.size, _ptr(codes))
    return codes, np.float32(inv)


def build_lut(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    out = np.empty(codes.size // 2 * 32, np.int8)
    lib().orc_build_lut(_ptr(codes), codes.size, _ptr(out))
    return out


def tl1_gemv_i32(w: np.ndarray, codes: np.ndarray, N: int, K: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    acc = np.empty(N, np.int32)
    lib().orc_tl1_gemv_i32(_ptr(w), _ptr(codes), N, K, _ptr(acc))
    return acc


def tl1_gemv(x: np.ndarray, w: np.ndarray, N: int, w_scale: float):
    x = f32(x)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.empty(N, np.float32)
    acc = np.empty(N, np.int32)
    inv = lib().orc_tl1_gemv(_ptr(x), _ptr(w), N, x.size, w_scale, _ptr(y), _ptr(acc))
    return y, acc, np.float32(inv)


def sumsq(x: np.ndarray) -> np.float32:
    x = f32(x)
    return np.float32(lib().orc_sumsq(_ptr(x), x.size))


def rsqrt_est(a: float) -> np.float32:
    return np.float32(lib().orc_rsqrt_est(float(a)))


def inv_rms(ss: float, dim: int, eps: float = 1e-5) -> np.float32:
    return np.float32(lib().orc_inv_rms(float(ss), int(dim), float(eps)))


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float = 1e-5) -> np.ndarray:
    x = f32(x)
    y = np.empty_like(x)
    wp = None
    if w is not None:
        w = f32(w)
        wp = _ptr(w)
    lib().orc_rms_norm(_ptr(x), wp, _ptr(y), x.size, eps)
    return y


def kv_quant(x: np.ndarray):
    x = f32(x)
    codes = np.empty(x.size, np.int8)
    s = lib().orc_kv_quant(_ptr(x), x.size, _ptr(codes))
    return codes, np.float32(s)


def rope_table(theta: float, pos: int, head_dim: int = 128) -> np.ndarray:
    cs = np.empty(head_dim, np.float32)
    lib().orc_rope_table(theta, head_dim, pos, _ptr(cs))
    return cs


def rope_apply(x: np.ndarray, cs: np.ndarray, head_dim: int = 128) -> np.ndarray:
    y = f32(x).copy()
    lib().orc_rope_apply(_ptr(y), y.size // head_dim, head_dim, _ptr(f32(cs)))
    return y


def attn_int8(q, kc, vc, ks, vs, Hq, Hkv, max_seq, seq_len) -> np.ndarray:
    q = f32(q)
    kc = np.ascontiguousarray(kc, np.int8)
    vc = np.ascontiguousarray(vc, np.int8)
    ks = f32(ks)
    vs = f32(vs)
    out = np.zeros(Hq * 128, np.float32)
    lib().orc_attn_int8(_ptr(q), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs), Hq, Hkv, max_seq,
                        seq_len, _ptr(out))
    return out


def attention_step(q, k, v, kc, vc, ks, vs, Hq, Hkv, max_seq, pos, rope_cs, f16_scales=False):
    """forward_attention_raw: mutates copies of q/k and the given cache arrays in place."""
    q = f32(q).copy()
    k = f32(k).copy()
    v = f32(v)
    out = np.zeros(Hq * 128, np.float32)
    for a in (kc, vc, ks, vs):
        assert a.flags["C_CONTIGUOUS"]
    lib().orc_attention_step(_ptr(q), _ptr(k), _ptr(v), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs),
                             Hq, Hkv, max_seq, pos, _ptr(f32(rope_cs)), int(bool(f16_scales)),
                             _ptr(out))
    return out, q, k


# ternary KV modes: 1 = tl1_fused, 2 = popcount_fused
KV_MODES = {"int8_fused": 0, "tl1_fused": 1, "popcount_fused": 2}


def tern_stats(x):
    """(threshold, scale) of one KV / query row (TenzoEngine.cpp:544-565)."""
    x = f32(x)
    th = ctypes.c_float()
    s = ctypes.c_float()
    lib().orc_tern_stats(_ptr(x), x.size, ctypes.byref(th), ctypes.byref(s))
    return np.float32(th.value), np.float32(s.value)


def tern_pack(x, th) -> np.ndarray:
    x = f32(x)
    out = np.empty(x.size // 4, np.uint8)
    lib().orc_tern_pack(_ptr(x), x.size, float(th), _ptr(out))
    return out


def tern_bitplanes(x, th) -> np.ndarray:
    x = f32(x)
    out = np.empty(4, np.uint64)
    lib().orc_tern_bitplanes(_ptr(x), float(th), _ptr(out))
    return out


def attn_tern(mode: int, q, kb, vb, ks, vs, Hq, Hkv, max_seq, seq_len) -> np.ndarray:
    q = f32(q)
    kb = np.ascontiguousarray(kb, np.uint8)
    vb = np.ascontiguousarray(vb, np.uint8)
    out = np.zeros(Hq * 128, np.float32)
    lib().orc_attn_tern(mode, _ptr(q), _ptr(kb), _ptr(vb), _ptr(f32(ks)), _ptr(f32(vs)), Hq,
                        Hkv, max_seq, seq_len, _ptr(out))
    return out


def attention_step_tern(mode: int, q, k, v, kb, vb, ks, vs, Hq, Hkv, max_seq, pos, rope_cs):
    """forward_attention_raw in a ternary mode: mutates the given cache arrays in place."""
    q = f32(q).copy()
    k = f32(k).copy()
    v = f32(v)
    out = np.zeros(Hq * 128, np.float32)
    for a in (kb, vb, ks, vs):
        assert a.flags["C_CONTIGUOUS"]
    lib().orc_attention_step_tern(mode, _ptr(q), _ptr(k), _ptr(v), _ptr(kb), _ptr(vb), _ptr(ks),
                                  _ptr(vs), Hq, Hkv, max_seq, pos, _ptr(f32(rope_cs)), _ptr(out))
    return out, q, k


PAGE = 16  # tokens per block of the paged_int8 cache (PagedKVCache::BLOCK_SIZE)


def attention_step_paged(q, k, v, pk, pv, pks, pvs, block_table, n_layers, layer, Hq, Hkv, pos,
                         rope_cs):
    """PagedKVCache::forward_attention_raw for one layer; pools [blocks][n_layers][Hkv][16][128]
    int8 and [blocks][n_layers][Hkv][16] fp32 are updated in place."""
    q = f32(q).copy()
    k = f32(k).copy()
    v = f32(v)
    bt = np.ascontiguousarray(block_table, np.int32)
    out = np.zeros(Hq * 128, np.float32)
    for a in (pk, pv, pks, pvs):
        assert a.flags["C_CONTIGUOUS"]
    lib().orc_attention_step_paged(_ptr(q), _ptr(k), _ptr(v), _ptr(pk), _ptr(pv), _ptr(pks),
                                   _ptr(pvs), _ptr(bt), n_layers, layer, Hq, Hkv, pos,
                                   _ptr(f32(rope_cs)), _ptr(out))
    return out, q, k


def lm_head(xn, W, scales):
    xn = f32(xn)
    W = np.ascontiguousarray(W, np.int8)
    scales = f32(scales)
    V, H = W.shape
    logits = np.empty(V, np.float32)
    codes = np.empty(H, np.int8)
    s = lib().orc_lm_head(_ptr(xn), _ptr(W), _ptr(scales), V, H, _ptr(logits), _ptr(codes))
    return logits, codes, np.float32(s)


def argmax(logits) -> int:
    logits = f32(logits)
    return int(lib().orc_argmax(_ptr(logits), logits.size))


def rep_penalty(logits, tokens, penalty: float) -> np.ndarray:
    out = f32(logits).copy()
    t = np.ascontiguousarray(tokens, np.int32)
    lib().orc_rep_penalty(_ptr(out), out.size, _ptr(t), int(t.size), float(penalty))
    return out


def quant_rows_i8(E):
    E = f32(E)
    V, H = E.shape
    codes = np.empty((V, H), np.int8)
    scales = np.empty(V, np.float32)
    lib().orc_quant_rows_i8(_ptr(E), V, H, _ptr(codes), _ptr(scales))
    return codes, scales


def sample_top_k_top_p(logits, top_k: int, top_p: float, temperature: float, r: float) -> int:
    logits = f32(logits)
    return int(lib().orc_sample_top_k_top_p(_ptr(logits), logits.size, int(top_k), float(top_p),
                                            float(temperature), float(r)))


def q4_0(a, w, K, N):
    a = f32(a)
    w = np.ascontiguousarray(w, np.uint8)
    y = np.empty(N, np.float32)
    lib().orc_q4_0(_ptr(a), _ptr(w), _ptr(y), K, N)
    return y


def q8_0(a, w, K, N):
    a = f32(a)
    w = np.ascontiguousarray(w, np.uint8)
    y = np.empty(N, np.float32)
    lib().orc_q8_0(_ptr(a), _ptr(w), _ptr(y), K, N)
    return y


def gptq(a, qweight, scales, qzeros, K, N, group=128):
    a = f32(a)
    qweight = np.ascontiguousarray(qweight, np.uint32)
    scales = f32(scales)
    qzeros = np.ascontiguousarray(qzeros, np.uint32)
    y = np.empty(N, np.float32)
    lib().orc_gptq(_ptr(a), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(y), K, N, group)
    return y


def awq(a, qweight, scales, qzeros, K, N, group=128):
    a = f32(a)
    qweight = np.ascontiguousarray(qweight, np.uint32)
    scales = f32(scales)
    qzeros = np.ascontiguousarray(qzeros, np.uint32)
    y = np.empty(N, np.float32)
    lib().orc_awq(_ptr(a), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(y), K, N, group)
    return y


def quantize_q8_0(x) -> np.ndarray:
    x = f32(x)
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0(_ptr(x), x.size, _ptr(out))
    return out


def q4_0_q8act(qa, w, K, N):
    qa = np.ascontiguousarray(qa, np.uint8)
    w = np.ascontiguousarray(w, np.uint8)
    y = np.empty(N, np.float32)
    lib().orc_q4_0_q8act(_ptr(qa), _ptr(w), _ptr(y), K, N)
    return y


class RefLayerWeights(ctypes.Structure):
    """The reference's tenzo_layer_weights_t (include/tenzo.h:75-87)."""
    _fields_ = [
        ("q_w", _P), ("q_scale", _F), ("k_w", _P), ("k_scale", _F),
        ("v_w", _P), ("v_scale", _F), ("out_w", _P), ("out_scale", _F),
        ("gate_w", _P), ("gate_scale", _F), ("up_w", _P), ("up_scale", _F),
        ("down_w", _P), ("down_scale", _F),
        ("in_norm", _P), ("attn_sub_norm", _P), ("post_norm", _P), ("ffn_sub_norm", _P),
    ]


def ref_layer_struct(sm, l):
    """tenzo_layer_weights_t of layer l of a tenzo_amd.synth.SynthModel (the
    arrays must stay alive while the reference engine uses them)."""
    lw = sm.layers[l]
    w = RefLayerWeights()
    for p, f in zip(("q", "k", "v", "o", "gate", "up", "down"),
                    ("q", "k", "v", "out", "gate", "up", "down")):
        setattr(w, f + "_w", _ptr(lw.tl1[p]).value)
        setattr(w, f + "_scale", float(lw.scale[p]))
    for f in ("in_norm", "attn_sub_norm", "post_norm", "ffn_sub_norm"):
        setattr(w, f, _ptr(getattr(lw, f)).value)
    return w


class Model(ctypes.Structure):
    """Mirror of orc_model_t."""
    _fields_ = [
        ("hidden", _I), ("n_q_heads", _I), ("n_kv_heads", _I), ("n_layers", _I),
        ("ffn", _I), ("vocab", _I), ("max_seq", _I),
        ("eps", _F), ("f16_kv_scales", _I),
        ("q_w", _P), ("k_w", _P), ("v_w", _P), ("o_w", _P),
        ("gate_w", _P), ("up_w", _P), ("down_w", _P),
        ("scales", _P),
        ("in_norm", _P), ("attn_sub_norm", _P), ("post_norm", _P), ("ffn_sub_norm", _P),
        ("final_norm", _P),
        ("embed", _P), ("embed_scales", _P),
        ("kc", _P), ("vc", _P), ("ks", _P), ("vs", _P),
        ("kv_mode", _I), ("block_table", _P),
    ]


class OracleModel:
    """Holds a synthetic model (see tenzo_amd.synth.SynthModel) for orc_decode_step.

    The KV arrays are owned here and updated in place by each step.
    """

    def __init__(self, sm, f16_kv_scales: bool = True, kv_mode: int = 0, kv=None):
        """kv_mode 1 / 2 (tl1_fused / popcount_fused) take kv = (kb, vb, ks, vs):
        [L][Hkv][max_seq][32] uint8 rows and [L][Hkv][max_seq] fp32 scales."""
        self.sm = sm
        c = sm.cfg
        self._keep = []
        m = Model()
        m.hidden, m.n_q_heads, m.n_kv_heads = c.hidden, c.n_q_heads, c.n_kv_heads
        m.n_layers, m.ffn, m.vocab, m.max_seq = c.n_layers, c.ffn, c.vocab, c.max_seq
        m.eps = c.eps
        m.f16_kv_scales = int(f16_kv_scales)

        def ptr_array(arrs):
            arr = (_P * len(arrs))(*[_ptr(a) for a in arrs])
            self._keep.append(arr)
            return ctypes.cast(arr, _P)

        names = ["q", "k", "v", "o", "gate", "up", "down"]
        for nm, field in zip(names, ["q_w", "k_w", "v_w", "o_w", "gate_w", "up_w", "down_w"]):
            setattr(m, field, ptr_array([lw.tl1[nm] for lw in sm.layers]))
        self.scales = np.ascontiguousarray(
            np.array([[lw.scale[nm] for nm in names] for lw in sm.layers], np.float32))
        m.scales = _ptr(self.scales)
        for field in ["in_norm", "attn_sub_norm", "post_norm", "ffn_sub_norm"]:
            setattr(m, field, ptr_array([getattr(lw, field) for lw in sm.layers]))
        m.final_norm = _ptr(sm.final_norm)
        m.embed = _ptr(sm.embed)
        m.embed_scales = _ptr(sm.embed_scales)
        if kv_mode == 3:  # kv = (pk, pv, pks, pvs, block_table)
            self.kc, self.vc, self.ks, self.vs = (np.ascontiguousarray(a).copy() for a in kv[:4])
            self.block_table = np.ascontiguousarray(kv[4], np.int32).copy()
            m.block_table = _ptr(self.block_table)
        elif kv_mode == 0:
            self.kc = sm.kc.copy()
            self.vc = sm.vc.copy()
            self.ks = sm.ks.copy()
            self.vs = sm.vs.copy()
        else:
            self.kc, self.vc, self.ks, self.vs = (np.ascontiguousarray(a).copy() for a in kv)
            assert self.kc.dtype == np.uint8 and self.kc.shape[-1] == 32
        m.kc, m.vc, m.ks, m.vs = _ptr(self.kc), _ptr(self.vc), _ptr(self.ks), _ptr(self.vs)
        m.kv_mode = kv_mode
        self.m = m

    def step(self, token: int, pos: int, theta: float):
        c = self.sm.cfg
        cs = rope_table(theta, pos)
        logits = np.empty(c.vocab, np.float32)
        hidden = np.empty(c.hidden, np.float32)
        tok = lib().orc_decode_step(ctypes.byref(self.m), token, pos, _ptr(cs), _ptr(logits),
                                    _ptr(hidden))
        return tok, logits, hidden

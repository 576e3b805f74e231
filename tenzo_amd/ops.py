"""Operator-level interface of the decode hot path on torch device tensors.

Mirrors the reference operator surface - ``ROCmRuntime::executeBitLinearTL1``
/ ``executeRMSNorm`` (reference ``src/runtime/ROCmRuntime.h:19-37``), the
free GEMV functions ``compute_linear_gguf_q4_0`` / ``_gptq`` / ``_awq``
(``TenzoEngine.cpp:1022-1175``), ``FusedKVCache::forward_attention_raw``
(``TenzoEngine.cpp:447-919``) and ``compute_logits`` (``:1634-1720``) - with
the same argument meaning. Every call goes through libtenzo_hip.so on the
current torch stream; tensors must live on the GPU.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

F32, F16 = 0, 1


def _ptr(t: torch.Tensor | None):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tenzo_amd ops take GPU tensors")
    if not t.is_contiguous():
        raise ValueError("tenzo_amd ops take contiguous tensors")
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float16:
        return F16
    raise ValueError(f"unsupported dtype {t.dtype}")


# ------------------------------------------------------------------ TL1 ----

def tl1_packed_bytes(N: int, K: int) -> int:
    return int(_lib.load().tenzo_hip_tl1_packed_bytes(N, K))


def tl1_repack(w_tl1: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """TL1 bytes [N/64][K/2][32] -> device GEMV layout (uint8 tensor)."""
    out = torch.empty(tl1_packed_bytes(N, K), dtype=torch.uint8, device=w_tl1.device)
    _lib.check(_lib.load().tenzo_hip_tl1_repack(_ptr(w_tl1), _ptr(out), N, K, _stream()),
               "tl1_repack")
    return out


def padded(K: int) -> int:
    return (K + 63) // 64 * 64


def rmsnorm_quant31(x: torch.Tensor, norm_w: torch.Tensor | None = None, eps: float = 1e-5,
                    do_norm: bool | None = None, want_y: bool = False):
    """build_lut's activation quantization of each row of x ([M][K] or [K]),
    optionally after rms_norm_raw. Returns (codes int8 [M][Kp], actq int32
    [M][2] viewed as {inv_scale(float bits), code_sum}, y or None)."""
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    codes = torch.empty((M, padded(K)), dtype=torch.int8, device=x.device)
    q = torch.empty((M, 2), dtype=torch.int32, device=x.device)
    norm = bool(do_norm) if do_norm is not None else norm_w is not None
    y = torch.empty_like(x2) if (want_y and norm) else None
    _lib.check(_lib.load().tenzo_hip_rmsnorm_quant31(
        _ptr(x2), _ptr(norm_w), int(norm), eps, M, K, _ptr(codes), _ptr(q), _ptr(y), _stream()),
        "rmsnorm_quant31")
    return codes, q, y


def actq_inv_scale(q: torch.Tensor) -> torch.Tensor:
    return q[:, 0].contiguous().view(torch.float32)


def bitlinear_tl1(codes: torch.Tensor, q: torch.Tensor, w_packed: torch.Tensor, w_scale: float,
                  N: int, K: int, want_acc: bool = False):
    M = codes.shape[0]
    y = torch.empty((M, N), dtype=torch.float32, device=codes.device)
    acc = torch.empty((M, N), dtype=torch.int32, device=codes.device) if want_acc else None
    _lib.check(_lib.load().tenzo_hip_bitlinear_tl1(
        _ptr(codes), _ptr(q), _ptr(w_packed), w_scale, M, N, K, _ptr(y), _ptr(acc), _stream()),
        "bitlinear_tl1")
    return y, acc


def bitlinear_tl1_lut(codes: torch.Tensor, q: torch.Tensor, w_packed: torch.Tensor,
                      w_scale: float, N: int, K: int, want_acc: bool = False,
                      y: torch.Tensor | None = None):
    """bitlinear_tl1 by the reference's table method (a 16-entry table per
    activation pair in LDS, looked up per 4-bit weight pair): the same bits;
    kept to measure the two methods against each other."""
    M = codes.shape[0]
    if y is None:
        y = torch.empty((M, N), dtype=torch.float32, device=codes.device)
    acc = torch.empty((M, N), dtype=torch.int32, device=codes.device) if want_acc else None
    _lib.check(_lib.load().tenzo_hip_bitlinear_tl1_lut(
        _ptr(codes), _ptr(q), _ptr(w_packed), w_scale, M, N, K, _ptr(y), _ptr(acc), _stream()),
        "bitlinear_tl1_lut")
    return y, acc


def bitlinear_tl1_into(codes: torch.Tensor, q: torch.Tensor, w_packed: torch.Tensor,
                       w_scale: float, N: int, K: int, y: torch.Tensor) -> torch.Tensor:
    """bitlinear_tl1 writing into a caller-owned y (no allocation per call)."""
    M = codes.shape[0]
    _lib.check(_lib.load().tenzo_hip_bitlinear_tl1(
        _ptr(codes), _ptr(q), _ptr(w_packed), w_scale, M, N, K, _ptr(y), None, _stream()),
        "bitlinear_tl1")
    return y


def bitlinear_tl1_batch(codes: torch.Tensor, q: torch.Tensor, w_packed: torch.Tensor,
                        w_scale: float, N: int, K: int, want_acc: bool = False,
                        tile: int = 0, y: torch.Tensor | None = None):
    """The TL1 contraction of all M token rows of codes at once on int8 MFMA
    (prefill): the results of bitlinear_tl1, bit for bit."""
    M = codes.shape[0]
    if y is None:
        y = torch.empty((M, N), dtype=torch.float32, device=codes.device)
    acc = torch.empty((M, N), dtype=torch.int32, device=codes.device) if want_acc else None
    _lib.check(_lib.load().tenzo_hip_bitlinear_tl1_batch(
        _ptr(codes), _ptr(q), _ptr(w_packed), w_scale, M, N, K, _ptr(y), _ptr(acc), tile,
        _stream()), "bitlinear_tl1_batch")
    return y, acc


def bitlinear_tl1_f32(x: torch.Tensor, w_packed: torch.Tensor, w_scale: float, N: int,
                      K: int) -> torch.Tensor:
    """executeBitLinearTL1(act, w, out, M, K, N, scale) on device tensors."""
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().tenzo_hip_bitlinear_tl1_f32(
        _ptr(x2), _ptr(w_packed), w_scale, M, N, K, _ptr(y), _stream()), "bitlinear_tl1_f32")
    return y


def rmsnorm(x: torch.Tensor, w: torch.Tensor | None, eps: float = 1e-5) -> torch.Tensor:
    """executeRMSNorm(in, w, out, dim, eps)."""
    y = torch.empty_like(x)
    _lib.check(_lib.load().tenzo_hip_rmsnorm(_ptr(x), _ptr(w), _ptr(y), x.numel(), eps,
                                             _stream()), "rmsnorm")
    return y


# ------------------------------------------------------------ attention ----

def rope_table(theta: float, pos0: int, n_pos: int, head_dim: int = 128) -> torch.Tensor:
    """Host-side cos/sin rows (reference RoPE angles) as a CPU float tensor."""
    cs = torch.empty((n_pos, head_dim), dtype=torch.float32)
    _lib.load().tenzo_hip_rope_table(theta, head_dim, pos0, n_pos,
                                     ctypes.c_void_p(cs.data_ptr()))
    return cs


def attn_int8_decode(q, k_new, v_new, kc, vc, ks, vs, rope_cs, pos: int, want_rot=False):
    """forward_attention_raw for B sequences at position pos.

    q [B][Hq*128], k_new/v_new [B][Hkv*128] fp32; kc/vc [B][Hkv][max_seq][128]
    int8 and ks/vs [B][Hkv][max_seq] fp16 (updated in place at pos);
    rope_cs [128] fp32 on the device. Returns out [B][Hq*128] (and rotated
    q, k when want_rot)."""
    B, Hkv, max_seq, D = kc.shape
    Hq = q.numel() // (B * D)
    out = torch.empty((B, Hq * D), dtype=torch.float32, device=q.device)
    q_rot = torch.empty_like(out) if want_rot else None
    k_rot = torch.empty((B, Hkv * D), dtype=torch.float32, device=q.device) if want_rot else None
    _lib.check(_lib.load().tenzo_hip_attn_int8_decode(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs), _ptr(rope_cs),
        B, Hq, Hkv, max_seq, pos, _ptr(out), _ptr(q_rot), _ptr(k_rot), _stream()),
        "attn_int8_decode")
    return (out, q_rot, k_rot) if want_rot else out


KV_TERN_MODES = {"tl1_fused": 1, "popcount_fused": 2}


def attn_tern_decode(mode, q, k_new, v_new, kb, vb, ks, vs, rope_cs, pos: int, want_rot=False):
    """forward_attention_raw in a ternary KV mode ("tl1_fused" / "popcount_fused",
    or 1 / 2) for B sequences at position pos.

    kb/vb [B][Hkv][max_seq][32] uint8 rows and ks/vs [B][Hkv][max_seq] fp32
    (updated in place at pos); the rest as attn_int8_decode."""
    mode = KV_TERN_MODES.get(mode, mode)
    B, Hkv, max_seq, R = kb.shape
    assert R == 32 and kb.dtype == torch.uint8 and ks.dtype == torch.float32
    D = 128
    Hq = q.numel() // (B * D)
    out = torch.empty((B, Hq * D), dtype=torch.float32, device=q.device)
    q_rot = torch.empty_like(out) if want_rot else None
    k_rot = torch.empty((B, Hkv * D), dtype=torch.float32, device=q.device) if want_rot else None
    _lib.check(_lib.load().tenzo_hip_attn_tern_decode(
        int(mode), _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(kb), _ptr(vb), _ptr(ks), _ptr(vs),
        _ptr(rope_cs), B, Hq, Hkv, max_seq, pos, _ptr(out), _ptr(q_rot), _ptr(k_rot), _stream()),
        "attn_tern_decode")
    return (out, q_rot, k_rot) if want_rot else out


def attn_paged_int8_decode(q, k_new, v_new, pk, pv, pks, pvs, block_table, layer: int, rope_cs,
                           pos: int):
    """PagedKVCache::forward_attention_raw for one layer at position pos (batch 1).

    pk/pv [blocks][n_layers][Hkv][16][128] int8 and pks/pvs [blocks][n_layers][Hkv][16]
    fp32 (updated in place at pos); block_table int32 covering position pos."""
    nb, n_layers, Hkv, page, D = pk.shape
    assert page == 16 and pk.dtype == torch.int8 and pks.dtype == torch.float32
    assert block_table.dtype == torch.int32 and block_table.numel() * 16 > pos
    Hq = q.numel() // D
    out = torch.empty((1, Hq * D), dtype=torch.float32, device=q.device)
    _lib.check(_lib.load().tenzo_hip_attn_paged_int8_decode(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(pk), _ptr(pv), _ptr(pks), _ptr(pvs),
        _ptr(block_table), n_layers, layer, _ptr(rope_cs), Hq, Hkv, pos, _ptr(out), _stream()),
        "attn_paged_int8_decode")
    return out


# -------------------------------------------------------- quantized GEMV ---

def gemv_q4_0(act: torch.Tensor, w: torch.Tensor, K: int, N: int) -> torch.Tensor:
    a = act.reshape(-1, K).contiguous()
    B = a.shape[0]
    y = torch.empty((B, N), dtype=torch.float32, device=act.device)
    _lib.check(_lib.load().tenzo_hip_gemv_q4_0(_ptr(a), _dtype_code(a), _ptr(w), _ptr(y), K, N,
                                               B, _stream()), "gemv_q4_0")
    return y


def gemv_q8_0(act: torch.Tensor, w: torch.Tensor, K: int, N: int) -> torch.Tensor:
    """compute_linear_gguf_q8_0 for B activation rows (fp32 or fp16) of K:
    w = N rows of K/32 blocks of 34 bytes. Returns [B][N] fp32."""
    a = act.reshape(-1, K).contiguous()
    B = a.shape[0]
    y = torch.empty((B, N), dtype=torch.float32, device=act.device)
    _lib.check(_lib.load().tenzo_hip_gemv_q8_0(_ptr(a), _dtype_code(a), _ptr(w), _ptr(y), K, N,
                                               B, _stream()), "gemv_q8_0")
    return y


def gemv_q4_0_q8_0(qa: torch.Tensor, w: torch.Tensor, K: int, N: int) -> torch.Tensor:
    B = qa.numel() // (K // 32 * 34)
    y = torch.empty((B, N), dtype=torch.float32, device=qa.device)
    _lib.check(_lib.load().tenzo_hip_gemv_q4_0_q8_0(_ptr(qa), _ptr(w), _ptr(y), K, N, B,
                                                    _stream()), "gemv_q4_0_q8_0")
    return y


def _gemv_gq(fn_name, act, qweight, scales, qzeros, K, N, group):
    a = act.reshape(-1, K).contiguous()
    B = a.shape[0]
    y = torch.empty((B, N), dtype=torch.float32, device=act.device)
    fn = getattr(_lib.load(), fn_name)
    _lib.check(fn(_ptr(a), _dtype_code(a), _ptr(qweight), _ptr(scales), _dtype_code(scales),
                  _ptr(qzeros), _ptr(y), K, N, group, B, _stream()), fn_name)
    return y


def gemv_gptq(act, qweight, scales, qzeros, K: int, N: int, group: int = 128):
    return _gemv_gq("tenzo_hip_gemv_gptq", act, qweight, scales, qzeros, K, N, group)


def gemv_awq(act, qweight, scales, qzeros, K: int, N: int, group: int = 128):
    return _gemv_gq("tenzo_hip_gemv_awq", act, qweight, scales, qzeros, K, N, group)


# -------------------------------------------------------------- LM head ----

def i8_packed_bytes(V: int, H: int) -> int:
    return int(_lib.load().tenzo_hip_i8_packed_bytes(V, H))


def i8_rows_repack(w: torch.Tensor, V: int, H: int) -> torch.Tensor:
    out = torch.empty(i8_packed_bytes(V, H), dtype=torch.uint8, device=w.device)
    _lib.check(_lib.load().tenzo_hip_i8_rows_repack(_ptr(w), _ptr(out), V, H, _stream()),
               "i8_rows_repack")
    return out


def lm_head_i8(x, norm_w, w_packed, scales, V: int, H: int, eps: float = 1e-5):
    logits = torch.empty(V, dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().tenzo_hip_lm_head_i8(_ptr(x), _ptr(norm_w), eps, _ptr(w_packed),
                                                _ptr(scales), _ptr(logits), V, H, _stream()),
               "lm_head_i8")
    return logits


def actquant127(x: torch.Tensor, norm_w: torch.Tensor | None = None, eps: float = 1e-5):
    """compute_logits' activation quantization of each row of x ([M][K] or
    [K]), after rms_norm_raw when norm_w is given. Returns (codes int8 [M][K],
    actq int32 [M][2])."""
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    codes = torch.empty((M, K), dtype=torch.int8, device=x.device)
    q = torch.empty((M, 2), dtype=torch.int32, device=x.device)
    _lib.check(_lib.load().tenzo_hip_rmsnorm_quant127(
        _ptr(x2), _ptr(norm_w), int(norm_w is not None), eps, M, K, _ptr(codes), _ptr(q),
        _stream()), "rmsnorm_quant127")
    return codes, q


def lm_head_i8_codes_into(codes, q, w_packed, scales, V: int, H: int, logits,
                          idx=None):
    """The LM-head GEMV on precomputed codes into caller-owned logits (and the
    fused greedy argmax into idx when given)."""
    _lib.check(_lib.load().tenzo_hip_lm_head_i8_codes(
        _ptr(codes), _ptr(q), _ptr(w_packed), _ptr(scales), _ptr(logits), V, H, _ptr(idx),
        _stream()), "lm_head_i8_codes")
    return logits


def argmax(logits: torch.Tensor) -> torch.Tensor:
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    _lib.check(_lib.load().tenzo_hip_argmax(_ptr(logits), logits.numel(), _ptr(out), _stream()),
               "argmax")
    return out


def sample_top_k_top_p(logits: torch.Tensor, top_k: int, top_p: float, temperature: float,
                       r: float) -> int:
    """sample_top_k_top_p's sampling branch on device logits with the draw r."""
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    _lib.check(_lib.load().tenzo_hip_sample_top_k_top_p(
        _ptr(logits), logits.numel(), int(top_k), float(top_p), float(temperature), float(r),
        _ptr(out), _stream()), "sample_top_k_top_p")
    return int(out.item())


def embed_i8(w_packed, scales, token: torch.Tensor, V: int, H: int) -> torch.Tensor:
    x = torch.empty(H, dtype=torch.float32, device=w_packed.device)
    _lib.check(_lib.load().tenzo_hip_embed_i8(_ptr(w_packed), _ptr(scales), _ptr(token), V, H,
                                              _ptr(x), _stream()), "embed_i8")
    return x

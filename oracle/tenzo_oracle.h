/*
 * tenzo_oracle.h - CPU restatement of Tenzo's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * CPU baseline legs may load this library, and only as the checker. The product
 * (tenzo_amd/, libtenzo_hip.so) never calls it.
 *
 * Every function restates one reference function (file:line into the reference
 * checkout, src/runtime/TenzoEngine.cpp unless noted). Plain scalar C, built with
 * -ffp-contract=off so that the only fused multiply-adds are the explicit fmaf()
 * calls, which stand where the reference's AVX2 code issues _mm256_fmadd_ps.
 *
 * Pinning (how each function is checked, in tests/test_oracle.py):
 *   orc_tl1_pack, orc_tl1_pack_raw   reference packers' layout (golden vectors
 *                                    from the compiled reference) + brute-force
 *                                    unpack round trip
 *   orc_quant31, orc_build_lut       compiled-reference goldens (bit-exact LUT
 *                                    bytes and scale) + closed form
 *   orc_tl1_gemv_i32 / orc_tl1_gemv  closed form sum_k W[n,k]*a_k (dense brute
 *                                    force) + compiled-reference goldens (bit-exact)
 *   orc_sumsq, orc_inv_rms,
 *   orc_rms_norm                     compiled reference (bit-exact at dims 1..8200,
 *                                    live and fixture) + fp64 brute force (1e-6)
 *                                    + the eight-chain order against an exact
 *                                    rational restatement on small rows
 *   orc_rsqrt_est                    the host's RSQRTSS over every positive normal
 *                                    float (Intel hosts) + exponent scaling
 *   orc_kv_quant                     compiled-reference goldens (bit-exact codes)
 *                                    + special cases (all-zero, single spike)
 *   orc_rope_table, orc_rope_apply   compiled reference (bit-exact rotated q/k) +
 *                                    fp64 closed form
 *   orc_attn_int8                    fp64 brute-force softmax attention over the
 *                                    dequantized cache (1e-3) + compiled reference
 *                                    + ctx=1 special case
 *   orc_lm_head                      closed-form int32 dot + compiled reference
 *   orc_q4_0, orc_q8_0               compiled reference (bit-exact: the lane chains
 *                                    and their pairwise sum, live at three shapes
 *                                    and the goldens) + fp64 brute force
 *   orc_gptq, orc_awq                fp64 brute force of each dequant formula +
 *                                    compiled-reference goldens (layout conventions;
 *                                    the build's vectorised order is not restated)
 *   orc_q4_0_q8act                   no reference counterpart: closed form (fp64
 *                                    brute force of the block formula)
 *   orc_quantize_q8_0                llama.cpp's published quantize_row_q8_0 (no
 *                                    reference counterpart), pinned by the
 *                                    properties its arithmetic fixes: amax -> +-127,
 *                                    |q| <= 127, zero block -> d = 0, fp16 scale of
 *                                    amax/127, half-step reconstruction bound, exact
 *                                    half-steps away from zero
 *   orc_decode_step                  compiled reference whole-engine step on small
 *                                    configs (logits 1e-3, greedy token equal)
 *   orc_argmax                       brute force (first maximum)
 *   orc_rep_penalty                  the compiled reference's sampler (its logits
 *                                    after the penalty, bit-exact) with repeated,
 *                                    negative, zero and out-of-range tokens + a
 *                                    check that a true division rounds differently
 *   orc_tern_stats, orc_tern_pack,
 *   orc_tern_bitplanes,
 *   orc_attention_step_tern          compiled reference (bit-exact rows and scales,
 *                                    outputs 1e-5; fixture and live) + special rows
 *                                    (zero, constant magnitude, one spike) + a check
 *                                    that index-order sums give other scales
 *                                    (tests/test_kv_tern.py)
 *   orc_attn_tern                    closed forms: seq_len 1 (out = w_v s_v, fields
 *                                    3 read 0) and two tokens (out = tanh(score/2)
 *                                    with a brute-force integer dot)
 *   orc_attention_step_paged         compiled reference (bit-exact pool rows and
 *                                    scales, outputs 1e-5, permuted block tables)
 *   orc_quant_rows_i8                the compiled reference's loader output (its
 *                                    int8 LM head and row scales, bit-exact) on
 *                                    synthetic model files
 *   orc_sample_top_k_top_p           the compiled reference's own sampler on the
 *                                    same logits and the same rand() draw (token
 *                                    equal) + special cases (top_k 1 = argmax,
 *                                    tiny temperature = argmax, top_p 1 keeps k)
 */
#ifndef TENZO_ORACLE_H
#define TENZO_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 helpers (IEEE binary16, round to nearest even) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- TL1 packing ---- */
/* Dense ternary [N][K] in {-1,0,1} -> TL1 [N/64][K/2][32]
 * (PybindModule.cpp:315-355). */
void orc_tl1_pack(const int8_t* tern, int64_t N, int64_t K, uint8_t* out);
/* HF 2-bit [N/4][K] (row r at byte r/4, shift 2*(r%4)) -> TL1 (TenzoEngine.cpp:1842-1884). */
void orc_tl1_pack_raw(const uint8_t* raw, int64_t N, int64_t K, uint8_t* out);
/* TL1 -> dense ternary [N][K] (inverse of orc_tl1_pack). */
void orc_tl1_unpack(const uint8_t* w, int64_t N, int64_t K, int8_t* tern);

/* ---- activation quantization for TL1 (build_lut, TenzoEngine.cpp:22-62) ---- */
/* codes[k] = round(x[k] * (31/absmax)); returns absmax/31. */
float orc_quant31(const float* x, int64_t K, int8_t* codes);
/* The 32-byte LUT record per k-pair, as build_lut writes it. */
void orc_build_lut(const int8_t* codes, int64_t K, int8_t* lut);

/* ---- TL1 GEMV (compute_single_block / compute_from_lut, :64-146) ---- */
void orc_tl1_gemv_i32(const uint8_t* w, const int8_t* codes, int64_t N, int64_t K,
                      int32_t* acc);
/* y[n] = float(acc[n]) * (absmax/31 * w_scale); acc optional. Returns absmax/31. */
float orc_tl1_gemv(const float* x, const uint8_t* w, int64_t N, int64_t K, float w_scale,
                   float* y, int32_t* acc);

/* ---- RMSNorm (rms_norm_raw, :148-166, as the reference build evaluates it) ---- */
/* Sum of squares: eight FMA chains (chain j over x[j], x[j+8], ...), the n % 8
 * tail added to chain 0, then ((c0+c4)+(c2+c6)) + ((c1+c5)+(c3+c7)). */
float orc_sumsq(const float* x, int64_t n);
/* RSQRTSS estimate of the reference's build host (table, exact for every
 * positive normal a). */
float orc_rsqrt_est(float a);
/* inv_rms = (y0 * -0.5) * fma(a * y0, y0, -3), a = ss / dim + eps, y0 = est(a). */
float orc_inv_rms(float ss, int64_t dim, float eps);
/* y = (x * w) * inv_rms, or x * inv_rms without weights. */
void orc_rms_norm(const float* x, const float* w, float* y, int64_t dim, float eps);

/* ---- INT8 KV cache (FusedKVCache, TenzoEngine.h:60-115, .cpp:506-533) ---- */
/* codes = clamp(round(x/s)), s = max(1e-8, amax)/127; returns s. */
float orc_kv_quant(const float* x, int d, int8_t* codes);
/* RoPE angle table for one position (:454-504 formula, theta as a parameter):
 * cs[i] = cosf(pos*f_i), cs[d/2+i] = sinf(pos*f_i) with f_i = 1/theta^(2i/d)
 * evaluated as the reference build does: expf(-(2i/d) * logf(theta)) in fp32,
 * angle = (float)pos * f_i in fp32, glibc cosf/sinf. */
void orc_rope_table(float theta, int head_dim, int pos, float* cs);
/* In-place NeoX half-split rotation of nheads heads (:460-504). */
void orc_rope_apply(float* x, int nheads, int head_dim, const float* cs);
/* Decode attention over t in [0, seq_len) for Hq query heads, GQA map
 * kvh = qh / (Hq/Hkv) (:657-919, int8 branches). Cache arrays are
 * [Hkv][max_seq][128] codes and [Hkv][max_seq] fp32 scales. */
void orc_attn_int8(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                   const float* vs, int Hq, int Hkv, int max_seq, int seq_len,
                   float* out);
/* forward_attention_raw as a whole: RoPE on q/k (in place), quantize-append k/v
 * at pos (scale stored as fp32, or fp16-rounded when f16_scales != 0), then
 * attention over pos+1 tokens. */
void orc_attention_step(float* q, float* k, const float* v, int8_t* kc, int8_t* vc,
                        float* ks, float* vs, int Hq, int Hkv, int max_seq, int pos,
                        const float* rope_cs, int f16_scales, float* out);

/* ---- int8 LM head (compute_logits, :1634-1720), input already normalized ---- */
/* Returns s_x; codes optional. */
/* ---- ternary KV modes (tl1_fused = 1, popcount_fused = 2; :534-648, :695-885) ---- */
void orc_tern_stats(const float* x, int d, float* th, float* s);
void orc_tern_pack(const float* x, int d, float th, uint8_t* out);
void orc_tern_bitplanes(const float* x, float th, uint64_t* out);
/* kb / vb [Hkv][max_seq][32] bytes, ks / vs [Hkv][max_seq] fp32 */
void orc_attn_tern(int mode, const float* q, const uint8_t* kb, const uint8_t* vb,
                   const float* ks, const float* vs, int Hq, int Hkv, int max_seq,
                   int seq_len, float* out);
void orc_attention_step_tern(int mode, float* q, float* k, const float* v, uint8_t* kb,
                             uint8_t* vb, float* ks, float* vs, int Hq, int Hkv, int max_seq,
                             int pos, const float* rope_cs, float* out);

/* ---- paged_int8 (PagedKVCache::forward_attention_raw :269-445), one layer ---- */
void orc_attention_step_paged(float* q, float* k, const float* v, int8_t* pk, int8_t* pv,
                              float* pks, float* pvs, const int32_t* block_table, int n_layers,
                              int layer, int Hq, int Hkv, int pos, const float* rope_cs,
                              float* out);

float orc_lm_head(const float* xn, const int8_t* W, const float* scales, int64_t V,
                  int64_t H, float* logits, int8_t* codes);
int orc_argmax(const float* logits, int64_t V);
/* Repetition penalty in place (:1735-1743 as built: positive logits times
 * 1/penalty, others times penalty; per occurrence; skipped at penalty 1). */
void orc_rep_penalty(float* logits, int64_t V, const int32_t* tokens, int n, float penalty);
/* load_model_from_files' LM-head quantization (:1925-1941), row-major [V][H]. */
void orc_quant_rows_i8(const float* E, int64_t V, int64_t H, int8_t* codes, float* scales);
/* sample_top_k_top_p (:1722-1807), temperature > 0, with the draw r in [0, 1]. */
int orc_sample_top_k_top_p(const float* logits, int64_t V, int top_k, float top_p,
                           float temperature, float r);
/* embedding_lookup int8 branch (:1294-1316). */
void orc_embed_i8(const int8_t* E, const float* scales, int64_t H, int token, float* x);

/* ---- quantized GEMVs (:1022-1175) ---- */
void orc_q4_0(const float* a, const uint8_t* w, float* y, int K, int N);
void orc_q8_0(const float* a, const uint8_t* w, float* y, int K, int N);
void orc_gptq(const float* a, const uint32_t* qweight, const float* scales,
              const uint32_t* qzeros, float* y, int K, int N, int group);
void orc_awq(const float* a, const uint32_t* qweight, const float* scales,
             const uint32_t* qzeros, float* y, int K, int N, int group);
/* Q8_0 activation blocks (34 B: fp16 d + 32 int8), llama.cpp quantize_row_q8_0. */
void orc_quantize_q8_0(const float* x, int K, uint8_t* out);
/* Q4_0 weights x Q8_0 activations (closed form; no reference counterpart). */
void orc_q4_0_q8act(const uint8_t* qa, const uint8_t* w, float* y, int K, int N);

/* ---- whole decode step (forward_layer_raw :1522-1632, generate_step :1821-1838) ---- */
typedef struct {
    int hidden, n_q_heads, n_kv_heads, n_layers, ffn, vocab, max_seq;
    float eps;            /* 1e-5 (rms_norm_raw default) */
    int f16_kv_scales;    /* store KV scales rounded to fp16 */
    /* per layer, TL1 [N/64][K/2][32] */
    const uint8_t** q_w; const uint8_t** k_w; const uint8_t** v_w; const uint8_t** o_w;
    const uint8_t** gate_w; const uint8_t** up_w; const uint8_t** down_w;
    const float* scales;  /* [n_layers][7]: q,k,v,o,gate,up,down */
    const float** in_norm; const float** attn_sub_norm; const float** post_norm;
    const float** ffn_sub_norm;
    const float* final_norm;
    const int8_t* embed;  /* [vocab][hidden] int8, tied LM head */
    const float* embed_scales;
    /* KV cache state, [n_layers][n_kv_heads][max_seq][128] / [..][max_seq];
     * kv_mode 1 / 2: rows of 32 bytes (see orc_attn_tern), fp32 scales */
    int8_t* kc; int8_t* vc; float* ks; float* vs;
    int kv_mode;          /* 0 int8_fused, 1 tl1_fused, 2 popcount_fused, 3 paged_int8 */
    /* paged_int8: kc / vc are the pools [blocks][n_layers][Hkv][16][128], ks / vs
     * their fp32 scales, block_table maps logical to physical blocks */
    const int32_t* block_table;
} orc_model_t;

/* Runs one token through all layers at position pos (appending to the cache),
 * then the LM head; writes logits (vocab) and the final hidden state (hidden),
 * either may be null. rope_cs is the per-position table (head_dim floats).
 * Returns the greedy token. */
int orc_decode_step(const orc_model_t* m, int token, int pos, const float* rope_cs,
                    float* logits, float* hidden);

#ifdef __cplusplus
}
#endif
#endif

/*
 * tenzo_hip.h - C ABI of the MI355X (gfx950) decode hot path.
 *
 * Operator-level entry points: every pointer is DEVICE memory unless stated,
 * sizes are element counts, `stream` is a hipStream_t passed as void*
 * (NULL = the null stream). Calls are stream-ordered and asynchronous; no
 * exception crosses the ABI. Return value: 0 on success or a negative
 * tenzo_status_t (include/tenzo.h); tenzo_hip_last_error() gives the message.
 * The caller owns every buffer it passes. Scratch memory (split-K partial
 * sums, attention partials) is owned by the library, one region per device,
 * grown on demand; calls that overlap on one device must be issued on one
 * stream.
 *
 * Each entry point names the reference function it replaces (file:line into
 * the reference checkout, src/runtime/ unless noted).
 */
#ifndef TENZO_HIP_H
#define TENZO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define TENZO_HIP_API __attribute__((visibility("default")))
#else
#define TENZO_HIP_API
#endif

/* Per-token activation quantization parameters, device resident (8 bytes). */
typedef struct {
    float inv_scale; /* absmax/31 (TL1) or absmax/127 (LM head), as fp32 */
    int32_t code_sum; /* sum of the int8 codes (TL1 kernels use it) */
} tenzo_hip_actq_t;

TENZO_HIP_API const char* tenzo_hip_version(void);
TENZO_HIP_API const char* tenzo_hip_last_error(void);
/* Number of visible HIP devices (0 when none). */
TENZO_HIP_API int tenzo_hip_device_count(void);
/* Frees the library-owned scratch of the current device. */
TENZO_HIP_API int tenzo_hip_release_scratch(void);

/* ---- TL1 ternary GEMV -------------------------------------------------- */

/* Bytes of the device layout that tenzo_hip_tl1_repack writes for an N x K
 * matrix: (N/64) * ceil(K/64) * 1024. */
TENZO_HIP_API size_t tenzo_hip_tl1_packed_bytes(int64_t N, int64_t K);

/* Repacks TL1 blocks [N/64][K/2][32] (the layout compute_single_block reads,
 * TenzoEngine.cpp:64-127, written by PybindModule.cpp:315-355 and
 * TenzoEngine.cpp:1842-1884) into the device GEMV layout. N % 64 == 0,
 * K % 2 == 0. */
TENZO_HIP_API int tenzo_hip_tl1_repack(const uint8_t* w_tl1, void* w_packed, int64_t N,
                                       int64_t K, void* stream);

/* The device layout straight from the raw 2-bit layout the model loader
 * reads (pack_ternary_weights_raw's input, TenzoEngine.cpp:1842-1884: byte
 * (r/4, c) of [N/4][K] holds row r, column c at bits 2(r%4) as w+1): the same
 * bytes as tenzo_hip_tl1_repack of the TL1 blocks that function produces.
 * N % 64 == 0. */
TENZO_HIP_API int tenzo_hip_tl1_repack_raw(const uint8_t* raw, void* w_packed, int64_t N,
                                           int64_t K, void* stream);

/* Activation quantization of build_lut (TenzoEngine.cpp:22-62) for M tokens
 * of K values: codes[m][k] = round(x * 31/absmax), written with a row stride
 * of ceil(K/64)*64 (zero padded); q[m] = {absmax/31, sum of codes}. When
 * norm_w is non-null or do_norm is set, x is first replaced by
 * rms_norm_raw(x, norm_w, eps) (TenzoEngine.cpp:148-166) and, if y_out is
 * non-null, the normalized values are written there. */
TENZO_HIP_API int tenzo_hip_rmsnorm_quant31(const float* x, const float* norm_w, int do_norm,
                                            float eps, int64_t M, int64_t K, int8_t* codes,
                                            tenzo_hip_actq_t* q, float* y_out, void* stream);

/* TL1 GEMV on quantized activations (compute_from_lut, TenzoEngine.cpp:129-146):
 * acc[m][n] = sum_k W[n][k] * codes[m][k] (exact int32),
 * y[m][n] = float(acc) * (q[m].inv_scale * w_scale). acc_out may be null. */
TENZO_HIP_API int tenzo_hip_bitlinear_tl1(const int8_t* codes, const tenzo_hip_actq_t* q,
                                          const void* w_packed, float w_scale, int64_t M,
                                          int64_t N, int64_t K, float* y, int32_t* acc_out,
                                          void* stream);

/* The same product as tenzo_hip_bitlinear_tl1 by the reference's own table
 * method (build_lut and compute_single_block, TenzoEngine.cpp:22-127): a
 * 16-entry table per activation pair in LDS, looked up with each 4-bit pair of
 * weight codes. Same arguments and bit-identical results; it is there to
 * measure the table method against the masked-v_dot4 kernel, not used by the
 * engine. K needs at most 64 KiB of tables per workgroup. */
TENZO_HIP_API int tenzo_hip_bitlinear_tl1_lut(const int8_t* codes, const tenzo_hip_actq_t* q,
                                              const void* w_packed, float w_scale, int64_t M,
                                              int64_t N, int64_t K, float* y, int32_t* acc_out,
                                              void* stream);

/* Multi-token TL1 contraction on int8 MFMA (prefill): the same results as M
 * separate compute_from_lut calls (TenzoEngine.cpp:129-146), which
 * prefill_token (TenzoEngine.cpp:1809-1819) makes one token at a time, from
 * one pass over the packed weights: acc[m][n] and y[m][n] as in
 * tenzo_hip_bitlinear_tl1, bit for bit. tile = 0 picks the workgroup shape;
 * 100 * KW + 10 * RW + CT forces 64*RW rows x 32*CT tokens with KW K groups
 * (142, 242, 442, 222, 422, 221, 421, 412, 411 or 811, with
 * (N/64) % RW == 0). No scratch memory is used. */
TENZO_HIP_API int tenzo_hip_bitlinear_tl1_batch(const int8_t* codes, const tenzo_hip_actq_t* q,
                                                const void* w_packed, float w_scale, int64_t M,
                                                int64_t N, int64_t K, float* y,
                                                int32_t* acc_out, int tile, void* stream);

/* executeBitLinearTL1(act, w, out, M, K, N, scale) (ROCmRuntime.h:20-28) on
 * device pointers: quantize each of the M activation rows then run the TL1
 * GEMV over the packed weights. */
TENZO_HIP_API int tenzo_hip_bitlinear_tl1_f32(const float* x, const void* w_packed,
                                              float w_scale, int64_t M, int64_t N, int64_t K,
                                              float* y, void* stream);

/* executeRMSNorm(in, w, out, dim, eps) (ROCmRuntime.h:31-37) on device pointers. */
TENZO_HIP_API int tenzo_hip_rmsnorm(const float* x, const float* w, float* y, int64_t dim,
                                    float eps, void* stream);

/* ---- INT8 KV-cache decode attention ------------------------------------ */

/* One decode step of FusedKVCache::forward_attention_raw (TenzoEngine.cpp:447-919,
 * int8_fused mode) for B sequences at the same position pos:
 *   q [B][Hq][128], k_new / v_new [B][Hkv][128] fp32;
 *   cache codes kc / vc [B][Hkv][max_seq][128] int8,
 *   scales ks / vs [B][Hkv][max_seq] fp16 (fp32 in the reference);
 *   rope_cs: cos[64] then sin[64] for position pos (tenzo_hip_rope_table);
 * RoPE is applied to q and k_new, k_new/v_new are quantized and appended at
 * pos, and out [B][Hq][128] receives attention over positions 0..pos.
 * q_rot / k_rot, when non-null, receive the rotated q / k (they must not
 * alias q / k_new). GQA: query head h reads kv head h / (Hq/Hkv). */
TENZO_HIP_API int tenzo_hip_attn_int8_decode(const float* q, const float* k_new,
                                             const float* v_new, int8_t* kc, int8_t* vc,
                                             uint16_t* ks, uint16_t* vs, const float* rope_cs,
                                             int B, int Hq, int Hkv, int max_seq, int pos,
                                             float* out, float* q_rot, float* k_rot,
                                             void* stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tenzo_hip_attn_int8_decode, same arguments and results,
 * with its chunk partials in a fixed 8 MiB array of device memory per device
 * that comes with the library's code object instead of the library scratch;
 * it calls no allocator. Calls whose partials exceed the array
 * (B * Hq * chunks * 520 bytes: e.g. B 1 up to ~200k tokens of context, B 16
 * up to 8k) return TENZO_ERROR_INVALID_ARGUMENT. Every call on a device
 * shares that device's array: calls that overlap on one device race. */
TENZO_HIP_API int tenzo_hip_attn_int8_decode_noalloc(const float* q, const float* k_new,
                                                     const float* v_new, int8_t* kc, int8_t* vc,
                                                     uint16_t* ks, uint16_t* vs,
                                                     const float* rope_cs, int B, int Hq, int Hkv,
                                                     int max_seq, int pos, float* out,
                                                     float* q_rot, float* k_rot, void* stream);

/* ---- Ternary KV-cache decode attention ----------------------------------- */

/* One decode step of FusedKVCache::forward_attention_raw in the ternary modes
 * (TenzoEngine.cpp:534-648 append, :695-805 scores, :852-885 values):
 * mode 1 = "tl1_fused", 2 = "popcount_fused". Arguments as
 * tenzo_hip_attn_int8_decode, with cache rows of 32 bytes per (kv head, token)
 * kb / vb [B][Hkv][max_seq][32] and fp32 scales ks / vs [B][Hkv][max_seq]:
 *   V rows and mode-1 K rows: byte i = dims 4i..4i+3 as 2-bit fields w + 1
 *   (w in {-1, 0, 1}, bit 2j for dim 4i + j; a field 3 reads as 0);
 *   mode-2 K rows: uint64 {kp0, kp1, kn0, kn1} sign bitplanes (bit d of
 *   kp0 / kn0: dim d above / below the row's threshold; kp1 / kn1 dims 64..127),
 *   the layout of the reference's PopcountBitplanes (TenzoEngine.h:87-89).
 * The new row is thresholded at half its mean |x| with scale = mean |x| over
 * the dims above it (reductions in the order of the reference build). */
TENZO_HIP_API int tenzo_hip_attn_tern_decode(int mode, const float* q, const float* k_new,
                                             const float* v_new, uint8_t* kb, uint8_t* vb,
                                             float* ks, float* vs, const float* rope_cs, int B,
                                             int Hq, int Hkv, int max_seq, int pos, float* out,
                                             float* q_rot, float* k_rot, void* stream);

/* ---- paged_int8 decode attention ----------------------------------------- */

/* One decode step of PagedKVCache::forward_attention_raw (TenzoEngine.cpp:269-445)
 * for one layer of a block pool: codes pk / pv [blocks][n_layers][Hkv][16][128]
 * int8, fp32 scales pks / pvs [blocks][n_layers][Hkv][16]; block_table[t / 16]
 * is the physical block of token t and must already hold the block of pos (the
 * reference allocates it on reaching a new block, :318-324). q / k_new / v_new
 * as tenzo_hip_attn_int8_decode (batch 1); the new row is quantized like
 * int8_fused with an fp32 scale; softmax 1 / (sum + 1e-8); tokens with weight
 * below 1e-7 add no value. */
TENZO_HIP_API int tenzo_hip_attn_paged_int8_decode(const float* q, const float* k_new,
                                                   const float* v_new, int8_t* pk, int8_t* pv,
                                                   float* pks, float* pvs,
                                                   const int32_t* block_table, int n_layers,
                                                   int layer, const float* rope_cs, int Hq,
                                                   int Hkv, int pos, float* out, void* stream);

/* HOST function: fills cs[pos - pos0][0..127] = cos/sin table rows for
 * positions pos0 .. pos0+n_pos-1 with the reference's RoPE angles
 * (TenzoEngine.cpp:465-469; theta is 10000 there and a parameter here). */
TENZO_HIP_API void tenzo_hip_rope_table(float theta, int head_dim, int pos0, int n_pos,
                                        float* cs_host);

/* ---- Quantized GEMVs (TenzoEngine.cpp:1022-1175) ------------------------ */

/* act_dtype / scale_dtype: 0 = fp32, 1 = fp16. B activation rows
 * ([B][K]), outputs [B][N] fp32. */

/* compute_linear_gguf_q4_0 (:1022-1075): w [N][K/32] blocks of 18 bytes. */
TENZO_HIP_API int tenzo_hip_gemv_q4_0(const void* act, int act_dtype, const uint8_t* w,
                                      float* y, int K, int N, int B, void* stream);
/* compute_linear_gguf_q8_0 (:1078-1114): w [N][K/32] blocks of 34 bytes
 * (fp16 d, 32 int8 codes), 2-byte aligned. */
TENZO_HIP_API int tenzo_hip_gemv_q8_0(const void* act, int act_dtype, const uint8_t* w,
                                      float* y, int K, int N, int B, void* stream);
/* Q4_0 weights x Q8_0 activations (no reference counterpart: the reference
 * has only fp32 activations for Q4_0): qa = B rows of K/32 blocks of 34 bytes. */
TENZO_HIP_API int tenzo_hip_gemv_q4_0_q8_0(const uint8_t* qa, const uint8_t* w, float* y,
                                           int K, int N, int B, void* stream);
/* compute_linear_gptq (:1117-1143): qweight [K/8][N] u32, scales [K/g][N],
 * qzeros [ceil(K/g/8)][N] u32 (nibble g%8, zero = nibble + 1). B <= 8
 * rows; 9..16 with 16-byte aligned fp16 activations, K % 512 == 0,
 * g in {32, 64, 128, 256, 512} and B (K + 4) fp16 within 152 KiB (fp16 MFMA,
 * which also serves batch 4..8 of that form). */
TENZO_HIP_API int tenzo_hip_gemv_gptq(const void* act, int act_dtype, const uint32_t* qweight,
                                      const void* scales, int scale_dtype,
                                      const uint32_t* qzeros, float* y, int K, int N,
                                      int group, int B, void* stream);
/* compute_linear_awq (:1146-1175): qweight [K/8][N] (nibble e holds element
 * k + {0,2,4,6,1,3,5,7}[e]), scales [K/g][N], qzeros [K/g][N/8]. Batch
 * limits as for GPTQ. */
TENZO_HIP_API int tenzo_hip_gemv_awq(const void* act, int act_dtype, const uint32_t* qweight,
                                     const void* scales, int scale_dtype,
                                     const uint32_t* qzeros, float* y, int K, int N, int group,
                                     int B, void* stream);

/* ---- int8 LM head, embedding, greedy sampling -------------------------- */

/* Bytes of the device layout tenzo_hip_i8_rows_repack writes for V x H:
 * ceil(V/64) * (H/16) * 1024. */
TENZO_HIP_API size_t tenzo_hip_i8_packed_bytes(int64_t V, int64_t H);
/* Row-major int8 [V][H] (H % 16 == 0) -> device LM-head layout. */
TENZO_HIP_API int tenzo_hip_i8_rows_repack(const int8_t* w, void* w_packed, int64_t V,
                                           int64_t H, void* stream);
/* compute_logits (TenzoEngine.cpp:1634-1720): final rms_norm_raw(x, norm_w),
 * int8 activation quantization (absmax/127), logits[v] =
 * float(sum x_i8 * W[v]) * (s_x * scales[v]). */
TENZO_HIP_API int tenzo_hip_lm_head_i8(const float* x, const float* norm_w, float eps,
                                       const void* w_packed, const float* scales,
                                       float* logits, int64_t V, int64_t H, void* stream);
/* The activation quantization of compute_logits (TenzoEngine.cpp:1666-1678)
 * for M rows of K values, after rms_norm_raw(x, norm_w, eps) when norm_w is
 * non-null or do_norm is set: codes[m][k] = clamp(round(x * 127/absmax),
 * -128, 127) (row stride K, K % 16 == 0), q[m] = {absmax/127, sum of codes}. */
TENZO_HIP_API int tenzo_hip_rmsnorm_quant127(const float* x, const float* norm_w, int do_norm,
                                             float eps, int64_t M, int64_t K, int8_t* codes,
                                             tenzo_hip_actq_t* q, void* stream);
/* The int8 GEMV of compute_logits (TenzoEngine.cpp:1689-1718) on codes from
 * tenzo_hip_rmsnorm_quant127: logits[v] = float(sum codes * W[v]) *
 * (q->inv_scale * scales[v]); when out_idx is non-null the same launch also
 * writes the greedy argmax (first maximum, TenzoEngine.cpp:1745-1755). */
TENZO_HIP_API int tenzo_hip_lm_head_i8_codes(const int8_t* codes, const tenzo_hip_actq_t* q,
                                             const void* w_packed, const float* scales,
                                             float* logits, int64_t V, int64_t H,
                                             int32_t* out_idx, void* stream);
/* Greedy branch of sample_top_k_top_p (TenzoEngine.cpp:1745-1755): index of
 * the first maximum, written to *out_idx (device int32). */
TENZO_HIP_API int tenzo_hip_argmax(const float* logits, int64_t V, int32_t* out_idx,
                                   void* stream);
/* The model loader's int8 LM-head quantization (load_model_from_files,
 * TenzoEngine.cpp:1925-1941) of V fp32 rows of H, as the reference is built
 * (-ffast-math): scales[v] = amax * (1/127) (amax floored at 1e-8), codes =
 * clamp(round(x * (127/amax)), -127, 127), row-major [V][H] int8. */
TENZO_HIP_API int tenzo_hip_quant_rows_i8(const float* E, int64_t V, int64_t H, int8_t* codes,
                                          float* scales, void* stream);
/* Sampling branch of sample_top_k_top_p (TenzoEngine.cpp:1757-1806),
 * temperature > 0, on logits that already carry the repetition penalty: top_k
 * clamped to [1, 64], softmax at the temperature over the top-k, top-p
 * cutoff, and the draw r in [0, 1] (the reference draws rand()/RAND_MAX; the
 * engine passes that same value). The token goes to *out_token (device
 * int32). Among logits equal to the k-th largest, the lowest indices are
 * kept. V <= 262144. */
TENZO_HIP_API int tenzo_hip_sample_top_k_top_p(const float* logits, int64_t V, int top_k,
                                               float top_p, float temperature, float r,
                                               int32_t* out_token, void* stream);
/* embedding_lookup, int8 branch (TenzoEngine.cpp:1294-1316), reading the
 * table in the LM-head device layout: x = float(E[token]) * scales[token].
 * token is read from device memory (token_dev). */
TENZO_HIP_API int tenzo_hip_embed_i8(const void* w_packed, const float* scales,
                                     const int32_t* token_dev, int64_t V, int64_t H, float* x,
                                     void* stream);

/* ---- host-pointer shims of the reference ROCm operator surface ----------
 * Synchronous, host memory in and out, return 1 on success and 0 on failure,
 * like ROCmRuntime::execute* (ROCmRuntime.h:20-37). Packed weights are cached
 * on the device keyed by the host pointer (the caller keeps them unchanged). */
TENZO_HIP_API int tenzo_hip_execute_bitlinear_tl1(const float* act, const uint8_t* w,
                                                  float* out, size_t M, size_t K, size_t N,
                                                  float scale);
TENZO_HIP_API int tenzo_hip_execute_rmsnorm(const float* in, const float* w, float* out,
                                            size_t dim, float eps);

/* HOST function: the byte offsets of the weights.bin tensors and the
 * projection scales that load_model_from_files (TenzoEngine.cpp:1943-1959)
 * reads from a model.mlir text: an index constant whose next non-blank line
 * is a memref.view of it, an f32 constant whose next non-blank line passes it
 * as the third operand of "tenzo.bitlinear_elut". Up to max_views / max_scales
 * values are written; *n_views / *n_scales receive the counts found. */
TENZO_HIP_API int tenzo_hip_parse_model_mlir(const char* text, uint64_t* views, int max_views,
                                             float* scales, int max_scales, int* n_views,
                                             int* n_scales);

/* ---- engine extensions (the engine itself is include/tenzo.h) ----------- */
struct tenzo_engine_opaque;
/* Prefills n prompt tokens (host array) at positions seq_len .. seq_len+n-1:
 * the KV cache, the hidden state and seq_len end as after n calls of
 * tenzo_prefill_token (TenzoEngine.cpp:1809-1819, C API :2187), which is how
 * the reference prefills a prompt (main_inference.cpp:470-472). Each layer
 * runs once per pass of up to 512 tokens: the TL1 projections as int8 MFMA
 * contractions (tenzo_hip_bitlinear_tl1_batch), then every token's attention
 * over its own prefix. exact != 0: the attention repeats a decode step's
 * chunking and arithmetic per token, so everything equals the per-token
 * kernels of the non-persistent modes bit for bit; exact == 0 (fast): one
 * streaming pass per token with an online softmax, equal up to fp32 rounding
 * of the softmax sums. */
TENZO_HIP_API int tenzo_hip_engine_prefill(struct tenzo_engine_opaque* e, const int32_t* tokens,
                                           int n, int exact);
/* Copies a prefilled KV cache into the engine and sets its sequence length;
 * pointers are device memory when is_device, else host. Layout by kv_mode:
 * int8_fused codes [L][Hkv][seq_len][128] int8 and fp16 scales [L][Hkv][seq_len];
 * tl1_fused / popcount_fused rows [L][Hkv][seq_len][32] bytes (the layouts of
 * tenzo_hip_attn_tern_decode) and fp32 scales [L][Hkv][seq_len]; paged_int8 the
 * int8_fused codes with fp32 scales, scattered into fresh blocks (the block
 * manager is reset first) and gathered back in block-table order. Mirrors
 * writing the public FusedKVCache state (TenzoEngine.h:60-115). */
TENZO_HIP_API int tenzo_hip_engine_set_kv(struct tenzo_engine_opaque* e, const void* kc,
                                          const void* vc, const void* ks, const void* vs,
                                          int seq_len, int is_device);
/* Reads back the cache (same layout, seq_len positions). */
TENZO_HIP_API int tenzo_hip_engine_get_kv(struct tenzo_engine_opaque* e, void* kc, void* vc,
                                          void* ks, void* vs, int seq_len);
/* Rewinds the sequence to seq_len <= the current length (positions past it
 * are overwritten by the next steps), e.g. to roll back rejected tokens or to
 * decode repeatedly at one position. No reference counterpart (the reference
 * only resets to 0, TenzoEngine.cpp:1249-1255). */
TENZO_HIP_API int tenzo_hip_engine_set_seq_len(struct tenzo_engine_opaque* e, int seq_len);
/* paged_int8 engines: copies up to cap entries of the sequence's block table
 * (PagedKVCache::block_table, TenzoEngine.h:160) and returns its length. */
TENZO_HIP_API int tenzo_hip_engine_block_table(struct tenzo_engine_opaque* e, int32_t* out,
                                               int cap);
/* RoPE theta (the reference hard-codes 10000; BitNet-2B uses 500000). */
TENZO_HIP_API int tenzo_hip_engine_set_rope_theta(struct tenzo_engine_opaque* e, float theta);
/* Copies the last step's logits (vocab fp32) to host memory. */
TENZO_HIP_API int tenzo_hip_engine_get_logits(struct tenzo_engine_opaque* e, float* logits);
/* Copies an engine buffer to host memory, by name: "x" (hidden state),
 * "qkv" (pre-RoPE q | k | v), "attn_out", "h1", "gate_up" (gate | up),
 * "logits" - the last layer's values of the last step. n is the capacity of
 * out in floats. */
TENZO_HIP_API int tenzo_hip_engine_get_buffer(struct tenzo_engine_opaque* e, const char* name,
                                              float* out, int64_t n);
/* Per-layer state of the last step when it ran the persistent kernel (mode 2),
 * for layer-by-layer checks against a CPU restatement of forward_layer_raw
 * (TenzoEngine.cpp:1522-1632); no reference counterpart. which: 0 the layer's
 * input x, 1 h1 = x + out projection, 2 the attention output (fp32, H / qd
 * floats); the int32 TL1 sums sum_k (w_k + 1) a_k (the activation codes' sum
 * is not yet subtracted) of 3 q|k|v, 4 the out projection, 5 gate|up, 6 down.
 * n is the capacity of out in 4-byte words. */
TENZO_HIP_API int tenzo_hip_engine_get_layer_state(struct tenzo_engine_opaque* e, int layer,
                                                   int which, void* out, int64_t n);
/* How a decode step is executed (no reference counterpart; the results are
 * the same up to fp32 reduction order in attention):
 *   2 (default) one persistent kernel per token (one workgroup per CU, all
 *     resident: an ordinary launch, and a cooperative one after a step has
 *     timed out), stages separated by in-kernel barriers (needs cooperative
 *     launch support, an int8 LM head, MLP weights in every layer, hidden and
 *     ffn multiples of 64 and <= 8192; otherwise mode 1 runs). Every in-kernel
 *     wait is bounded (TENZO_HIP_SPIN_LIMIT polls, read when the engine is
 *     made; default 262144): a wait that gives up fails the call, and the
 *     engine state is then invalid;
 *   1 one kernel per stage, replayed from a captured HIP graph;
 *   0 one kernel per stage, launched eagerly. */
TENZO_HIP_API int tenzo_hip_engine_set_mode(struct tenzo_engine_opaque* e, int mode);
/* The mode the next step will use (after the fallback above). */
TENZO_HIP_API int tenzo_hip_engine_get_mode(struct tenzo_engine_opaque* e);
/* Greedy decode of n tokens with the tokens chained on the device (no host
 * round trip per token; no reference counterpart - the reference's decode
 * loop calls tenzo_generate_step per token): step i consumes token (i = 0)
 * or step i-1's greedy token, at position seq_len + i. out (host, n ints)
 * receives the n greedy tokens; *ms (optional) the HIP-event time of the n
 * steps on the engine stream. Repetition penalty and sampling are not
 * applied. */
TENZO_HIP_API int tenzo_hip_engine_decode(struct tenzo_engine_opaque* e, int token, int n,
                                          int32_t* out, float* ms);
/* Step trace of the persistent kernel (mode 2; no reference counterpart):
 * while on, each step records for every stage s (5 per layer, then the LM
 * head) and workgroup w the wall-clock ticks (100 MHz) at which w reached
 * and left the barrier after s: out[(s * nwg + w) * 2 + {0, 1}].
 * get_trace returns the word count (out may be null to query it) or -1. */
TENZO_HIP_API int tenzo_hip_engine_trace(struct tenzo_engine_opaque* e, int on);
TENZO_HIP_API int64_t tenzo_hip_engine_get_trace(struct tenzo_engine_opaque* e, uint64_t* out,
                                                 int64_t n);
/* use_graph(1) = set_mode(1), use_graph(0) = set_mode(0). */
TENZO_HIP_API int tenzo_hip_engine_use_graph(struct tenzo_engine_opaque* e, int on);
/* The engine's HIP stream (hipStream_t as void*). */
TENZO_HIP_API void* tenzo_hip_engine_stream(struct tenzo_engine_opaque* e);

#ifdef __cplusplus
}
#endif
#endif /* TENZO_HIP_H */

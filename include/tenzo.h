/*
 * tenzo.h - engine C API served by libtenzo_hip.so on an MI355X.
 *
 * Same symbols, struct layouts and status codes as the reference's public
 * header (include/tenzo.h:39-193 in the reference checkout, implemented at
 * src/runtime/TenzoEngine.cpp:2086-2204), so its callers
 * (src/main_inference.cpp, examples/basic_inference.cpp) link against this
 * library unchanged. Differences, by design:
 *   - the decode step runs on the GPU whatever `device` says (this library
 *     has no CPU path); `kv_mode` is "int8_fused" (or NULL), "tl1_fused",
 *     "popcount_fused" or "paged_int8" (the reference's fp32 fallback for
 *     other strings is not provided: create returns NULL); every mode runs
 *     in the persistent decode kernel (paged_int8 up to the context its
 *     in-kernel softmax wait supports, the stage kernels beyond), and the
 *     modes other than int8_fused fill the cache token by token in
 *     tenzo_hip_engine_prefill;
 *   - weights are copied to device memory when they are set, so the caller may
 *     free its copies afterwards (the reference keeps non-owning pointers to
 *     layer weights and the final norm); the pointers may be host or device
 *     memory;
 *   - a null engine/weights pointer, a missing q/k/v/out matrix, a token
 *     outside [0, vocab), a step on a full KV cache or a step before the
 *     weights are set return an error (-1 from generate_step) instead of
 *     the reference's undefined behaviour;
 *   - tenzo_create_engine returns NULL when no GPU is usable or the config is
 *     unsupported (the reference never returns NULL);
 *   - sampling with temperature > 0 runs on the device with the reference's
 *     algorithm and draw (rand()/RAND_MAX from the process's libc); among
 *     logits equal to the k-th largest the lowest indices are kept, where the
 *     reference's heap keeps an insertion-order-dependent subset;
 *   - tenzo_load_model takes the projection shapes from the config (the
 *     reference hard-codes BitNet-2B's 2560/640 there) and returns
 *     TENZO_ERROR_MODEL_PARSE when weights.bin is smaller than the fp32
 *     embedding table (the reference reads past the end); otherwise it
 *     follows the reference's offsets, scales and fallbacks.
 */
#ifndef TENZO_H
#define TENZO_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) && __GNUC__ >= 4
#define TENZO_API __attribute__((visibility("default")))
#else
#define TENZO_API
#endif

#define TENZO_VERSION_MAJOR 1
#define TENZO_VERSION_MINOR 0
#define TENZO_VERSION_PATCH 0
#define TENZO_VERSION_STRING "1.0.0-mi355x"

typedef struct tenzo_engine_opaque* tenzo_engine_t;

typedef enum {
    TENZO_SUCCESS = 0,
    TENZO_ERROR_INVALID_ARGUMENT = -1,
    TENZO_ERROR_OUT_OF_MEMORY = -2,
    TENZO_ERROR_IO = -3,
    TENZO_ERROR_MODEL_PARSE = -4,
    TENZO_ERROR_UNSUPPORTED = -5
} tenzo_status_t;

typedef struct {
    int hidden_size;     /* 2560 for BitNet-b1.58-2B */
    int num_q_heads;     /* 20 */
    int num_kv_heads;    /* 5 */
    int head_dim;        /* 128 (the only supported value) */
    int num_layers;      /* 30 */
    int ffn_dim;         /* 6912 */
    int vocab_size;      /* 128256 */
    int max_seq_len;     /* 8192 */
    const char* kv_mode; /* "int8_fused", "tl1_fused", "popcount_fused", "paged_int8" */
    const char* device;  /* ignored: always the GPU */
} tenzo_config_t;

typedef struct {
    float temperature;        /* <= 0: greedy argmax */
    float top_p;
    int top_k;
    float repetition_penalty; /* applied on the device before the argmax */
} tenzo_sampling_params_t;

/* TL1-packed ternary weights [N/64][K/2][32] with per-tensor fp32 scales and
 * fp32 RMSNorm weights (reference include/tenzo.h:75-87). */
typedef struct {
    const int8_t* q_w;    float q_scale;
    const int8_t* k_w;    float k_scale;
    const int8_t* v_w;    float v_scale;
    const int8_t* out_w;  float out_scale;
    const int8_t* gate_w; float gate_scale;
    const int8_t* up_w;   float up_scale;
    const int8_t* down_w; float down_scale;
    const float* in_norm;
    const float* attn_sub_norm;
    const float* post_norm;
    const float* ffn_sub_norm;
} tenzo_layer_weights_t;

TENZO_API const char* tenzo_get_version(void);
TENZO_API tenzo_config_t tenzo_default_config(void);
TENZO_API tenzo_sampling_params_t tenzo_default_sampling_params(void);
TENZO_API tenzo_engine_t tenzo_create_engine(const tenzo_config_t* config);
TENZO_API void tenzo_destroy_engine(tenzo_engine_t engine);
TENZO_API void tenzo_reset(tenzo_engine_t engine);
TENZO_API int tenzo_get_seq_len(tenzo_engine_t engine);
TENZO_API tenzo_status_t tenzo_set_layer_weights(tenzo_engine_t engine, int layer_idx,
                                                 const tenzo_layer_weights_t* weights);
TENZO_API tenzo_status_t tenzo_set_final_norm(tenzo_engine_t engine, const float* norm_w);
TENZO_API tenzo_status_t tenzo_set_lm_head_f32(tenzo_engine_t engine, const float* embed_w,
                                               int vocab_size, int hidden_size);
TENZO_API tenzo_status_t tenzo_set_lm_head_i8(tenzo_engine_t engine, const int8_t* embed_w,
                                              const float* embed_scales, int vocab_size,
                                              int hidden_size);
TENZO_API tenzo_status_t tenzo_load_model(tenzo_engine_t engine, const char* weights_path,
                                          const char* mlir_path);
TENZO_API tenzo_status_t tenzo_prefill_token(tenzo_engine_t engine, int token_id);
TENZO_API int tenzo_generate_step(tenzo_engine_t engine, int cur_token,
                                  const tenzo_sampling_params_t* params,
                                  const int* past_tokens, int past_tokens_len);

#ifdef __cplusplus
}
#endif
#endif /* TENZO_H */

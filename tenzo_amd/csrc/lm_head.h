// Internal interface of the LM-head, argmax and embedding kernels (used by the
// C ABI and the engine).
#pragma once

#include "common.h"

namespace tz {

// Greedy-argmax workspace: one (value, index) pair per producing block, a
// completion counter that must start at zero (the kernels leave it at zero),
// and the result.
struct ArgmaxWs {
    float2* part = nullptr;    // [max blocks]
    uint32_t* counter = nullptr;
    int32_t* out_idx = nullptr;
};

// Bytes of the workspace for V logits (partials + counter), 256-aligned.
size_t argmax_ws_bytes(int64_t V);
// Carves an ArgmaxWs out of `base` (argmax_ws_bytes(V) bytes); out_idx is
// supplied by the caller.
ArgmaxWs argmax_ws_at(void* base, int64_t V, int32_t* out_idx);

int launch_i8_repack(const int8_t* w, void* w_packed, int64_t V, int64_t H, hipStream_t st);
// logits[v] = float(sum codes * W[v]) * (aq->inv_scale * scales[v]); when
// am.out_idx is set, also the index of the first maximum.
int launch_lm_head_i8(const int8_t* codes, const tenzo_hip_actq_t* aq, const void* w_packed,
                      const float* scales, float* logits, int64_t V, int64_t H,
                      const ArgmaxWs& am, hipStream_t st);
// fp32 LM head (set_lm_head_f32): logits[v] = sum xn * E[v] over a row-major
// [V][H] fp32 table.
int launch_lm_head_f32(const float* xn, const float* E, float* logits, int64_t V, int64_t H,
                       hipStream_t st);
int launch_argmax(const float* logits, int64_t V, const ArgmaxWs& am, hipStream_t st);
// x = float(E[token]) * scales[token] from the packed int8 table; tokens
// outside [0, V) give x = 0. n tokens (token_dev[0..n)) fill n rows of x.
int launch_embed_i8(const void* w_packed, const float* scales, const int32_t* token_dev,
                    int64_t V, int64_t H, float* x, hipStream_t st, int n = 1);
// x = E[token] from a row-major fp32 table.
int launch_embed_f32(const float* E, const int32_t* token_dev, int64_t V, int64_t H, float* x,
                     hipStream_t st, int n = 1);
// Repetition penalty of sample_top_k_top_p (TenzoEngine.cpp:1735-1743), in
// place and in the order given (a token listed twice is penalised twice).
// The model loader's LM-head quantization of V fp32 rows of H (TenzoEngine.cpp:1925-1941).
int launch_quant_rows_i8(const float* E, int64_t V, int64_t H, int8_t* codes, float* scales,
                         hipStream_t st);
// sample_top_k_top_p (TenzoEngine.cpp:1722-1807) for temperature > 0 with the
// draw r: the token goes to *out_token (device). ws: sample_ws_bytes(V).
constexpr int kSampleSlice = 2048;  // logits per first-stage workgroup
constexpr int kSampleK = 64;        // the reference clamps top_k to [1, 64]
size_t sample_ws_bytes(int64_t V);
int launch_sample(const float* logits, int64_t V, int top_k, float top_p, float temperature,
                  float r, void* ws, int32_t* out_token, hipStream_t st);
int launch_rep_penalty(float* logits, int64_t V, const int32_t* tokens, int n, float penalty,
                       hipStream_t st);

}  // namespace tz

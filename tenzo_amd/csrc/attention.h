// Internal interface of the attention kernels (used by the C ABI and the engine).
#pragma once

#include "common.h"

namespace tz {

constexpr int kMaxChunk = 256;   // tokens per workgroup, upper bound
constexpr int kPartStride = 130; // m, l, o[128] per (query head, chunk)

struct AttnLaunch {
    const float* q = nullptr;
    const float* k_new = nullptr;
    const float* v_new = nullptr;
    int8_t* kc = nullptr;
    int8_t* vc = nullptr;
    uint16_t* ks = nullptr;
    uint16_t* vs = nullptr;
    const float* rope = nullptr;
    const int* pos_dev = nullptr;  // device position (graph replays); else pos
    int pos = 0;
    int rope_indexed = 0;          // rope points at a [max_seq][128] table
    int B = 1, Hq = 0, Hkv = 0, max_seq = 0;
    int T = 64;                    // tokens per chunk (multiple of 32, <= kMaxChunk)
    int max_chunks = 1;            // grid size along the context
    float* out = nullptr;
    float* part = nullptr;         // partials; library scratch when null
    float* q_rot = nullptr;
    float* k_rot = nullptr;
};

int attn_pick_chunk(int seq_len, int Hkv, int B);
int launch_attn(const AttnLaunch& L, hipStream_t st);

}  // namespace tz

// Internal interface of the persistent decode-step kernel (used by the engine).
#pragma once

#include "common.h"

namespace tz {

// Per-layer device pointers and scales (an array of these lives in HBM).
// Slot s of mat/norm belongs to the stage that reads it: 0 Q|K|V (in_norm),
// 1 O (attn_sub_norm), 2 gate|up (post_norm), 3 down (ffn_sub_norm).
struct DsLayer {
    const uint4* mat[4];   // TL1 GEMV layout; Q|K|V and gate|up row-concatenated
    const float* norm[4];  // null = no weight
    float sc[7];           // q, k, v, o, gate, up, down
};

struct DsParams {
    const DsLayer* layers;
    const float* final_norm;
    const uint4* head;          // packed int8 LM head (lm_head.hip layout)
    const float* head_scales;
    const float* rope;          // [max_seq][128] cos | sin
    int8_t* kc;                 // [L][Hkv][max_seq][128] (paged: the code pools)
    int8_t* vc;
    uint16_t* ks;               // [L][Hkv][max_seq] fp16 (unused when paged)
    uint16_t* vs;
    // paged_int8 (block_table non-null): pools of 16-token blocks, codes
    // kc/vc [blocks][L][Hkv][16][128] and fp32 scales pks/pvs [blocks][L][Hkv][16];
    // block_table[t / 16] is the pool block of token t
    const int32_t* block_table;
    float* pks;                 // fp32 scales: paged pools, or [L][Hkv][max_seq] (ternary)
    float* pvs;
    int kv_mode;                // 0 int8_fused, 1 tl1_fused, 2 popcount_fused, 3 paged_int8
                                // (ternary: kc / vc hold 32-byte rows [L][Hkv][max_seq][32])
    // host-visible vectors of the last layer (x: the final hidden state)
    float* x;                   // [H] hidden state
    float* qkv;                 // [qd + 2 kvd]
    float* attn;                // [qd]
    float* h1;                  // [H]
    float* gu;                  // [2F]
    float* logits;              // [V]
    // per-layer copies the kernel reads back (each written once per launch)
    float* xs;                  // [L][H]  input of layer l
    float* h1s;                 // [L][H]  x + o of layer l
    float* attns;               // [L][qd] attention output of layer l
    float* part;                // [Hkv][C][G][kDsPartStride] attention partials
    float2* am_part;            // [nwg] argmax partials
    unsigned* sync;             // ds_sync_words() words, zero before each launch
    // grid-barrier counters (kDsCounters words 256 bytes apart) and the error
    // word after them, in uncached memory (polled with scalar loads): the
    // counters carry on from launch to launch, bar_base generations of them
    // having been completed by earlier launches (kDsBarWords words, zeroed by
    // the host before the first launch and after a launch that aborted)
    unsigned* bar;
    unsigned bar_base;
    int* acc;                   // ds_acc_words() int32 GEMV accumulators, zero before
                                // each launch: per layer q|k|v, o, gate|up, down
    int32_t* io;                // [0] token in, [2] greedy token out (also copied to [0]),
                                // [3] set to 1 when a wait timed out (cleared by the host)
    int32_t* out_tokens;        // optional: the greedy token is also stored at [step]
    int step;
    int H, F, Hq, Hkv, L, V, max_seq;
    int pos, C, T;              // this step's position and attention chunking
    int nwg;
    int split[4];               // K slices per row block of the QKV, O, GU, DOWN GEMVs
    int split_chunks[4];        // 64-column chunks per K slice: ceil(K / 64 / split)
    unsigned split_mul[4];      // ds_div_mul(split[i])
    unsigned c_mul;             // ds_div_mul(C)
    int with_head;              // 0: stop after the layers (prefill)
    unsigned spin_limit;        // polls before a wait gives up (kDsSpinLimit)
    float eps;
    // optional step trace: for stage s and workgroup w, [(s * nwg + w) * 2]
    // = wall clock (100 MHz) when w arrives at the barrier after stage s,
    // [.. + 1] = when it leaves it
    uint64_t* trace;
};

constexpr int kDsThreads = 512;
constexpr int kDsMaxChunk = 256;            // context tokens per attention task, at most
constexpr unsigned kDsSpinLimit = 1u << 18;  // ~0.3 s of polling; a barrier waits < 0.1 ms
constexpr int kDsPartStride = 132;  // floats per attention partial record (16-byte aligned)
constexpr int kDsCounters = 16;
constexpr int kDsBarWords = (kDsCounters + 1) * 64;  // counters, then the error word
constexpr int kDsMaxLayers = 64;    // the layer table is staged in LDS
constexpr int kDsMaxBlocks = 1024;  // paged: the block table is staged in LDS (16384 tokens)

// uint32 words of the sync region for L layers and Hkv kv heads (a multiple of
// 64, so the accumulators can follow it in one allocation).
size_t ds_sync_words(int L, int Hkv);
// int32 words of the accumulator region.
size_t ds_acc_words(int L, int H, int F, int Hq, int Hkv);
// floats of the per-layer vector region (xs, h1s, attns).
size_t ds_vec_floats(int L, int H, int Hq);
// K slices per row block for each GEMV stage (fills p.split, p.split_chunks
// and p.split_mul from the shapes and p.nwg; p.c_mul from p.C).
void ds_plan_splits(DsParams& p);
// Multiplier for t / d (1 <= d < 2^15, 0 <= t < 2^16) as
// umulhi(2 t, ceil(2^31 / d)): the product exceeds t / d by less than
// t / 2^31 < 2^-15, too little to reach the next integer.
inline unsigned ds_div_mul(int d) { return (unsigned)((0x80000000ull + (unsigned)d - 1) / (unsigned)d); }
// Workgroup count the kernel runs with on the current device (a multiple of
// kDsCounters, all co-resident), or 0 when cooperative launch is unavailable.
int ds_grid_size();
// Chunks per kv head the attention stage aims for (one task per workgroup).
int ds_chunk_budget(int nwg, int Hkv);
// Attention chunking (C chunks of T tokens per kv head) for context ctx.
void ds_chunking(int ctx, int Hkv, int nwg, int* C, int* T);
// Longest context the kernel's attention merge supports for G query heads per
// kv head (its chunk statistics live in LDS).
int ds_max_context(int G);
// Grid barriers per launch of L layers (bar_base advances by this much).
inline unsigned ds_barriers(int L) { return 5u * (unsigned)L; }
// Returned by launch_decode_step when a cooperative launch was asked for and
// the runtime refused it (nothing was launched).
constexpr int kDsCoopRefused = 1000;
// Launches one decode step: an ordinary launch, or with coop a cooperative
// one (kDsCoopRefused when the runtime refuses it). The sync region must be
// zero. A launch whose io[3] is already set returns at once (a chained decode
// stops at the first step that aborted).
int launch_decode_step(const DsParams& p, int G, bool coop, hipStream_t st);

}  // namespace tz

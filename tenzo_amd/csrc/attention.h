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

// Merge of the chunk partials [B][Hq][max_chunks][130] of a decode step at
// position pos (pos_dev when non-null) with chunks of T tokens into out.
int launch_attn_combine(const float* part, float* out, int B, int Hq, int Hkv, int T,
                        int max_chunks, const int* pos_dev, int pos, hipStream_t st);

// Decode attention over a ternary KV cache (attention_tern.hip): mode 1
// tl1_fused, 2 popcount_fused; rows of 32 bytes per (kv head, token) in kb / vb
// ([B][Hkv][max_seq][32]) and fp32 scales ks / vs ([B][Hkv][max_seq]).
struct AttnTernLaunch {
    int mode = 0;
    const float* q = nullptr;
    const float* k_new = nullptr;
    const float* v_new = nullptr;
    uint8_t* kb = nullptr;
    uint8_t* vb = nullptr;
    float* ks = nullptr;
    float* vs = nullptr;
    const float* rope = nullptr;
    const int* pos_dev = nullptr;
    int pos = 0;
    int rope_indexed = 0;
    int B = 1, Hq = 0, Hkv = 0, max_seq = 0;
    int T = 64;
    int max_chunks = 1;
    float* out = nullptr;
    float* part = nullptr;
    float* q_rot = nullptr;
    float* k_rot = nullptr;
};
int launch_attn_tern(const AttnTernLaunch& L, hipStream_t st);

// paged_int8 decode attention (attention_paged.hip) over one layer of block
// pools pk / pv [blocks][n_layers][Hkv][16][128] int8 with fp32 scales pks / pvs
// [blocks][n_layers][Hkv][16]; block_table[t / 16] is the physical block of
// token t (the block of pos included). ws: paged_ws_bytes bytes, or null for
// the library scratch. Batch 1.
struct AttnPagedLaunch {
    const float* q = nullptr;
    const float* k_new = nullptr;
    const float* v_new = nullptr;
    int8_t* pk = nullptr;
    int8_t* pv = nullptr;
    float* pks = nullptr;
    float* pvs = nullptr;
    const int32_t* block_table = nullptr;
    const float* rope = nullptr;
    const int* pos_dev = nullptr;
    int pos = 0;
    int rope_indexed = 0;
    int n_layers = 1, layer = 0, Hq = 0, Hkv = 0;
    int T = 64;
    int max_chunks = 1;
    float* ws = nullptr;
    float* out = nullptr;
};
size_t paged_ws_bytes(int Hq, int max_chunks, int T);
int launch_attn_paged(const AttnPagedLaunch& L, hipStream_t st);

// Attention for n prompt tokens at positions pos0 .. pos0+n-1 over one INT8
// cache: the k/v rows of all n tokens are RoPE'd, quantized and appended
// first (as n decode steps would), then query i attends to positions
// 0 .. pos0+i. exact: with the chunking and arithmetic of a decode step at
// that position (chunk by chunk, then the decode merge), so every output
// equals the one n sequential decode steps produce bit for bit; otherwise a
// streaming pass per query (one wave, 64-token blocks, online softmax), equal
// to within fp32 rounding of the softmax sums and far faster. q / k_new /
// v_new are rows of row_stride elements (q at column 0, k and v where the
// pointers say); out rows are out_stride apart.
struct AttnPrefill {
    const float* q = nullptr;
    const float* k_new = nullptr;
    const float* v_new = nullptr;
    int64_t row_stride = 0;
    int8_t* kc = nullptr;
    int8_t* vc = nullptr;
    uint16_t* ks = nullptr;
    uint16_t* vs = nullptr;
    const float* rope = nullptr;  // [max_seq][128]
    int pos0 = 0, n = 0, Hq = 0, Hkv = 0, max_seq = 0;
    float* out = nullptr;
    int64_t out_stride = 0;
    int exact = 0;
};
int launch_attn_prefill(const AttnPrefill& P, hipStream_t st);

}  // namespace tz

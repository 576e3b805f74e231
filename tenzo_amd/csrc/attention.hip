// INT8 KV-cache decode attention on gfx950 (FusedKVCache::forward_attention_raw,
// reference src/runtime/TenzoEngine.cpp:447-919, int8_fused branches).
//
// One workgroup per (context chunk, kv head, sequence). It holds the G query
// heads that share the kv head (GQA), so each K/V byte is read from HBM once
// for all of them. Within a chunk: RoPE on q (and, for the chunk that holds
// the new token, on k), quantize-append of the new k/v, then
//   scores   s[g][t] = (q_g . k_t) * (s_k[t] / sqrt(128))
//   weights  p[g][t] = exp(s[g][t] - m_chunk[g]),  l[g] = sum_t p[g][t]
//   values   o[g][d] = sum_t p[g][t] * s_v[t] * v_t[d]
// and the chunk partials (m, l, o) are merged by a combine kernel
// (out = sum_c e^{m_c - M} o_c / sum_c e^{m_c - M} l_c).
//
// Scores and values run on fp16 MFMA over tiles of 16 tokens (score_tile,
// value_tile below): K and V codes are exact in fp16, the fp32 query rows and
// weights enter as fp16 hi + lo pairs. A wave takes tiles wave, wave + 4, ...;
// every wave load covers whole 128-byte cache rows.
#include <algorithm>
#include <mutex>

#include "attention.h"
#include "common.h"

namespace tz {

constexpr int kD = 128;
constexpr float kScaleFactor = 0.08838834764831845f;  // 1/sqrt(128)

// Tokens per chunk for a context of seq_len: ~512 workgroups over the chip,
// chunks of 64 .. kMaxChunk tokens (a 32-token chunk would leave two of the
// chunk kernel's four waves without a 16-token tile).
__host__ __device__ inline int pick_chunk(int seq_len, int Hkv, int B) {
    const int target = (512 + Hkv * B - 1) / (Hkv * B);
    int T = (seq_len + target - 1) / target;
    T = (T + 31) / 32 * 32;
    if (T < 64) T = 64;
    if (T > kMaxChunk) T = kMaxChunk;
    return T;
}

struct AttnArgs {
    const float* q;      // [B][Hq][128]
    const float* k_new;  // [B][Hkv][128]
    const float* v_new;
    int8_t* kc;          // [B][Hkv][max_seq][128] (batch stride given below)
    int8_t* vc;
    uint16_t* ks;        // [B][Hkv][max_seq]
    uint16_t* vs;
    const float* rope;   // cos[64] | sin[64], per position when rope_indexed
    const int* pos_dev;  // position read from device memory when non-null
    int pos;
    int rope_indexed;
    int Hq, Hkv, max_seq, T;
    int64_t cache_batch_stride;  // elements between sequences' caches
    int64_t q_stride;            // elements between the rows of q (per sequence / token)
    int64_t kv_stride;           // elements between the rows of k_new / v_new
    int64_t out_stride;          // elements between the rows of out
    // Prefill: row b of q / out is the query of position pos + b over one
    // cache whose k/v rows (through pos + b) are already appended; each query
    // takes the chunk size decode would pick at its position (attn_pick_chunk).
    int prefill;
    int pos_n;  // streaming prefill: number of query rows
    float* out;          // [B][Hq][128] (used when nchunks == 1)
    float* part;         // [B][Hq][max_chunks][130] partials
    int max_chunks;
    float* q_rot;        // optional
    float* k_rot;        // optional
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t att_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Scores on fp16 MFMA (v_mfma_f32_16x16x16_f16), shared by the decode chunk
// kernel and the prefill kernel so both give the same bits. A wave takes 16
// tokens at a time: lane l holds token n = l % 16 of the tile and its dims
// 32 q .. 32 q + 31 (q = l / 16, 32 bytes of the cache row), and the dims of
// MFMA step j are {32 q + 4 j + e} (q, e < 4). K codes are exact in fp16
// (u = k ^ 0x80 placed under the fp16 exponent of 1024, then 1152
// subtracted); the fp32 query rows are the A operand as two fp16 parts of
// q' = q 2^e (e per head, so that its largest |q'| is in [2^13, 2^14) and the
// parts stay normal numbers): hi = fp16(q'), lo = fp16(q' - hi), the hi step
// first, and the sums are scaled back by 2^-e (exact). Products are exact and
// summed in fp32; D row m = head m of the tile's column n, held by lanes
// 16 (m / 4) .. +15 as element m % 4.
typedef _Float16 h2a __attribute__((ext_vector_type(2)));
typedef _Float16 h4a __attribute__((ext_vector_type(4)));
typedef float f4a __attribute__((ext_vector_type(4)));

// The exponent that brings a magnitude up to [2^13, 2^14): x * 2^e then stays
// below fp16's largest finite value and its fp16 remainder x * 2^e - hi stays a
// normal number down to ~1.5e-5 of the magnitude (fp16 subnormals would lose it).
__device__ __forceinline__ int fp16_span_exp(float mx) {
    if (!(mx > 0.0f)) return 0;
    int E;
    (void)frexpf(mx, &E);  // mx = f 2^E, f in [0.5, 1)
    return min(14 - E, 100);
}

// the A operands of the G query heads for this lane (head l % 16, zero past G), each
// head scaled by a power of two (fp16_span_exp of its largest |q|); qin[e] = the inverse
// scale of D row 4 (l / 16) + e (the head of lane 4 (l / 16) + e)
template <int G>
__device__ __forceinline__ void q_operands(const float (&qs)[G][kD], h4a (&qh)[8], h4a (&ql)[8],
                                           float (&qin)[4]) {
    const int lane = threadIdx.x & 63, m = lane & 15, q = lane >> 4;
    const float* qrow = &qs[m < G ? m : 0][32 * q];
    float mx = 0.0f;  // (two passes over the LDS row keep 32 registers free)
#pragma unroll
    for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(qrow[i]));
    mx = m < G ? mx : 0.0f;
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const int sh = fp16_span_exp(mx);
    const float up = ldexpf(1.0f, sh), down = ldexpf(1.0f, -sh);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float xs = (m < G ? qrow[4 * j + e] : 0.0f) * up;  // (exact: a power of two)
            const _Float16 hi = (_Float16)xs;
            qh[j][e] = hi;
            ql[j][e] = (_Float16)(xs - (float)hi);
        }
#pragma unroll
    for (int e = 0; e < 4; ++e) qin[e] = __shfl(down, 4 * q + e, 64);
}

// e64 = 0x64006400 in a VGPR (a VGPR operand of v_perm_b32), made once by the caller
__device__ __forceinline__ h4a i8x4_h4(uint32_t w, uint32_t e64) {
    const uint32_t x = w ^ 0x80808080u;
    const h2a bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2a p0 = __builtin_bit_cast(h2a, __builtin_amdgcn_perm(e64, x, 0x07010500u)) + bias;
    const h2a p1 = __builtin_bit_cast(h2a, __builtin_amdgcn_perm(e64, x, 0x07030502u)) + bias;
    return h4a{p0.x, p0.y, p1.x, p1.y};
}

__device__ __forceinline__ f4a score_tile(const h4a (&qh)[8], const h4a (&ql)[8],
                                          const uint4 k0, const uint4 k1) {
    const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    uint32_t e64 = 0x64006400u;
    asm volatile("" : "+v"(e64));
    f4a d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const h4a b = i8x4_h4(kw[j], e64);
        d = __builtin_amdgcn_mfma_f32_16x16x16f16(qh[j], b, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x16f16(ql[j], b, d, 0, 0, 0);
    }
    return d;
}

// Values on fp16 MFMA for the same 16-token tiles: O[g][d] += sum_t W[g][t] V[t][d]
// with the tile's 16 tokens as the MFMA's k. Lane l = (n, q) = (l % 16, l / 16) holds
// tokens 4 q .. 4 q + 3 of the tile and dims 8 n .. 8 n + 7 of each (v[e]: 8 bytes of
// token 4 q + e), and MFMA dt (0..7) takes dim 8 n + dt as its column n, so a lane's
// 4 x 8 block, transposed in registers (byte permutes), gives its B operands: 4 tokens of
// one dim, exact in fp16. The A operand is W = p * s_v of head l % 16 at the lane's 4
// tokens, scaled by a power of two per wave and split into fp16 hi + lo parts (the hi
// MFMA first). acc[dt] row g = D[g][dim 8 n + dt], held by lanes 16 (g / 4) .. +15 as
// element g % 4.
__device__ __forceinline__ void value_tile(const h4a (&wh)[1], const h4a (&wl)[1],
                                           const uint2 (&v)[4], f4a (&acc)[8]) {
    uint32_t e64 = 0x64006400u;  // (a VGPR operand of v_perm_b32)
    asm volatile("" : "+v"(e64));
    const h2a bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {  // dims 4 hf .. 4 hf + 3 of the lane's 8
        uint32_t x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = (hf ? v[e].y : v[e].x) ^ 0x80808080u;
        // (token 0, token 1) and (token 2, token 3) interleaved: dims 0, 1 / dims 2, 3
        const uint32_t t01a = __builtin_amdgcn_perm(x[1], x[0], 0x05010400u);
        const uint32_t t01b = __builtin_amdgcn_perm(x[1], x[0], 0x07030602u);
        const uint32_t t23a = __builtin_amdgcn_perm(x[3], x[2], 0x05010400u);
        const uint32_t t23b = __builtin_amdgcn_perm(x[3], x[2], 0x07030602u);
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const uint32_t sel = (f & 1) ? 0x07030502u : 0x07010500u;
            const h2a p01 =
                __builtin_bit_cast(h2a, __builtin_amdgcn_perm(e64, f < 2 ? t01a : t01b, sel)) + bias;
            const h2a p23 =
                __builtin_bit_cast(h2a, __builtin_amdgcn_perm(e64, f < 2 ? t23a : t23b, sel)) + bias;
            const h4a b = {p01.x, p01.y, p23.x, p23.y};
            const int dt = 4 * hf + f;
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(wh[0], b, acc[dt], 0, 0, 0);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(wl[0], b, acc[dt], 0, 0, 0);
        }
    }
}

// the A operand of a value tile: W[g][t] = p[g][t] * s_v[t] of head g = l % 16 at tokens
// tile * 16 + 4 (l / 16) + e, zero past G or past the chunk, scaled by 2^wsh (a power of
// two that keeps the wave's largest s_v, and so every W of its tiles, within fp16's
// normal span)
template <int G>
__device__ __forceinline__ void w_operands(const float (&sc)[G][kMaxChunk], int tile, int nt,
                                           const float (&svf)[4], float wup, h4a (&wh)[1],
                                           h4a (&wl)[1]) {
    const int lane = threadIdx.x & 63, m = lane & 15, q = lane >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int tl = tile * 16 + 4 * q + e;
        const float w =
            (m < G && tl < nt) ? __fmul_rn(sc[m < G ? m : 0][tl], svf[e]) * wup : 0.0f;
        const _Float16 hi = (_Float16)w;
        wh[0][e] = hi;
        wl[0][e] = (_Float16)(w - (float)hi);
    }
}

// KV append quantization (:516-531 as built): s = amax*(1/127), code =
// clamp(round(x * (127/amax)), -128, 127). 64 lanes x 2 values.
__device__ __forceinline__ void quant_kv_pair(float x0, float x1, int8_t* codes_out,
                                              int lane, float* s_out) {
    float amax = fmaxf(fabsf(x0), fabsf(x1));
    amax = fmaxf(wave_max(amax), 1e-8f);
    const float inv = __fdiv_rn(127.0f, amax);
    float r0 = roundf(__fmul_rn(x0, inv));
    float r1 = roundf(__fmul_rn(x1, inv));
    r0 = fminf(fmaxf(r0, -128.0f), 127.0f);
    r1 = fminf(fmaxf(r1, -128.0f), 127.0f);
    codes_out[lane] = (int8_t)r0;
    codes_out[lane + 64] = (int8_t)r1;
    *s_out = __fmul_rn(amax, 1.0f / 127.0f);
}

// The decode chunk kernel (attn_prefill_exact_kernel repeats its arithmetic per
// row, so prefill and decode agree bit for bit). The loads are arranged for
// latency: each lane's K and V rows of the chunk (U = T / 32, so
// (U + 1) / 2 tiles of 16 tokens per wave; rows past the context read the
// chunk's last row and are not used) are issued right after the query loads,
// so they stream while q is rotated and the new token appended; the new
// token's row comes from LDS (its cache row is written by this workgroup in
// the same launch).
template <int G, int U>
__global__ void __launch_bounds__(256, 3) attn_int8_chunk_kernel(AttnArgs a) {  // (3 waves per SIMD)
    __shared__ float qs[G][kD];
    __shared__ float sc[G][kMaxChunk];
    __shared__ float ow[4][G][kD];
    __shared__ float mstat[G], lstat[G];
    __shared__ __align__(16) int8_t newk[kD];
    __shared__ __align__(16) int8_t newv[kD];
    __shared__ float news[2];
    __shared__ uint16_t news_h[2];

    const int c = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos) + (a.prefill ? b : 0);
    const int seq_len = pos + 1;
    const int T = a.prefill ? pick_chunk(seq_len, a.Hkv, 1) : a.T;
    const int t0 = c * T;
    if (t0 >= seq_len) return;  // chunks past the context (fixed-size grids)
    const int t1 = min(t0 + T, seq_len);
    const int nt = t1 - t0;
    const int nchunks = (seq_len + T - 1) / T;
    const float* rope = a.rope + (a.rope_indexed ? (int64_t)pos * kD : 0);
    const int64_t cache_head = (int64_t)b * a.cache_batch_stride + (int64_t)h * a.max_seq;
    const int8_t* kbase = a.kc + cache_head * kD;
    const int8_t* vbase = a.vc + cache_head * kD;
    const uint16_t* ksb = a.ks + cache_head;
    const uint16_t* vsb = a.vs + cache_head;

    // ---- the queries' loads first (RoPE and the append wait for them alone), then this
    // lane's K (and V) rows ----
    constexpr int kQI = (G * 64 + 255) / 256;  // RoPE pairs per thread
    float qx0[kQI], qx1[kQI], qcs[kQI], qsn[kQI];
#pragma unroll
    for (int r = 0; r < kQI; ++r) {
        const int i = min(tid + 256 * r, G * 64 - 1);
        const int g = i >> 6, j = i & 63;
        const float* qv = a.q + (int64_t)b * a.q_stride + (int64_t)(h * G + g) * kD;
        qx0[r] = qv[j];
        qx1[r] = qv[j + 64];
        qcs[r] = rope[j];
        qsn[r] = rope[64 + j];
    }
    // the new token's k (wave 0) or v (wave 1) row and its rotation, loaded by every wave
    // (no branch: waves 2 and 3 load k again and do not use it)
    const float* nsrc = (wave == 1 ? a.v_new : a.k_new) + (int64_t)b * a.kv_stride + (int64_t)h * kD;
    const float nx0 = nsrc[lane], nx1 = nsrc[lane + 64];
    const float ncs = rope[lane], nsn = rope[64 + lane];
    asm volatile("" ::: "memory");  // (keeps the K / V loads behind those loads)
    // K and V in the tiles' mappings (tile wave + 4 i of 16 tokens): K lane token l % 16,
    // dims 32 (l / 16) ..; V lane tokens 4 (l / 16) .. +3, dims 8 (l % 16) .. +7
    constexpr int NTW = (U + 1) / 2;  // 16-token tiles per wave
    const int kn = lane & 15, kq = lane >> 4;
    // (buffer loads from the chunk's first row: 32-bit offsets, no per-lane 64-bit address)
    const __amdgpu_buffer_rsrc_t rk = att_rsrc(kbase + (int64_t)t0 * kD, (uint32_t)nt * kD);
    const __amdgpu_buffer_rsrc_t rv = att_rsrc(vbase + (int64_t)t0 * kD, (uint32_t)nt * kD);
    const __amdgpu_buffer_rsrc_t rks = att_rsrc(ksb + t0, (uint32_t)nt * 2);
    const __amdgpu_buffer_rsrc_t rvs = att_rsrc(vsb + t0, (uint32_t)nt * 2);
    uint4 kr[NTW][2];
    uint16_t ksr[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i) {
        const uint32_t tl = (uint32_t)min((wave + 4 * i) * 16 + kn, nt - 1);
        const uint32_t off = tl * kD + 32 * kq;
        kr[i][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
        kr[i][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, off + 16, 0, 0));
        ksr[i] = __builtin_amdgcn_raw_buffer_load_b16(rks, tl * 2, 0, 0);
    }
    uint2 vm[NTW][4];
    uint16_t vms[NTW][4];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t tl = (uint32_t)min((wave + 4 * i) * 16 + 4 * kq + e, nt - 1);
            vm[i][e] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, tl * kD + 8 * kn, 0, 0));
            vms[i][e] = __builtin_amdgcn_raw_buffer_load_b16(rvs, tl * 2, 0, 0);
        }

    // ---- RoPE on the G query heads (:460-481) ----
#pragma unroll
    for (int r = 0; r < kQI; ++r) {
        const int i = tid + 256 * r;
        if (i < G * 64) {
            const int g = i >> 6, j = i & 63;
            const int qh = h * G + g;
            const float r0 = __builtin_fmaf(qx0[r], qcs[r], -__fmul_rn(qx1[r], qsn[r]));
            const float r1 = __builtin_fmaf(qx0[r], qsn[r], __fmul_rn(qx1[r], qcs[r]));
            qs[g][j] = r0;
            qs[g][j + 64] = r1;
            if (a.q_rot && c == 0) {
                float* qr = a.q_rot + ((int64_t)b * a.Hq + qh) * kD;
                qr[j] = r0;
                qr[j + 64] = r1;
            }
        }
    }
    // ---- new token: RoPE on k, quantize-append k and v (:482-533) ----
    const bool has_new = !a.prefill && pos >= t0 && pos < t1;
    if (has_new && wave < 2) {
        float x0 = nx0, x1 = nx1;
        if (wave == 0) {
            const float cs = ncs, sn = nsn;
            const float r0 = __builtin_fmaf(x0, cs, -__fmul_rn(x1, sn));
            const float r1 = __builtin_fmaf(x0, sn, __fmul_rn(x1, cs));
            x0 = r0;
            x1 = r1;
            if (a.k_rot) {
                float* kr2 = a.k_rot + ((int64_t)b * a.Hkv + h) * kD;
                kr2[lane] = r0;
                kr2[lane + 64] = r1;
            }
        }
        float s;
        quant_kv_pair(x0, x1, wave == 0 ? newk : newv, lane, &s);
        const uint16_t sh = float_to_half_bits(s);
        int8_t* dst = (wave == 0 ? a.kc : a.vc) + (cache_head + pos) * kD;
        dst[lane] = (wave == 0 ? newk : newv)[lane];
        dst[lane + 64] = (wave == 0 ? newk : newv)[lane + 64];
        if (lane == 0) {
            (wave == 0 ? a.ks : a.vs)[cache_head + pos] = sh;
            news[wave] = half_bits_to_float(sh);
            news_h[wave] = sh;
        }
    }
    // (LDS only: the new row's cache copy is not read back in this launch)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (has_new) {  // (workgroup-uniform) the new row replaces the stale one read for token pos
        const int pl = pos - t0;  // (= nt - 1: the rows past the chunk read it too)
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            if (min((wave + 4 * i) * 16 + kn, nt - 1) == pl) {
                kr[i][0] = *reinterpret_cast<const uint4*>(newk + 32 * kq);
                kr[i][1] = *reinterpret_cast<const uint4*>(newk + 32 * kq + 16);
                ksr[i] = news_h[0];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (min((wave + 4 * i) * 16 + 4 * kq + e, nt - 1) == pl) {
                    vm[i][e] = *reinterpret_cast<const uint2*>(newv + 8 * kn);
                    vms[i][e] = news_h[1];
                }
        }
    }

    // ---- scores (:678-694) on MFMA ----
    {
        h4a qh[8], ql[8];
        float qin[4];
        q_operands<G>(qs, qh, ql, qin);
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int tile = wave + 4 * i;
            if (tile * 16 >= nt) break;  // (wave-uniform)
            const int tl = tile * 16 + kn;
            const f4a d = score_tile(qh, ql, kr[i][0], kr[i][1]);
            if (tl < nt) {
                const float f = __fmul_rn(half_bits_to_float(ksr[i]), kScaleFactor);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int g = 4 * kq + e;
                    if (g < G) sc[g][tl] = __fmul_rn(d[e] * qin[e], f);
                }
            }
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- chunk softmax statistics (:824-830) ----
    for (int g = wave; g < G; g += 4) {
        float m = -1e30f;
        for (int i = lane; i < nt; i += 64) m = fmaxf(m, sc[g][i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < nt; i += 64) {
            const float e = expf(sc[g][i] - m);
            sc[g][i] = e;
            l += e;
        }
        l = wave_sum_tree(l);
        if (lane == 0) {
            mstat[g] = m;
            lstat[g] = l;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- weighted values (:842-851) ----
    {  // on MFMA, tile by tile (value_tile)
        // the wave's largest V scale over its tiles' tokens sets its power-of-two scale
        float vmax = 0.0f;
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            if ((wave + 4 * i) * 16 >= nt) break;  // (wave-uniform)
#pragma unroll
            for (int e = 0; e < 4; ++e) vmax = fmaxf(vmax, half_bits_to_float(vms[i][e]));
        }
        const int wsh = fp16_span_exp(wave_max(vmax));
        const float wup = ldexpf(1.0f, wsh), wdown = ldexpf(1.0f, -wsh);
        f4a acc8[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc8[dt] = f4a{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int tile = wave + 4 * i;
            if (tile * 16 >= nt) break;  // (wave-uniform)
            float svf[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) svf[e] = half_bits_to_float(vms[i][e]);
            h4a wh[1], wl[1];
            w_operands<G>(sc, tile, nt, svf, wup, wh, wl);
            value_tile(wh, wl, vm[i], acc8);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int g = 4 * kq + e;
            if (g < G) {
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) ow[wave][g][8 * kn + dt] = acc8[dt][e] * wdown;
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < G * kD; i += 256) {
        const int g = i >> 7, d = i & 127;
        const float o = (ow[0][g][d] + ow[1][g][d]) + (ow[2][g][d] + ow[3][g][d]);
        const int qh = h * G + g;
        if (nchunks == 1) {
            a.out[(int64_t)b * a.out_stride + (int64_t)qh * kD + d] = __fdiv_rn(o, lstat[g]);
        } else {
            float* pp = a.part + (((int64_t)b * a.Hq + qh) * a.max_chunks + c) * kPartStride;
            pp[2 + d] = o;
            if (d == 0) {
                pp[0] = mstat[g];
                pp[1] = lstat[g];
            }
        }
    }
}

// Merge of the chunk partials; one 128-thread block per (query head, sequence):
//   M = max_c m_c,  L = sum_c e^{m_c - M} l_c,  o = sum_c e^{m_c - M} o_c,
// summed in chunk order with one fma per term. The chunks' (m, l) are staged
// in LDS by the whole block (M reduced across the block as they are), each
// chunk's weight e^{m_c - M} is evaluated once
// into LDS, and each thread's o_c loads are issued kMergeU at a time (the first
// batch together with the statistics' loads), so the loop waits for memory
// once per kMergeU chunks instead of once per chunk; the arithmetic (and so
// the result) is that of the plain loop.
// Decode: kMergeU = 64, kMergeLds = 1024 (contexts of 32K at 32-token chunks). The
// exact prefill's merge (a few chunks per query, thousands of blocks) takes 16 and 128:
// fewer registers and less LDS per block, so more blocks per CU.
template <int kMergeU, int kMergeLds>
__global__ void __launch_bounds__(128) attn_combine_kernel(AttnArgs a) {
    __shared__ float ms[kMergeLds], ls[kMergeLds], es[kMergeLds];
    __shared__ float wm[2];
    const int qh = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos) + (a.prefill ? b : 0);
    const int T = a.prefill ? pick_chunk(pos + 1, a.Hkv, 1) : a.T;
    const int nchunks = (pos + 1 + T - 1) / T;
    if (nchunks == 1) return;  // the chunk kernel wrote the output
    const float* pp = a.part + ((int64_t)b * a.Hq + qh) * a.max_chunks * kPartStride;
    float M = -1e30f, L = 0.0f, o = 0.0f;
    if (nchunks > kMergeLds) {
        for (int c = 0; c < nchunks; ++c) M = fmaxf(M, pp[c * kPartStride]);
        for (int c = 0; c < nchunks; ++c) {
            const float e = expf(pp[c * kPartStride] - M);
            L = __builtin_fmaf(e, pp[c * kPartStride + 1], L);
            o = __builtin_fmaf(e, pp[c * kPartStride + 2 + d], o);
        }
    } else {
        // the first kMergeU value loads go out before the statistics are
        // staged (they do not depend on M), so both share one wait
        float ov[kMergeU];
#pragma unroll
        for (int u = 0; u < kMergeU; ++u)
            ov[u] = u < nchunks ? pp[u * kPartStride + 2 + d] : 0.0f;
        float mloc = -1e30f;
        for (int c = d; c < nchunks; c += 128) {
            const float m = pp[c * kPartStride];
            ms[c] = m;
            ls[c] = pp[c * kPartStride + 1];
            mloc = fmaxf(mloc, m);
        }
        // M over the block (a maximum: the same in any order) from the two
        // waves' maxima, instead of a serial pass over the staged statistics
        mloc = wave_max(mloc);
        if ((d & 63) == 0) wm[d >> 6] = mloc;
        __syncthreads();
        M = fmaxf(wm[0], wm[1]);
        // each chunk's weight e^{m_c - M} once per block (the same expf the
        // plain loop evaluates in every thread)
        for (int c = d; c < nchunks; c += 128) es[c] = expf(ms[c] - M);
        __syncthreads();
        for (int c0 = 0; c0 < nchunks; c0 += kMergeU) {
            if (c0 > 0) {
#pragma unroll
                for (int u = 0; u < kMergeU; ++u)
                    ov[u] = c0 + u < nchunks ? pp[(c0 + u) * kPartStride + 2 + d] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < kMergeU; ++u) {
                if (c0 + u < nchunks) {
                    const float e = es[c0 + u];
                    L = __builtin_fmaf(e, ls[c0 + u], L);
                    o = __builtin_fmaf(e, ov[u], o);
                }
            }
        }
    }
    a.out[(int64_t)b * a.out_stride + (int64_t)qh * kD + d] = __fdiv_rn(o, L);
}

// The merge of more than kWideMin chunk partials (decode launches of more than
// kWideMin chunks, and the exact prefill's rows with as many), on 512 threads:
// four groups of 128 (one thread per dim) each merge a contiguous quarter of the
// chunks in chunk order, one fma per term, and the four sums are added as
// (g0 + g1) + (g2 + g3) before the division; the quarters' value loads go out
// together, where one 128-thread block would wait for its batches one after
// another (b1 8k, 86 chunks: 17.5 -> 14.3 us; b1 32k, 128 chunks: 28.1 -> 22.7).
// A row with kWideMin chunks or fewer (a decode grid sized for longer contexts)
// is merged by group 0 alone, exactly as attn_combine_kernel merges it, and
// one with more than kWideLds by attn_combine_kernel's plain loop, so the
// chunk count alone decides the arithmetic: a prefill row and a decode step at
// the same position give the same bits. M, the chunks' weights e^{m_c - M} and
// L are those of attn_combine_kernel.
// (64: the exact prefill's rows up to 64 chunks keep the 128-thread merge, one
// block per row being the better shape for thousands of rows: 2048 prompt tokens
// ran 65.3k tok/s that way, 64.1k on the wide merge)
constexpr int kWideMin = 64;
constexpr int kWideLds = 1024;
template <int kU>
__global__ void __launch_bounds__(512) attn_combine_wide_kernel(AttnArgs a) {
    __shared__ float ms[kWideLds], ls[kWideLds], es[kWideLds];
    __shared__ float wm[8];
    __shared__ float po[3][kD], pl[3];
    const int qh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int d = tid & 127, grp = tid >> 7, lane = tid & 63;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos) + (a.prefill ? b : 0);
    const int T = a.prefill ? pick_chunk(pos + 1, a.Hkv, 1) : a.T;
    const int nchunks = (pos + 1 + T - 1) / T;
    if (nchunks == 1) return;  // the chunk kernel wrote the output
    const float* pp = a.part + ((int64_t)b * a.Hq + qh) * a.max_chunks * kPartStride;
    float* dst = a.out + (int64_t)b * a.out_stride + (int64_t)qh * kD + d;
    if (nchunks > kWideLds) {  // statistics past the LDS arrays: attn_combine_kernel's plain loop
        if (grp == 0) {
            float M = -1e30f, L = 0.0f, o = 0.0f;
            for (int c = 0; c < nchunks; ++c) M = fmaxf(M, pp[c * kPartStride]);
            for (int c = 0; c < nchunks; ++c) {
                const float e = expf(pp[c * kPartStride] - M);
                L = __builtin_fmaf(e, pp[c * kPartStride + 1], L);
                o = __builtin_fmaf(e, pp[c * kPartStride + 2 + d], o);
            }
            *dst = __fdiv_rn(o, L);
        }
        return;
    }
    const int ng = nchunks > kWideMin ? 4 : 1;
    const int per = (nchunks + ng - 1) / ng;
    const int cb = grp * per, ce = grp < ng ? min(nchunks, cb + per) : cb;
    // this group's first batch of value loads, before the statistics
    float ov[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) ov[u] = cb + u < ce ? pp[(cb + u) * kPartStride + 2 + d] : 0.0f;
    float mloc = -1e30f;
    for (int c = tid; c < nchunks; c += 512) {
        const float m = pp[c * kPartStride];
        ms[c] = m;
        ls[c] = pp[c * kPartStride + 1];
        mloc = fmaxf(mloc, m);
    }
    mloc = wave_max(mloc);
    if (lane == 0) wm[tid >> 6] = mloc;
    __syncthreads();
    float M = wm[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) M = fmaxf(M, wm[w]);
    for (int c = tid; c < nchunks; c += 512) es[c] = expf(ms[c] - M);
    __syncthreads();
    float L = 0.0f, o = 0.0f;
    for (int c0 = cb; c0 < ce; c0 += kU) {
        if (c0 > cb) {
#pragma unroll
            for (int u = 0; u < kU; ++u)
                ov[u] = c0 + u < ce ? pp[(c0 + u) * kPartStride + 2 + d] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            if (c0 + u < ce) {
                const float e = es[c0 + u];
                L = __builtin_fmaf(e, ls[c0 + u], L);
                o = __builtin_fmaf(e, ov[u], o);
            }
        }
    }
    if (ng == 1) {
        if (grp == 0) *dst = __fdiv_rn(o, L);
        return;
    }
    if (grp > 0) {
        po[grp - 1][d] = o;
        if (d == 0) pl[grp - 1] = L;
    }
    __syncthreads();
    if (grp == 0) {
        o = (o + po[0][d]) + (po[1][d] + po[2][d]);
        L = (L + pl[0]) + (pl[1] + pl[2]);
        *dst = __fdiv_rn(o, L);
    }
}

// Exact prefill attention, batched: the decode chunk kernel's arithmetic for
// QB = 16 / G queries at once. A workgroup takes chunk c (decode's chunk size
// T at those positions, the same for the launch) of kv head h for the queries
// qb QB .. qb QB + QB - 1; the 16 MFMA rows are (query j, head g) = row
// j G + g, so every score and value tile is one MFMA for all of them. MFMA
// rows do not interact, and each row's operands are the ones decode forms for
// that query (its query vector's own power-of-two scale; its chunk's valid
// tokens nt_j, zero weights past them; its own V-scale exponent per wave over
// the same tiles; the same statistics reduction per row), so each row's
// partial (m, l, o) -- and after attn_combine_kernel its output -- equals the
// token-by-token decode step's bit for bit. Queries whose context ends before
// chunk c contribute no rows.
template <int G, int U>
__global__ void __launch_bounds__(256) attn_prefill_exact_kernel(AttnArgs a) {
    constexpr int QB = 16 / G;
    constexpr int NTW = (U + 1) / 2;  // 16-token tiles per wave (T = 32 U)
    __shared__ float qs[16][kD];
    __shared__ float sc[16][kMaxChunk + 4];  // (+4: the W reads of 16 rows hit 16 bank groups)
    __shared__ float ow[4][16][kD];
    __shared__ float mstat[16], lstat[16];
    const int c = blockIdx.x, h = blockIdx.y, qb = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kn = lane & 15, kq = lane >> 4;
    const int T = a.T;
    const int t0 = c * T;
    const int b0 = qb * QB;
    const int nq = min(QB, a.pos_n - b0);
    // the block's last query has the longest context
    const int nt_max = min(T, a.pos + b0 + nq - t0);
    if (nt_max <= 0) return;
    auto nt_of = [&](int j) {  // valid tokens of chunk c for query j (<= 0: none)
        return j < nq ? min(T, a.pos + b0 + j + 1 - t0) : 0;
    };
    const int64_t cache_head = (int64_t)h * a.max_seq;
    const int8_t* kbase = a.kc + cache_head * kD;
    const int8_t* vbase = a.vc + cache_head * kD;
    const uint16_t* ksb = a.ks + cache_head;
    const uint16_t* vsb = a.vs + cache_head;

    // ---- every load first: the rows' query pairs and RoPE factors, then this lane's K and
    // V rows of the wave's tiles (tokens past the block's context read its last row) ----
    constexpr int kQI = 16 * 64 / 256;
    float qx0[kQI], qx1[kQI], qcs[kQI], qsn[kQI];
#pragma unroll
    for (int r = 0; r < kQI; ++r) {
        const int i = tid + 256 * r;
        const int row = i >> 6, jd = i & 63;
        const int j = min(row / G, nq - 1), g = row % G;  // (rows past nq: a valid query)
        const int b = b0 + j;
        const float* qv = a.q + (int64_t)b * a.q_stride + (int64_t)(h * G + g) * kD;
        const float* rope = a.rope + (int64_t)(a.pos + b) * kD;
        qx0[r] = qv[jd];
        qx1[r] = qv[jd + 64];
        qcs[r] = rope[jd];
        qsn[r] = rope[64 + jd];
    }
    asm volatile("" ::: "memory");
    uint4 kr[NTW][2];
    uint16_t ksr[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i) {
        const int t = t0 + min((wave + 4 * i) * 16 + kn, nt_max - 1);
        const uint4* kp = reinterpret_cast<const uint4*>(kbase + (int64_t)t * kD + 32 * kq);
        kr[i][0] = kp[0];
        kr[i][1] = kp[1];
        ksr[i] = ksb[t];
    }
    uint2 vm[NTW][4];
    uint16_t vms[NTW][4];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = t0 + min((wave + 4 * i) * 16 + 4 * kq + e, nt_max - 1);
            vm[i][e] = *reinterpret_cast<const uint2*>(vbase + (int64_t)t * kD + 8 * kn);
            vms[i][e] = vsb[t];
        }

    // ---- RoPE on the rows' query vectors (:460-481) ----
#pragma unroll
    for (int r = 0; r < kQI; ++r) {
        const int i = tid + 256 * r;
        const int row = i >> 6, jd = i & 63;
        const bool live = row / G < nq;
        qs[row][jd] = live ? __builtin_fmaf(qx0[r], qcs[r], -__fmul_rn(qx1[r], qsn[r])) : 0.0f;
        qs[row][jd + 64] = live ? __builtin_fmaf(qx0[r], qsn[r], __fmul_rn(qx1[r], qcs[r])) : 0.0f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- scores (:678-694) on MFMA: rows 4 kq + e of lane (kn, kq) ----
    {
        h4a qh[8], ql[8];
        float qin[4];
        q_operands<16>(qs, qh, ql, qin);
        int ntr[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ntr[e] = nt_of((4 * kq + e) / G);
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int tile = wave + 4 * i;
            if (tile * 16 >= nt_max) break;  // (wave-uniform)
            const int tl = tile * 16 + kn;
            const f4a d = score_tile(qh, ql, kr[i][0], kr[i][1]);
            const float f = __fmul_rn(half_bits_to_float(ksr[i]), kScaleFactor);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (tl < ntr[e]) sc[4 * kq + e][tl] = __fmul_rn(d[e] * qin[e], f);
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- chunk softmax statistics (:824-830), row by row as decode does per head ----
    for (int row = wave; row < 16; row += 4) {
        const int nt = nt_of(row / G);
        if (nt <= 0) continue;  // (wave-uniform)
        float m = -1e30f;
        for (int i = lane; i < nt; i += 64) m = fmaxf(m, sc[row][i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < nt; i += 64) {
            const float e = expf(sc[row][i] - m);
            sc[row][i] = e;
            l += e;
        }
        l = wave_sum_tree(l);
        if (lane == 0) {
            mstat[row] = m;
            lstat[row] = l;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- weighted values (:842-851) on MFMA (value_tile) ----
    {
        // per query, the wave's largest V scale over its tiles' valid tokens sets its
        // power-of-two scale (decode: the same tiles, the tokens clamped to the chunk, whose
        // repeats of the last valid token do not change the maximum)
        float vmq[QB];
#pragma unroll
        for (int j = 0; j < QB; ++j) vmq[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            if ((wave + 4 * i) * 16 >= nt_max) break;  // (wave-uniform)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tl = (wave + 4 * i) * 16 + 4 * kq + e;
                const float sv = half_bits_to_float(vms[i][e]);
#pragma unroll
                for (int j = 0; j < QB; ++j)
                    if (tl < nt_of(j)) vmq[j] = fmaxf(vmq[j], sv);
            }
        }
        // this lane's W row (kn) and D rows (4 kq + e): their queries' exponents
        float wup_row = 1.0f, wdn[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        int nt_w = 0;
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            const int sh = fp16_span_exp(wave_max(vmq[j]));
            const float up = ldexpf(1.0f, sh), down = ldexpf(1.0f, -sh);
            if (kn / G == j) {
                wup_row = up;
                nt_w = nt_of(j);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if ((4 * kq + e) / G == j) wdn[e] = down;
        }
        f4a acc8[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc8[dt] = f4a{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int tile = wave + 4 * i;
            if (tile * 16 >= nt_max) break;  // (wave-uniform)
            float svf[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) svf[e] = half_bits_to_float(vms[i][e]);
            // w_operands' arithmetic with this row's valid length and scale
            const float4 p4 = *reinterpret_cast<const float4*>(&sc[kn][tile * 16 + 4 * kq]);
            const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
            h4a wh[1], wl[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tl = tile * 16 + 4 * kq + e;
                const float w = tl < nt_w ? __fmul_rn(pv[e], svf[e]) * wup_row : 0.0f;
                const _Float16 hi = (_Float16)w;
                wh[0][e] = hi;
                wl[0][e] = (_Float16)(w - (float)hi);
            }
            value_tile(wh, wl, vm[i], acc8);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) ow[wave][4 * kq + e][8 * kn + dt] = acc8[dt][e] * wdn[e];
    }
    __syncthreads();
    for (int i = tid; i < 16 * kD; i += 256) {
        const int row = i >> 7, d = i & 127;
        const int j = row / G, g = row % G;
        if (nt_of(j) <= 0) continue;
        const int b = b0 + j;
        const int qh = h * G + g;
        const float o = (ow[0][row][d] + ow[1][row][d]) + (ow[2][row][d] + ow[3][row][d]);
        if (a.pos + b + 1 <= T) {  // one chunk: the output itself
            a.out[(int64_t)b * a.out_stride + (int64_t)qh * kD + d] = __fdiv_rn(o, lstat[row]);
        } else {
            float* pp = a.part + (((int64_t)b * a.Hq + qh) * a.max_chunks + c) * kPartStride;
            pp[2 + d] = o;
            if (d == 0) {
                pp[0] = mstat[row];
                pp[1] = lstat[row];
            }
        }
    }
}

// attn_prefill_exact_kernel for 64-token chunks: decode's four waves each take
// one 16-token tile of the chunk, and so do this kernel's, for QB = 16 / G
// queries at once (row j G + g: query j, head g). Each row's statistics are
// decode's single-wave pass over its 64 tokens (token i in lane i), its V-scale
// exponent per wave over the wave's valid tokens, and its partial decode's
// (ow0 + ow1) + (ow2 + ow3): waves 0 and 2 hand their sums over LDS, waves 1 and 3
// add theirs (the lanes of every wave hold the same rows and dims), wave 3 hands
// (ow2 + ow3) back and wave 1 adds it to its (ow0 + ow1). LDS 28 KB: five
// workgroups per CU.
template <int G>
__global__ void __launch_bounds__(256) attn_prefill_exact64_kernel(AttnArgs a) {
    constexpr int QB = 16 / G;
    constexpr int T = 64;
    __shared__ float qs[16][kD];
    __shared__ float sc[16][T + 4];
    __shared__ float ow[2][16][kD];
    __shared__ float mstat[16], lstat[16];
    const int c = blockIdx.x, h = blockIdx.y, qb = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kn = lane & 15, kq = lane >> 4;
    const int b0 = qb * QB;
    const int nq = min(QB, a.pos_n - b0);
    const int last_len = a.pos + b0 + nq;  // the block's longest context
    const int t0 = c * T;
    const int nt_max = min(T, last_len - t0);
    if (nt_max <= 0) return;
    auto nt_of = [&](int j) {  // valid tokens of the chunk for query j
        return j < nq ? min(T, a.pos + b0 + j + 1 - t0) : 0;
    };
    const int64_t cache_head = (int64_t)h * a.max_seq;
    const int8_t* kbase = a.kc + cache_head * kD;
    const int8_t* vbase = a.vc + cache_head * kD;
    const uint16_t* ksb = a.ks + cache_head;
    const uint16_t* vsb = a.vs + cache_head;

    // ---- every load first (tokens past the context read the context's last row) ----
    constexpr int kQI = 16 * 64 / 256;
    float qx0[kQI], qx1[kQI], qcs[kQI], qsn[kQI];
#pragma unroll
    for (int r = 0; r < kQI; ++r) {
        const int i = tid + 256 * r;
        const int row = i >> 6, jd = i & 63;
        const int j = min(row / G, nq - 1), g = row % G;
        const int b = b0 + j;
        const float* qv = a.q + (int64_t)b * a.q_stride + (int64_t)(h * G + g) * kD;
        const float* rope = a.rope + (int64_t)(a.pos + b) * kD;
        qx0[r] = qv[jd];
        qx1[r] = qv[jd + 64];
        qcs[r] = rope[jd];
        qsn[r] = rope[64 + jd];
    }
    asm volatile("" ::: "memory");
    const int tlast = last_len - 1;
    uint4 k0, k1;
    uint16_t ksr;
    {
        const int t = min(t0 + wave * 16 + kn, tlast);
        const uint4* kp = reinterpret_cast<const uint4*>(kbase + (int64_t)t * kD + 32 * kq);
        k0 = kp[0];
        k1 = kp[1];
        ksr = ksb[t];
    }
    uint2 vm[4];
    uint16_t vms[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = min(t0 + wave * 16 + 4 * kq + e, tlast);
        vm[e] = *reinterpret_cast<const uint2*>(vbase + (int64_t)t * kD + 8 * kn);
        vms[e] = vsb[t];
    }

    // ---- RoPE on the rows' query vectors (:460-481) ----
#pragma unroll
    for (int r = 0; r < kQI; ++r) {
        const int i = tid + 256 * r;
        const int row = i >> 6, jd = i & 63;
        const bool live = row / G < nq;
        qs[row][jd] = live ? __builtin_fmaf(qx0[r], qcs[r], -__fmul_rn(qx1[r], qsn[r])) : 0.0f;
        qs[row][jd + 64] = live ? __builtin_fmaf(qx0[r], qsn[r], __fmul_rn(qx1[r], qcs[r])) : 0.0f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- scores (:678-694) on MFMA: rows 4 kq + e of lane (kn, kq) ----
    if (wave * 16 < nt_max) {  // (wave-uniform)
        h4a qh[8], ql[8];
        float qin[4];
        q_operands<16>(qs, qh, ql, qin);
        const int tl = wave * 16 + kn;
        const f4a d = score_tile(qh, ql, k0, k1);
        const float f = __fmul_rn(half_bits_to_float(ksr), kScaleFactor);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (tl < nt_of((4 * kq + e) / G)) sc[4 * kq + e][tl] = __fmul_rn(d[e] * qin[e], f);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- chunk softmax statistics (:824-830): decode's pass, one row per wave pass ----
    for (int row = wave; row < 16; row += 4) {
        const int nt = nt_of(row / G);
        if (nt <= 0) continue;  // (wave-uniform)
        const float x = lane < nt ? sc[row][lane] : -1e30f;
        const float m = wave_max(x);
        float l = 0.0f;
        if (lane < nt) {
            const float e = expf(x - m);
            sc[row][lane] = e;
            l += e;
        }
        l = wave_sum_tree(l);
        if (lane == 0) {
            mstat[row] = m;
            lstat[row] = l;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- weighted values (:842-851) on MFMA (value_tile) ----
    {
        const bool has_tile = wave * 16 < nt_max;  // (wave-uniform)
        float vmq[QB];
#pragma unroll
        for (int j = 0; j < QB; ++j) vmq[j] = 0.0f;
        if (has_tile) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tl = wave * 16 + 4 * kq + e;
                const float sv = half_bits_to_float(vms[e]);
#pragma unroll
                for (int j = 0; j < QB; ++j)
                    if (tl < nt_of(j)) vmq[j] = fmaxf(vmq[j], sv);
            }
        }
        float wup_row = 1.0f, wdn[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        int nt_w = 0;
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            const int sh = fp16_span_exp(wave_max(vmq[j]));
            const float up = ldexpf(1.0f, sh), down = ldexpf(1.0f, -sh);
            if (kn / G == j) {
                wup_row = up;
                nt_w = nt_of(j);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if ((4 * kq + e) / G == j) wdn[e] = down;
        }
        f4a acc8[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc8[dt] = f4a{0.0f, 0.0f, 0.0f, 0.0f};
        if (has_tile) {
            float svf[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) svf[e] = half_bits_to_float(vms[e]);
            const float4 p4 = *reinterpret_cast<const float4*>(&sc[kn][wave * 16 + 4 * kq]);
            const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
            h4a wh[1], wl[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tl = wave * 16 + 4 * kq + e;
                const float w = tl < nt_w ? __fmul_rn(pv[e], svf[e]) * wup_row : 0.0f;
                const _Float16 hi = (_Float16)w;
                wh[0][e] = hi;
                wl[0][e] = (_Float16)(w - (float)hi);
            }
            value_tile(wh, wl, vm, acc8);
        }
        // decode's o = (ow0 + ow1) + (ow2 + ow3)
        const int slot = wave >> 1;
        if ((wave & 1) == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) ow[slot][4 * kq + e][8 * kn + dt] = acc8[dt][e] * wdn[e];
        }
        __syncthreads();
        float s2[4][8];
        if (wave & 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
                    s2[e][dt] = ow[slot][4 * kq + e][8 * kn + dt] + acc8[dt][e] * wdn[e];
        }
        if (wave == 3) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) ow[1][4 * kq + e][8 * kn + dt] = s2[e][dt];
        }
        __syncthreads();
        if (wave == 1) {  // the partial (or, with one chunk, the output) of each row
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = 4 * kq + e;
                const int j = row / G, g = row % G;
                if (nt_of(j) <= 0) continue;
                const int bq = b0 + j;
                const int qh = h * G + g;
                float o[8];
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) o[dt] = s2[e][dt] + ow[1][row][8 * kn + dt];
                if (a.pos + bq + 1 <= T) {  // one chunk: the output itself
                    float* dst = a.out + (int64_t)bq * a.out_stride + (int64_t)qh * kD + 8 * kn;
                    const float L = lstat[row];
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) dst[dt] = __fdiv_rn(o[dt], L);
                } else {
                    float* pp = a.part +
                                (((int64_t)bq * a.Hq + qh) * a.max_chunks + c) * kPartStride;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) pp[2 + 8 * kn + dt] = o[dt];
                    if (kn == 0) {
                        pp[0] = mstat[row];
                        pp[1] = lstat[row];
                    }
                }
            }
        }
    }
}

// Prefill attention on fp16 MFMA, streaming form (an online softmax over the
// causal prefix): a workgroup takes QP = 16 / G consecutive queries of one kv
// head as the 16 MFMA rows (row m: query m / G, head m % G) and its 4 waves
// split the prefix's 16-token tiles (wave w: tiles w, w + 4, ...), each with
// its own running max m, sum l and value sums, merged in LDS at the end. Per
// tile: the scores on score_tile (the rows' query vectors scaled per row as in
// decode), masked to each row's causal prefix; the row statistics over the 16
// lanes that hold a row (DPP within 16-lane rows); the probabilities move from
// the score D layout to the value A layout through LDS (a 16 x 16 tile per
// wave); the values on value_tile with W = p * s_v scaled per wave. The
// longest prefixes (last queries) are dispatched first.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    return fmaxf(v, dpp_f<kDppMirror>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    return v + dpp_f<kDppMirror>(v);
}

template <int G>
__global__ void __launch_bounds__(256) attn_prefill_mfma_kernel(AttnArgs a) {
    constexpr int QP = 16 / G;  // queries per workgroup
    __shared__ float qs[16][kD];
    __shared__ __align__(16) float pt[4][16][20];  // per wave: the P tile, rows padded
    __shared__ float wm[4][16], wls[4][16];
    __shared__ float wo[4][16][kD];
    const int h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kn = lane & 15, kq = lane >> 4;
    const int qb = (gridDim.x - 1 - blockIdx.x) * QP;  // the group's first query row
    const int nq = min(QP, a.pos_n - qb);              // its live queries
    // ---- RoPE on the 16 rows (:460-481); rows of dead queries are zero ----
    for (int i = tid; i < 16 * 64; i += 256) {
        const int m = i >> 6, j = i & 63, qi = m / G, g = m % G;
        const bool live = qi < nq;
        const int b = qb + (live ? qi : 0);
        const float* rope = a.rope + (int64_t)(a.pos + b) * kD;
        const float* qv = a.q + (int64_t)b * a.q_stride + (int64_t)(h * G + g) * kD;
        const float x0 = live ? qv[j] : 0.0f, x1 = live ? qv[j + 64] : 0.0f;
        const float cs = rope[j], sn = rope[64 + j];
        qs[m][j] = __builtin_fmaf(x0, cs, -__fmul_rn(x1, sn));
        qs[m][j + 64] = __builtin_fmaf(x0, sn, __fmul_rn(x1, cs));
    }
    __syncthreads();
    // the rows' A operands, each row scaled by its own power of two
    h4a qh[8], ql[8];
    float qin[4];
    {
        const float* qrow = &qs[kn][32 * kq];
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(qrow[i]));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const int sh = fp16_span_exp(mx);
        const float up = ldexpf(1.0f, sh), down = ldexpf(1.0f, -sh);
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float xs = qrow[4 * j + e] * up;
                const _Float16 hi = (_Float16)xs;
                qh[j][e] = hi;
                ql[j][e] = (_Float16)(xs - (float)hi);
            }
#pragma unroll
        for (int e = 0; e < 4; ++e) qin[e] = __shfl(down, 4 * kq + e, 64);
    }
    // this lane's D rows 4 kq + i: their query positions (-1: a dead row, all masked)
    int prow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int qi = (4 * kq + i) / G;
        prow[i] = qi < nq ? a.pos + qb + qi : -1;
    }
    const int nkey = a.pos + qb + nq;  // keys 0 .. the last live query
    const int ntile = (nkey + 15) / 16;
    const int64_t cache_head = (int64_t)h * a.max_seq;
    const int8_t* kbase = a.kc + cache_head * kD;
    const int8_t* vbase = a.vc + cache_head * kD;
    const uint16_t* ksb = a.ks + cache_head;
    const uint16_t* vsb = a.vs + cache_head;
    // the wave's power-of-two scale for W = p * s_v: its tiles' largest V scale
    float vmax = 0.0f;
    for (int tile = wave; tile < ntile; tile += 4)
        vmax = fmaxf(vmax, half_bits_to_float(vsb[min(tile * 16 + kn, nkey - 1)]));
    const int wsh = fp16_span_exp(wave_max(vmax));
    const float wup = ldexpf(1.0f, wsh), wdown = ldexpf(1.0f, -wsh);
    float mr[4], lr[4];
    f4a acc8[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        mr[i] = -1e30f;
        lr[i] = 0.0f;
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc8[dt] = f4a{0.0f, 0.0f, 0.0f, 0.0f};
    for (int tile = wave; tile < ntile; tile += 4) {
        // the tile's K (lane token kn) and V (lane tokens 4 kq + e) rows and scales
        const int tk = min(tile * 16 + kn, nkey - 1);
        const uint4* kp = reinterpret_cast<const uint4*>(kbase + (int64_t)tk * kD + 32 * kq);
        const uint4 k0 = kp[0], k1 = kp[1];
        const float f = __fmul_rn(half_bits_to_float(ksb[tk]), kScaleFactor);
        uint2 v[4];
        float svf[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int tv = min(tile * 16 + 4 * kq + e, nkey - 1);
            v[e] = *reinterpret_cast<const uint2*>(vbase + (int64_t)tv * kD + 8 * kn);
            svf[e] = half_bits_to_float(vsb[tv]);
        }
        const f4a d = score_tile(qh, ql, k0, k1);
        const int tok = tile * 16 + kn;
        float p[4], rs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float sv = tok <= prow[i] ? __fmul_rn(d[i] * qin[i], f) : -1e30f;
            const float mn = fmaxf(mr[i], row16_max(sv));
            rs[i] = expf(mr[i] - mn);
            p[i] = tok <= prow[i] ? expf(sv - mn) : 0.0f;
            lr[i] = __builtin_fmaf(lr[i], rs[i], row16_sum(p[i]));
            mr[i] = mn;
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc8[dt][i] *= rs[i];
        // P from the score layout (row 4 kq + i, token kn) to the value A layout (row kn,
        // tokens 4 kq ..): through this wave's LDS tile (in order within the wave)
#pragma unroll
        for (int i = 0; i < 4; ++i) pt[wave][4 * kq + i][kn] = p[i];
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        asm volatile("" ::: "memory");
        const float4 pr = *reinterpret_cast<const float4*>(&pt[wave][kn][4 * kq]);
        const float pw[4] = {pr.x, pr.y, pr.z, pr.w};
        h4a wh[1], wl[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float w = __fmul_rn(pw[e], svf[e]) * wup;
            const _Float16 hi = (_Float16)w;
            wh[0][e] = hi;
            wl[0][e] = (_Float16)(w - (float)hi);
        }
        asm volatile("" ::: "memory");  // (the next tile's LDS writes stay behind this read)
        value_tile(wh, wl, v, acc8);
    }
    // merge the 4 waves: (m, l) per row, value sums unscaled
    if (kn == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            wm[wave][4 * kq + i] = mr[i];
            wls[wave][4 * kq + i] = lr[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) wo[wave][4 * kq + i][8 * kn + dt] = acc8[dt][i] * wdown;
    __syncthreads();
    for (int o = tid; o < 16 * kD; o += 256) {
        const int m = o >> 7, dd = o & 127, qi = m / G, g = m % G;
        if (qi >= nq) continue;
        const float M = fmaxf(fmaxf(wm[0][m], wm[1][m]), fmaxf(wm[2][m], wm[3][m]));
        float L = 0.0f, acc = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float e = expf(wm[w][m] - M);
            L = __builtin_fmaf(e, wls[w][m], L);
            acc = __builtin_fmaf(e, wo[w][m][dd], acc);
        }
        a.out[(int64_t)(qb + qi) * a.out_stride + (int64_t)(h * G + g) * kD + dd] = __fdiv_rn(acc, L);
    }
}

// Prefill append: RoPE on k and the INT8 quantization of k and v for the
// tokens at positions pos .. pos + n - 1, with the arithmetic of the decode
// kernel's append (so the cache matches one decode step per token). Grid
// (n, Hkv), 128 threads: wave 0 k, wave 1 v.
__global__ void __launch_bounds__(128) attn_append_kernel(AttnArgs a) {
    __shared__ __align__(16) int8_t codes[2][kD];
    const int i = blockIdx.x, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int pos = a.pos + i;
    const float* rope = a.rope + (int64_t)pos * kD;
    const float* src = (wave == 0 ? a.k_new : a.v_new) + (int64_t)i * a.kv_stride + (int64_t)h * kD;
    float x0 = src[lane], x1 = src[lane + 64];
    if (wave == 0) {
        const float cs = rope[lane], sn = rope[64 + lane];
        const float r0 = __builtin_fmaf(x0, cs, -__fmul_rn(x1, sn));
        const float r1 = __builtin_fmaf(x0, sn, __fmul_rn(x1, cs));
        x0 = r0;
        x1 = r1;
    }
    float s;
    quant_kv_pair(x0, x1, codes[wave], lane, &s);
    const int64_t row = (int64_t)h * a.max_seq + pos;
    int8_t* dst = (wave == 0 ? a.kc : a.vc) + row * kD;
    dst[lane] = codes[wave][lane];
    dst[lane + 64] = codes[wave][lane + 64];
    if (lane == 0) (wave == 0 ? a.ks : a.vs)[row] = float_to_half_bits(s);
}

int attn_pick_chunk(int seq_len, int Hkv, int B) { return pick_chunk(seq_len, Hkv, B); }

int launch_attn(const AttnLaunch& L, hipStream_t st) {
    const int G = L.Hq / L.Hkv;
    AttnArgs a{};
    a.q = L.q;
    a.k_new = L.k_new;
    a.v_new = L.v_new;
    a.kc = L.kc;
    a.vc = L.vc;
    a.ks = L.ks;
    a.vs = L.vs;
    a.rope = L.rope;
    a.pos_dev = L.pos_dev;
    a.pos = L.pos;
    a.rope_indexed = L.rope_indexed;
    a.Hq = L.Hq;
    a.Hkv = L.Hkv;
    a.max_seq = L.max_seq;
    a.T = L.T;
    a.cache_batch_stride = (int64_t)L.Hkv * L.max_seq;
    a.q_stride = (int64_t)L.Hq * kD;
    a.kv_stride = (int64_t)L.Hkv * kD;
    a.out_stride = (int64_t)L.Hq * kD;
    a.prefill = 0;
    a.out = L.out;
    a.max_chunks = L.max_chunks;
    a.q_rot = L.q_rot;
    a.k_rot = L.k_rot;
    const size_t part_bytes = (size_t)L.B * L.Hq * L.max_chunks * kPartStride * 4;
    if (L.max_chunks > 1) {
        a.part = L.part ? L.part : (float*)Scratch::get(kScratchAttn, part_bytes, st);
        if (!a.part) return TENZO_ERROR_OUT_OF_MEMORY;
    }
    dim3 grid(L.max_chunks, L.Hkv, L.B);
    if (G != 1 && G != 2 && G != 4 && G != 8) {
        set_error("attention: query heads per kv head must be 1, 2, 4 or 8 (got %d)", G);
        return TENZO_ERROR_UNSUPPORTED;
    }
    if (L.T < 32 || L.T > kMaxChunk || L.T % 32 != 0) {
        set_error("attention: tokens per chunk must be a multiple of 32 in [32, %d] (got %d)",
                  kMaxChunk, L.T);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    const int U = L.T / 32;  // groups of 8 tokens per wave
#define ATT_CASE(GG, UU)                                                                      \
    if (G == GG && U == UU)                                                                   \
        hipLaunchKernelGGL((attn_int8_chunk_kernel<GG, UU>), grid, dim3(256), 0, st, a);
#define ATT_G(GG)                                                                             \
    ATT_CASE(GG, 1) ATT_CASE(GG, 2) ATT_CASE(GG, 3) ATT_CASE(GG, 4) ATT_CASE(GG, 5)           \
    ATT_CASE(GG, 6) ATT_CASE(GG, 7) ATT_CASE(GG, 8)
    ATT_G(1) ATT_G(2) ATT_G(4) ATT_G(8)
#undef ATT_G
#undef ATT_CASE
    int rc = launch_status("attn_int8_chunk_kernel");
    if (rc) return rc;
    if (L.max_chunks > 1) {
        // (the same arithmetic for every narrow instantiation; 17-32 chunks in one
        // batch of 32 loads: b1 1k 10.4 -> 9.9 us; past kWideMin the four-group merge)
        const dim3 cg((unsigned)L.Hq, (unsigned)L.B);
        if (L.max_chunks > 16 && L.max_chunks <= 32)
            hipLaunchKernelGGL((attn_combine_kernel<32, 128>), cg, dim3(128), 0, st, a);
        else if (L.max_chunks <= kWideMin)
            hipLaunchKernelGGL((attn_combine_kernel<16, 128>), cg, dim3(128), 0, st, a);
        else
            hipLaunchKernelGGL((attn_combine_wide_kernel<32>), cg, dim3(512), 0, st, a);
        rc = launch_status("attn_combine_kernel");
    }
    return rc;
}

int launch_attn_combine(const float* part, float* out, int B, int Hq, int Hkv, int T,
                        int max_chunks, const int* pos_dev, int pos, hipStream_t st) {
    AttnArgs a{};
    a.part = const_cast<float*>(part);
    a.out = out;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.T = T;
    a.max_chunks = max_chunks;
    a.pos_dev = pos_dev;
    a.pos = pos;
    a.out_stride = (int64_t)Hq * kD;
    hipLaunchKernelGGL((attn_combine_kernel<64, 1024>), dim3(Hq, B), dim3(128), 0, st, a);
    return launch_status("attn_combine_kernel");
}

int attn_prefill_max_chunks(int pos0, int n, int Hkv) {
    int mx = 1;
    for (int i = 0; i < n; ++i) {
        const int sl = pos0 + i + 1, T = pick_chunk(sl, Hkv, 1);
        mx = std::max(mx, (sl + T - 1) / T);
    }
    return mx;
}

int launch_attn_prefill(const AttnPrefill& P, hipStream_t st) {
    const int G = P.Hq / P.Hkv;
    AttnArgs a{};
    a.q = P.q;
    a.k_new = P.k_new;
    a.v_new = P.v_new;
    a.kc = P.kc;
    a.vc = P.vc;
    a.ks = P.ks;
    a.vs = P.vs;
    a.rope = P.rope;
    a.pos = P.pos0;
    a.rope_indexed = 1;
    a.Hq = P.Hq;
    a.Hkv = P.Hkv;
    a.max_seq = P.max_seq;
    a.cache_batch_stride = 0;
    a.q_stride = P.row_stride;
    a.kv_stride = P.row_stride;
    a.out_stride = P.out_stride;
    a.out = P.out;
    a.prefill = 1;
    hipLaunchKernelGGL(attn_append_kernel, dim3(P.n, P.Hkv), dim3(128), 0, st, a);
    int rc = launch_status("attn_append_kernel");
    if (rc) return rc;
    if (!P.exact && (G == 1 || G == 2 || G == 4 || G == 8)) {
        a.pos_n = P.n;
        dim3 grid((unsigned)ceil_div(P.n, 16 / G), P.Hkv);
        switch (G) {
            case 1: hipLaunchKernelGGL(attn_prefill_mfma_kernel<1>, grid, dim3(256), 0, st, a); break;
            case 2: hipLaunchKernelGGL(attn_prefill_mfma_kernel<2>, grid, dim3(256), 0, st, a); break;
            case 4: hipLaunchKernelGGL(attn_prefill_mfma_kernel<4>, grid, dim3(256), 0, st, a); break;
            default: hipLaunchKernelGGL(attn_prefill_mfma_kernel<8>, grid, dim3(256), 0, st, a); break;
        }
        return launch_status("attn_prefill_mfma_kernel");
    }
    // exact form (attn_prefill_exact_kernel, then decode's merge): runs of queries with one
    // chunk size (it changes only at a few context lengths), in groups whose chunk partials
    // fit 256 MiB of scratch
    if (G != 1 && G != 2 && G != 4 && G != 8) {
        set_error("attention: query heads per kv head must be 1, 2, 4 or 8 (got %d)", G);
        return TENZO_ERROR_UNSUPPORTED;
    }
    const int QB = 16 / G;
    for (int s0 = 0; s0 < P.n;) {
        const int T = pick_chunk(P.pos0 + s0 + 1, P.Hkv, 1);
        int s1 = s0 + 1;
        while (s1 < P.n && pick_chunk(P.pos0 + s1 + 1, P.Hkv, 1) == T) ++s1;
        const int mc = (int)ceil_div(P.pos0 + s1, T);  // chunks of the run's last query
        const size_t per_query = (size_t)P.Hq * mc * kPartStride * 4;
        const int qg_max =
            mc > 1 ? (int)std::max<size_t>(1, std::min<size_t>(s1 - s0, (256u << 20) / per_query))
                   : s1 - s0;
        for (int i0 = s0; i0 < s1; i0 += qg_max) {
            const int n = std::min(qg_max, s1 - i0);
            a.pos = P.pos0 + i0;
            a.pos_n = n;
            a.T = T;
            a.q = P.q + (int64_t)i0 * P.row_stride;
            a.out = P.out + (int64_t)i0 * P.out_stride;
            a.max_chunks = mc;
            a.part = nullptr;
            if (mc > 1) {
                a.part = (float*)Scratch::get(kScratchAttn, (size_t)n * per_query, st);
                if (!a.part) return TENZO_ERROR_OUT_OF_MEMORY;
            }
            const dim3 grid((unsigned)mc, (unsigned)P.Hkv, (unsigned)ceil_div(n, QB));
            const int U = T / 32;  // 2 .. 8 (pick_chunk: multiples of 32 from 64 to kMaxChunk)
            if (U == 2) {  // 64-token chunks: the kernel with the score tile sized to them
                switch (G) {
                    case 1: hipLaunchKernelGGL(attn_prefill_exact64_kernel<1>, grid, dim3(256), 0, st, a); break;
                    case 2: hipLaunchKernelGGL(attn_prefill_exact64_kernel<2>, grid, dim3(256), 0, st, a); break;
                    case 4: hipLaunchKernelGGL(attn_prefill_exact64_kernel<4>, grid, dim3(256), 0, st, a); break;
                    default: hipLaunchKernelGGL(attn_prefill_exact64_kernel<8>, grid, dim3(256), 0, st, a); break;
                }
            } else {
#define PX_CASE(GG, UU)                                                                       \
    if (G == GG && U == UU)                                                                   \
        hipLaunchKernelGGL((attn_prefill_exact_kernel<GG, UU>), grid, dim3(256), 0, st, a);
#define PX_G(GG)                                                                              \
    PX_CASE(GG, 3) PX_CASE(GG, 4) PX_CASE(GG, 5) PX_CASE(GG, 6) PX_CASE(GG, 7) PX_CASE(GG, 8)
            PX_G(1) PX_G(2) PX_G(4) PX_G(8)
#undef PX_G
#undef PX_CASE
            }
            if ((rc = launch_status("attn_prefill_exact_kernel"))) return rc;
            if (mc > 1) {
                // rows with up to kWideMin chunks on the one-group kernel, the rest on
                // decode's wide merge (a row's chunk count grows with its position;
                // the two kernels give the same bits for the short rows)
                const int nr = std::max(0, std::min(n, kWideMin * T - a.pos));
                if (nr > 0) {
                    hipLaunchKernelGGL((attn_combine_kernel<16, 128>), dim3(P.Hq, nr), dim3(128), 0,
                                       st, a);
                    if ((rc = launch_status("attn_combine_kernel"))) return rc;
                }
                if (nr < n) {
                    AttnArgs w = a;
                    w.pos = a.pos + nr;
                    w.out = a.out + (int64_t)nr * a.out_stride;
                    w.part = a.part + (int64_t)nr * P.Hq * mc * kPartStride;
                    hipLaunchKernelGGL((attn_combine_wide_kernel<32>), dim3(P.Hq, n - nr), dim3(512),
                                       0, st, w);
                    if ((rc = launch_status("attn_combine_wide_kernel"))) return rc;
                }
            }
        }
        s0 = s1;
    }
    return TENZO_SUCCESS;
}

}  // namespace tz

using namespace tz;

namespace tz {
namespace {

// The chunk partials of tenzo_hip_attn_int8_decode_noalloc (kPartStride
// floats per sequence, query head and chunk): a fixed array in device memory,
// one copy per device, loaded with the code object and held until the
// process ends, so the entry point allocates nothing. In host code `scratch`
// only names the variable: its device address comes from
// hipGetSymbolAddress, per device.
constexpr size_t kNoAllocPartFloats = (size_t)2 << 20;  // 8 MiB
static __device__ __align__(256) float scratch[kNoAllocPartFloats];

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
float* g_noalloc_part[kNoAllocMaxDevices];  // device address of `scratch`, per device

// The current device's copy of `scratch` (looked up on the first call on a
// device, with that device current), or null with the error set.
float* noalloc_part() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        hip_fail(e, "attn_int8_decode_noalloc: hipGetDevice");
        return nullptr;
    }
    if (dev < 0 || dev >= kNoAllocMaxDevices) {
        set_error("attn_int8_decode_noalloc: device %d beyond the %d supported", dev,
                  kNoAllocMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_part[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                     "attn_int8_decode_noalloc: hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        g_noalloc_part[dev] = static_cast<float*>(ptr);
    }
    return g_noalloc_part[dev];
}

}  // namespace
}  // namespace tz

extern "C" {

TENZO_HIP_API void tenzo_hip_rope_table(float theta, int head_dim, int pos0, int n_pos,
                                        float* cs) {
    // The reference evaluates freq = 1/powf(theta, 2i/d) under -ffast-math as
    // expf(-(2i/d) * logf(theta)) and takes glibc cosf/sinf of the fp32 angle
    // pos * freq (TenzoEngine.cpp:465-469 as built).
    const int half = head_dim / 2;
    const float ln_theta = logf(theta);
    for (int p = 0; p < n_pos; ++p) {
        float* row = cs + (int64_t)p * head_dim;
        for (int i = 0; i < half; ++i) {
            const float e = (float)(2 * i) / (float)head_dim;
            const float freq = expf(-e * ln_theta);
            const float angle = (float)(pos0 + p) * freq;
            row[i] = cosf(angle);
            row[half + i] = sinf(angle);
        }
    }
}

// Checks the arguments of the int8 decode entry points and fills L.
static int attn_int8_args(tz::AttnLaunch& L, const float* q, const float* k_new,
                          const float* v_new, int8_t* kc, int8_t* vc, uint16_t* ks, uint16_t* vs,
                          const float* rope_cs, int B, int Hq, int Hkv, int max_seq, int pos,
                          float* out, float* q_rot, float* k_rot) {
    using namespace tz;
    TZ_CHECK(q && k_new && v_new && kc && vc && ks && vs && rope_cs && out,
             "attn_int8_decode: null pointer");
    TZ_CHECK(B > 0 && B <= 65535 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0,
             "attn_int8_decode: bad head counts (Hq=%d Hkv=%d)", Hq, Hkv);
    TZ_CHECK(pos >= 0 && pos < max_seq, "attn_int8_decode: pos %d outside [0, %d)", pos,
             max_seq);
    TZ_CHECK(q_rot != q && k_rot != k_new, "attn_int8_decode: q_rot/k_rot must not alias q/k");
    L.q = q;
    L.k_new = k_new;
    L.v_new = v_new;
    L.kc = kc;
    L.vc = vc;
    L.ks = ks;
    L.vs = vs;
    L.rope = rope_cs;
    L.pos = pos;
    L.B = B;
    L.Hq = Hq;
    L.Hkv = Hkv;
    L.max_seq = max_seq;
    L.T = attn_pick_chunk(pos + 1, Hkv, B);
    L.max_chunks = (int)ceil_div(pos + 1, L.T);
    L.out = out;
    L.q_rot = q_rot;
    L.k_rot = k_rot;
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_attn_int8_decode(const float* q, const float* k_new,
                                             const float* v_new, int8_t* kc, int8_t* vc,
                                             uint16_t* ks, uint16_t* vs, const float* rope_cs,
                                             int B, int Hq, int Hkv, int max_seq, int pos,
                                             float* out, float* q_rot, float* k_rot,
                                             void* stream) {
    tz::AttnLaunch L{};
    const int rc = attn_int8_args(L, q, k_new, v_new, kc, vc, ks, vs, rope_cs, B, Hq, Hkv,
                                  max_seq, pos, out, q_rot, k_rot);
    if (rc) return rc;
    return tz::launch_attn(L, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_attn_int8_decode_noalloc(const float* q, const float* k_new,
                                                     const float* v_new, int8_t* kc, int8_t* vc,
                                                     uint16_t* ks, uint16_t* vs,
                                                     const float* rope_cs, int B, int Hq, int Hkv,
                                                     int max_seq, int pos, float* out,
                                                     float* q_rot, float* k_rot, void* stream) {
    using namespace tz;
    AttnLaunch L{};
    const int rc = attn_int8_args(L, q, k_new, v_new, kc, vc, ks, vs, rope_cs, B, Hq, Hkv,
                                  max_seq, pos, out, q_rot, k_rot);
    if (rc) return rc;
    if (L.max_chunks > 1) {  // (one chunk writes the output directly: no partials)
        const size_t need = (size_t)B * Hq * L.max_chunks * kPartStride;
        TZ_CHECK(need <= kNoAllocPartFloats,
                 "attn_int8_decode_noalloc: %zu bytes of chunk partials (B=%d Hq=%d, %d chunks) "
                 "exceed its fixed %zu-byte array; use tenzo_hip_attn_int8_decode",
                 need * 4, B, Hq, L.max_chunks, kNoAllocPartFloats * 4);
        L.part = noalloc_part();
        if (!L.part) return TENZO_ERROR_UNSUPPORTED;
    }
    return launch_attn(L, (hipStream_t)stream);
}

}  // extern "C"

// Device arithmetic of the ternary KV modes (tl1_fused, popcount_fused) of
// FusedKVCache (reference src/runtime/TenzoEngine.cpp: append :534-648, query
// codes :700-714 / :766-791, scores :720-760 / :793-804, values :852-885),
// shared by the chunk-attention kernel (attention_tern.hip) and the
// persistent decode kernel (decode_step.hip) so both compute the same bits.
//
// Cache rows are 32 bytes per (kv head, token), scales fp32 per row:
//   tl1_fused K and every V: byte i holds dims 4i..4i+3 as 2-bit fields
//     (w + 1) from bit 0, w in {-1, 0, +1} (a field 3 reads as 0, as the
//     reference's LUT_W0 / LUT_W1 decode it);
//   popcount_fused K: uint64 {kp0, kp1, kn0, kn1}, bit d of kp0 / kn0 set when
//     dim d is above / below the threshold, kp1 / kn1 for dims 64..127.
#pragma once

#include "common.h"

namespace tz {

constexpr int kTernRowW = 8;  // dwords per cache row
constexpr float kTernScale = 0.08838834764831845f;  // 1/sqrt(128)

// Sum over the 128 dims of x of |x_d| (masked: only the |x_d| > th) in the
// order the reference build evaluates its loops (-O3 -mavx2 -ffast-math,
// :544-561): eight partial sums over dims j, j+8, ..., j+120 in index order,
// then (l0+l4, l1+l5, l2+l6, l3+l7), (a0+a2, a1+a3), b0+b1 -- the xor
// butterfly over lanes 4, 2, 1 of lanes 0..7. Called by a whole wave; the
// result is returned in every lane. Adding 0 for a masked dim leaves a
// partial sum unchanged, as the build's masked vector add does.
__device__ __forceinline__ float tern_abs_sum(const float* x, int lane, bool masked, float th) {
    float l = 0.0f;
    if (lane < 8) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float a = fabsf(x[lane + 8 * i]);
            l += (!masked || a > th) ? a : 0.0f;
        }
    }
    l += __shfl_xor(l, 4, 64);
    l += __shfl_xor(l, 2, 64);
    l += __shfl_xor(l, 1, 64);
    return __shfl(l, 0, 64);
}

// Threshold and scale of a 128-dim row (:544-565).
__device__ __forceinline__ void tern_stats(const float* x, int lane, float* th_out, float* s_out) {
    const float mean = tern_abs_sum(x, lane, false, 0.0f) * (1.0f / 128.0f);
    const float th = 0.5f * mean;
    const float nz = tern_abs_sum(x, lane, true, th);
    const int cnt = __popcll(__ballot(fabsf(x[lane]) > th)) +
                    __popcll(__ballot(fabsf(x[lane + 64]) > th));
    *th_out = th;
    *s_out = cnt > 0 ? __fdiv_rn(nz, (float)cnt) : mean + 1e-6f;
}

__device__ __forceinline__ uint32_t tern_field(float v, float th) {
    return v > th ? 2u : (v < -th ? 0u : 1u);
}

// Dword w (dims 16w .. 16w+15) of a 2-bit row (:567-582).
__device__ __forceinline__ uint32_t tern_word(const float* x, int w, float th) {
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) r |= tern_field(x[16 * w + i], th) << (2 * i);
    return r;
}

// Dword w = lane % 8 of the row's sign bitplanes {kp0, kp1, kn0, kn1} (:622-633).
__device__ __forceinline__ uint32_t plane_word(const float* x, int lane, float th) {
    const uint64_t p0 = __ballot(x[lane] > th), p1 = __ballot(x[lane + 64] > th);
    const uint64_t n0 = __ballot(x[lane] < -th), n1 = __ballot(x[lane + 64] < -th);
    const int w = lane & 7;
    const uint64_t v = w < 2 ? p0 : (w < 4 ? p1 : (w < 6 ? n0 : n1));
    return (uint32_t)(w & 1 ? v >> 32 : v);
}

// A field 3 decodes as 0: clear bit 1 of every field whose bit 0 is set.
__device__ __forceinline__ uint32_t canon_fields(uint32_t w) { return w & ~((w & 0x55555555u) << 1); }

// Query codes of one head (a whole wave, q = the rotated head in LDS):
// MODE 1: int8 codes round(q * 127 / max|q|) (as built; s_q = max|q| / 127)
// into qw (dword 8f + w = dims 16w + 4j + f, byte j), their sum into *qsum;
// MODE 2: the query's bitplanes thresholded like a K row into qw[0..7].
// *qeff = s_q / sqrt(128) (lane 0 writes).
template <int MODE>
__device__ __forceinline__ void tern_query(const float* q, int lane, uint32_t* qw, int* qsum,
                                           float* qeff) {
    if (MODE == 1) {
        const float x0 = q[lane], x1 = q[lane + 64];
        const float mx = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
        const float s_q = mx > 0.0f ? __fmul_rn(mx, 1.0f / 127.0f) : 1.0f;
        const float inv = mx > 0.0f ? __fdiv_rn(127.0f, mx) : 1.0f;
        const int c0 = (int)roundf(__fmul_rn(x0, inv));
        const int c1 = (int)roundf(__fmul_rn(x1, inv));
        int8_t* qb = reinterpret_cast<int8_t*>(qw);
        const int d0 = lane, d1 = lane + 64;
        qb[4 * (8 * (d0 & 3) + (d0 >> 4)) + ((d0 & 15) >> 2)] = (int8_t)c0;
        qb[4 * (8 * (d1 & 3) + (d1 >> 4)) + ((d1 & 15) >> 2)] = (int8_t)c1;
        const int sum = wave_sum_i32(c0 + c1);
        if (lane == 0) {
            *qsum = sum;
            *qeff = __fmul_rn(s_q, kTernScale);
        }
    } else {
        float th, s;
        tern_stats(q, lane, &th, &s);
        const uint32_t w = plane_word(q, lane, th);
        if (lane < kTernRowW) qw[lane] = w;
        if (lane == 0) *qeff = __fmul_rn(s, kTernScale);
    }
}

// The appended row of the new token's k (kv 0) or v (kv 1) (a whole wave):
// dword lane of the row in lanes 0..7, the row's scale in *s (every lane).
template <int MODE>
__device__ __forceinline__ uint32_t tern_row(const float* x, int kv, int lane, float* s) {
    float th;
    tern_stats(x, lane, &th, s);
    uint32_t w = (MODE == 2 && kv == 0) ? plane_word(x, lane, th) : 0u;
    if (lane < kTernRowW && !(MODE == 2 && kv == 0)) w = tern_word(x, lane, th);
    return w;
}

// Score of one K row against the G query heads: float(dot) * (qeff * s_k).
// tl1: dot = sum_d q_d (field_d - 1) as v_dot4 on the fields masked in place;
// popcount: sign agreements minus disagreements.
template <int G, int MODE>
__device__ __forceinline__ void tern_scores(const uint32_t (&kr)[kTernRowW],
                                            const uint32_t (*qw)[32], const int* qsum,
                                            const float* qeff, float skf, float (&out)[G]) {
    if (MODE == 1) {
        uint32_t m0[kTernRowW], m1[kTernRowW], m2[kTernRowW], m3[kTernRowW];
#pragma unroll
        for (int w = 0; w < kTernRowW; ++w) {
            const uint32_t f = canon_fields(kr[w]);
            m0[w] = f & 0x03030303u;         // field 0 of each byte
            m1[w] = f & 0x0C0C0C0Cu;         // 4 x field 1
            m2[w] = f & 0x30303030u;         // 16 x field 2
            m3[w] = (f >> 2) & 0x30303030u;  // 16 x field 3
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int* Q = reinterpret_cast<const int*>(qw[g]);
            int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int w = 0; w < kTernRowW; ++w) {
                a0 = sdot4(m0[w], Q[w], a0);
                a1 = sdot4(m1[w], Q[8 + w], a1);
                a2 = sdot4(m2[w], Q[16 + w], a2);
                a2 = sdot4(m3[w], Q[24 + w], a2);
            }
            // sum_d q_d (field_d - 1): the scaled sums are exact multiples
            const int dot = a0 + (a1 >> 2) + (a2 >> 4) - qsum[g];
            out[g] = __fmul_rn((float)dot, __fmul_rn(qeff[g], skf));
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint32_t* Q = qw[g];
            int pm = 0, nm = 0;
#pragma unroll
            for (int i = 0; i < kTernRowW; ++i) {
                pm += __popc(Q[i] & kr[i]);
                nm += __popc(Q[i] & kr[i ^ 4]);
            }
            out[g] = __fmul_rn((float)(pm - nm), __fmul_rn(qeff[g], skf));
        }
    }
}

// The four values w - 1 of the 2-bit fields of byte b of a V row.
__device__ __forceinline__ void tern_value4(uint32_t b, float (&w)[4]) {
    const uint32_t f = canon_fields(b & 0xffu);
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = (float)((int)((f >> (2 * k)) & 3u) - 1);
}

}  // namespace tz

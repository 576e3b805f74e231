/*
 * tenzo_oracle.c - CPU restatement of Tenzo's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see tenzo_oracle.h for the pinning of each
 * function). Citations are file:line into the reference checkout,
 * src/runtime/TenzoEngine.cpp unless another file is named.
 *
 * Floating-point notes. The reference is built with -ffast-math
 * (CMakeLists.txt:43-45). Under it GCC rewrites a division by a constant into
 * a multiplication by the rounded reciprocal, so "amax / 31.0f" is evaluated as
 * amax * (1/31.0f); the compiled reference was checked to do exactly this. The
 * restatement writes those reciprocal multiplications out, so integer codes
 * derived from them are bit-exact with the reference as built. Likewise
 * "s = amax / 127; inv = 1 / s" is folded to s = amax * (1/127) and
 * inv = 127 / amax (one division), and 1/powf(theta, e) to
 * expf(-e * logf(theta)); both were read off the reference's x86 code as built
 * here and confirmed on exact rounding ties.
 */
#include "tenzo_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* fp16                                                                       */
/* ------------------------------------------------------------------------- */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalize */
            int e = -1;
            do { man <<= 1; ++e; } while (!(man & 0x400));
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000;
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t man = x & 0x7fffff;
    if (exp == 255) return (uint16_t)(sign | 0x7c00 | (man ? 0x200 : 0));
    int32_t e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t r = man >> shift;
        if (rem > half || (rem == half && (r & 1))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) ++r; /* may carry into exp: ok */
    return (uint16_t)(sign | r);
}

/* ------------------------------------------------------------------------- */
/* TL1 packing                                                                */
/* ------------------------------------------------------------------------- */

/* PybindModule.cpp:315-355: byte [b][k][c] = idx(row 64b+c) | idx(row 64b+32+c) << 4,
 * idx = (w0+1) | ((w1+1) << 2) for the column pair (2k, 2k+1). */
void orc_tl1_pack(const int8_t* tern, int64_t N, int64_t K, uint8_t* out) {
    int64_t nb = N / 64, kh = K / 2;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t k = 0; k < kh; ++k)
            for (int c = 0; c < 32; ++c) {
                const int8_t* lo = tern + (b * 64 + c) * K + 2 * k;
                const int8_t* hi = tern + (b * 64 + 32 + c) * K + 2 * k;
                unsigned il = (unsigned)((lo[0] + 1) | ((lo[1] + 1) << 2));
                unsigned ih = (unsigned)((hi[0] + 1) | ((hi[1] + 1) << 2));
                out[(b * kh + k) * 32 + c] = (uint8_t)((il & 15u) | ((ih & 15u) << 4));
            }
}

/* TenzoEngine.cpp:1842-1884 (get_tern at :1854-1859). */
void orc_tl1_pack_raw(const uint8_t* raw, int64_t N, int64_t K, uint8_t* out) {
    int64_t nb = N / 64, kh = K / 2;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t k = 0; k < kh; ++k)
            for (int c = 0; c < 32; ++c) {
                int w[4];
                int64_t rows[2] = {b * 64 + c, b * 64 + 32 + c};
                for (int h = 0; h < 2; ++h)
                    for (int j = 0; j < 2; ++j) {
                        int64_t r = rows[h], col = 2 * k + j;
                        uint8_t byte = raw[(r / 4) * K + col];
                        w[2 * h + j] = (int)((byte >> ((r % 4) * 2)) & 3) - 1;
                    }
                unsigned n0 = (unsigned)((w[0] + 1) | ((w[1] + 1) << 2));
                unsigned n1 = (unsigned)((w[2] + 1) | ((w[3] + 1) << 2));
                out[(b * kh + k) * 32 + c] = (uint8_t)((n0 & 15u) | ((n1 & 15u) << 4));
            }
}

void orc_tl1_unpack(const uint8_t* w, int64_t N, int64_t K, int8_t* tern) {
    int64_t nb = N / 64, kh = K / 2;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t k = 0; k < kh; ++k)
            for (int c = 0; c < 32; ++c) {
                uint8_t byte = w[(b * kh + k) * 32 + c];
                unsigned lo = byte & 15u, hi = byte >> 4;
                int8_t* rl = tern + (b * 64 + c) * K + 2 * k;
                int8_t* rh = tern + (b * 64 + 32 + c) * K + 2 * k;
                rl[0] = (int8_t)((int)(lo & 3u) - 1);
                rl[1] = (int8_t)((int)(lo >> 2) - 1);
                rh[0] = (int8_t)((int)(hi & 3u) - 1);
                rh[1] = (int8_t)((int)(hi >> 2) - 1);
            }
}

/* ------------------------------------------------------------------------- */
/* build_lut (:22-62)                                                         */
/* ------------------------------------------------------------------------- */

float orc_quant31(const float* x, int64_t K, int8_t* codes) {
    float max_abs = 1e-6f;                                   /* :28-32 */
    for (int64_t k = 0; k < K; ++k) {
        float v = fabsf(x[k]);
        if (v > max_abs) max_abs = v;
    }
    const float scale_act = 31.0f / max_abs;                 /* :34 */
    const float inv_scale_act = max_abs * (1.0f / 31.0f);    /* :35, as built */
    for (int64_t k = 0; k < K; ++k)                          /* :41-42 */
        codes[k] = (int8_t)(int16_t)roundf(x[k] * scale_act);
    return inv_scale_act;
}

void orc_build_lut(const int8_t* codes, int64_t K, int8_t* lut) {
    for (int64_t k = 0; k < K / 2; ++k) {                    /* :40-60 */
        int a0 = codes[2 * k], a1 = codes[2 * k + 1];
        int8_t* rec = lut + k * 32;
        memset(rec, 0, 32);
        for (int w0 = -1; w0 <= 1; ++w0)
            for (int w1 = -1; w1 <= 1; ++w1) {
                int idx = (w0 + 1) | ((w1 + 1) << 2);
                int s = w0 * a0 + w1 * a1;
                if (s < -128) s = -128;
                if (s > 127) s = 127;
                rec[idx] = (int8_t)s;
                rec[idx + 16] = (int8_t)s;
            }
    }
}

/* ------------------------------------------------------------------------- */
/* TL1 GEMV (:64-146)                                                         */
/* ------------------------------------------------------------------------- */

void orc_tl1_gemv_i32(const uint8_t* w, const int8_t* codes, int64_t N, int64_t K,
                      int32_t* acc) {
    int64_t nb = N / 64, kh = K / 2;
    int8_t* lut = (int8_t*)malloc((size_t)kh * 32);
    orc_build_lut(codes, K, lut);
    #pragma omp parallel for schedule(dynamic, 4)
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t* bw = w + b * kh * 32;
        int32_t a32[64];
        memset(a32, 0, sizeof(a32));
        int64_t k = 0;
        while (k < kh) {                                      /* :83-116 */
            int64_t chunk = kh - k < 64 ? kh - k : 64;
            int16_t a16[64];
            memset(a16, 0, sizeof(a16));
            for (int64_t c = 0; c < chunk; ++c, ++k) {
                const uint8_t* rec = bw + k * 32;
                const int8_t* l = lut + k * 32;
                for (int ch = 0; ch < 32; ++ch) {
                    a16[ch] = (int16_t)(a16[ch] + l[rec[ch] & 15]);
                    a16[32 + ch] = (int16_t)(a16[32 + ch] + l[rec[ch] >> 4]);
                }
            }
            for (int r = 0; r < 64; ++r) a32[r] += a16[r];
        }
        memcpy(acc + b * 64, a32, sizeof(a32));
    }
    free(lut);
}

float orc_tl1_gemv(const float* x, const uint8_t* w, int64_t N, int64_t K, float w_scale,
                   float* y, int32_t* acc) {
    int8_t* codes = (int8_t*)malloc((size_t)K);
    int32_t* a = acc ? acc : (int32_t*)malloc((size_t)N * 4);
    float inv = orc_quant31(x, K, codes);
    orc_tl1_gemv_i32(w, codes, N, K, a);
    float total = inv * w_scale;                              /* :1554, :1586 */
    for (int64_t n = 0; n < N; ++n) y[n] = (float)a[n] * total;   /* :118-126 */
    if (!acc) free(a);
    free(codes);
    return inv;
}

/* ------------------------------------------------------------------------- */
/* RMSNorm (:148-166)                                                         */
/* ------------------------------------------------------------------------- */

/* The reference build (-O3 -mavx2 -mfma -ffast-math) vectorises rms_norm_raw's
 * "omp simd reduction(+:sum_sq)" loop into one 8-lane accumulator: lane j is an
 * FMA chain over x[j], x[j+8], ... in index order; the n % 8 tail elements are
 * then added to lane 0 one at a time, and the lanes are summed as
 * ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) (vextractf128 / vmovhlps / vshufps). */
float orc_sumsq(const float* x, int64_t n) {
    float l[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    const int64_t n8 = n / 8 * 8;
    for (int64_t i = 0; i < n8; i += 8)
        for (int j = 0; j < 8; ++j) l[j] = fmaf(x[i + j], x[i + j], l[j]);
    for (int64_t i = n8; i < n; ++i) l[0] = fmaf(x[i], x[i], l[0]);
    return ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
}

/* x86 RSQRTSS of the host the reference was built and its goldens written on:
 * indexed by the exponent's parity and the top 10 mantissa bits (a in [0.5, 2)),
 * the estimate's exponent moving by half the input's (gen_rsqrt_est.c). */
static const uint32_t kRsqrtEst[2048] = {
#include "rsqrt_est_table.inc"
};

float orc_rsqrt_est(float a) {
    uint32_t b;
    memcpy(&b, &a, 4);
    const int32_t e = (int32_t)(b >> 23), odd = e & 1, e0 = odd ? 127 : 126;
    const uint32_t t = kRsqrtEst[odd * 1024 + ((b >> 13) & 1023u)];
    const uint32_t r = (uint32_t)((int32_t)t - ((e - e0) / 2) * (1 << 23));
    float f;
    memcpy(&f, &r, 4);
    return f;
}

/* inv_rms of :154 as built: 1/std::sqrt(a) becomes the estimate y0 = rsqrtss(a)
 * and one Newton step, evaluated as (y0 * -0.5f) * fmaf(a * y0, y0, -3.0f); the
 * mean is a true division (vdivss). */
float orc_inv_rms(float ss, int64_t dim, float eps) {
    const float a = ss / (float)dim + eps;
    const float y0 = orc_rsqrt_est(a);
    return (y0 * -0.5f) * fmaf(a * y0, y0, -3.0f);
}

/* :155-165 as built: the weighted product is reassociated to (x * w) * inv_rms. */
void orc_rms_norm(const float* x, const float* w, float* y, int64_t dim, float eps) {
    const float inv_rms = orc_inv_rms(orc_sumsq(x, dim), dim, eps);
    for (int64_t i = 0; i < dim; ++i) y[i] = w ? (x[i] * w[i]) * inv_rms : x[i] * inv_rms;
}

/* ------------------------------------------------------------------------- */
/* INT8 KV cache + attention (:447-919)                                       */
/* ------------------------------------------------------------------------- */

float orc_kv_quant(const float* x, int d, int8_t* codes) {
    float amax = 1e-8f;                                       /* :516-520 */
    for (int i = 0; i < d; ++i) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float s = amax * (1.0f / 127.0f);                         /* :521, as built */
    float inv = 127.0f / amax;                                /* :526: 1/s folded as built */
    for (int i = 0; i < d; ++i) {                             /* :528-531 */
        float r = roundf(x[i] * inv);
        if (r < -128.0f) r = -128.0f;
        if (r > 127.0f) r = 127.0f;
        codes[i] = (int8_t)r;
    }
    return s;
}

void orc_rope_table(float theta, int head_dim, int pos, float* cs) {
    /* :465-469 as built: under -ffast-math GCC turns 1/powf(theta, e) into
     * expf(-e * logf(theta)); cos/sin are glibc cosf/sinf of the fp32 angle.
     * Checked against the compiled reference for all 64 frequencies. */
    int half = head_dim / 2;
    const float ln_theta = logf(theta);
    for (int i = 0; i < half; ++i) {
        float e = (float)(2 * i) / (float)head_dim;
        float freq = expf(-e * ln_theta);
        float angle = (float)pos * freq;
        cs[i] = cosf(angle);
        cs[half + i] = sinf(angle);
    }
}

void orc_rope_apply(float* x, int nheads, int head_dim, const float* cs) {
    int half = head_dim / 2;
    for (int h = 0; h < nheads; ++h) {                        /* :472-477 */
        float* v = x + h * head_dim;
        for (int i = 0; i < half; ++i) {
            float x0 = v[i], x1 = v[i + half], c = cs[i], s = cs[half + i];
            v[i] = fmaf(x0, c, -(x1 * s));
            v[i + half] = fmaf(x0, s, x1 * c);
        }
    }
}

void orc_attn_int8(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                   const float* vs, int Hq, int Hkv, int max_seq, int seq_len,
                   float* out) {
    const int D = 128;
    const int gqa = Hq / Hkv;                                 /* :659 */
    const float scale_factor = 1.0f / sqrtf((float)D);        /* :660 */
    if (seq_len <= 0 || Hkv <= 0) return;
    float* scores = (float*)malloc((size_t)seq_len * 4);
    for (int qh = 0; qh < Hq; ++qh) {
        int kvh = qh / gqa;
        const float* qv = q + qh * D;
        const int8_t* kb = kc + (size_t)kvh * max_seq * D;
        const int8_t* vb = vc + (size_t)kvh * max_seq * D;
        const float* ksb = ks + (size_t)kvh * max_seq;
        const float* vsb = vs + (size_t)kvh * max_seq;
        float max_score = -1e30f;
        for (int t = 0; t < seq_len; ++t) {                   /* :678-694 */
            float lane[8] = {0};
            for (int d = 0; d < D; d += 8)
                for (int j = 0; j < 8; ++j)
                    lane[j] = fmaf(qv[d + j], (float)kb[(size_t)t * D + d + j], lane[j]);
            float dot = lane[0];
            for (int j = 1; j < 8; ++j) dot += lane[j];
            dot = dot * (ksb[t] * scale_factor);
            scores[t] = dot;
            if (dot > max_score) max_score = dot;
        }
        float sum = 0.0f;                                     /* :824-830 */
        for (int t = 0; t < seq_len; ++t) {
            scores[t] = expf(scores[t] - max_score);
            sum += scores[t];
        }
        float inv_sum = 1.0f / sum;
        for (int t = 0; t < seq_len; ++t) scores[t] *= inv_sum;
        float acc[128] = {0};                                 /* :842-851 */
        for (int t = 0; t < seq_len; ++t) {
            float wsc = scores[t] * vsb[t];
            for (int d = 0; d < D; ++d)
                acc[d] = fmaf((float)vb[(size_t)t * D + d], wsc, acc[d]);
        }
        memcpy(out + qh * D, acc, sizeof(acc));               /* :911-913 */
    }
    free(scores);
}

void orc_attention_step(float* q, float* k, const float* v, int8_t* kc, int8_t* vc,
                        float* ks, float* vs, int Hq, int Hkv, int max_seq, int pos,
                        const float* rope_cs, int f16_scales, float* out) {
    const int D = 128;
    orc_rope_apply(q, Hq, D, rope_cs);                        /* :458-481 */
    orc_rope_apply(k, Hkv, D, rope_cs);                       /* :482-504 */
    for (int h = 0; h < Hkv; ++h) {                           /* :507-533 */
        size_t off = ((size_t)h * max_seq + pos) * D;
        size_t soff = (size_t)h * max_seq + pos;
        float sk = orc_kv_quant(k + h * D, D, kc + off);
        float sv = orc_kv_quant(v + h * D, D, vc + off);
        if (f16_scales) {
            sk = orc_f16_to_f32(orc_f32_to_f16(sk));
            sv = orc_f16_to_f32(orc_f32_to_f16(sv));
        }
        ks[soff] = sk;
        vs[soff] = sv;
    }
    orc_attn_int8(q, kc, vc, ks, vs, Hq, Hkv, max_seq, pos + 1, out);
}

/* ------------------------------------------------------------------------- */
/* Ternary KV modes: tl1_fused (2-bit K and V, :534-587 append, :695-763 and  */
/* :852-885 attention) and popcount_fused (K as sign bitplanes, 2-bit V,       */
/* :588-648 append, :764-805 and :852-885 attention). Cache rows are 32 bytes  */
/* per (kv head, token): tl1 K / every V byte i holds dims 4i..4i+3 as 2-bit   */
/* fields (w + 1) from bit 0; popcount K is uint64 {kp0, kp1, kn0, kn1} (bit d */
/* of kp0 / kn0: dim d > th / < -th; kp1 / kn1: dims 64..127). Scales fp32.    */
/* ------------------------------------------------------------------------- */

/* Sum of |x[i]| (over the i with |x[i]| > th when masked) in the order the
 * reference build evaluates it (-O3 -mavx2 -ffast-math): eight lanes i mod 8,
 * each summed in index order, then ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)). */
static float tern_abs_sum(const float* x, int d, int masked, float th, int* cnt) {
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int c = 0;
    for (int i = 0; i < d; ++i) {
        const float a = fabsf(x[i]);
        if (!masked || a > th) {
            l[i & 7] += a;
            ++c;
        }
    }
    if (cnt) *cnt = c;
    const float a0 = l[0] + l[4], a1 = l[1] + l[5], a2 = l[2] + l[6], a3 = l[3] + l[7];
    return (a0 + a2) + (a1 + a3);
}

/* :544-565: mean |x|, threshold 0.5 mean, scale = mean of the |x| above it
 * (mean + 1e-6 when none is). */
void orc_tern_stats(const float* x, int d, float* th, float* s) {
    const float mean = tern_abs_sum(x, d, 0, 0.0f, NULL) / (float)d;
    const float t = 0.5f * mean;
    int cnt = 0;
    const float nz = tern_abs_sum(x, d, 1, t, &cnt);
    *th = t;
    *s = cnt > 0 ? nz / (float)cnt : mean + 1e-6f;
}

static int tern_code(float v, float th) { return v > th ? 1 : (v < -th ? -1 : 0); }

/* :567-582: four dims per byte, field (w + 1) at bit 2j for dim 4i + j. */
void orc_tern_pack(const float* x, int d, float th, uint8_t* out) {
    for (int i = 0; i < d; i += 4) {
        unsigned b = 0;
        for (int j = 0; j < 4; ++j) b |= (unsigned)(tern_code(x[i + j], th) + 1) << (2 * j);
        out[i / 4] = (uint8_t)b;
    }
}

/* :622-633: {kp0, kp1, kn0, kn1} for a 128-dim row. */
void orc_tern_bitplanes(const float* x, float th, uint64_t* out) {
    uint64_t p0 = 0, p1 = 0, n0 = 0, n1 = 0;
    for (int i = 0; i < 64; ++i) {
        if (x[i] > th) p0 |= 1ull << i;
        else if (x[i] < -th) n0 |= 1ull << i;
        if (x[64 + i] > th) p1 |= 1ull << i;
        else if (x[64 + i] < -th) n1 |= 1ull << i;
    }
    out[0] = p0; out[1] = p1; out[2] = n0; out[3] = n1;
}

/* The 2-bit field decode of the reference's LUT_W0 / LUT_W1 (:697-698):
 * 0 -> -1, 1 -> 0, 2 -> +1, 3 -> 0. */
static int tern_field(unsigned f) { return f == 3 ? 0 : (int)f - 1; }

void orc_attn_tern(int mode, const float* q, const uint8_t* kb, const uint8_t* vb,
                   const float* ks, const float* vs, int Hq, int Hkv, int max_seq,
                   int seq_len, float* out) {
    const int D = 128;
    const int gqa = Hq / Hkv;                                 /* :659 */
    const float scale_factor = 1.0f / sqrtf((float)D);        /* :660 */
    if (seq_len <= 0 || Hkv <= 0) return;
    float* scores = (float*)malloc((size_t)seq_len * 4);
    for (int qh = 0; qh < Hq; ++qh) {
        const int kvh = qh / gqa;
        const float* qv = q + qh * D;
        const uint8_t* kbase = kb + (size_t)kvh * max_seq * 32;
        const uint8_t* vbase = vb + (size_t)kvh * max_seq * 32;
        const float* ksb = ks + (size_t)kvh * max_seq;
        const float* vsb = vs + (size_t)kvh * max_seq;
        float max_score = -1e30f;
        if (mode == 1) {
            /* :700-714 as built: s_q = max|q| * (1/127) (1 when q = 0), codes
             * round(q * (127 / max|q|)) (1/s_q re-associated) */
            float max_q = 0.0f;
            for (int d = 0; d < D; ++d) max_q = fmaxf(max_q, fabsf(qv[d]));
            const float s_q = max_q > 0.0f ? max_q * (1.0f / 127.0f) : 1.0f;
            const float inv = max_q > 0.0f ? 127.0f / max_q : 1.0f;
            int qi[128];
            for (int d = 0; d < D; ++d) qi[d] = (int)roundf(qv[d] * inv);
            const float q_eff = s_q * scale_factor;
            for (int t = 0; t < seq_len; ++t) {               /* :720-760 */
                const uint8_t* kr = kbase + (size_t)t * 32;
                int32_t isum = 0;
                for (int d = 0; d < D; ++d)
                    isum += qi[d] * tern_field((kr[d / 4] >> (2 * (d % 4))) & 3u);
                const float dot = (float)isum * (q_eff * ksb[t]);
                scores[t] = dot;
                if (dot > max_score) max_score = dot;
            }
        } else {
            /* :766-791: q's own threshold, scale and bitplanes */
            float th_q, s_q;
            orc_tern_stats(qv, D, &th_q, &s_q);
            uint64_t qp[4];
            orc_tern_bitplanes(qv, th_q, qp);
            const float q_eff = s_q * scale_factor;
            for (int t = 0; t < seq_len; ++t) {               /* :793-804 */
                uint64_t kp[4];
                memcpy(kp, kbase + (size_t)t * 32, 32);
                const int pm = __builtin_popcountll(qp[0] & kp[0]) + __builtin_popcountll(qp[1] & kp[1]) +
                               __builtin_popcountll(qp[2] & kp[2]) + __builtin_popcountll(qp[3] & kp[3]);
                const int nm = __builtin_popcountll(qp[0] & kp[2]) + __builtin_popcountll(qp[1] & kp[3]) +
                               __builtin_popcountll(qp[2] & kp[0]) + __builtin_popcountll(qp[3] & kp[1]);
                const float dot = (float)(pm - nm) * (q_eff * ksb[t]);
                scores[t] = dot;
                if (dot > max_score) max_score = dot;
            }
        }
        float sum = 0.0f;                                     /* :824-830 */
        for (int t = 0; t < seq_len; ++t) {
            scores[t] = expf(scores[t] - max_score);
            sum += scores[t];
        }
        const float inv_sum = 1.0f / sum;
        for (int t = 0; t < seq_len; ++t) scores[t] *= inv_sum;
        float acc[128] = {0};                                 /* :852-885 */
        for (int t = 0; t < seq_len; ++t) {
            const uint8_t* vr = vbase + (size_t)t * 32;
            const float wsc = scores[t] * vsb[t];
            for (int d = 0; d < D; ++d)
                acc[d] = fmaf((float)tern_field((vr[d / 4] >> (2 * (d % 4))) & 3u), wsc, acc[d]);
        }
        memcpy(out + qh * D, acc, sizeof(acc));
    }
    free(scores);
}

void orc_attention_step_tern(int mode, float* q, float* k, const float* v, uint8_t* kb,
                             uint8_t* vb, float* ks, float* vs, int Hq, int Hkv, int max_seq,
                             int pos, const float* rope_cs, float* out) {
    const int D = 128;
    orc_rope_apply(q, Hq, D, rope_cs);                        /* :458-481 */
    orc_rope_apply(k, Hkv, D, rope_cs);                       /* :482-504 */
    for (int h = 0; h < Hkv; ++h) {                           /* :534-648 */
        const size_t row = (size_t)h * max_seq + pos;
        float th_k, s_k, th_v, s_v;
        orc_tern_stats(k + h * D, D, &th_k, &s_k);
        orc_tern_stats(v + h * D, D, &th_v, &s_v);
        ks[row] = s_k;
        vs[row] = s_v;
        if (mode == 1) {
            orc_tern_pack(k + h * D, D, th_k, kb + row * 32);
        } else {
            uint64_t planes[4];
            orc_tern_bitplanes(k + h * D, th_k, planes);
            memcpy(kb + row * 32, planes, 32);
        }
        orc_tern_pack(v + h * D, D, th_v, vb + row * 32);
    }
    orc_attn_tern(mode, q, kb, vb, ks, vs, Hq, Hkv, max_seq, pos + 1, out);
}

/* ------------------------------------------------------------------------- */
/* paged_int8 (PagedKVCache, :218-445): pools [blocks][L][Hkv][16][128] int8,  */
/* fp32 scales [blocks][L][Hkv][16], a block table per sequence.               */
/* ------------------------------------------------------------------------- */

static size_t paged_row(int blk, int n_layers, int layer, int Hkv, int h) {
    return ((size_t)blk * n_layers + layer) * Hkv + h;  /* then x 16 slots */
}

void orc_attention_step_paged(float* q, float* k, const float* v, int8_t* pk, int8_t* pv,
                              float* pks, float* pvs, const int32_t* block_table, int n_layers,
                              int layer, int Hq, int Hkv, int pos, const float* rope_cs,
                              float* out) {
    const int D = 128, BS = 16;
    orc_rope_apply(q, Hq, D, rope_cs);                        /* :271-292 */
    orc_rope_apply(k, Hkv, D, rope_cs);                       /* :294-315 */
    const int lb = pos / BS, slot = pos % BS;                 /* :318-326 */
    const int phys = block_table[lb];
    for (int h = 0; h < Hkv; ++h) {                           /* :328-352: the int8_fused quantizer */
        const size_t r = paged_row(phys, n_layers, layer, Hkv, h) * BS + slot;
        pks[r] = orc_kv_quant(k + h * D, D, pk + r * D);
        pvs[r] = orc_kv_quant(v + h * D, D, pv + r * D);
    }
    const int total = pos + 1;                                /* :355-445 */
    const int gqa = Hq / Hkv;
    const float qk_scale = 1.0f / sqrtf((float)D);
    float* scores = (float*)malloc((size_t)total * 4);
    for (int qh = 0; qh < Hq; ++qh) {
        const int kvh = qh / gqa;
        const float* qv = q + qh * D;
        float max_score = -1e30f;
        for (int t = 0; t < total; ++t) {                     /* :366-393 */
            const size_t r = paged_row(block_table[t / BS], n_layers, layer, Hkv, kvh) * BS + t % BS;
            const int8_t* kr = pk + r * D;
            float a0[8] = {0}, a1[8] = {0};
            for (int d = 0; d < D; d += 16)
                for (int j = 0; j < 8; ++j) {
                    a0[j] = fmaf(qv[d + j], (float)kr[d + j], a0[j]);
                    a1[j] = fmaf(qv[d + 8 + j], (float)kr[d + 8 + j], a1[j]);
                }
            float dot = 0.0f;
            for (int j = 0; j < 8; ++j) dot += a0[j] + a1[j];
            const float score = dot * pks[r] * qk_scale;
            scores[t] = score;
            if (score > max_score) max_score = score;
        }
        float sum = 0.0f;                                     /* :396-405 */
        for (int t = 0; t < total; ++t) {
            scores[t] = expf(scores[t] - max_score);
            sum += scores[t];
        }
        const float inv_sum = 1.0f / (sum + 1e-8f);
        for (int t = 0; t < total; ++t) scores[t] *= inv_sum;
        float* o = out + qh * D;                              /* :408-443 */
        memset(o, 0, D * sizeof(float));
        for (int t = 0; t < total; ++t) {
            const float alpha = scores[t];
            if (alpha < 1e-7f) continue;
            const size_t r = paged_row(block_table[t / BS], n_layers, layer, Hkv, kvh) * BS + t % BS;
            const float w = alpha * pvs[r];
            for (int d = 0; d < D; ++d) o[d] = fmaf(w, (float)pv[r * D + d], o[d]);
        }
    }
    free(scores);
}

/* ------------------------------------------------------------------------- */
/* LM head (:1634-1720), argmax (:1745-1755), embedding (:1294-1316)          */
/* ------------------------------------------------------------------------- */

float orc_lm_head(const float* xn, const int8_t* W, const float* scales, int64_t V,
                  int64_t H, float* logits, int8_t* codes_out) {
    float amax = 1e-8f;                                       /* :1666-1670 */
    for (int64_t i = 0; i < H; ++i) {
        float a = fabsf(xn[i]);
        if (a > amax) amax = a;
    }
    float s_x = amax * (1.0f / 127.0f);                       /* :1671, as built */
    float inv = 127.0f / amax;                                /* :1672: 1/s_x folded as built */
    int8_t* c = codes_out ? codes_out : (int8_t*)malloc((size_t)H);
    for (int64_t i = 0; i < H; ++i) {                         /* :1674-1678 */
        float r = roundf(xn[i] * inv);
        if (r < -128.0f) r = -128.0f;
        if (r > 127.0f) r = 127.0f;
        c[i] = (int8_t)r;
    }
    #pragma omp parallel for schedule(static)
    for (int64_t v = 0; v < V; ++v) {                         /* :1689-1718 */
        const int8_t* row = W + v * H;
        int32_t s = 0;
        for (int64_t i = 0; i < H; ++i) s += (int32_t)c[i] * (int32_t)row[i];
        logits[v] = (float)s * (s_x * scales[v]);
    }
    if (!codes_out) free(c);
    return s_x;
}

int orc_argmax(const float* logits, int64_t V) {
    int64_t best = 0;
    float bv = logits[0];
    for (int64_t i = 1; i < V; ++i)
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    return (int)best;
}

/* The loader's LM-head quantization (:1925-1941) as the reference is built
 * (-ffast-math): per row amax (floor 1e-8), stored scale = amax * (1/127) (the
 * divide by the constant folded into a multiply), codes = clamp(round(x *
 * (127 / amax)), -127, 127) (1 / (amax * (1/127)) re-associated to 127 /
 * amax; x * (1 / scale) differs at exact .5 ties). */
void orc_quant_rows_i8(const float* E, int64_t V, int64_t H, int8_t* codes, float* scales) {
    for (int64_t v = 0; v < V; ++v) {
        const float* row = E + v * H;
        float amax = 1e-8f;
        for (int64_t i = 0; i < H; ++i) amax = fmaxf(amax, fabsf(row[i]));
        const float scale = amax * (1.0f / 127.0f);
        scales[v] = scale;
        const float inv_s = 127.0f / amax;
        for (int64_t i = 0; i < H; ++i) {
            float c = roundf(row[i] * inv_s);
            c = c < -127.0f ? -127.0f : (c > 127.0f ? 127.0f : c);
            codes[v * H + i] = (int8_t)c;
        }
    }
}

/* The repetition penalty of sample_top_k_top_p (:1735-1743): applied in place,
 * once per occurrence, only when penalty != 1. As built (-ffast-math) the
 * division is hoisted: inv = 1 / penalty once, positive logits times inv,
 * the others times penalty. */
void orc_rep_penalty(float* logits, int64_t V, const int32_t* tokens, int n, float penalty) {
    if (penalty == 1.0f || !tokens || n <= 0) return;
    const float inv = 1.0f / penalty;
    for (int k = 0; k < n; ++k) {
        const int32_t t = tokens[k];
        if (t >= 0 && t < V) {
            const float l = logits[t];
            logits[t] = l > 0.0f ? l * inv : l * penalty;
        }
    }
}

/* sample_top_k_top_p (:1722-1807) for temperature > 0 after the penalty, with
 * the uniform draw r passed in (the reference draws rand()/RAND_MAX there).
 * Top-k by the reference's min-heap rule: the first k logits enter; a later
 * logit replaces the heap's least (value, index) pair only when its value is
 * strictly greater. Candidates then run in descending (value, index) order. */
static int orc_pair_less(float a, int ia, float b, int ib) {
    return a < b || (a == b && ia < ib);
}

int orc_sample_top_k_top_p(const float* logits, int64_t V, int top_k, float top_p,
                           float temperature, float r) {
    int k = top_k < 1 ? 1 : (top_k > 64 ? 64 : top_k);
    float hv[64];
    int hi[64];
    int n = 0;
    for (int64_t i = 0; i < V; ++i) {                          /* :1759-1767 */
        const float l = logits[i];
        if (n < k) {
            hv[n] = l;
            hi[n] = (int)i;
            ++n;
            continue;
        }
        int m = 0;                                             /* heap top: least pair */
        for (int j = 1; j < n; ++j)
            if (orc_pair_less(hv[j], hi[j], hv[m], hi[m])) m = j;
        if (l > hv[m]) {
            hv[m] = l;
            hi[m] = (int)i;
        }
    }
    /* descending (value, index): the heap popped least-first into candidates[n-1..0] */
    for (int a = 0; a < n; ++a)
        for (int b = a + 1; b < n; ++b)
            if (orc_pair_less(hv[a], hi[a], hv[b], hi[b])) {
                float tv = hv[a]; hv[a] = hv[b]; hv[b] = tv;
                int ti = hi[a]; hi[a] = hi[b]; hi[b] = ti;
            }
    float probs[64];
    const float max_l = hv[0];
    float sum_exp = 0.0f;
    for (int i = 0; i < n; ++i) {                              /* :1776-1782 */
        probs[i] = expf((hv[i] - max_l) / temperature);
        sum_exp += probs[i];
    }
    for (int i = 0; i < n; ++i) probs[i] /= sum_exp;
    float cum_p = 0.0f;
    int cutoff = n;
    for (int i = 0; i < n; ++i) {                              /* :1784-1792 */
        cum_p += probs[i];
        if (cum_p >= top_p) {
            cutoff = i + 1;
            break;
        }
    }
    float sub_sum = 0.0f;
    for (int i = 0; i < cutoff; ++i) sub_sum += probs[i];
    for (int i = 0; i < cutoff; ++i) probs[i] /= sub_sum;
    float acc = 0.0f;
    for (int i = 0; i < cutoff; ++i) {                         /* :1798-1804 */
        acc += probs[i];
        if (r <= acc) return hi[i];
    }
    return hi[0];
}

void orc_embed_i8(const int8_t* E, const float* scales, int64_t H, int token, float* x) {
    const int8_t* row = E + (int64_t)token * H;
    float s = scales[token];
    for (int64_t i = 0; i < H; ++i) x[i] = (float)row[i] * s;
}

/* ------------------------------------------------------------------------- */
/* Quantized GEMVs (:1022-1175)                                               */
/* ------------------------------------------------------------------------- */

/* tmp[0] + ... + tmp[7] of the reference's Q4_0 / Q8_0 loops (:1072, :1112) as
 * its build evaluates it (-O3 -ffast-math; the generated code of
 * oracle/_ref): adjacent pairs, then the pairs of pairs. */
static float orc_lanes8_sum(const float* t) {
    return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

/* :1022-1075. Eight fp32 lanes: lane j takes block elements j, 8+j, 16+j, 24+j;
 * elements 0..15 are the low nibbles of qs[0..15], 16..31 the high nibbles. */
void orc_q4_0(const float* a, const uint8_t* w, float* y, int K, int N) {
    int nbk = K / 32;
    #pragma omp parallel for schedule(dynamic, 8)
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = w + (size_t)n * nbk * 18;
        float acc[8] = {0};
        for (int b = 0; b < nbk; ++b) {
            const uint8_t* blk = row + b * 18;
            float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            const uint8_t* qs = blk + 2;
            const float* ab = a + b * 32;
            for (int j = 0; j < 8; ++j) {
                float w0 = (float)((int)(qs[j] & 15) - 8);
                float w1 = (float)((int)(qs[8 + j] & 15) - 8);
                float w2 = (float)((int)(qs[j] >> 4) - 8);
                float w3 = (float)((int)(qs[8 + j] >> 4) - 8);
                float bd = ab[j] * w0;
                bd = fmaf(ab[8 + j], w1, bd);
                bd = fmaf(ab[16 + j], w2, bd);
                bd = fmaf(ab[24 + j], w3, bd);
                acc[j] = fmaf(bd, d, acc[j]);
            }
        }
        y[n] = orc_lanes8_sum(acc);
    }
}

/* :1078-1114 */
void orc_q8_0(const float* a, const uint8_t* w, float* y, int K, int N) {
    int nbk = K / 32;
    #pragma omp parallel for schedule(dynamic, 8)
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = w + (size_t)n * nbk * 34;
        float acc[8] = {0};
        for (int b = 0; b < nbk; ++b) {
            const uint8_t* blk = row + b * 34;
            float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            const int8_t* qs = (const int8_t*)(blk + 2);
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 8; ++j)
                    acc[j] = fmaf(a[b * 32 + i * 8 + j] * (float)qs[i * 8 + j], d, acc[j]);
        }
        y[n] = orc_lanes8_sum(acc);
    }
}

/* :1117-1143. qzeros packed along groups: word (g/8)*N + n, nibble g%8, plus one. */
void orc_gptq(const float* a, const uint32_t* qweight, const float* scales,
              const uint32_t* qzeros, float* y, int K, int N, int group) {
    #pragma omp parallel for schedule(dynamic, 8)
    for (int n = 0; n < N; ++n) {
        float total = 0.0f;
        for (int k = 0; k < K; k += 8) {
            int g = k / group;
            float s = scales[(size_t)g * N + n];
            uint32_t zp = qzeros[(size_t)(g / 8) * N + n];
            int z = (int)((zp >> ((g % 8) * 4)) & 15u) + 1;
            uint32_t qw = qweight[(size_t)(k / 8) * N + n];
            for (int e = 0; e < 8; ++e) {
                int q = (int)((qw >> (e * 4)) & 15u);
                float wd = (float)(q - z) * s;
                total = fmaf(a[k + e], wd, total);
            }
        }
        y[n] = total;
    }
}

/* :1146-1175. Nibble e of qweight[(k/8)*N+n] holds element k + order[e];
 * qzeros packed along N: word g*(N/8) + n/8, nibble n%8, no offset. */
void orc_awq(const float* a, const uint32_t* qweight, const float* scales,
             const uint32_t* qzeros, float* y, int K, int N, int group) {
    static const int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    #pragma omp parallel for schedule(dynamic, 8)
    for (int n = 0; n < N; ++n) {
        float total = 0.0f;
        for (int k = 0; k < K; k += 8) {
            int g = k / group;
            float s = scales[(size_t)g * N + n];
            uint32_t zp = qzeros[(size_t)g * (N / 8) + n / 8];
            int z = (int)((zp >> ((n % 8) * 4)) & 15u);
            uint32_t qw = qweight[(size_t)(k / 8) * N + n];
            for (int e = 0; e < 8; ++e) {
                int q = (int)((qw >> (e * 4)) & 15u);
                float wd = (float)(q - z) * s;
                total = fmaf(a[k + order[e]], wd, total);
            }
        }
        y[n] = total;
    }
}

/* llama.cpp quantize_row_q8_0 (ggml-quants.c): d = amax/127, q = round(x/d). */
void orc_quantize_q8_0(const float* x, int K, uint8_t* out) {
    for (int b = 0; b < K / 32; ++b) {
        const float* xb = x + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float v = fabsf(xb[j]);
            if (v > amax) amax = v;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = orc_f32_to_f16(d);
        uint8_t* blk = out + b * 34;
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
    }
}

/* y_n = sum_b fp16(d_w) * fp16(d_a) * sum_j (q_j - 8) * qa_j; the int32 block
 * dot is exact, the block scale product and the running sum are fp32. */
void orc_q4_0_q8act(const uint8_t* qa, const uint8_t* w, float* y, int K, int N) {
    int nbk = K / 32;
    #pragma omp parallel for schedule(dynamic, 8)
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = w + (size_t)n * nbk * 18;
        float total = 0.0f;
        for (int b = 0; b < nbk; ++b) {
            const uint8_t* blk = row + b * 18;
            const uint8_t* ab = qa + b * 34;
            float dw = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            float da = orc_f16_to_f32((uint16_t)(ab[0] | (ab[1] << 8)));
            const int8_t* q8 = (const int8_t*)(ab + 2);
            int32_t s = 0;
            for (int j = 0; j < 16; ++j) {
                s += ((int)(blk[2 + j] & 15) - 8) * q8[j];
                s += ((int)(blk[2 + j] >> 4) - 8) * q8[16 + j];
            }
            total = fmaf((float)s, dw * da, total);
        }
        y[n] = total;
    }
}

/* ------------------------------------------------------------------------- */
/* Whole decode step (:1522-1632, :1634-1838)                                 */
/* ------------------------------------------------------------------------- */

int orc_decode_step(const orc_model_t* m, int token, int pos, const float* rope_cs,
                    float* logits, float* hidden) {
    const int H = m->hidden, F = m->ffn, D = 128;
    const int qd = m->n_q_heads * D, kvd = m->n_kv_heads * D;
    const float eps = m->eps;
    float* x = (float*)malloc((size_t)H * 4);
    float* nx = (float*)malloc((size_t)(F > H ? F : H) * 4);
    float* q = (float*)malloc((size_t)qd * 4);
    float* k = (float*)malloc((size_t)kvd * 4);
    float* v = (float*)malloc((size_t)kvd * 4);
    float* attn = (float*)malloc((size_t)qd * 4);
    float* o = (float*)malloc((size_t)H * 4);
    float* h1 = (float*)malloc((size_t)H * 4);
    float* g = (float*)malloc((size_t)F * 4);
    float* u = (float*)malloc((size_t)F * 4);
    float* act = (float*)malloc((size_t)F * 4);
    float* dn = (float*)malloc((size_t)H * 4);
    int8_t* codes = (int8_t*)malloc((size_t)(F > H ? F : H));
    int32_t* acc = (int32_t*)malloc((size_t)(2 * F + qd + 2 * kvd) * 4);

    orc_embed_i8(m->embed, m->embed_scales, H, token, x);     /* :1827 */
    for (int l = 0; l < m->n_layers; ++l) {
        const float* sc = m->scales + l * 7;
        size_t cache_off = (size_t)l * m->n_kv_heads * m->max_seq;
        /* :1542-1572 */
        orc_rms_norm(x, m->in_norm[l], nx, H, eps);
        float inv = orc_quant31(nx, H, codes);
        orc_tl1_gemv_i32(m->q_w[l], codes, qd, H, acc);
        for (int i = 0; i < qd; ++i) q[i] = (float)acc[i] * (inv * sc[0]);
        orc_tl1_gemv_i32(m->k_w[l], codes, kvd, H, acc);
        for (int i = 0; i < kvd; ++i) k[i] = (float)acc[i] * (inv * sc[1]);
        orc_tl1_gemv_i32(m->v_w[l], codes, kvd, H, acc);
        for (int i = 0; i < kvd; ++i) v[i] = (float)acc[i] * (inv * sc[2]);
        /* :1578 */
        if (m->kv_mode == 3)
            orc_attention_step_paged(q, k, v, m->kc, m->vc, m->ks, m->vs, m->block_table,
                                     m->n_layers, l, m->n_q_heads, m->n_kv_heads, pos, rope_cs,
                                     attn);
        else if (m->kv_mode == 0)
            orc_attention_step(q, k, v, m->kc + cache_off * D, m->vc + cache_off * D,
                               m->ks + cache_off, m->vs + cache_off, m->n_q_heads,
                               m->n_kv_heads, m->max_seq, pos, rope_cs, m->f16_kv_scales,
                               attn);
        else
            orc_attention_step_tern(m->kv_mode, q, k, v, (uint8_t*)m->kc + cache_off * 32,
                                    (uint8_t*)m->vc + cache_off * 32, m->ks + cache_off,
                                    m->vs + cache_off, m->n_q_heads, m->n_kv_heads,
                                    m->max_seq, pos, rope_cs, attn);
        /* :1582-1590 */
        orc_rms_norm(attn, m->attn_sub_norm[l], nx, H, eps);
        inv = orc_quant31(nx, H, codes);
        orc_tl1_gemv_i32(m->o_w[l], codes, H, H, acc);
        for (int i = 0; i < H; ++i) o[i] = (float)acc[i] * (inv * sc[3]);
        for (int i = 0; i < H; ++i) h1[i] = x[i] + o[i];
        /* :1594-1628 */
        orc_rms_norm(h1, m->post_norm[l], nx, H, eps);
        inv = orc_quant31(nx, H, codes);
        orc_tl1_gemv_i32(m->gate_w[l], codes, F, H, acc);
        for (int i = 0; i < F; ++i) g[i] = (float)acc[i] * (inv * sc[4]);
        orc_tl1_gemv_i32(m->up_w[l], codes, F, H, acc);
        for (int i = 0; i < F; ++i) u[i] = (float)acc[i] * (inv * sc[5]);
        for (int i = 0; i < F; ++i) {
            float r = g[i] > 0.0f ? g[i] : 0.0f;
            act[i] = (r * r) * u[i];
        }
        orc_rms_norm(act, m->ffn_sub_norm[l], nx, F, eps);
        inv = orc_quant31(nx, F, codes);
        orc_tl1_gemv_i32(m->down_w[l], codes, H, F, acc);
        for (int i = 0; i < H; ++i) dn[i] = (float)acc[i] * (inv * sc[6]);
        for (int i = 0; i < H; ++i) x[i] = h1[i] + dn[i];
    }
    if (hidden) memcpy(hidden, x, (size_t)H * 4);
    /* :1638-1720 */
    orc_rms_norm(x, m->final_norm, nx, H, eps);
    float* lg = logits ? logits : (float*)malloc((size_t)m->vocab * 4);
    orc_lm_head(nx, m->embed, m->embed_scales, m->vocab, H, lg, NULL);
    int tok = orc_argmax(lg, m->vocab);
    if (!logits) free(lg);
    free(x); free(nx); free(q); free(k); free(v); free(attn); free(o); free(h1);
    free(g); free(u); free(act); free(dn); free(codes); free(acc);
    return tok;
}

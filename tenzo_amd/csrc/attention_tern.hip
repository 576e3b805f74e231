// Ternary KV-cache decode attention on gfx950: the tl1_fused and
// popcount_fused modes of FusedKVCache::forward_attention_raw (reference
// src/runtime/TenzoEngine.cpp: append :534-648, scores :695-805, values
// :852-885).
//
// Cache rows are 32 bytes per (kv head, token), scales fp32 per row:
//   tl1_fused K and every V: byte i holds dims 4i..4i+3 as 2-bit fields
//     (w + 1) from bit 0, w in {-1, 0, +1} (a field 3 reads as 0, as the
//     reference's LUT_W0 / LUT_W1 decode it);
//   popcount_fused K: uint64 {kp0, kp1, kn0, kn1}, bit d of kp0 / kn0 set when
//     dim d is above / below the threshold, kp1 / kn1 for dims 64..127.
// The append thresholds each row at half its mean |x| and keeps the mean |x|
// above the threshold as its scale. Scores are exact integer dot products
// times an fp32 scale:
//   tl1_fused:      q quantized to int8 per head (round(q * 127 / max|q|)),
//                   dot = sum_d q_d w_d over the K fields (v_dot4 on the
//                   fields masked in place);
//   popcount_fused: q thresholded like K, dot = popcount of sign agreements
//                   minus popcount of disagreements (v_bcnt);
//   score = float(dot) * (s_q / sqrt(128) * s_k[t]).
// Softmax and the value sum (o = sum_t w_t p_t s_v[t]) follow the INT8 kernel:
// one workgroup per (context chunk, kv head, sequence) holding the G query
// heads of the kv head, chunk partials (m, l, o) merged by attn_combine_kernel.
#include "attention.h"
#include "common.h"
#include "tern_kv.h"

namespace tz {
namespace {

constexpr int kD = 128;
constexpr int kRowW = kTernRowW;  // dwords per cache row
constexpr int kParts = 8;   // token sets of the value pass (32 threads each)

struct TernArgs {
    const float* q;
    const float* k_new;
    const float* v_new;
    uint8_t* kb;  // [B][Hkv][max_seq][32]
    uint8_t* vb;
    float* ks;    // [B][Hkv][max_seq]
    float* vs;
    const float* rope;
    const int* pos_dev;
    int pos;
    int rope_indexed;
    int Hq, Hkv, max_seq, T, max_chunks;
    float* out;   // [B][Hq][128]
    float* part;  // [B][Hq][max_chunks][130]
    float* q_rot;
    float* k_rot;
};

template <int MODE, int G>
__global__ void __launch_bounds__(256) attn_tern_chunk_kernel(TernArgs a) {
    __shared__ float qs[G][kD];
    __shared__ uint32_t qw[G][32];  // tl1: code bytes, dword 8f + w = dims 16w + 4j + f (byte j);
                                    // popcount: the query's bitplanes in dwords 0..7
    __shared__ int qsum[G];
    __shared__ float qeff[G];
    __shared__ float xn[2][kD];     // the new token's rotated k and its v
    __shared__ uint32_t nrow[2][kRowW];
    __shared__ float nsc[2];
    __shared__ float sc[G][kMaxChunk];
    __shared__ float vsc[kMaxChunk];
    __shared__ uint4 vt[kMaxChunk][2];
    __shared__ float ow[kParts][G][kD];
    __shared__ float mstat[G], lstat[G];

    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = a.pos_dev ? *a.pos_dev : a.pos;
    const int seq_len = pos + 1;
    const int T = a.T;
    const int t0 = c * T;
    if (t0 >= seq_len) return;  // chunks past the context (fixed-size grids)
    const int nt = min(T, seq_len - t0);
    const int nchunks = (seq_len + T - 1) / T;
    const float* rope = a.rope + (a.rope_indexed ? (int64_t)pos * kD : 0);
    const int64_t head = ((int64_t)b * a.Hkv + h) * a.max_seq;  // first row of this kv head
    const bool has_new = pos >= t0 && pos < t0 + nt;

    // ---- RoPE on the G query heads and on the new k (:454-504) ----
    for (int i = tid; i < G * 64; i += 256) {
        const int g = i >> 6, j = i & 63;
        const int qh = h * G + g;
        const float* qv = a.q + ((int64_t)b * a.Hq + qh) * kD;
        const float x0 = qv[j], x1 = qv[j + 64];
        const float cs = rope[j], sn = rope[64 + j];
        const float r0 = __builtin_fmaf(x0, cs, -__fmul_rn(x1, sn));
        const float r1 = __builtin_fmaf(x0, sn, __fmul_rn(x1, cs));
        qs[g][j] = r0;
        qs[g][j + 64] = r1;
        if (a.q_rot && c == 0) {
            float* qr = a.q_rot + ((int64_t)b * a.Hq + qh) * kD;
            qr[j] = r0;
            qr[j + 64] = r1;
        }
    }
    if (has_new && wave < 2) {
        const float* src = (wave == 0 ? a.k_new : a.v_new) + ((int64_t)b * a.Hkv + h) * kD;
        float x0 = src[lane], x1 = src[lane + 64];
        if (wave == 0) {
            const float cs = rope[lane], sn = rope[64 + lane];
            const float r0 = __builtin_fmaf(x0, cs, -__fmul_rn(x1, sn));
            const float r1 = __builtin_fmaf(x0, sn, __fmul_rn(x1, cs));
            x0 = r0;
            x1 = r1;
            if (a.k_rot) {
                float* kr = a.k_rot + ((int64_t)b * a.Hkv + h) * kD;
                kr[lane] = r0;
                kr[lane + 64] = r1;
            }
        }
        xn[wave][lane] = x0;
        xn[wave][lane + 64] = x1;
    }
    __syncthreads();

    // ---- per-head query codes (:700-714, :766-791) and the new rows (:534-648) ----
    const int jobs = G + (has_new ? 2 : 0);
    for (int j = wave; j < jobs; j += 4) {
        if (j < G) {
            tern_query<MODE>(qs[j], lane, qw[j], &qsum[j], &qeff[j]);
        } else {
            const int kv = j - G;  // 0: k, 1: v
            float s;
            const uint32_t w = tern_row<MODE>(xn[kv], kv, lane, &s);
            if (lane < kRowW) {
                nrow[kv][lane] = w;
                uint32_t* dst = reinterpret_cast<uint32_t*>((kv == 0 ? a.kb : a.vb) +
                                                            (head + pos) * 32);
                dst[lane] = w;
            }
            if (lane == 0) {
                (kv == 0 ? a.ks : a.vs)[head + pos] = s;
                nsc[kv] = s;
            }
        }
    }
    __syncthreads();

    // ---- scores (:720-760 / :793-804); token tid of the chunk, V row staged ----
    if (tid < nt) {
        const int t = t0 + tid;
        uint32_t kr[kRowW];
        float skf;
        if (has_new && t == pos) {
#pragma unroll
            for (int i = 0; i < kRowW; ++i) kr[i] = nrow[0][i];
            vt[tid][0] = make_uint4(nrow[1][0], nrow[1][1], nrow[1][2], nrow[1][3]);
            vt[tid][1] = make_uint4(nrow[1][4], nrow[1][5], nrow[1][6], nrow[1][7]);
            skf = nsc[0];
            vsc[tid] = nsc[1];
        } else {
            const uint4* kp = reinterpret_cast<const uint4*>(a.kb + (head + t) * 32);
            const uint4* vp = reinterpret_cast<const uint4*>(a.vb + (head + t) * 32);
            const uint4 k0 = kp[0], k1 = kp[1];
            vt[tid][0] = vp[0];
            vt[tid][1] = vp[1];
            kr[0] = k0.x; kr[1] = k0.y; kr[2] = k0.z; kr[3] = k0.w;
            kr[4] = k1.x; kr[5] = k1.y; kr[6] = k1.z; kr[7] = k1.w;
            skf = a.ks[head + t];
            vsc[tid] = a.vs[head + t];
        }
        float scv[G];
        tern_scores<G, MODE>(kr, qw, qsum, qeff, skf, scv);
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g][tid] = scv[g];
    }
    __syncthreads();

    // ---- chunk softmax statistics (:824-830); weight kept = e^{s-m} s_v ----
    for (int g = wave; g < G; g += 4) {
        float m = -1e30f;
        for (int i = lane; i < nt; i += 64) m = fmaxf(m, sc[g][i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < nt; i += 64) {
            const float e = expf(sc[g][i] - m);
            sc[g][i] = __fmul_rn(e, vsc[i]);
            l += e;
        }
        l = wave_sum_tree(l);
        if (lane == 0) {
            mstat[g] = m;
            lstat[g] = l;
        }
    }
    __syncthreads();

    // ---- weighted values (:852-885): thread (byte bi, token set p) ----
    {
        const int bi = tid & 31, p = tid >> 5;
        float o[G][4];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 4; ++k) o[g][k] = 0.0f;
        const int word = bi >> 2, sh = 8 * (bi & 3);
        for (int t = p; t < nt; t += kParts) {
            const uint32_t* row = reinterpret_cast<const uint32_t*>(vt[t]);
            float w[4];
            tern_value4(row[word] >> sh, w);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float wt = sc[g][t];
#pragma unroll
                for (int k = 0; k < 4; ++k) o[g][k] = __builtin_fmaf(w[k], wt, o[g][k]);
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 4; ++k) ow[p][g][4 * bi + k] = o[g][k];
    }
    __syncthreads();
    for (int i = tid; i < G * kD; i += 256) {
        const int g = i >> 7, d = i & 127;
        float o = ow[0][g][d];
#pragma unroll
        for (int p = 1; p < kParts; ++p) o += ow[p][g][d];
        const int qh = h * G + g;
        if (nchunks == 1) {
            a.out[((int64_t)b * a.Hq + qh) * kD + d] = __fdiv_rn(o, lstat[g]);
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

template <int MODE>
int launch_mode(const TernArgs& a, dim3 grid, int G, hipStream_t st) {
    switch (G) {
        case 1: hipLaunchKernelGGL((attn_tern_chunk_kernel<MODE, 1>), grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((attn_tern_chunk_kernel<MODE, 2>), grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((attn_tern_chunk_kernel<MODE, 4>), grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL((attn_tern_chunk_kernel<MODE, 8>), grid, dim3(256), 0, st, a); break;
        default:
            set_error("attention: query heads per kv head must be 1, 2, 4 or 8 (got %d)", G);
            return TENZO_ERROR_UNSUPPORTED;
    }
    return launch_status("attn_tern_chunk_kernel");
}

}  // namespace

int launch_attn_tern(const AttnTernLaunch& L, hipStream_t st) {
    if (L.mode != 1 && L.mode != 2) {
        set_error("attention: ternary KV mode must be 1 (tl1_fused) or 2 (popcount_fused)");
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    if (L.T <= 0 || L.T > kMaxChunk || L.max_chunks <= 0) {
        set_error("attention: chunk of %d tokens (at most %d)", L.T, kMaxChunk);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    TernArgs a{};
    a.q = L.q;
    a.k_new = L.k_new;
    a.v_new = L.v_new;
    a.kb = L.kb;
    a.vb = L.vb;
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
    a.max_chunks = L.max_chunks;
    a.out = L.out;
    a.q_rot = L.q_rot;
    a.k_rot = L.k_rot;
    if (L.max_chunks > 1) {
        const size_t part_bytes = (size_t)L.B * L.Hq * L.max_chunks * kPartStride * 4;
        a.part = L.part ? L.part : (float*)Scratch::get(kScratchAttn, part_bytes, st);
        if (!a.part) return TENZO_ERROR_OUT_OF_MEMORY;
    }
    const dim3 grid(L.max_chunks, L.Hkv, L.B);
    const int G = L.Hq / L.Hkv;
    int rc = L.mode == 1 ? launch_mode<1>(a, grid, G, st) : launch_mode<2>(a, grid, G, st);
    if (rc || L.max_chunks == 1) return rc;
    return launch_attn_combine(a.part, L.out, L.B, L.Hq, L.Hkv, L.T, L.max_chunks, L.pos_dev,
                               L.pos, st);
}

}  // namespace tz

extern "C" {

TENZO_HIP_API int tenzo_hip_attn_tern_decode(int mode, const float* q, const float* k_new,
                                             const float* v_new, uint8_t* kb, uint8_t* vb,
                                             float* ks, float* vs, const float* rope_cs, int B,
                                             int Hq, int Hkv, int max_seq, int pos, float* out,
                                             float* q_rot, float* k_rot, void* stream) {
    using namespace tz;
    TZ_CHECK(mode == 1 || mode == 2, "attn_tern_decode: mode %d is not 1 (tl1_fused) or 2 "
             "(popcount_fused)", mode);
    TZ_CHECK(q && k_new && v_new && kb && vb && ks && vs && rope_cs && out,
             "attn_tern_decode: null pointer");
    TZ_CHECK(B > 0 && B <= 65535 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0,
             "attn_tern_decode: bad head counts (Hq=%d Hkv=%d)", Hq, Hkv);
    TZ_CHECK(pos >= 0 && pos < max_seq, "attn_tern_decode: pos %d outside [0, %d)", pos, max_seq);
    TZ_CHECK(q_rot != q && k_rot != k_new, "attn_tern_decode: q_rot/k_rot must not alias q/k");
    AttnTernLaunch L{};
    L.mode = mode;
    L.q = q;
    L.k_new = k_new;
    L.v_new = v_new;
    L.kb = kb;
    L.vb = vb;
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
    return launch_attn_tern(L, (hipStream_t)stream);
}

}  // extern "C"

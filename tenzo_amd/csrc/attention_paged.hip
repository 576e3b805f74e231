// paged_int8 decode attention on gfx950 (PagedKVCache::forward_attention_raw,
// reference src/runtime/TenzoEngine.cpp:269-445).
//
// The cache is a pool of 16-token blocks, codes [blocks][n_layers][Hkv][16][128]
// int8 and fp32 scales [blocks][n_layers][Hkv][16]; a block table maps the
// sequence's logical block t / 16 to its physical block. The append quantizes
// like int8_fused (scale amax/127, codes round(x*127/amax)) but keeps fp32
// scales; the attention normalizes with 1 / (sum + 1e-8) and skips the values
// of tokens whose softmax weight is below 1e-7. That cut-off needs the
// normalized weights, so the step runs as passes over the context instead of
// one online-softmax pass:
//   1. paged_scores_kernel  (chunk, kv head): RoPE, append, raw scores
//      s_t = (q.k_t * s_k[t]) / sqrt(128) of the kv head's G query heads into a
//      score buffer, and each chunk's maximum;
//   2. paged_softmax_kernel (query head): M = max, e_t = exp(s_t - M),
//      L = sum e_t, p_t = e_t / (L + 1e-8) in place;
//   3. paged_values_kernel  (chunk, kv head): o_c = sum over the chunk's tokens
//      with p_t >= 1e-7 of (p_t s_v[t]) v_t;
//   4. paged_sum_kernel     (query head): out = sum_c o_c in chunk order.
#include "attention.h"
#include "common.h"

namespace tz {
namespace {

constexpr int kD = 128;
constexpr int kPage = 16;
constexpr float kQkScale = 0.08838834764831845f;  // 1/sqrt(128)
constexpr int kSumU = 32;

struct PagedArgs {
    const float* q;
    const float* k_new;
    const float* v_new;
    int8_t* pk;
    int8_t* pv;
    float* pks;
    float* pvs;
    const int32_t* block_table;
    const float* rope;
    const int* pos_dev;
    int pos;
    int rope_indexed;
    int n_layers, layer, Hq, Hkv, T, max_chunks, score_stride;
    float* scores;  // [Hq][score_stride]
    float* cmax;    // [Hq][max_chunks]
    float* part;    // [Hq][max_chunks][128]
    float* out;     // [Hq][128]
};

// Row index (in 128-byte rows / scales) of token t of kv head h.
__device__ __forceinline__ int64_t page_row(const PagedArgs& a, int t, int h) {
    const int64_t blk = a.block_table[t / kPage];
    return ((blk * a.n_layers + a.layer) * a.Hkv + h) * kPage + t % kPage;
}

__device__ __forceinline__ int step_pos(const PagedArgs& a) { return a.pos_dev ? *a.pos_dev : a.pos; }

// KV append quantization (:334-350 as built): s = amax*(1/127) with amax
// floored at 1e-8, code = clamp(round(x * (127/amax)), -128, 127). 64 lanes x 2.
__device__ __forceinline__ float quant_row(float x0, float x1, int8_t* codes, int lane) {
    const float amax = fmaxf(wave_max(fmaxf(fabsf(x0), fabsf(x1))), 1e-8f);
    const float inv = __fdiv_rn(127.0f, amax);
    codes[lane] = (int8_t)fminf(fmaxf(roundf(__fmul_rn(x0, inv)), -128.0f), 127.0f);
    codes[lane + 64] = (int8_t)fminf(fmaxf(roundf(__fmul_rn(x1, inv)), -128.0f), 127.0f);
    return __fmul_rn(amax, 1.0f / 127.0f);
}

template <int G>
__global__ void __launch_bounds__(256) paged_scores_kernel(PagedArgs a) {
    __shared__ float qs[G][kD];
    __shared__ float sc[G][kMaxChunk];
    __shared__ __align__(16) int8_t newk[kD];
    __shared__ float newks;
    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = step_pos(a);
    const int seq_len = pos + 1;
    const int t0 = c * a.T;
    if (t0 >= seq_len) return;
    const int nt = min(a.T, seq_len - t0);
    const float* rope = a.rope + (a.rope_indexed ? (int64_t)pos * kD : 0);
    const bool has_new = pos >= t0 && pos < t0 + nt;

    // RoPE on the G query heads (:271-292)
    for (int i = tid; i < G * 64; i += 256) {
        const int g = i >> 6, j = i & 63;
        const float* qv = a.q + (int64_t)(h * G + g) * kD;
        const float x0 = qv[j], x1 = qv[j + 64];
        const float cs = rope[j], sn = rope[64 + j];
        qs[g][j] = __builtin_fmaf(x0, cs, -__fmul_rn(x1, sn));
        qs[g][j + 64] = __builtin_fmaf(x0, sn, __fmul_rn(x1, cs));
    }
    // the new token: RoPE on k, quantize into its block slot (:294-352)
    if (has_new && wave < 2) {
        __shared__ __align__(16) int8_t newv[kD];
        const float* src = (wave == 0 ? a.k_new : a.v_new) + (int64_t)h * kD;
        float x0 = src[lane], x1 = src[lane + 64];
        if (wave == 0) {
            const float cs = rope[lane], sn = rope[64 + lane];
            const float r0 = __builtin_fmaf(x0, cs, -__fmul_rn(x1, sn));
            const float r1 = __builtin_fmaf(x0, sn, __fmul_rn(x1, cs));
            x0 = r0;
            x1 = r1;
        }
        int8_t* codes = wave == 0 ? newk : newv;
        const float s = quant_row(x0, x1, codes, lane);
        const int64_t r = page_row(a, pos, h);
        int8_t* dst = (wave == 0 ? a.pk : a.pv) + r * kD;
        dst[lane] = codes[lane];
        dst[lane + 64] = codes[lane + 64];
        if (lane == 0) {
            (wave == 0 ? a.pks : a.pvs)[r] = s;
            if (wave == 0) newks = s;
        }
    }
    __syncthreads();

    // scores (:366-393): lane (wave, l) takes token r*32 + wave*8 + l/8 and dims
    // (l%8)*16 .. +15; the 8 lanes of a token meet through DPP adds
    const int sub = lane >> 3, d0 = (lane & 7) * 16;
    float qr[G][16];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 16; ++j) qr[g][j] = qs[g][d0 + j];
    for (int tb = wave * 8; tb < nt; tb += 32) {
        const int tl = tb + sub, t = t0 + tl;
        float kf[16];
        float skf = 0.0f;
        if (tl < nt) {
            uint4 kv;
            if (has_new && t == pos) {
                kv = *reinterpret_cast<const uint4*>(newk + d0);
                skf = newks;
            } else {
                const int64_t r = page_row(a, t, h);
                kv = *reinterpret_cast<const uint4*>(a.pk + r * kD + d0);
                skf = a.pks[r];
            }
            const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) kf[4 * i + j] = (float)(int8_t)((w[i] >> (8 * j)) & 0xff);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) kf[j] = 0.0f;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) s = __builtin_fmaf(qr[g][j], kf[j], s);
            s += dpp_f<kDppXor1>(s);
            s += dpp_f<kDppXor2>(s);
            s += dpp_f<kDppHalfMirror>(s);
            if (tl < nt && (lane & 7) == (g & 7)) sc[g][tl] = __fmul_rn(__fmul_rn(s, skf), kQkScale);
        }
    }
    __syncthreads();
    for (int g = wave; g < G; g += 4) {
        float m = -1e30f;
        float* dst = a.scores + (int64_t)(h * G + g) * a.score_stride + t0;
        for (int i = lane; i < nt; i += 64) {
            dst[i] = sc[g][i];
            m = fmaxf(m, sc[g][i]);
        }
        m = wave_max(m);
        if (lane == 0) a.cmax[(h * G + g) * a.max_chunks + c] = m;
    }
}

// Softmax of one query head over the whole context (:395-405), in place.
__global__ void __launch_bounds__(256) paged_softmax_kernel(PagedArgs a) {
    __shared__ float red[4];
    __shared__ float stat;
    const int qh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int seq_len = step_pos(a) + 1;
    const int nchunks = (seq_len + a.T - 1) / a.T;
    const float* cm = a.cmax + qh * a.max_chunks;
    float M = -1e30f;
    for (int c = 0; c < nchunks; ++c) M = fmaxf(M, cm[c]);
    float* s = a.scores + (int64_t)qh * a.score_stride;
    // thread tid takes t = tid, tid + 256, ... in order; a read-only pass sums
    // the exponentials (its loads issued kU at a time), a second pass writes
    // the normalized weights (the same expf of the same score)
    constexpr int kU = 8;
    float l = 0.0f;
    for (int t0 = tid; t0 < seq_len; t0 += 256 * kU) {
        float v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = t0 + 256 * u < seq_len ? s[t0 + 256 * u] : 0.0f;
#pragma unroll
        for (int u = 0; u < kU; ++u)
            if (t0 + 256 * u < seq_len) l += expf(v[u] - M);
    }
    l = wave_sum_tree(l);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    if (tid == 0) stat = __fdiv_rn(1.0f, ((red[0] + red[1]) + (red[2] + red[3])) + 1e-8f);
    __syncthreads();
    const float inv = stat;
    for (int t0 = tid; t0 < seq_len; t0 += 256 * kU) {
        float v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = t0 + 256 * u < seq_len ? s[t0 + 256 * u] : 0.0f;
#pragma unroll
        for (int u = 0; u < kU; ++u)
            if (t0 + 256 * u < seq_len) s[t0 + 256 * u] = __fmul_rn(expf(v[u] - M), inv);
    }
}

// Weighted values of one chunk (:408-443): thread (d4, p) owns dims 4 d4 .. +3
// of every query head and takes the chunk's tokens p, p + 8, ...
template <int G>
__global__ void __launch_bounds__(256) paged_values_kernel(PagedArgs a) {
    __shared__ float ow[8][G][kD];
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int seq_len = step_pos(a) + 1;
    const int t0 = c * a.T;
    if (t0 >= seq_len) return;
    const int nt = min(a.T, seq_len - t0);
    const int nchunks = (seq_len + a.T - 1) / a.T;
    const int d4 = tid & 31, p = tid >> 5;
    float o[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) o[g][k] = 0.0f;
    for (int i = p; i < nt; i += 8) {
        const int t = t0 + i;
        const int64_t r = page_row(a, t, h);
        const uint32_t vb = *reinterpret_cast<const uint32_t*>(a.pv + r * kD + 4 * d4);
        const float sv = a.pvs[r];
        float vf[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) vf[k] = (float)(int8_t)((vb >> (8 * k)) & 0xff);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float alpha = a.scores[(int64_t)(h * G + g) * a.score_stride + t];
            const float w = alpha < 1e-7f ? 0.0f : __fmul_rn(alpha, sv);
#pragma unroll
            for (int k = 0; k < 4; ++k) o[g][k] = __builtin_fmaf(w, vf[k], o[g][k]);
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) ow[p][g][4 * d4 + k] = o[g][k];
    __syncthreads();
    for (int i = tid; i < G * kD; i += 256) {
        const int g = i >> 7, d = i & 127;
        float v = ow[0][g][d];
#pragma unroll
        for (int q = 1; q < 8; ++q) v += ow[q][g][d];
        const int qh = h * G + g;
        if (nchunks == 1)
            a.out[(int64_t)qh * kD + d] = v;
        else
            a.part[((int64_t)qh * a.max_chunks + c) * kD + d] = v;
    }
}

// out = sum of the chunk sums in chunk order, kSumU loads in flight.
__global__ void __launch_bounds__(128) paged_sum_kernel(PagedArgs a) {
    const int qh = blockIdx.x, d = threadIdx.x;
    const int seq_len = step_pos(a) + 1;
    const int nchunks = (seq_len + a.T - 1) / a.T;
    if (nchunks == 1) return;
    const float* pp = a.part + (int64_t)qh * a.max_chunks * kD + d;
    float o = 0.0f;
    for (int c0 = 0; c0 < nchunks; c0 += kSumU) {
        float v[kSumU];
#pragma unroll
        for (int u = 0; u < kSumU; ++u) v[u] = c0 + u < nchunks ? pp[(int64_t)(c0 + u) * kD] : 0.0f;
#pragma unroll
        for (int u = 0; u < kSumU; ++u)
            if (c0 + u < nchunks) o += v[u];
    }
    a.out[(int64_t)qh * kD + d] = o;
}

}  // namespace

size_t paged_ws_bytes(int Hq, int max_chunks, int T) {
    const size_t stride = (size_t)max_chunks * T;
    return (size_t)Hq * (stride + max_chunks + (size_t)max_chunks * kD) * 4;
}

int launch_attn_paged(const AttnPagedLaunch& L, hipStream_t st) {
    const int G = L.Hq / L.Hkv;
    if (L.T <= 0 || L.T > kMaxChunk || L.T % kPage || L.max_chunks <= 0) {
        set_error("paged attention: chunk of %d tokens (a multiple of 16, at most %d)", L.T,
                  kMaxChunk);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    PagedArgs a{};
    a.q = L.q;
    a.k_new = L.k_new;
    a.v_new = L.v_new;
    a.pk = L.pk;
    a.pv = L.pv;
    a.pks = L.pks;
    a.pvs = L.pvs;
    a.block_table = L.block_table;
    a.rope = L.rope;
    a.pos_dev = L.pos_dev;
    a.pos = L.pos;
    a.rope_indexed = L.rope_indexed;
    a.n_layers = L.n_layers;
    a.layer = L.layer;
    a.Hq = L.Hq;
    a.Hkv = L.Hkv;
    a.T = L.T;
    a.max_chunks = L.max_chunks;
    a.score_stride = L.max_chunks * L.T;
    float* ws = L.ws ? L.ws
                     : (float*)Scratch::get(kScratchAttn, paged_ws_bytes(L.Hq, L.max_chunks, L.T), st);
    if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
    a.scores = ws;
    a.cmax = ws + (size_t)L.Hq * a.score_stride;
    a.part = a.cmax + (size_t)L.Hq * L.max_chunks;
    a.out = L.out;
    const dim3 grid(L.max_chunks, L.Hkv);
    switch (G) {
        case 1: hipLaunchKernelGGL(paged_scores_kernel<1>, grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(paged_scores_kernel<2>, grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(paged_scores_kernel<4>, grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL(paged_scores_kernel<8>, grid, dim3(256), 0, st, a); break;
        default:
            set_error("attention: query heads per kv head must be 1, 2, 4 or 8 (got %d)", G);
            return TENZO_ERROR_UNSUPPORTED;
    }
    int rc = launch_status("paged_scores_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(paged_softmax_kernel, dim3(L.Hq), dim3(256), 0, st, a);
    if ((rc = launch_status("paged_softmax_kernel"))) return rc;
    switch (G) {
        case 1: hipLaunchKernelGGL(paged_values_kernel<1>, grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(paged_values_kernel<2>, grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(paged_values_kernel<4>, grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL(paged_values_kernel<8>, grid, dim3(256), 0, st, a); break;
    }
    if ((rc = launch_status("paged_values_kernel"))) return rc;
    if (L.max_chunks == 1) return TENZO_SUCCESS;
    hipLaunchKernelGGL(paged_sum_kernel, dim3(L.Hq), dim3(128), 0, st, a);
    return launch_status("paged_sum_kernel");
}

}  // namespace tz

extern "C" {

TENZO_HIP_API int tenzo_hip_attn_paged_int8_decode(const float* q, const float* k_new,
                                                   const float* v_new, int8_t* pk, int8_t* pv,
                                                   float* pks, float* pvs,
                                                   const int32_t* block_table, int n_layers,
                                                   int layer, const float* rope_cs, int Hq,
                                                   int Hkv, int pos, float* out, void* stream) {
    using namespace tz;
    TZ_CHECK(q && k_new && v_new && pk && pv && pks && pvs && block_table && rope_cs && out,
             "attn_paged_int8_decode: null pointer");
    TZ_CHECK(Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "attn_paged_int8_decode: bad head counts "
             "(Hq=%d Hkv=%d)", Hq, Hkv);
    TZ_CHECK(n_layers > 0 && layer >= 0 && layer < n_layers && pos >= 0,
             "attn_paged_int8_decode: layer %d of %d, pos %d", layer, n_layers, pos);
    AttnPagedLaunch L{};
    L.q = q;
    L.k_new = k_new;
    L.v_new = v_new;
    L.pk = pk;
    L.pv = pv;
    L.pks = pks;
    L.pvs = pvs;
    L.block_table = block_table;
    L.rope = rope_cs;
    L.pos = pos;
    L.n_layers = n_layers;
    L.layer = layer;
    L.Hq = Hq;
    L.Hkv = Hkv;
    L.T = attn_pick_chunk(pos + 1, Hkv, 1);
    L.max_chunks = (int)ceil_div(pos + 1, L.T);
    L.out = out;
    return launch_attn_paged(L, (hipStream_t)stream);
}

}  // extern "C"

// Persistent decode-step kernel for gfx950: one cooperative launch runs the
// embedding, all layers and the LM head of one token
// (forward_layer_raw / compute_logits / the greedy sampler of the reference,
// src/runtime/TenzoEngine.cpp:1522-1755), with every CU resident for the
// whole step.
//
// Schedule. The step is a sequence of stages: per layer QKV, ATT, O, GU
// (gate|up), DOWN, then HEAD. Each stage has a list of tasks (a 64-row block
// of a TL1 matrix, an attention chunk of one kv head, a row block of the LM
// head); stage s's tasks go to workgroups off_s, off_s+1, ... (mod nwg) with
// off_{s+1} = off_s + ntasks_s, so consecutive stages mostly use different
// workgroups. A workgroup issues the loads of its weight tile first thing in a
// stage, so they are in flight while it reads and normalizes the stage input.
// Per stage each CU reads at most ~110 KB of weights: the critical path is the
// chain of barriers and input reads, not bandwidth.
//
// Synchronisation. Stage outputs are written with device-coherent stores and
// read with device-coherent loads (sc1: through to the memory side, so no
// L2 write-back / invalidate fence is needed); before arriving at a barrier
// every wave waits for its stores to be acknowledged (s_waitcnt). The barrier
// is 16 counters on separate 256-byte lines (one per workgroup residue mod
// 16) polled together by one wave. The attention split-K combine is done by
// the last workgroup to finish a kv head (a per-head arrival counter). Every
// wait is bounded: on timeout a workgroup raises the error word and all
// others abort at their next poll, so the grid always drains.
//
// Arithmetic is the reference's, in the same rounding steps as the
// multi-kernel path (tl1.hip, attention.hip, lm_head.hip): RMSNorm with the
// fixed 256-partial summation order, +-31 / +-127 activation codes, exact
// int32 TL1 / int8 sums, fp32 epilogues.
#include "attention.h"
#include "decode_step.h"

namespace tz {
namespace {

constexpr int kT = kDsThreads;   // 512 threads = 8 waves
constexpr int kW = kT / 64;
constexpr int kPF = 10;          // tile uint4 per lane preloaded (all of K <= 2560)
constexpr int kNC = kDsCounters;
constexpr int kD = 128;
constexpr int kPS = kDsPartStride;  // partial record: m, l, -, -, o[128]
constexpr int kTmax = 1024;      // attention tokens per task (LDS score buffer)
constexpr int kRT = kW * 8;      // attention tokens per round (8 per wave)
constexpr int kAR = 4;           // attention rounds preloaded in registers
constexpr unsigned kSpinLimit = 1u << 22;
constexpr float kAttnScale = 0.08838834764831845f;  // 1/sqrt(128)

enum Stage { S_QKV = 0, S_ATT = 1, S_O = 2, S_GU = 3, S_DOWN = 4, S_HEAD = 5 };

__device__ __forceinline__ float ldc(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ldcu(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-coherent 16-byte loads through a raw buffer resource (cache policy
// sc1: the read is served from the memory side, as the relaxed agent-scope
// atomics above). Lanes past the resource's byte count read zeros.
typedef float f4v __attribute__((ext_vector_type(4)));
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, gfx9 family

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRsrcWord3);
}
__device__ __forceinline__ f4v ldc16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}

// dst[0..n) = src[0..n) (n % 4 == 0, src 16-byte aligned), all loads of a
// thread issued before any is used.
__device__ __forceinline__ void load_vec(float* dst, const float* src, int n) {
    constexpr int U = 8;
    const __amdgpu_buffer_rsrc_t r = rsrc(src, (uint32_t)n * 4);
    const int n4 = n >> 2;
    for (int base = threadIdx.x; base < n4; base += U * kDsThreads) {
        f4v v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = ldc16(r, (uint32_t)(base + u * kDsThreads) * 16);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * kDsThreads;
            if (i < n4) {
                dst[4 * i] = v[u].x;
                dst[4 * i + 1] = v[u].y;
                dst[4 * i + 2] = v[u].z;
                dst[4 * i + 3] = v[u].w;
            }
        }
    }
}

// dst[0..n) = src[0..n) for read-only data (the norm weights), plain loads
// issued together. n % 4 == 0, src 16-byte aligned.
__device__ __forceinline__ void load_ro(float* dst, const float* __restrict__ src, int n) {
    constexpr int U = 8;
    const int n4 = n >> 2;
    const float4* s4 = reinterpret_cast<const float4*>(src);
    for (int base = threadIdx.x; base < n4; base += U * kDsThreads) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * kDsThreads;
            if (i < n4) v[u] = s4[i];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * kDsThreads;
            if (i < n4) {
                dst[4 * i] = v[u].x;
                dst[4 * i + 1] = v[u].y;
                dst[4 * i + 2] = v[u].z;
                dst[4 * i + 3] = v[u].w;
            }
        }
    }
}

// dst[i] = max(0, gate[i])^2 * up[i] (:1616-1620) for the gate | up vector.
__device__ __forceinline__ void load_act(float* dst, const float* gu, int F) {
    constexpr int U = 8;
    const __amdgpu_buffer_rsrc_t r = rsrc(gu, (uint32_t)F * 8);
    const int n4 = F >> 2;
    for (int base = threadIdx.x; base < n4; base += U * kDsThreads) {
        f4v g[U], u[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t off = (uint32_t)(base + k * kDsThreads) * 16;
            g[k] = ldc16(r, off);
            u[k] = ldc16(r, off + (uint32_t)F * 4);
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int i = base + k * kDsThreads;
            if (i < n4) {
                const float gg[4] = {g[k].x, g[k].y, g[k].z, g[k].w};
                const float uu[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float rr = fmaxf(0.0f, gg[j]);
                    dst[4 * i + j] = (rr * rr) * uu[j];
                }
            }
        }
    }
}

// ---------------------------------------------------------------- layout --

__host__ __device__ inline size_t w_err(int, int) { return (size_t)kNC * 64; }
__host__ __device__ inline size_t w_am(int, int) { return (size_t)(kNC + 1) * 64; }
__host__ __device__ inline size_t w_head(int l, int h, int Hkv) {
    return (size_t)(kNC + 2 + l * Hkv + h) * 64;
}

struct Shared {
    float xs[8192];                 // stage input / normalized values
    float ws[8192];                 // RMSNorm weights of the stage
    int8_t codes[8192] __attribute__((aligned(16)));
    int red_i[kW][64];
    float red_f[kW];
    int red_i8[kW];
    float inv_scale;
    int code_sum;
    int flag;
};

struct AttnShared {
    float qs[8][kD];
    float sc[8][kTmax];
    float ow[kW][8][kD];
    float mstat[8], lstat[8];
    int8_t newk[kD] __attribute__((aligned(16)));
    int8_t newv[kD] __attribute__((aligned(16)));
    float news[2];
    int last;
};

union SharedAll {
    Shared s;
    AttnShared a;
};

// -------------------------------------------------------------- schedule --

__device__ __forceinline__ int ntasks(const DsParams& p, int st) {
    const int qd = p.Hq * kD, kvd = p.Hkv * kD;
    switch (st) {
        case S_QKV: return (qd + 2 * kvd) / 64;
        case S_ATT: return p.Hkv * p.C;
        case S_O: return p.H / 64;
        case S_GU: return 2 * p.F / 64;
        case S_DOWN: return p.H / 64;
        default: return (p.V + 63) / 64;
    }
}

// Stage index s = 5*layer + kind for the layers, 5*L for the head.
__device__ __forceinline__ int kind_of(const DsParams& p, int s) {
    return s >= 5 * p.L ? S_HEAD : s % 5;
}

// ------------------------------------------------------------- barrier ----

__device__ bool grid_barrier(const DsParams& p, unsigned& gen, int* s_abort) {
    ++gen;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are acknowledged
    __syncthreads();
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        if (l == 0)
            __hip_atomic_fetch_add(p.sync + (blockIdx.x % kNC) * 64, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        const unsigned target = gen * (unsigned)(p.nwg / kNC);
        bool done = l >= kNC;
        unsigned spins = 0;
        bool abort = false;
        while (true) {
            if (!done) done = ldcu(p.sync + l * 64) >= target;
            if (__all(done)) break;
            if ((++spins & 63) == 0) {
                if (ldcu(p.sync + w_err(p.L, p.Hkv)) != 0) {
                    abort = true;
                    break;
                }
                if (spins > kSpinLimit) {
                    if (l == 0)
                        __hip_atomic_store(p.sync + w_err(p.L, p.Hkv), 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    abort = true;
                    break;
                }
            }
        }
        if (l == 0) *s_abort = abort ? 1 : 0;
    }
    __syncthreads();
    return *s_abort == 0;
}

// ------------------------------------------------------------ prologue ----

// Sum of squares of xs[0..K) in the order of the CPU oracle (orc_sumsq):
// threads 0..255 accumulate strided partials, then a balanced tree.
__device__ __forceinline__ float wg_sumsq(const float* xs, int K, float* red) {
    const int t = threadIdx.x;
    float s = 0.0f;
    if (t < 256)
        for (int i = t; i < K; i += 256) s = __builtin_fmaf(xs[i], xs[i], s);
    s = wave_sum_tree(s);
    if ((t & 63) == 0 && t < 256) red[t >> 6] = s;
    __syncthreads();
    const float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float wg_max(float v, float* red) {
    v = wave_max(v);
    const int t = threadIdx.x;
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kW; ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int wg_sum_i(int v, int* red) {
    v = wave_sum_i32(v);
    const int t = threadIdx.x;
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int w = 0; w < kW; ++w) r += red[w];
    __syncthreads();
    return r;
}

// xs[0..K) holds the stage input. Normalizes in place (rms_norm_raw with
// weight w, :148-166) and quantizes to codes (QMAX 31: build_lut :28-42,
// QMAX 127: compute_logits :1666-1678), codes zero-padded to a multiple of 64.
// w is the LDS copy of the norm weights, or null for none.
template <int QMAX>
__device__ void norm_quant(SharedAll& sh, int K, const float* w, float eps) {
    Shared& s = sh.s;
    const int t = threadIdx.x;
    const float inv_rms = inv_rms_from_sumsq(wg_sumsq(s.xs, K, s.red_f), K, eps);
    float amax = QMAX == 31 ? 1e-6f : 1e-8f;
    for (int i = t; i < K; i += kT) {
        const float y = norm_apply(s.xs[i], inv_rms, w, i);
        s.xs[i] = y;
        amax = fmaxf(amax, fabsf(y));
    }
    amax = wg_max(amax, s.red_f);
    const float scale = (float)QMAX / amax;
    const int Kp = (K + 63) & ~63;
    int csum = 0;
    for (int i = t; i < Kp; i += kT) {
        int c = 0;
        if (i < K) {
            float r = roundf(s.xs[i] * scale);
            if (QMAX == 127) r = fminf(fmaxf(r, -128.0f), 127.0f);
            c = (int)r;
        }
        s.codes[i] = (int8_t)c;
        csum += c;
    }
    csum = wg_sum_i(csum, s.red_i8);
    if (t == 0) {
        s.inv_scale = amax * (1.0f / (float)QMAX);
        s.code_sum = csum;
    }
    __syncthreads();
}

// ---------------------------------------------------------------- GEMV ----

__device__ __forceinline__ int dot64(const uint4 v, const int4* c4, int acc) {
    // 64 columns of 2-bit codes (tl1.hip layout) against 64 int8 codes
    const uint32_t M = 0x03030303u;
    const int4 a0 = c4[0], a1 = c4[1], a2 = c4[2], a3 = c4[3];
    acc = sdot4(v.x & M, a0.x, acc);
    acc = sdot4((v.x >> 2) & M, a0.y, acc);
    acc = sdot4((v.x >> 4) & M, a0.z, acc);
    acc = sdot4((v.x >> 6) & M, a0.w, acc);
    acc = sdot4(v.y & M, a1.x, acc);
    acc = sdot4((v.y >> 2) & M, a1.y, acc);
    acc = sdot4((v.y >> 4) & M, a1.z, acc);
    acc = sdot4((v.y >> 6) & M, a1.w, acc);
    acc = sdot4(v.z & M, a2.x, acc);
    acc = sdot4((v.z >> 2) & M, a2.y, acc);
    acc = sdot4((v.z >> 4) & M, a2.z, acc);
    acc = sdot4((v.z >> 6) & M, a2.w, acc);
    acc = sdot4(v.w & M, a3.x, acc);
    acc = sdot4((v.w >> 2) & M, a3.y, acc);
    acc = sdot4((v.w >> 4) & M, a3.z, acc);
    acc = sdot4((v.w >> 6) & M, a3.w, acc);
    return acc;
}

// Loads the first kPF chunks per lane of TL1 row block rb (KS super-chunks).
__device__ __forceinline__ void load_tl1_tile(uint4* pf, const uint4* __restrict__ W, int rb,
                                              int KS) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint4* base = W + (size_t)rb * KS * 64 + lane;
#pragma unroll
    for (int i = 0; i < kPF; ++i) {
        const int c = wave + kW * i;
        if (c < KS) pf[i] = base[(size_t)c * 64];
    }
}

// One TL1 row block: returns the exact int32 sum sum_k u_k a_k (u = w+1) in
// wave 0, lane = row (other waves: 0).
__device__ __forceinline__ int tl1_rowblock(SharedAll& sh, const uint4* cur,
                                            const uint4* __restrict__ W, int rb, int KS) {
    Shared& s = sh.s;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int4* c4 = reinterpret_cast<const int4*>(s.codes);
    int acc = 0;
#pragma unroll
    for (int i = 0; i < kPF; ++i) {
        const int c = wave + kW * i;
        if (c < KS) acc = dot64(cur[i], c4 + c * 4, acc);
    }
    // K beyond the preloaded window (the down projection): 8 loads in flight
    const uint4* base = W + (size_t)rb * KS * 64 + lane;
    for (int c0 = wave + kW * kPF; c0 < KS; c0 += 8 * kW) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kW;
            if (c < KS) v[u] = base[(size_t)c * 64];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kW;
            if (c < KS) acc = dot64(v[u], c4 + c * 4, acc);
        }
    }
    s.red_i[wave][lane] = acc;
    __syncthreads();
    int tot = 0;
    if (wave == 0) {
#pragma unroll
        for (int w = 0; w < kW; ++w) tot += s.red_i[w][lane];
    }
    __syncthreads();
    return tot;
}

// ----------------------------------------------------------- attention ----

// KV append quantization (:516-531 as built), 64 lanes x 2 values.
__device__ __forceinline__ void quant_kv(float x0, float x1, int8_t* codes, int lane,
                                         float* s_out) {
    float amax = fmaxf(fabsf(x0), fabsf(x1));
    amax = fmaxf(wave_max(amax), 1e-8f);
    const float inv = 127.0f / amax;
    const float r0 = fminf(fmaxf(roundf(x0 * inv), -128.0f), 127.0f);
    const float r1 = fminf(fmaxf(roundf(x1 * inv), -128.0f), 127.0f);
    codes[lane] = (int8_t)r0;
    codes[lane + 64] = (int8_t)r1;
    *s_out = amax * (1.0f / 127.0f);
}

__device__ __forceinline__ void unpack16(const uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) f[4 * i + j] = (float)(int8_t)((w[i] >> (8 * j)) & 0xff);
}

// Attention tile: the first kAR rounds of kRT tokens; lane (wave, l) holds 16
// bytes of token r*kRT + wave*8 + l/8 at dims (l%8)*16 of K (pf[2r]) and V
// (pf[2r+1]) and its two fp16 scales (pfs[r]). Later rounds are read in the
// loops that use them.
__device__ __forceinline__ void load_att_tile(uint4* pf, uint32_t* pfs, const DsParams& p,
                                              int l, int h, int c) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = c * p.T;
    const int ctx = p.pos + 1;
    const int nt = min(p.T, ctx - t0);
    const size_t head = ((size_t)l * p.Hkv + h) * p.max_seq;
    const int d0 = (lane & 7) * 16;
#pragma unroll
    for (int r = 0; r < kAR; ++r) {
        const int tl = r * kRT + wave * 8 + (lane >> 3);
        const int t = t0 + tl;
        if (tl < nt && t != p.pos) {
            pf[2 * r] = *reinterpret_cast<const uint4*>(p.kc + (head + t) * kD + d0);
            pf[2 * r + 1] = *reinterpret_cast<const uint4*>(p.vc + (head + t) * kD + d0);
            pfs[r] = (uint32_t)p.ks[head + t] | ((uint32_t)p.vs[head + t] << 16);
        }
    }
}

template <int G>
__device__ void attn_task(SharedAll& sh, const DsParams& p, const uint4* cur,
                          const uint32_t* curs, int l, int h, int c) {
    AttnShared& a = sh.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ctx = p.pos + 1;
    const int t0 = c * p.T;
    const int nt = min(p.T, ctx - t0);
    const int qd = p.Hq * kD, kvd = p.Hkv * kD;
    const float* rope = p.rope + (size_t)p.pos * kD;
    const size_t head = ((size_t)l * p.Hkv + h) * p.max_seq;
    // RoPE on the G query heads (:460-481)
    for (int i = tid; i < G * 64; i += kT) {
        const int g = i >> 6, j = i & 63;
        const float* qv = p.qkv + (size_t)(h * G + g) * kD;
        const float x0 = ldc(qv + j), x1 = ldc(qv + j + 64);
        const float cs = rope[j], sn = rope[64 + j];
        a.qs[g][j] = __builtin_fmaf(x0, cs, -(x1 * sn));
        a.qs[g][j + 64] = __builtin_fmaf(x0, sn, x1 * cs);
    }
    // the new token: RoPE on k, quantize-append k and v (:482-533)
    const bool has_new = p.pos >= t0 && p.pos < t0 + nt;
    if (has_new && wave < 2) {
        const float* src = p.qkv + qd + (wave == 0 ? 0 : kvd) + (size_t)h * kD;
        float x0 = ldc(src + lane), x1 = ldc(src + lane + 64);
        if (wave == 0) {
            const float cs = rope[lane], sn = rope[64 + lane];
            const float r0 = __builtin_fmaf(x0, cs, -(x1 * sn));
            const float r1 = __builtin_fmaf(x0, sn, x1 * cs);
            x0 = r0;
            x1 = r1;
        }
        float s;
        int8_t* nb = wave == 0 ? a.newk : a.newv;
        quant_kv(x0, x1, nb, lane, &s);
        const uint16_t sh16 = float_to_half_bits(s);
        int8_t* dst = (wave == 0 ? p.kc : p.vc) + (head + p.pos) * kD;
        dst[lane] = nb[lane];
        dst[lane + 64] = nb[lane + 64];
        if (lane == 0) {
            (wave == 0 ? p.ks : p.vs)[head + p.pos] = sh16;
            a.news[wave] = half_bits_to_float(sh16);
        }
    }
    __syncthreads();

    const int sub = lane >> 3, d0 = (lane & 7) * 16;
    // scores (:678-694)
    {
        float qr[G][16];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 16; ++j) qr[g][j] = a.qs[g][d0 + j];
        const int rounds = (nt + kRT - 1) / kRT;
        for (int r = 0; r < rounds; ++r) {
            const int tl = r * kRT + wave * 8 + sub;
            const int t = t0 + tl;
            float kf[16];
            float skf = 0.0f;
            if (tl < nt) {
                uint4 kv;
                if (t == p.pos) {
                    kv = *reinterpret_cast<const uint4*>(a.newk + d0);
                    skf = a.news[0];
                } else if (r < kAR) {
                    kv = cur[2 * r];
                    skf = half_bits_to_float((uint16_t)(curs[r] & 0xffffu));
                } else {
                    kv = *reinterpret_cast<const uint4*>(p.kc + (head + t) * kD + d0);
                    skf = half_bits_to_float(p.ks[head + t]);
                }
                unpack16(kv, kf);
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) kf[j] = 0.0f;
            }
            float pr[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) s = __builtin_fmaf(qr[g][j], kf[j], s);
                s += __shfl_xor(s, 1, 64);
                s += __shfl_xor(s, 2, 64);
                s += __shfl_xor(s, 4, 64);
                pr[g] = s;
            }
            if (tl < nt) {
                const float f = skf * kAttnScale;
#pragma unroll
                for (int g = 0; g < G; ++g)
                    if ((lane & 7) == (g & 7)) a.sc[g][tl] = pr[g] * f;
            }
        }
    }
    __syncthreads();
    // chunk softmax statistics (:824-830)
    for (int g = wave; g < G; g += kW) {
        float m = -1e30f;
        for (int i = lane; i < nt; i += 64) m = fmaxf(m, a.sc[g][i]);
        m = wave_max(m);
        float lsum = 0.0f;
        for (int i = lane; i < nt; i += 64) {
            const float e = expf(a.sc[g][i] - m);
            a.sc[g][i] = e;
            lsum += e;
        }
        lsum = wave_sum_tree(lsum);
        if (lane == 0) {
            a.mstat[g] = m;
            a.lstat[g] = lsum;
        }
    }
    __syncthreads();
    // weighted values (:842-851)
    float acc[G][16];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[g][j] = 0.0f;
    {
        const int rounds = (nt + kRT - 1) / kRT;
        for (int r = 0; r < rounds; ++r) {
            const int tl = r * kRT + wave * 8 + sub;
            const int t = t0 + tl;
            if (tl < nt) {
                uint4 vv;
                float svf;
                if (t == p.pos) {
                    vv = *reinterpret_cast<const uint4*>(a.newv + d0);
                    svf = a.news[1];
                } else if (r < kAR) {
                    vv = cur[2 * r + 1];
                    svf = half_bits_to_float((uint16_t)(curs[r] >> 16));
                } else {
                    vv = *reinterpret_cast<const uint4*>(p.vc + (head + t) * kD + d0);
                    svf = half_bits_to_float(p.vs[head + t]);
                }
                float vf[16];
                unpack16(vv, vf);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float wgt = a.sc[g][tl] * svf;
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[g][j] = __builtin_fmaf(vf[j], wgt, acc[g][j]);
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            float v = acc[g][j];
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[g][j] = v;
        }
    if (lane < 8) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 16; ++j) a.ow[wave][g][d0 + j] = acc[g][j];
    }
    __syncthreads();
    const int stride = kPS;
    for (int i = tid; i < G * kD; i += kT) {
        const int g = i >> 7, d = i & 127;
        static_assert(kW == 4, "the wave reduction below sums 4 waves");
        const float o = (a.ow[0][g][d] + a.ow[1][g][d]) + (a.ow[2][g][d] + a.ow[3][g][d]);
        if (p.C == 1) {
            stc(p.attn + (size_t)(h * G + g) * kD + d, o / a.lstat[g]);
        } else {
            float* pp = p.part + (((size_t)h * p.C + c) * G + g) * stride;
            stc(pp + 4 + d, o);
            if (d == 0) {
                stc(pp, a.mstat[g]);
                stc(pp + 1, a.lstat[g]);
            }
        }
    }
    if (p.C == 1) return;
    // the last chunk of this kv head to finish merges the partials
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(p.sync + w_head(l, h, p.Hkv), 1u,
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.last = old == (unsigned)(p.C - 1);
    }
    __syncthreads();
    if (!a.last) return;
    // merge (same formula as attn_combine_kernel): out = sum_c e^{m_c-M} o_c /
    // sum_c e^{m_c-M} l_c. 1) every (chunk, head) statistic into LDS, loads
    // issued together; 2) weights e^{m_c-M}, L per head; 3) o, a float4 of
    // dims per thread, its chunks' loads issued 8 at a time.
    const float* base = p.part + (size_t)h * p.C * G * stride;
    const __amdgpu_buffer_rsrc_t r = rsrc(base, (uint32_t)(p.C * G * stride) * 4);
    const int npairs = p.C * G;
    float* wts = &a.sc[0][0];  // [C][G] weights (the scores are no longer needed)
    float* lcs = wts + npairs;
    for (int i0 = tid; i0 < npairs; i0 += 4 * kT) {
        f4v v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = ldc16(r, (uint32_t)(i0 + u * kT) * stride * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * kT;
            if (i < npairs) {
                wts[i] = v[u].x;
                lcs[i] = v[u].y;
            }
        }
    }
    __syncthreads();
    for (int g = wave; g < G; g += kW) {  // one wave per head, lanes over chunks
        float M = -1e30f;
        for (int cc = lane; cc < p.C; cc += 64) M = fmaxf(M, wts[cc * G + g]);
        M = wave_max(M);
        float L = 0.0f;
        for (int cc = lane; cc < p.C; cc += 64) {
            const float e = expf(wts[cc * G + g] - M);
            wts[cc * G + g] = e;
            L = __builtin_fmaf(e, lcs[cc * G + g], L);
        }
        L = wave_sum_tree(L);
        if (lane == 0) a.mstat[g] = L;
    }
    __syncthreads();
    constexpr int kSlots = G * kD / 4;          // float4 slots of the G outputs
    constexpr int kSplit = kT / kSlots > 0 ? kT / kSlots : 1;  // threads per slot
    const int slot = tid % kSlots, part = tid / kSlots;
    f4v acc4 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (part < kSplit) {
        const int g = slot / (kD / 4), d4 = slot % (kD / 4);
        for (int c0 = part; c0 < p.C; c0 += 8 * kSplit) {
            f4v v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int cc = c0 + u * kSplit;
                v[u] = ldc16(r, (uint32_t)((cc * G + g) * stride + 4 + 4 * d4) * 4);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int cc = c0 + u * kSplit;
                if (cc < p.C) {
                    const float e = wts[cc * G + g];
                    acc4.x = __builtin_fmaf(e, v[u].x, acc4.x);
                    acc4.y = __builtin_fmaf(e, v[u].y, acc4.y);
                    acc4.z = __builtin_fmaf(e, v[u].z, acc4.z);
                    acc4.w = __builtin_fmaf(e, v[u].w, acc4.w);
                }
            }
        }
    }
    float* red = &a.ow[0][0][0];  // [kSplit][G*128]
    if (part < kSplit) {
        red[part * G * kD + 4 * slot] = acc4.x;
        red[part * G * kD + 4 * slot + 1] = acc4.y;
        red[part * G * kD + 4 * slot + 2] = acc4.z;
        red[part * G * kD + 4 * slot + 3] = acc4.w;
    }
    __syncthreads();
    for (int i = tid; i < G * kD; i += kT) {
        const int g = i >> 7, d = i & 127;
        float o = 0.0f;
        for (int q = 0; q < kSplit; ++q) o += red[q * G * kD + i];
        stc(p.attn + (size_t)(h * G + g) * kD + d, o / a.mstat[g]);
    }
}

// ------------------------------------------------------------ LM head -----

__device__ __forceinline__ void am_combine(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(i, o, 64);
        am_combine(v, i, ov, oi);
    }
}

// ---------------------------------------------------------------- kernel --

template <int G>
__global__ void __launch_bounds__(kT, 1) decode_step_kernel(DsParams p) {
    __shared__ SharedAll sh;
    __shared__ int s_abort;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wg = blockIdx.x;
    const int qd = p.Hq * kD, kvd = p.Hkv * kD;
    const int KSH = p.H / 64, KSF = p.F / 64;
    const int nstages = 5 * p.L + (p.with_head ? 1 : 0);
    unsigned gen = 0;

    int off = 0;  // first workgroup of the current stage
    for (int s = 0; s < nstages; ++s) {
        const int kind = kind_of(p, s);
        const int l = s / 5;
        const int n = ntasks(p, s < 5 * p.L ? kind : S_HEAD);
        const int first = (wg - off + p.nwg) % p.nwg;  // my first task index here
        const bool have = first < n;

        if (kind == S_ATT) {
            for (int t = first; t < n; t += p.nwg) {
                uint4 tile[2 * kAR];
                uint32_t tiles[kAR];
                load_att_tile(tile, tiles, p, l, t / p.C, t % p.C);
                attn_task<G>(sh, p, tile, tiles, l, t / p.C, t % p.C);
                __syncthreads();
            }
        } else if (have || kind == S_HEAD) {
            const DsLayer& Lw = p.layers[l < p.L ? l : 0];
            const int slot = kind == S_QKV ? 0 : kind - 1;  // 0..3 for the TL1 stages
            const uint4* W = kind == S_HEAD ? nullptr : Lw.mat[slot];
            const int KS = slot == 3 ? KSF : KSH;
            // the first weight tile is in flight while the input is normalized
            uint4 tile[kPF];
            if (kind != S_HEAD && have) load_tl1_tile(tile, W, first, KS);
            // prologue: the stage input vector and the norm weights into LDS
            // (all loads issued together), then norm + quantize
            const float* nw = kind == S_HEAD ? p.final_norm : Lw.norm[slot];
            int K = kind == S_DOWN ? p.F : p.H;
            if (nw) load_ro(sh.s.ws, nw, K);
            if (kind == S_QKV) {
                if (l == 0) {  // embedding_lookup (:1294-1316) from the packed head
                    const int tok = p.io[0];
                    const float es = p.head_scales[tok];
                    const uint8_t* hb = reinterpret_cast<const uint8_t*>(p.head);
                    const size_t b = tok >> 6, r = tok & 63;
                    for (int i = tid; i < p.H; i += kT) {
                        const int8_t e =
                            (int8_t)hb[((b * (p.H / 16) + (i >> 4)) * 64 + r) * 16 + (i & 15)];
                        sh.s.xs[i] = (float)e * es;
                    }
                } else {
                    load_vec(sh.s.xs, p.x, p.H);
                }
            } else if (kind == S_O) {
                load_vec(sh.s.xs, p.attn, p.H);
            } else if (kind == S_GU) {
                load_vec(sh.s.xs, p.h1, p.H);
            } else if (kind == S_DOWN) {
                load_act(sh.s.xs, p.gu, p.F);
            } else {  // S_HEAD
                load_vec(sh.s.xs, p.x, p.H);
            }
            __syncthreads();
            const float* nws = nw ? sh.s.ws : nullptr;
            if (kind == S_HEAD) norm_quant<127>(sh, K, nws, p.eps);
            else norm_quant<31>(sh, K, nws, p.eps);
            const float inv = sh.s.inv_scale;
            const int csum = sh.s.code_sum;

            if (kind == S_HEAD) {
                // int8 GEMV over row blocks wg, wg+nwg, ... with the greedy argmax
                const int HC = p.H / 16;
                const int4* c4 = reinterpret_cast<const int4*>(sh.s.codes);
                float best = -INFINITY;
                int besti = INT_MAX;
                for (int t = first; t < n; t += p.nwg) {
                    const uint4* wb = p.head + (size_t)t * HC * 64 + lane;
                    int acc = 0;
                    for (int c0 = wave; c0 < HC; c0 += 8 * kW) {
                        uint4 v[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            const int c = c0 + u * kW;
                            v[u] = c < HC ? wb[(size_t)c * 64] : make_uint4(0, 0, 0, 0);
                        }
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            const int c = c0 + u * kW;
                            if (c < HC) {
                                const int4 a4 = c4[c];
                                acc = sdot4(v[u].x, a4.x, acc);
                                acc = sdot4(v[u].y, a4.y, acc);
                                acc = sdot4(v[u].z, a4.z, acc);
                                acc = sdot4(v[u].w, a4.w, acc);
                            }
                        }
                    }
                    sh.s.red_i[wave][lane] = acc;
                    __syncthreads();
                    if (wave == 0) {
                        int tot = 0;
#pragma unroll
                        for (int w = 0; w < kW; ++w) tot += sh.s.red_i[w][lane];
                        const int row = t * 64 + lane;
                        if (row < p.V) {
                            const float val = (float)tot * (inv * p.head_scales[row]);
                            p.logits[row] = val;
                            am_combine(best, besti, val, row);
                        }
                    }
                    __syncthreads();
                }
                // per-workgroup partial, then the last workgroup reduces (:1745-1755)
                if (wave == 0) {
                    wave_argmax(best, besti);
                    if (lane == 0) {
                        stc(&p.am_part[wg].x, best);
                        stc(&p.am_part[wg].y, __int_as_float(besti));
                    }
                }
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                if (tid == 0) {
                    const unsigned old =
                        __hip_atomic_fetch_add(p.sync + w_am(p.L, p.Hkv), 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                    sh.s.flag = old == (unsigned)(p.nwg - 1);
                }
                __syncthreads();
                if (sh.s.flag && wave == 0) {
                    float v = -INFINITY;
                    int vi = INT_MAX;
                    for (int q = lane; q < p.nwg; q += 64)
                        am_combine(v, vi, ldc(&p.am_part[q].x),
                                   __float_as_int(ldc(&p.am_part[q].y)));
                    wave_argmax(v, vi);
                    if (lane == 0) {
                        p.io[2] = vi;
                        p.io[0] = vi;  // the next step's input when steps are chained
                        if (p.out_tokens) p.out_tokens[p.step] = vi;
                    }
                }
                if (p.trace && tid == 0) {
                    const uint64_t now = wall_clock64();
                    p.trace[((size_t)s * p.nwg + wg) * 2] = now;
                    p.trace[((size_t)s * p.nwg + wg) * 2 + 1] = now;
                }
                return;
            }

            // TL1 stages
            for (int t = first; t < n; t += p.nwg) {
                if (t != first) load_tl1_tile(tile, W, t, KS);
                const int tot = tl1_rowblock(sh, tile, W, t, KS);
                if (wave == 0) {
                    const int row = t * 64 + lane;
                    const int v = tot - csum;
                    float sc;
                    if (kind == S_QKV) sc = row < qd ? Lw.sc[0] : row < qd + kvd ? Lw.sc[1] : Lw.sc[2];
                    else if (kind == S_O) sc = Lw.sc[3];
                    else if (kind == S_GU) sc = row < p.F ? Lw.sc[4] : Lw.sc[5];
                    else sc = Lw.sc[6];
                    const float y = (float)v * (inv * sc);  // :1554, :118-126
                    if (kind == S_QKV) stc(p.qkv + row, y);
                    else if (kind == S_O) {
                        // residual 1 (:1590); layer 0 reads the embedding WG 0 wrote
                        stc(p.h1 + row, ldc(p.x + row) + y);
                    } else if (kind == S_GU) stc(p.gu + row, y);
                    else stc(p.x + row, ldc(p.h1 + row) + y);  // residual 2 (:1628)
                }
            }
        }
        // layer 0: workgroup 0 publishes the embedded token for the O residual
        if (s == 0 && wg == 0) {
            const int tok = p.io[0];
            const float es = p.head_scales[tok];
            const uint8_t* hb = reinterpret_cast<const uint8_t*>(p.head);
            const size_t b = tok >> 6, r = tok & 63;
            for (int i = tid; i < p.H; i += kT) {
                const int8_t e = (int8_t)hb[((b * (p.H / 16) + (i >> 4)) * 64 + r) * 16 + (i & 15)];
                stc(p.x + i, (float)e * es);
            }
        }
        off = (off + n) % p.nwg;
        if (p.trace && tid == 0) p.trace[((size_t)s * p.nwg + wg) * 2] = wall_clock64();
        if (!grid_barrier(p, gen, &s_abort)) return;
        if (p.trace && tid == 0) p.trace[((size_t)s * p.nwg + wg) * 2 + 1] = wall_clock64();
    }
}

}  // namespace

size_t ds_sync_words(int L, int Hkv) { return (size_t)(kNC + 2 + L * Hkv) * 64; }
size_t ds_error_word(int L, int Hkv) { return w_err(L, Hkv); }

int ds_grid_size() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    int coop = 0, cus = 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess ||
        !coop)
        return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<4>, kT, 0) !=
            hipSuccess ||
        per_cu < 1)
        return 0;
    const int n = (cus / kNC) * kNC;
    return n;
}

void ds_chunking(int ctx, int Hkv, int nwg, int* C, int* T) {
    int c = (nwg * 3 / 4) / Hkv;  // leave room for the QKV tasks of the stage before
    if (c < 1) c = 1;
    if (c > ctx) c = ctx;
    int t = (ctx + c - 1) / c;
    if (t > kTmax) {
        t = kTmax;
        c = (ctx + t - 1) / t;
    }
    c = (ctx + t - 1) / t;  // no empty chunks
    *C = c;
    *T = t;
    // the merge keeps C x G chunk statistics (2 floats each) in the score
    // buffer: C * G <= 8 * kTmax / 2 holds for every C chosen here
    // (C <= max(3 nwg / 4, ctx / kTmax) with G <= 8)
}

int launch_decode_step(const DsParams& p, int G, hipStream_t st) {
    void* args[] = {const_cast<DsParams*>(&p)};
    void* fn = nullptr;
    switch (G) {
        case 1: fn = (void*)decode_step_kernel<1>; break;
        case 2: fn = (void*)decode_step_kernel<2>; break;
        case 4: fn = (void*)decode_step_kernel<4>; break;
        case 8: fn = (void*)decode_step_kernel<8>; break;
        default:
            set_error("decode step: query heads per kv head must be 1, 2, 4 or 8");
            return TENZO_ERROR_UNSUPPORTED;
    }
    hipError_t e = hipLaunchCooperativeKernel(fn, dim3(p.nwg), dim3(kT), args, 0, st);
    if (e != hipSuccess) return hip_fail(e, "hipLaunchCooperativeKernel(decode_step)");
    return TENZO_SUCCESS;
}

}  // namespace tz

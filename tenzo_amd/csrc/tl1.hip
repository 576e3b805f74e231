// TL1 ternary GEMV on gfx950: device weight layout, activation quantization
// (optionally fused with RMSNorm) and a split-K GEMV on v_dot4_i32_i8.
//
// Reference: src/runtime/TenzoEngine.cpp:22-166 (build_lut,
// compute_single_block, compute_from_lut, rms_norm_raw).
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "common.h"
#include "tl1.h"

namespace tz {

// ------------------------------------------------------------------------
// Device layout. For row block b (64 rows) and super-chunk s (64 columns)
// there are 64 x 16 bytes: the 16 bytes of row r hold its 64 columns as four
// dwords; dword q covers columns 64s+16q+c (c = 0..15) as 2-bit codes
// u = w + 1 in {0, 1, 2} at bit 8*(c%4) + 2*(c/4). So (dword >> 2j) & 0x03030303
// has the codes of columns 16q+4j .. 16q+4j+3 in byte order, ready for one
// v_dot4 against four consecutive activation codes, and
//     sum_k w_k a_k = sum_k u_k a_k - sum_k a_k.
// A wave reads one super-chunk of its row block as 1 KiB contiguous (lane =
// row); columns past K are padded with u = 1 (w = 0).
// ------------------------------------------------------------------------

__global__ void tl1_repack_kernel(const uint8_t* __restrict__ src, uint32_t* __restrict__ dst,
                                  int64_t nb, int64_t kh, int64_t KS) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nb * KS * 256) return;
    const int q = (int)(idx & 3);
    const int r = (int)((idx >> 2) & 63);
    const int64_t bs = idx >> 8;
    const int64_t s = bs % KS;
    const int64_t b = bs / KS;
    uint32_t out = 0;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int64_t kp = s * 32 + q * 8 + m;  // column pair (2kp, 2kp+1)
        uint32_t nib = 5u;                      // (w0, w1) = (0, 0)
        if (kp < kh) {
            const uint32_t byte = src[(b * kh + kp) * 32 + (r & 31)];
            nib = (r < 32) ? (byte & 15u) : (byte >> 4);
        }
        const int c0 = 2 * m, c1 = 2 * m + 1;
        out |= (nib & 3u) << (8 * (c0 & 3) + 2 * (c0 >> 2));
        out |= (nib >> 2) << (8 * (c1 & 3) + 2 * (c1 >> 2));
    }
    dst[idx] = out;
}

// The same device layout straight from the raw 2-bit layout the model
// loader reads (pack_ternary_weights_raw, TenzoEngine.cpp:1842-1884): byte
// (r/4, c) of a [N/4][K] array holds row r's column c at bits 2(r%4), as
// w + 1. Columns past K are padded with u = 1.
__global__ void tl1_repack_raw_kernel(const uint8_t* __restrict__ raw, uint32_t* __restrict__ dst,
                                      int64_t nb, int64_t K, int64_t KS) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nb * KS * 256) return;
    const int q = (int)(idx & 3);
    const int r = (int)((idx >> 2) & 63);
    const int64_t bs = idx >> 8;
    const int64_t s = bs % KS;
    const int64_t b = bs / KS;
    const int64_t row = b * 64 + r;
    const uint8_t* src = raw + (row >> 2) * K;
    const int shift = 2 * (int)(row & 3);
    uint32_t out = 0;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const int64_t col = s * 64 + q * 16 + c;
        const uint32_t u = col < K ? (uint32_t)((src[col] >> shift) & 3) : 1u;
        out |= u << (8 * (c & 3) + 2 * (c >> 2));
    }
    dst[idx] = out;
}

// ------------------------------------------------------------------------
// Activation quantization, one 256-thread block per token.
//   QMAX 31  : build_lut (:28-42): amax floor 1e-6, code = round(v * (31/amax)),
//              inv_scale = amax * (1/31) (the reference build folds the divide).
//   QMAX 127 : compute_logits (:1666-1678): amax floor 1e-8, code =
//              clamp(round(v * (127/amax)), -128, 127), inv_scale = amax * (1/127).
// MODE 0: codes of x; MODE 1: codes of rms_norm_raw(x, w); MODE 2: only the
// normalized vector (executeRMSNorm); MODE 3: x holds gate | up (2K values)
// and the row is act = max(0, gate)^2 * up (:1616-1620) before the norm.
// ------------------------------------------------------------------------
template <int MODE>
__device__ __forceinline__ float act_in(const float* __restrict__ xm, int64_t K, int64_t i) {
    if (MODE == 3) {
        const float r = fmaxf(0.0f, xm[i]);
        return __fmul_rn(__fmul_rn(r, r), xm[K + i]);
    }
    return xm[i];
}

// Rows up to this length are staged in LDS (chain layout) for the sum of
// squares; longer rows (the operator entry points accept any length) run the
// same chains from memory.
constexpr int64_t kChainMaxK = 16128;  // 8 * chain_ld(K) floats fit in 64 KiB

// inv_rms of rms_norm_raw for row xm (act_in values), in the reference build's
// arithmetic. ct: dynamic LDS of 8 * chain_ld(K) floats when K <= kChainMaxK;
// s_inv: a float of LDS. All 256 threads call it; the row is in ct (chain
// layout) afterwards.
template <int MODE>
__device__ __forceinline__ float act_inv_rms(const float* __restrict__ xm, int64_t K, float eps,
                                             float* ct, float* s_inv) {
    const int t = threadIdx.x;
    if (K <= kChainMaxK) {
        const int ld = chain_ld(K);
        for (int64_t i = t; i < K; i += 256) ct[chain_pos(i, ld)] = act_in<MODE>(xm, K, i);
        __syncthreads();
        if (t < 64) {
            const float ss = chain_sumsq_wave(ct, ld, K);
            if (t == 0) *s_inv = inv_rms_ref(ss, K, eps, kRsqrtEstTab);
        }
    } else if (t < 64) {
        // chain j = t % 8 over elements j, j + 8, ... from memory
        const int j = t & 7;
        const int64_t n8 = K >> 3;
        float s = 0.0f;
        for (int64_t k = 0; k < n8; ++k) {
            const float v = act_in<MODE>(xm, K, 8 * k + j);
            s = __builtin_fmaf(v, v, s);
        }
        if (j == 0)
            for (int64_t i = 8 * n8; i < K; ++i) {
                const float v = act_in<MODE>(xm, K, i);
                s = __builtin_fmaf(v, v, s);
            }
        const float c0 = lane_f(s, 0), c1 = lane_f(s, 1), c2 = lane_f(s, 2), c3 = lane_f(s, 3);
        const float c4 = lane_f(s, 4), c5 = lane_f(s, 5), c6 = lane_f(s, 6), c7 = lane_f(s, 7);
        const float ss = ((c0 + c4) + (c2 + c6)) + ((c1 + c5) + (c3 + c7));
        if (t == 0) *s_inv = inv_rms_ref(ss, K, eps, kRsqrtEstTab);
    }
    __syncthreads();
    return *s_inv;
}

template <int MODE, int QMAX>
__global__ void __launch_bounds__(256)
actquant_kernel(const float* __restrict__ x, const float* __restrict__ w, float eps, int64_t K,
                int64_t Kp, int8_t* __restrict__ codes, tenzo_hip_actq_t* __restrict__ q,
                float* __restrict__ y_out) {
    extern __shared__ float ct[];  // chain layout of the row (MODE >= 1, K <= kChainMaxK)
    __shared__ float redf[4];
    __shared__ int redi[4];
    __shared__ float s_inv;
    const int t = threadIdx.x;
    const int64_t m = blockIdx.x;
    const float* xm = x + m * (MODE == 3 ? 2 * K : K);
    float inv_rms = 1.0f;
    if (MODE >= 1) inv_rms = act_inv_rms<MODE>(xm, K, eps, ct, &s_inv);
    if (MODE == 2) {
        for (int64_t i = t; i < K; i += 256) y_out[m * K + i] = norm_apply(xm[i], inv_rms, w, i);
        return;
    }
    float amax = QMAX == 31 ? 1e-6f : 1e-8f;
    for (int64_t i = t; i < K; i += 256) {
        const float a = act_in<MODE>(xm, K, i);
        const float v = MODE >= 1 ? norm_apply(a, inv_rms, w, i) : a;
        amax = fmaxf(amax, fabsf(v));
    }
    amax = block256_max(amax, redf);
    const float scale_act = __fdiv_rn((float)QMAX, amax);
    int csum = 0;
    int8_t* cm = codes + m * Kp;
    for (int64_t i = t; i < Kp; i += 256) {
        int c = 0;
        if (i < K) {
            const float a = act_in<MODE>(xm, K, i);
            const float v = MODE >= 1 ? norm_apply(a, inv_rms, w, i) : a;
            if (MODE >= 1 && y_out) y_out[m * K + i] = v;
            float r = roundf(__fmul_rn(v, scale_act));
            if (QMAX == 127) r = fminf(fmaxf(r, -128.0f), 127.0f);
            c = (int)r;
        }
        cm[i] = (int8_t)c;
        csum += c;
    }
    csum = block256_sum_i32(csum, redi);
    if (t == 0) {
        q[m].inv_scale = __fmul_rn(amax, 1.0f / (float)QMAX);
        q[m].code_sum = csum;
    }
}

// Dynamic LDS of actquant_kernel for a row of K.
static size_t actquant_lds(int mode, int64_t K) {
    return mode >= 1 && K <= kChainMaxK ? (size_t)8 * chain_ld(K) * 4 : 0;
}

// The same quantization with the row held in registers: thread t loads its
// float4 groups t + 256 j (j < J) once, which is also the order of the
// sum of squares above (p[k] accumulates element 4t + 1024 j + k over j), so
// every result equals actquant_kernel's; the row is read from memory once
// instead of three times. K % 4 == 0 and K <= 1024 J.
template <int MODE, int QMAX, int J>
__global__ void __launch_bounds__(256)
actquant_reg_kernel(const float* __restrict__ x, const float* __restrict__ w, float eps,
                    int64_t K, int64_t Kp, int8_t* __restrict__ codes,
                    tenzo_hip_actq_t* __restrict__ q, float* __restrict__ y_out) {
    __shared__ float redf[4];
    __shared__ int redi[4];
    const int t = threadIdx.x;
    const int64_t m = blockIdx.x;
    const float* xm = x + m * (MODE == 3 ? 2 * K : K);
    float4 v[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t i = 4 * t + 1024 * j;
        v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < K) {
            const float4 a = *reinterpret_cast<const float4*>(xm + i);
            if (MODE == 3) {
                const float4 u = *reinterpret_cast<const float4*>(xm + K + i);
                const float r0 = fmaxf(0.0f, a.x), r1 = fmaxf(0.0f, a.y), r2 = fmaxf(0.0f, a.z),
                            r3 = fmaxf(0.0f, a.w);
                v[j] = make_float4(__fmul_rn(__fmul_rn(r0, r0), u.x), __fmul_rn(__fmul_rn(r1, r1), u.y),
                                   __fmul_rn(__fmul_rn(r2, r2), u.z), __fmul_rn(__fmul_rn(r3, r3), u.w));
            } else {
                v[j] = a;
            }
        }
    }
    if (MODE >= 1) {
        // the row into LDS in chain layout; wave 0 sums its squares in the
        // reference build's order
        constexpr int LD = (1024 * J / 8 + 27) / 32 * 32 + 4;  // chain_ld(1024 J)
        __shared__ float ct[8 * LD];
        __shared__ float s_inv;
        const int ld = chain_ld(K);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int64_t i = 4 * t + 1024 * j;
            if (i < K) {
                ct[chain_pos(i, ld)] = v[j].x;
                ct[chain_pos(i + 1, ld)] = v[j].y;
                ct[chain_pos(i + 2, ld)] = v[j].z;
                ct[chain_pos(i + 3, ld)] = v[j].w;
            }
        }
        __syncthreads();
        if (t < 64) {
            const float ss = chain_sumsq_wave(ct, ld, K);
            if (t == 0) s_inv = inv_rms_ref(ss, K, eps, kRsqrtEstTab);
        }
        __syncthreads();
        const float inv_rms = s_inv;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int64_t i = 4 * t + 1024 * j;
            if (i < K) {
                v[j].x = norm_apply(v[j].x, inv_rms, w, i);
                v[j].y = norm_apply(v[j].y, inv_rms, w, i + 1);
                v[j].z = norm_apply(v[j].z, inv_rms, w, i + 2);
                v[j].w = norm_apply(v[j].w, inv_rms, w, i + 3);
                if (y_out) *reinterpret_cast<float4*>(y_out + m * K + i) = v[j];
            }
        }
        if (MODE == 2) return;
    }
    float amax = QMAX == 31 ? 1e-6f : 1e-8f;
#pragma unroll
    for (int j = 0; j < J; ++j)
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)),
                                 fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    amax = block256_max(amax, redf);
    const float scale_act = __fdiv_rn((float)QMAX, amax);
    int csum = 0;
    int8_t* cm = codes + m * Kp;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t i = 4 * t + 1024 * j;
        if (i >= Kp) continue;
        int c[4] = {0, 0, 0, 0};
        if (i < K) {
            const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float r = roundf(__fmul_rn(e[k], scale_act));
                if (QMAX == 127) r = fminf(fmaxf(r, -128.0f), 127.0f);
                c[k] = (int)r;
            }
        }
        csum += (c[0] + c[1]) + (c[2] + c[3]);
        *reinterpret_cast<uint32_t*>(cm + i) = (uint32_t)(c[0] & 0xff) | ((uint32_t)(c[1] & 0xff) << 8) |
                                              ((uint32_t)(c[2] & 0xff) << 16) | ((uint32_t)(c[3] & 0xff) << 24);
    }
    csum = block256_sum_i32(csum, redi);
    if (t == 0) {
        q[m].inv_scale = __fmul_rn(amax, 1.0f / (float)QMAX);
        q[m].code_sum = csum;
    }
}

// ------------------------------------------------------------------------
// GEMV. Grid (row_blocks * splits, M); 256 threads = 4 waves. A block owns
// one row block (lane = row) and a contiguous range of super-chunks, which
// its 4 waves interleave. Activation codes are wave-uniform and come in
// through scalar loads. Partial int32 sums are exact: with splits > 1 they
// are added atomically into a zeroed accumulator and the last block of the
// row block converts and re-zeroes it.
// ------------------------------------------------------------------------

__device__ __forceinline__ int dot16(const uint4 v, const int32_t* __restrict__ a, int acc) {
    const uint32_t M = 0x03030303u;
    acc = sdot4(v.x & M, a[0], acc);
    acc = sdot4((v.x >> 2) & M, a[1], acc);
    acc = sdot4((v.x >> 4) & M, a[2], acc);
    acc = sdot4((v.x >> 6) & M, a[3], acc);
    acc = sdot4(v.y & M, a[4], acc);
    acc = sdot4((v.y >> 2) & M, a[5], acc);
    acc = sdot4((v.y >> 4) & M, a[6], acc);
    acc = sdot4((v.y >> 6) & M, a[7], acc);
    acc = sdot4(v.z & M, a[8], acc);
    acc = sdot4((v.z >> 2) & M, a[9], acc);
    acc = sdot4((v.z >> 4) & M, a[10], acc);
    acc = sdot4((v.z >> 6) & M, a[11], acc);
    acc = sdot4(v.w & M, a[12], acc);
    acc = sdot4((v.w >> 2) & M, a[13], acc);
    acc = sdot4((v.w >> 4) & M, a[14], acc);
    acc = sdot4((v.w >> 6) & M, a[15], acc);
    return acc;
}

// y = float(acc) * (inv_scale * w_scale) (:1554, :118-126), plus the residual
// add of :1590 / :1628 when resid is given (resid + y, one fp32 add).
__device__ __forceinline__ void tl1_finalize(int tot, int64_t m, int64_t row, int64_t N,
                                             const tenzo_hip_actq_t* __restrict__ aq,
                                             const RowScales& rs, float* y,
                                             const float* resid,
                                             int32_t* __restrict__ acc_out) {
    const tenzo_hip_actq_t a = aq[m];
    const int v = tot - a.code_sum;
    int j = 0;
    while (j < rs.n - 1 && row >= rs.end[j]) ++j;
    float out = (float)v * __fmul_rn(a.inv_scale, rs.scale[j]);
    if (resid) out = __fadd_rn(resid[m * N + row], out);
    y[m * N + row] = out;
    if (acc_out) acc_out[m * N + row] = v;
}

constexpr int kTl1J = 16;     // super-chunk loads a lane keeps in flight
constexpr int kTl1CU = 1024;  // 16-byte units of staged codes (256 super-chunks per block)

__global__ void __launch_bounds__(256)
tl1_gemv_kernel(const uint4* __restrict__ w, const int8_t* __restrict__ codes,
                const tenzo_hip_actq_t* __restrict__ aq, int64_t N, int64_t KS, int splits,
                RowScales rs, float* y, const float* resid, int32_t* __restrict__ acc_out,
                int32_t* __restrict__ ws_acc, uint32_t* __restrict__ ws_cnt) {
    __shared__ int red[4][64];
    __shared__ int is_last;
    __shared__ uint4 cs[kTl1CU + 256];  // codes, then one spare slot per thread
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nb = N >> 6;
    const int64_t b = blockIdx.x / splits;
    const int sp = (int)(blockIdx.x - b * splits);
    const int64_t m = blockIdx.y;
    const int64_t per = (KS + splits - 1) / splits;
    const int64_t s0 = sp * per;
    const int64_t s1 = s0 + per < KS ? s0 + per : KS;
    const uint4* wb = w + b * KS * 64 + lane;
    const uint4* c4 = reinterpret_cast<const uint4*>(codes + m * KS * 64);
    // the block's activation codes (64 bytes per super-chunk) into LDS first, one 16-byte
    // load per thread (past the end: into the thread's own spare slot, no branch), so the
    // dot steps read them as LDS broadcasts instead of one scalar-load round trip per
    // super-chunk; then the wave's super-chunks s0 + wave + 4 j, all of their weight loads
    // in flight together (up to kTl1J; beyond, in further rounds)
    const int cu = (int)(s1 - s0) * 4;  // 16-byte units of the block's codes
    {
        const int t = threadIdx.x;
        const uint4 cv = c4[min(s0, KS - 1) * 4 + max(0, min(t, cu - 1))];  // (empty split: any)
        const int64_t nj = s1 > s0 + wave ? (s1 - s0 - wave + 3) / 4 : 0;  // wave-uniform
        uint4 v[kTl1J];
#pragma unroll
        for (int j = 0; j < kTl1J; ++j)
            if (j < nj) v[j] = ld_nt16(&wb[(s0 + wave + 4 * j) * 64]);
        cs[t < cu ? t : kTl1CU + t] = cv;
        for (int u = t + 256; u < cu; u += 256) cs[u] = c4[s0 * 4 + u];
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int32_t* a32 = reinterpret_cast<const int32_t*>(cs);
        int acc = 0;
#pragma unroll
        for (int j = 0; j < kTl1J; ++j)
            if (j < nj) acc = dot16(v[j], a32 + (wave + 4 * j) * 16, acc);
        for (int64_t j0 = kTl1J; j0 < nj; j0 += kTl1J) {
#pragma unroll
            for (int j = 0; j < kTl1J; ++j)
                if (j0 + j < nj) v[j] = ld_nt16(&wb[(s0 + wave + 4 * (j0 + j)) * 64]);
#pragma unroll
            for (int j = 0; j < kTl1J; ++j)
                if (j0 + j < nj) acc = dot16(v[j], a32 + (wave + 4 * (j0 + j)) * 16, acc);
        }
        red[wave][lane] = acc;
    }

    __syncthreads();
    const int64_t row = b * 64 + lane;
    if (splits == 1) {
        if (wave == 0) {
            const int tot = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
            tl1_finalize(tot, m, row, N, aq, rs, y, resid, acc_out);
        }
        return;
    }
    if (wave == 0) {
        const int tot = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
        atomicAdd(&ws_acc[m * N + row], tot);
    }
    partials_acked();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = atomicAdd(&ws_cnt[m * nb + b], 1u);
        is_last = prev == (unsigned)(splits - 1);
    }
    __syncthreads();
    if (is_last && wave == 0) {
        const int tot = atomicExch(&ws_acc[m * N + row], 0);
        tl1_finalize(tot, m, row, N, aq, rs, y, resid, acc_out);
        if (lane == 0) atomicExch(&ws_cnt[m * nb + b], 0u);
    }
}

// ------------------------------------------------------------------------
// The GEMV on fp32 activations -- the unit of executeBitLinearTL1
// (ROCmRuntime.h:20-28): build_lut's quantization then compute_from_lut
// (TenzoEngine.cpp:22-146) -- as one launch. Every block quantizes row m of x
// itself with actquant_kernel<0, 31>'s arithmetic (absmax with the 1e-6
// floor, scale 31 / absmax correctly rounded, codes roundf(x * scale),
// inv_scale = absmax * (1/31)) into its LDS code stage while its weight loads
// are in flight, then takes tl1_gemv_kernel's dot steps over whole rows
// (no K split). Every block forms the same codes, so the outputs equal the
// two-launch path's bit for bit. J float4 groups of x per thread: the padded
// row (KS * 64 codes) is at most 1024 J; K % 4 == 0.
// ------------------------------------------------------------------------
template <int J>
__global__ void __launch_bounds__(256)
tl1_gemv_f32_kernel(const uint4* __restrict__ w, const float* __restrict__ x, int64_t N,
                    int64_t K, int64_t KS, RowScales rs, float* __restrict__ y) {
    __shared__ int red[4][64];
    __shared__ float redf[4];
    __shared__ int redi[4];
    __shared__ uint32_t cs[J * 256];  // the row's codes, four to a word (zero past K)
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int64_t b = blockIdx.x, m = blockIdx.y;
    const uint4* wb = w + b * KS * 64 + lane;
    // the row first (vector loads return in issue order), then every weight
    // load of the wave (up to kTl1J; beyond, in further rounds below)
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + m * K), 0, (int)(K * 4), 0x00020000);
    float xv[J][4];
#pragma unroll
    for (int j = 0; j < J; ++j) {  // groups past K read zeros (outside the resource)
        const uint4 u = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, (t + 256 * j) * 16, 0, 0));
        xv[j][0] = __uint_as_float(u.x);
        xv[j][1] = __uint_as_float(u.y);
        xv[j][2] = __uint_as_float(u.z);
        xv[j][3] = __uint_as_float(u.w);
    }
    const int64_t nj = KS > wave ? (KS - wave + 3) / 4 : 0;  // wave-uniform
    uint4 v[kTl1J];
#pragma unroll
    for (int j = 0; j < kTl1J; ++j)
        if (j < nj) v[j] = ld_nt16(&wb[(wave + 4 * j) * 64]);
    float amax = 1e-6f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(xv[j][e]));
    amax = block256_max(amax, redf);
    const float scale = __fdiv_rn(31.0f, amax);
    int csum = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        int c[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) c[e] = (int)roundf(__fmul_rn(xv[j][e], scale));
        cs[t + 256 * j] = (uint32_t)(c[0] & 0xff) | (uint32_t)(c[1] & 0xff) << 8 |
                          (uint32_t)(c[2] & 0xff) << 16 | (uint32_t)(c[3] & 0xff) << 24;
        csum += (c[0] + c[1]) + (c[2] + c[3]);
    }
    csum = block256_sum_i32(csum, redi);  // (its block barriers publish the codes)
    const int32_t* a32 = reinterpret_cast<const int32_t*>(cs);
    int acc = 0;
#pragma unroll
    for (int j = 0; j < kTl1J; ++j)
        if (j < nj) acc = dot16(v[j], a32 + (wave + 4 * j) * 16, acc);
    for (int64_t j0 = kTl1J; j0 < nj; j0 += kTl1J) {
#pragma unroll
        for (int j = 0; j < kTl1J; ++j)
            if (j0 + j < nj) v[j] = ld_nt16(&wb[(wave + 4 * (j0 + j)) * 64]);
#pragma unroll
        for (int j = 0; j < kTl1J; ++j)
            if (j0 + j < nj) acc = dot16(v[j], a32 + (wave + 4 * (j0 + j)) * 16, acc);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const int tot = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
        const int64_t row = b * 64 + lane;
        int j = 0;
        while (j < rs.n - 1 && row >= rs.end[j]) ++j;
        const float inv_scale = __fmul_rn(amax, 1.0f / 31.0f);
        y[m * N + row] = (float)(tot - csum) * __fmul_rn(inv_scale, rs.scale[j]);
    }
}

// ------------------------------------------------------------------------
// The same GEMV by the reference's own method (build_lut :22-62,
// compute_single_block :64-127): a 16-entry int8 table per activation pair
// (entry u0 | u1 << 2 = (u0 - 1) a0 + (u1 - 1) a1), staged in LDS, looked up
// with each 4-bit pair of weight codes. It reads the same packed weights as
// tl1_gemv_kernel, whose 4-bit nibbles pair the columns (16i + b, 16i + 4 + b)
// (low nibble of byte b of dword i) and (16i + 8 + b, 16i + 12 + b) (high
// nibble) of a super-chunk; the lookup is two byte permutes (v_perm, the
// pshufb of the reference) and a select. The tables hold the reference's
// values (w in {-1, 0, +1}), so the sum is sum w a directly; tl1_finalize
// takes sum (w + 1) a - code_sum, hence the code sum added back before it.
// The int32 sums are exact, so the
// results equal tl1_gemv_kernel's bit for bit; the kernel exists to measure
// the table method against the masked v_dot4 one (same grid, same splits).
// ------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
tl1_lut_gemv_kernel(const uint4* __restrict__ w, const int8_t* __restrict__ codes,
                    const tenzo_hip_actq_t* __restrict__ aq, int64_t N, int64_t KS, int splits,
                    RowScales rs, float* y, int32_t* __restrict__ acc_out,
                    int32_t* __restrict__ ws_acc, uint32_t* __restrict__ ws_cnt) {
    extern __shared__ uint4 lut[];  // [(s1 - s0) * 32 pairs] tables of 16 bytes
    __shared__ int red[4][64];
    __shared__ int is_last;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nb = N >> 6;
    const int64_t b = blockIdx.x / splits;
    const int sp = (int)(blockIdx.x - b * splits);
    const int64_t m = blockIdx.y;
    const int64_t per = (KS + splits - 1) / splits;
    const int64_t s0 = sp * per;
    const int64_t s1 = s0 + per < KS ? s0 + per : KS;
    const int8_t* cm = codes + m * KS * 64;
    // the tables of the block's super-chunks
    for (int64_t q = threadIdx.x; q < (s1 - s0) * 32; q += 256) {
        const int64_t sc = s0 + q / 32;
        const int i = (int)(q % 32) / 8, bb = (int)(q % 8) / 2, hh = (int)(q % 2);
        const int64_t c0 = sc * 64 + 16 * i + 8 * hh + bb;
        const int a0 = cm[c0], a1 = cm[c0 + 4];
        uint32_t t[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int u1 = 0; u1 < 3; ++u1)
#pragma unroll
            for (int u0 = 0; u0 < 3; ++u0) {
                const int idx = u0 | (u1 << 2);
                const int v = min(max((u0 - 1) * a0 + (u1 - 1) * a1, -128), 127);
                t[idx >> 2] |= (uint32_t)(v & 0xff) << (8 * (idx & 3));
            }
        lut[q] = make_uint4(t[0], t[1], t[2], t[3]);
    }
    __syncthreads();
    const uint4* wb = w + b * KS * 64 + lane;
    int acc = 0;
    for (int64_t s = s0 + wave; s < s1; s += 4) {
        const uint4 v = wb[s * 64];
        const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
        const uint4* tb = lut + (s - s0) * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 8; ++k) {  // nibble k: byte k / 2, half k % 2
                const uint4 tab = tb[i * 8 + k];  // the same address in every lane
                const uint32_t nib = (ws[i] >> (4 * k)) & 15u;
                const uint32_t sel = nib & 7u;
                const uint32_t lo = __builtin_amdgcn_perm(tab.y, tab.x, sel);
                const uint32_t hi = __builtin_amdgcn_perm(tab.w, tab.z, sel);
                acc += (int)(int8_t)((nib & 8u) ? hi : lo);
            }
    }
    red[wave][lane] = acc;
    __syncthreads();
    const int64_t row = b * 64 + lane;
    if (splits == 1) {
        if (wave == 0) {
            const int tot = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
            tl1_finalize(tot + aq[m].code_sum, m, row, N, aq, rs, y, nullptr, acc_out);
        }
        return;
    }
    if (wave == 0) {
        const int tot = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
        atomicAdd(&ws_acc[m * N + row], tot);
    }
    partials_acked();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = atomicAdd(&ws_cnt[m * nb + b], 1u);
        is_last = prev == (unsigned)(splits - 1);
    }
    __syncthreads();
    if (is_last && wave == 0) {
        const int tot = atomicExch(&ws_acc[m * N + row], 0);
        tl1_finalize(tot + aq[m].code_sum, m, row, N, aq, rs, y, nullptr, acc_out);
        if (lane == 0) atomicExch(&ws_cnt[m * nb + b], 0u);
    }
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

int tl1_pick_splits(int64_t nb, int64_t KS, int64_t M) {
    // A block's waves keep all their super-chunk loads in flight, so a block can take
    // about 28 super-chunks (7 per wave) before a K split pays for its partials' atomics
    // and the last block's read-back (memory round trips in series); and no more splits
    // than fill the 256 CUs. Measured per call, splits 1 / 2 / 3 / 4 / 6: 6912 x 2560
    // 5.08 / 5.47 / 5.54 / 5.70 / 6.21 us; 2560 x 6912 8.92 / 6.85 / 6.03 / 5.86 / 5.96;
    // 3840 x 2560 4.97 / 5.18 / 5.19 / 5.40 / 5.88.
    int64_t want = (KS + 14) / 28;
    const int64_t fill = ceil_div(256, nb * M);
    if (want > fill) want = fill;
    if (want < 1) want = 1;
    return (int)want;
}

int launch_actquant(int mode, int qmax, const float* x, const float* norm_w, float eps,
                    int64_t M, int64_t K, int64_t Kp, int8_t* codes, tenzo_hip_actq_t* q,
                    float* y_out, hipStream_t st) {
    const dim3 grid((unsigned)M), blk(256);
    if (K % 4 == 0 && K <= 16384) {
        const int J = (int)ceil_div(K, 1024);
#define AQR_CASE(MO, QM, JJ)                                                                  \
    if (mode == MO && qmax == QM && J <= JJ) {                                                \
        hipLaunchKernelGGL((actquant_reg_kernel<MO, QM, JJ>), grid, blk, 0, st, x, norm_w, eps, K, \
                           Kp, codes, q, y_out);                                              \
        return launch_status("actquant_reg_kernel");                                          \
    }
#define AQR_MODE(MO, QM) AQR_CASE(MO, QM, 2) AQR_CASE(MO, QM, 4) AQR_CASE(MO, QM, 8) AQR_CASE(MO, QM, 16)
        AQR_MODE(0, 31) AQR_MODE(1, 31) AQR_MODE(3, 31) AQR_MODE(0, 127) AQR_MODE(1, 127)
#undef AQR_MODE
#undef AQR_CASE
    }
#define AQ_CASE(MO, QM)                                                                  \
    if (mode == MO && qmax == QM) {                                                      \
        hipLaunchKernelGGL((actquant_kernel<MO, QM>), grid, blk, actquant_lds(MO, K), st, x,  \
                           norm_w, eps, K, Kp, codes, q, y_out);                         \
        return launch_status("actquant_kernel");                                         \
    }
    AQ_CASE(0, 31) AQ_CASE(1, 31) AQ_CASE(3, 31) AQ_CASE(0, 127) AQ_CASE(1, 127)
#undef AQ_CASE
    set_error("actquant: unsupported mode %d / range %d", mode, qmax);
    return TENZO_ERROR_UNSUPPORTED;
}

int launch_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps,
                   hipStream_t st) {
    hipLaunchKernelGGL((actquant_kernel<2, 31>), dim3(1), dim3(256), actquant_lds(2, dim), st, x,
                       w, eps, dim, dim,
                       (int8_t*)nullptr, (tenzo_hip_actq_t*)nullptr, y);
    return launch_status("rmsnorm");
}

int launch_quant31(const float* x, const float* norm_w, bool do_norm, float eps, int64_t M,
                   int64_t K, int8_t* codes, tenzo_hip_actq_t* q, float* y_out,
                   hipStream_t st) {
    return launch_actquant(do_norm ? 1 : 0, 31, x, norm_w, eps, M, K, ceil_div(K, 64) * 64,
                           codes, q, y_out, st);
}

size_t tl1_ws_bytes(int64_t M, int64_t N) { return (size_t)(M * N + M * (N / 64)) * 4; }

int launch_tl1_gemv(const int8_t* codes, const tenzo_hip_actq_t* q, const void* w_packed,
                    const RowScales& rs, int64_t M, int64_t N, int64_t K, float* y,
                    const float* resid, int32_t* acc_out, hipStream_t st, int splits,
                    void* ws) {
    const int64_t nb = N / 64;
    const int64_t KS = ceil_div(K, 64);
    if (splits <= 0) splits = tl1_pick_splits(nb, KS, M);
    if (splits > KS) splits = (int)KS;
    while (ceil_div(KS, splits) * 4 > kTl1CU) ++splits;  // a block's codes fit the LDS stage
    int32_t* ws_acc = nullptr;
    uint32_t* ws_cnt = nullptr;
    if (splits > 1) {
        if (!ws) ws = Scratch::get(kScratchGemvAcc, tl1_ws_bytes(M, N), st);
        if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
        ws_acc = (int32_t*)ws;
        ws_cnt = (uint32_t*)((char*)ws + (size_t)M * N * 4);
    }
    hipLaunchKernelGGL(tl1_gemv_kernel, dim3((unsigned)(nb * splits), (unsigned)M), dim3(256),
                       0, st, (const uint4*)w_packed, codes, q, N, KS, splits, rs, y, resid,
                       acc_out, ws_acc, ws_cnt);
    return launch_status("tl1_gemv_kernel");
}

int launch_tl1_repack_raw(const uint8_t* raw, void* w_packed, int64_t N, int64_t K,
                          hipStream_t st) {
    const int64_t nb = N / 64, KS = ceil_div(K, 64);
    const int64_t total = nb * KS * 256;
    hipLaunchKernelGGL(tl1_repack_raw_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                       st, raw, (uint32_t*)w_packed, nb, K, KS);
    return launch_status("tl1_repack_raw_kernel");
}

int launch_tl1_repack(const uint8_t* w_tl1, void* w_packed, int64_t N, int64_t K,
                      hipStream_t st) {
    const int64_t nb = N / 64, kh = K / 2, KS = ceil_div(K, 64);
    const int64_t total = nb * KS * 256;
    hipLaunchKernelGGL(tl1_repack_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                       st, w_tl1, (uint32_t*)w_packed, nb, kh, KS);
    return launch_status("tl1_repack_kernel");
}

}  // namespace tz

using namespace tz;

namespace {
std::mutex g_shim_mu;
struct ShimWeights {
    void* packed = nullptr;
    int64_t N = 0, K = 0;
};
std::map<const void*, ShimWeights> g_shim_cache;

int shim_upload(const uint8_t* w, int64_t N, int64_t K, void** out) {
    auto it = g_shim_cache.find(w);
    if (it != g_shim_cache.end() && it->second.N == N && it->second.K == K) {
        *out = it->second.packed;
        return TENZO_SUCCESS;
    }
    if (it != g_shim_cache.end()) {
        TZ_HIP(hipFree(it->second.packed));
        g_shim_cache.erase(it);
    }
    const size_t raw = (size_t)N * K / 4;
    void* staging = nullptr;
    void* packed = nullptr;
    TZ_HIP(hipMalloc(&staging, raw));
    TZ_HIP(hipMalloc(&packed, tenzo_hip_tl1_packed_bytes(N, K)));
    TZ_HIP(hipMemcpy(staging, w, raw, hipMemcpyHostToDevice));
    int st = launch_tl1_repack((const uint8_t*)staging, packed, N, K, nullptr);
    if (st) return st;
    TZ_HIP(hipDeviceSynchronize());
    TZ_HIP(hipFree(staging));
    g_shim_cache[w] = ShimWeights{packed, N, K};
    *out = packed;
    return TENZO_SUCCESS;
}
}  // namespace

extern "C" {

TENZO_HIP_API size_t tenzo_hip_tl1_packed_bytes(int64_t N, int64_t K) {
    return (size_t)(N / 64) * (size_t)ceil_div(K, 64) * 1024;
}

TENZO_HIP_API int tenzo_hip_tl1_repack(const uint8_t* w_tl1, void* w_packed, int64_t N,
                                       int64_t K, void* stream) {
    TZ_CHECK(w_tl1 && w_packed, "tl1_repack: null pointer");
    TZ_CHECK(N > 0 && K > 0 && N % 64 == 0 && K % 2 == 0,
             "tl1_repack: need N %% 64 == 0 and K %% 2 == 0 (N=%lld K=%lld)", (long long)N,
             (long long)K);
    return launch_tl1_repack(w_tl1, w_packed, N, K, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_tl1_repack_raw(const uint8_t* raw, void* w_packed, int64_t N,
                                           int64_t K, void* stream) {
    TZ_CHECK(raw && w_packed, "tl1_repack_raw: null pointer");
    TZ_CHECK(N > 0 && K > 0 && N % 64 == 0,
             "tl1_repack_raw: need N %% 64 == 0 (N=%lld K=%lld)", (long long)N, (long long)K);
    return launch_tl1_repack_raw(raw, w_packed, N, K, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_rmsnorm_quant31(const float* x, const float* norm_w, int do_norm,
                                            float eps, int64_t M, int64_t K, int8_t* codes,
                                            tenzo_hip_actq_t* q, float* y_out, void* stream) {
    TZ_CHECK(x && codes && q, "rmsnorm_quant31: null pointer");
    TZ_CHECK(M > 0 && M <= 65535 && K > 0, "rmsnorm_quant31: bad sizes");
    return launch_quant31(x, norm_w, do_norm || norm_w, eps, M, K, codes, q, y_out,
                          (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_bitlinear_tl1(const int8_t* codes, const tenzo_hip_actq_t* q,
                                          const void* w_packed, float w_scale, int64_t M,
                                          int64_t N, int64_t K, float* y, int32_t* acc_out,
                                          void* stream) {
    TZ_CHECK(codes && q && w_packed && y, "bitlinear_tl1: null pointer");
    TZ_CHECK(M > 0 && M <= 65535 && N > 0 && N % 64 == 0 && K > 0,
             "bitlinear_tl1: need N %% 64 == 0 (N=%lld)", (long long)N);
    RowScales rs = RowScales::single(w_scale);
    return launch_tl1_gemv(codes, q, w_packed, rs, M, N, K, y, nullptr, acc_out,
                           (hipStream_t)stream, 0, nullptr);
}

TENZO_HIP_API int tenzo_hip_bitlinear_tl1_lut(const int8_t* codes, const tenzo_hip_actq_t* q,
                                              const void* w_packed, float w_scale, int64_t M,
                                              int64_t N, int64_t K, float* y, int32_t* acc_out,
                                              void* stream) {
    TZ_CHECK(codes && q && w_packed && y, "bitlinear_tl1_lut: null pointer");
    TZ_CHECK(M > 0 && M <= 65535 && N > 0 && N % 64 == 0 && K > 0,
             "bitlinear_tl1_lut: need N %% 64 == 0 (N=%lld)", (long long)N);
    hipStream_t st = (hipStream_t)stream;
    const int64_t nb = N / 64, KS = ceil_div(K, 64);
    // its own best split: about one block per CU (the table build is per block, so fewer
    // and longer blocks cost it more than they save: 6912 x 2560 takes 17.8 us with 1
    // split, 10.0 with 3)
    int64_t want = ceil_div(256, nb * M);
    if (want > KS / 4) want = KS / 4;
    int splits = want < 1 ? 1 : (int)want;
    const int64_t per = ceil_div(KS, splits);
    const size_t lds = (size_t)per * 32 * 16;
    TZ_CHECK(lds <= 64 * 1024, "bitlinear_tl1_lut: K=%lld needs %zu bytes of tables", (long long)K,
             lds);
    int32_t* ws_acc = nullptr;
    uint32_t* ws_cnt = nullptr;
    if (splits > 1) {
        void* ws = Scratch::get(kScratchGemvAcc, tl1_ws_bytes(M, N), st);
        if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
        ws_acc = (int32_t*)ws;
        ws_cnt = (uint32_t*)((char*)ws + (size_t)M * N * 4);
    }
    hipLaunchKernelGGL(tl1_lut_gemv_kernel, dim3((unsigned)(nb * splits), (unsigned)M), dim3(256),
                       lds, st, (const uint4*)w_packed, codes, q, N, KS, splits,
                       RowScales::single(w_scale), y, acc_out, ws_acc, ws_cnt);
    return launch_status("tl1_lut_gemv_kernel");
}

TENZO_HIP_API int tenzo_hip_bitlinear_tl1_f32(const float* x, const void* w_packed,
                                              float w_scale, int64_t M, int64_t N, int64_t K,
                                              float* y, void* stream) {
    TZ_CHECK(x && w_packed && y, "bitlinear_tl1_f32: null pointer");
    TZ_CHECK(M > 0 && M <= 65535 && N > 0 && N % 64 == 0 && K > 0,
             "bitlinear_tl1_f32: need N %% 64 == 0");
    hipStream_t st = (hipStream_t)stream;
    const int64_t Kp = ceil_div(K, 64) * 64;
    RowScales rs = RowScales::single(w_scale);
    // one launch (tl1_gemv_f32_kernel) where whole rows per block is the GEMV's
    // own choice (tl1_pick_splits) and the padded row fits its stage
    const int64_t KS = Kp / 64;
    if (K % 4 == 0 && Kp <= 8192 && tl1_pick_splits(N / 64, KS, M) == 1) {
        const dim3 grid((unsigned)(N / 64), (unsigned)M), blk(256);
        const uint4* wp = (const uint4*)w_packed;
        if (Kp <= 2048)
            hipLaunchKernelGGL(tl1_gemv_f32_kernel<2>, grid, blk, 0, st, wp, x, N, K, KS, rs, y);
        else if (Kp <= 4096)
            hipLaunchKernelGGL(tl1_gemv_f32_kernel<4>, grid, blk, 0, st, wp, x, N, K, KS, rs, y);
        else
            hipLaunchKernelGGL(tl1_gemv_f32_kernel<8>, grid, blk, 0, st, wp, x, N, K, KS, rs, y);
        return launch_status("tl1_gemv_f32_kernel");
    }
    char* ws = (char*)Scratch::get(kScratchAct, (size_t)(M * Kp + M * 8 + 256), st);
    if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
    tenzo_hip_actq_t* q = (tenzo_hip_actq_t*)ws;
    int8_t* codes = (int8_t*)(ws + ((M * 8 + 255) / 256) * 256);
    int rc = launch_quant31(x, nullptr, false, 0.0f, M, K, codes, q, nullptr, st);
    if (rc) return rc;
    return launch_tl1_gemv(codes, q, w_packed, rs, M, N, K, y, nullptr, nullptr, st, 0, nullptr);
}

TENZO_HIP_API int tenzo_hip_rmsnorm(const float* x, const float* w, float* y, int64_t dim,
                                    float eps, void* stream) {
    TZ_CHECK(x && y && dim > 0, "rmsnorm: bad arguments");
    return launch_rmsnorm(x, w, y, dim, eps, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_execute_bitlinear_tl1(const float* act, const uint8_t* w,
                                                  float* out, size_t M, size_t K, size_t N,
                                                  float scale) {
    if (!act || !w || !out || M == 0 || N % 64 || K % 2) {
        set_error("execute_bitlinear_tl1: bad arguments");
        return 0;
    }
    std::lock_guard<std::mutex> lk(g_shim_mu);
    void* packed = nullptr;
    if (shim_upload(w, (int64_t)N, (int64_t)K, &packed)) return 0;
    float* dx = nullptr;
    float* dy = nullptr;
    if (hipMalloc(&dx, M * K * 4) != hipSuccess) return 0;
    if (hipMalloc(&dy, M * N * 4) != hipSuccess) {
        (void)hipFree(dx);
        return 0;
    }
    bool ok = hipMemcpy(dx, act, M * K * 4, hipMemcpyHostToDevice) == hipSuccess &&
              tenzo_hip_bitlinear_tl1_f32(dx, packed, scale, (int64_t)M, (int64_t)N,
                                          (int64_t)K, dy, nullptr) == 0 &&
              hipMemcpy(out, dy, M * N * 4, hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(dx);
    (void)hipFree(dy);
    return ok ? 1 : 0;
}

TENZO_HIP_API int tenzo_hip_execute_rmsnorm(const float* in, const float* w, float* out,
                                            size_t dim, float eps) {
    if (!in || !out || dim == 0) {
        set_error("execute_rmsnorm: bad arguments");
        return 0;
    }
    float* dx = nullptr;
    float* dw = nullptr;
    float* dy = nullptr;
    bool ok = hipMalloc(&dx, dim * 4) == hipSuccess && hipMalloc(&dy, dim * 4) == hipSuccess &&
              (!w || hipMalloc(&dw, dim * 4) == hipSuccess) &&
              hipMemcpy(dx, in, dim * 4, hipMemcpyHostToDevice) == hipSuccess &&
              (!w || hipMemcpy(dw, w, dim * 4, hipMemcpyHostToDevice) == hipSuccess) &&
              tenzo_hip_rmsnorm(dx, w ? dw : nullptr, dy, (int64_t)dim, eps, nullptr) == 0 &&
              hipMemcpy(out, dy, dim * 4, hipMemcpyDeviceToHost) == hipSuccess;
    if (dx) (void)hipFree(dx);
    if (dw) (void)hipFree(dw);
    if (dy) (void)hipFree(dy);
    return ok ? 1 : 0;
}

}  // extern "C"

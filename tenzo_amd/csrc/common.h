// Shared device helpers and host plumbing for libtenzo_hip.so (gfx950).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/tenzo.h"
#include "../../include/tenzo_hip.h"

namespace tz {

constexpr int kWave = 64;

// ---------------------------------------------------------------- host ----

// Thread-local error message behind tenzo_hip_last_error().
void set_error(const char* fmt, ...);
// Maps a HIP error to a status (and records the message).
int hip_fail(hipError_t e, const char* what);

#define TZ_HIP(call)                                            \
    do {                                                        \
        hipError_t e_ = (call);                                 \
        if (e_ != hipSuccess) return ::tz::hip_fail(e_, #call); \
    } while (0)

#define TZ_CHECK(cond, ...)                       \
    do {                                          \
        if (!(cond)) {                            \
            ::tz::set_error(__VA_ARGS__);         \
            return TENZO_ERROR_INVALID_ARGUMENT;  \
        }                                         \
    } while (0)

// Checks the launch that was just issued.
int launch_status(const char* what);

// Library-owned scratch, one region per device, grown on demand. Regions are
// zero-filled when (re)allocated; users that need zero-initialised memory
// restore zeros before they return (the split-K accumulators do).
struct Scratch {
    // Returns a device pointer of at least `bytes` for slot `slot` on the
    // current device, or nullptr (error recorded).
    static void* get(int slot, size_t bytes, hipStream_t stream);
};
enum ScratchSlot {
    kScratchGemvAcc = 0,   // int32 split-K accumulators + counters
    kScratchAttn = 1,      // attention partials
    kScratchAct = 2,       // quantized activations of the *_f32 entry points
    kScratchTmp = 3,
    kScratchHead = 4,      // argmax partials + counter
    kScratchSlots = 5
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// --------------------------------------------------------------- device ---

// Cross-lane moves inside 16-lane rows (DPP): lane i receives lane
// i^1, i^2 (quad permutations), 7-i within its half-row and 15-i within its
// row. After the first two steps of a butterfly every lane of a quad holds the
// same value, and after the third every lane of a half-row does, so the two
// mirrors then act as the xor-4 and xor-8 partners.
// (mov_dpp leaves no old value to keep, so the compiler folds each move into
// the add or max that uses it: one v_add_f32_dpp per butterfly step.)
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Sum over a wave (all 64 lanes active) as the balanced pairwise tree over the
// lanes in lane order: lane pairs (0,1), (2,3), ... first, then pairs of
// pairs, ...; the four 16-lane row sums are combined as (r0+r1)+(r2+r3). The
// result is identical in every lane. (Floating-point addition is commutative,
// so which operand of a pair comes first does not change it.)
__device__ __forceinline__ float wave_sum_tree(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    v += dpp_f<kDppMirror>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ int wave_sum_i32(int v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppHalfMirror>(v);
    v += dpp_i<kDppMirror>(v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Block-wide max / integer sum for 256 threads (order-independent).
__device__ __forceinline__ float block256_max(float v, float* red) {
    v = wave_max(v);
    const int t = threadIdx.x;
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block256_sum_i32(int v, int* red) {
    v = wave_sum_i32(v);
    const int t = threadIdx.x;
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    int r = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return r;
}

// The library is compiled with -ffp-contract=off, so a*b+c is two rounded
// operations unless written as __builtin_fmaf; HIP's default '/' and sqrtf
// are correctly rounded (__fsqrt_rn is not: without
// OCML_BASIC_ROUNDED_OPERATIONS it maps to the native approximation).

// ---- rms_norm_raw (TenzoEngine.cpp:148-166) as the reference build evaluates it ----
//
// The reference is compiled with -O3 -mavx2 -mfma -ffast-math, under which
//  * the "omp simd reduction(+:sum_sq)" loop is one 8-lane FMA accumulator:
//    chain j runs over x[j], x[j+8], ... in index order, the n % 8 tail is
//    added to chain 0, and the chains are summed as
//    ((c0+c4)+(c2+c6)) + ((c1+c5)+(c3+c7));
//  * 1.0f / std::sqrt(a) is the RSQRTSS estimate y0 refined by one Newton
//    step, (y0 * -0.5f) * fma(a * y0, y0, -3.0f), with a = ss / dim + eps;
//  * the weighted product x * inv_rms * w is reassociated to (x * w) * inv_rms.
// The activation codes that follow a norm depend on every one of these
// roundings, so the kernels reproduce them exactly.

// RSQRTSS of the host the reference was built on, for a in [0.5, 2): entry
// 1024 * (exponent parity) + top 10 mantissa bits (gen_rsqrt_est.c).
constexpr int kRsqrtEstWords = 2048;
__device__ static const uint32_t kRsqrtEstTab[kRsqrtEstWords] = {
#include "rsqrt_est_table.inc"
};

// The estimate for a positive normal a; tab is kRsqrtEstTab or a copy of it
// (in LDS). Its exponent moves by half the input's, exactly.
__device__ __forceinline__ float rsqrt_est(float a, const uint32_t* tab) {
    const uint32_t b = __float_as_uint(a);
    const int e = (int)(b >> 23), odd = e & 1, e0 = odd ? 127 : 126;
    const uint32_t t = tab[odd * 1024 + ((b >> 13) & 1023u)];
    return __uint_as_float((uint32_t)((int)t - ((e - e0) / 2) * (1 << 23)));
}

// inv_rms of :154 from the sum of squares.
__device__ __forceinline__ float inv_rms_ref(float ss, int64_t dim, float eps,
                                             const uint32_t* tab) {
    const float a = __fadd_rn(__fdiv_rn(ss, (float)dim), eps);
    const float y0 = rsqrt_est(a, tab);
    return __fmul_rn(__fmul_rn(y0, -0.5f), __builtin_fmaf(__fmul_rn(a, y0), y0, -3.0f));
}

// y = (x * w) * inv_rms, or x * inv_rms without weights (:155-165 as built).
__device__ __forceinline__ float norm_apply(float x, float inv_rms, const float* __restrict__ w,
                                            int64_t i) {
    return w ? __fmul_rn(__fmul_rn(x, w[i]), inv_rms) : __fmul_rn(x, inv_rms);
}

// Chain layout of a row in LDS: element i at ct[(i % 8) * ld + i / 8], so
// chain j is row j. ld >= ceil(n / 8) is a multiple of 4 and 4 mod 32 words,
// so the eight rows start in distinct banks.
__host__ __device__ inline int chain_ld(int64_t n) {
    const int c = (int)((n + 7) / 8);
    return (c + 27) / 32 * 32 + 4;
}
__device__ __forceinline__ int chain_pos(int64_t i, int ld) {
    return (int)(i & 7) * ld + (int)(i >> 3);
}

// FMAs of the squares of B float4 of a chain row into s, in order; the B
// LDS reads are issued together, ahead of the FMAs.
template <int B>
__device__ __forceinline__ void chain_block(const float4* row, float& s) {
    float4 v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) v[u] = row[u];
#pragma unroll
    for (int u = 0; u < B; ++u) {
        s = __builtin_fmaf(v[u].x, v[u].x, s);
        s = __builtin_fmaf(v[u].y, v[u].y, s);
        s = __builtin_fmaf(v[u].z, v[u].z, s);
        s = __builtin_fmaf(v[u].w, v[u].w, s);
    }
}

// Sum of squares of the n-element row in chain layout (ct, ld), in the
// reference build's order (orc_sumsq), by one wave: lanes 0..7 run chains
// 0..7, one FMA per term. The chains are bound by the latency of dependent
// FMAs (about 8 cycles each on the MI355X: 1.07 us for n = 2560, 2.88 us for
// 6912, measured), so the LDS reads only have to stay out of their way: a
// block of 16 float4 per lane is read before its 64 FMAs (one LDS wait per
// block), and what is left of a row goes in blocks of 8 and 4 rather than
// one float4 (one wait) at a time. Only lanes 0..7 read: an LDS read then
// returns 8 x 16 bytes instead of 64 x 16. The n % 8 tail is added to chain
// 0; the result is returned in every lane of the wave.
__device__ __forceinline__ float chain_sumsq_wave(const float* ct, int ld, int64_t n) {
    const int j = threadIdx.x & 7;
    const int n8 = (int)(n >> 3), nq = n8 >> 2;  // whole float4s of a chain
    float s = 0.0f;
    if ((threadIdx.x & 63) < 8) {
        const float4* row = reinterpret_cast<const float4*>(ct + j * ld);
        int q = 0;
        for (; q + 16 <= nq; q += 16) chain_block<16>(row + q, s);
        if (q + 8 <= nq) {
            chain_block<8>(row + q, s);
            q += 8;
        }
        if (q + 4 <= nq) {
            chain_block<4>(row + q, s);
            q += 4;
        }
        for (; q < nq; ++q) chain_block<1>(row + q, s);
        for (int k = nq * 4; k < n8; ++k) s = __builtin_fmaf(ct[j * ld + k], ct[j * ld + k], s);
        if (j == 0)
            for (int64_t t = (int64_t)n8 * 8; t < n; ++t) {
                const float v = ct[(int)(t & 7) * ld + n8];
                s = __builtin_fmaf(v, v, s);
            }
    }
    const float c0 = lane_f(s, 0), c1 = lane_f(s, 1), c2 = lane_f(s, 2), c3 = lane_f(s, 3);
    const float c4 = lane_f(s, 4), c5 = lane_f(s, 5), c6 = lane_f(s, 6), c7 = lane_f(s, 7);
    return ((c0 + c4) + (c2 + c6)) + ((c1 + c5) + (c3 + c7));
}

// Signed 8-bit dot of 4 lanes + accumulator (v_dot4_i32_i8).
__device__ __forceinline__ int sdot4(uint32_t a, int32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, b, c, false);
}

// A 16-byte load with the nontemporal hint, for weights a kernel reads once: on a pure
// 330 MB read it gives ~6% more bandwidth than a plain load and leaves the caches to the
// data that is read again. (The decode chunk kernel's K/V loads stay plain: there the
// hint, on the K or on the V loads, made attention 20-30% slower at 8k-32k contexts.)
__device__ __forceinline__ uint4 ld_nt16(const uint4* p) {
    typedef unsigned u4nt __attribute__((ext_vector_type(4)));
    const u4nt v = __builtin_nontemporal_load(reinterpret_cast<const u4nt*>(p));
    return uint4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// fp16 of an fp32 value that was rounded on its own. The empty asm keeps the
// compiler from fusing the conversion with the operation that produced f:
// v_fma_mixlo_f16 would round a product once, straight to fp16, which differs
// from fp16(fp32(a * b)) where fp32(a * b) sits on an fp16 rounding tie.
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    asm volatile("" : "+v"(f));
    return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float i8_to_f32(int v) { return (float)v; }

// Hand-off of split-K partials between workgroups. The partials are written
// as device-scope atomics or device-coherent stores (both performed past the
// XCD's L2 and read back with device-scope loads or atomics), so once this
// wave's vector memory operations are acknowledged they are visible to every
// workgroup, and a counter atomic issued after a block barrier can announce
// them. __threadfence() would add a write-back and invalidation of the whole
// L2 of the XCD (buffer_wbl2 / buffer_inv) to every arrival.
__device__ __forceinline__ void partials_acked() { __builtin_amdgcn_s_waitcnt(0); }
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace tz

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

// Sum of squares of x[0..n) in the fixed order shared with the CPU oracle
// (orc_sumsq): 1024 strided partials p[m] = fma-accumulated x[m], x[m+1024],
// ...; then a balanced pairwise tree over p[0..1023] in index order. Thread t
// of 256 owns p[4t..4t+3] (and adds them as the tree's first two levels); the
// butterfly over the wave and the 4-wave sum are the remaining levels. Must be
// called by all threads of a 256-thread block; `red` is 4 floats of LDS.
__device__ __forceinline__ float block256_sumsq(const float* __restrict__ x, int64_t n,
                                                float* red) {
    const int t = threadIdx.x;
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    for (int64_t i = 4 * t; i < n; i += 1024) {
        p0 = __builtin_fmaf(x[i], x[i], p0);
        if (i + 1 < n) p1 = __builtin_fmaf(x[i + 1], x[i + 1], p1);
        if (i + 2 < n) p2 = __builtin_fmaf(x[i + 2], x[i + 2], p2);
        if (i + 3 < n) p3 = __builtin_fmaf(x[i + 3], x[i + 3], p3);
    }
    float s = (p0 + p1) + (p2 + p3);
    s = wave_sum_tree(s);
    if ((t & 63) == 0) red[t >> 6] = s;
    __syncthreads();
    float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
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

// inv_rms of rms_norm_raw (TenzoEngine.cpp:154): 1 / sqrt(ss/dim + eps), each
// operation correctly rounded.
__device__ __forceinline__ float inv_rms_from_sumsq(float ss, int64_t dim, float eps) {
    const float mean = ss / (float)dim;
    return 1.0f / sqrtf(mean + eps);
}

// y = x * inv_rms * w evaluated left to right (TenzoEngine.cpp:158).
__device__ __forceinline__ float norm_apply(float x, float inv_rms, const float* __restrict__ w,
                                            int64_t i) {
    float v = __fmul_rn(x, inv_rms);
    return w ? __fmul_rn(v, w[i]) : v;
}

// Signed 8-bit dot of 4 lanes + accumulator (v_dot4_i32_i8).
__device__ __forceinline__ int sdot4(uint32_t a, int32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, b, c, false);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
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

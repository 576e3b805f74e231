// Quantized GEMVs on gfx950: GGUF Q4_0 (fp32/fp16 or Q8_0 activations), GGUF
// Q8_0, GPTQ and AWQ (reference src/runtime/TenzoEngine.cpp:1022-1175).
#include <type_traits>

#include "common.h"

namespace tz {

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return half_bits_to_float(v); }

// ------------------------------------------------------------------------
// Q4_0: rows of K/32 blocks of 18 bytes (fp16 d, then 16 bytes: low nibble of
// byte j is element j, high nibble element j+16), y_n = sum_b d_b * sum_j
// a_j (q_j - 8). Rows start 16-byte aligned whenever K % 256 == 0 (row
// stride 18*K/32), and 8 consecutive blocks are 144 bytes = 9 x 16, so a lane
// takes groups of 8 blocks with nine 16-byte loads. LPR lanes share a row
// (power of two); a 256-thread block holds 256/LPR rows. The activation row
// is staged in LDS as fp32.
// ------------------------------------------------------------------------

__device__ __forceinline__ uint32_t byte_at(const uint32_t* dw, int o) {
    return (dw[o >> 2] >> (8 * (o & 3))) & 0xffu;
}

__device__ __forceinline__ float q4_block_dot(const uint32_t* dw, int off, const float* a) {
    // block at byte offset `off` of the 36-dword window; a = its 32 activations
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t byte = byte_at(dw, off + 2 + j);
        s = __builtin_fmaf(a[j], (float)((int)(byte & 15u) - 8), s);
        s = __builtin_fmaf(a[16 + j], (float)((int)(byte >> 4) - 8), s);
    }
    return s;
}

// fp32 activation staging for the row-per-lane GEMVs (FULL path: K % 256 ==
// 0, 16-byte aligned operands). Element k sits at float k + 4 (k / 256): 16
// bytes of padding per 256 elements, the span of one lane's group of 8
// blocks, so the lanes of a row (one group apart) read different LDS banks.
// A thread's first kR 16-byte loads are issued before its weights and stored
// without a branch (units past the end go to the thread's own 32-byte spare
// slot behind the padded row); the rest, for K beyond kR * 256 loads, follow
// in a loop.
__host__ __device__ constexpr int f32s_size(int K) { return K + 4 * ((K + 255) / 256); }
// Floats past the staged row that F32Stage::store writes its idle first-round
// loads to (none when those kR * 256 loads are all within the row).
template <typename TA>
__host__ __device__ constexpr int f32s_dump(int K) {
    return K / (16 / (int)sizeof(TA)) >= (sizeof(TA) == 2 ? 2 : 4) * 256 ? 0 : 2048;
}
template <typename TA>
struct F32Stage {
    static constexpr int kE = 16 / (int)sizeof(TA);     // elements per 16-byte load
    static constexpr int kR = sizeof(TA) == 2 ? 2 : 4;  // loads per thread issued first
    uint4 v[kR];
    __device__ void load(const TA* a, int K) {
        const int units = K / kE;
#pragma unroll
        for (int j = 0; j < kR; ++j)
            v[j] = reinterpret_cast<const uint4*>(a)[min((int)threadIdx.x + j * 256, units - 1)];
    }
    __device__ static void put(float* d, const uint4 x) {
        if (sizeof(TA) == 2) {
            reinterpret_cast<float4*>(d)[0] =
                float4{half_bits_to_float((uint16_t)(x.x & 0xffffu)), half_bits_to_float((uint16_t)(x.x >> 16)),
                       half_bits_to_float((uint16_t)(x.y & 0xffffu)), half_bits_to_float((uint16_t)(x.y >> 16))};
            reinterpret_cast<float4*>(d)[1] =
                float4{half_bits_to_float((uint16_t)(x.z & 0xffffu)), half_bits_to_float((uint16_t)(x.z >> 16)),
                       half_bits_to_float((uint16_t)(x.w & 0xffffu)), half_bits_to_float((uint16_t)(x.w >> 16))};
        } else {
            *reinterpret_cast<uint4*>(d) = x;
        }
    }
    __device__ void store(float* a_s, const TA* a, int K) const {
        const int units = K / kE;
#pragma unroll
        for (int j = 0; j < kR; ++j) {
            const int u = (int)threadIdx.x + j * 256, k0 = u * kE;
            put(u < units ? a_s + k0 + 4 * (k0 >> 8) : a_s + f32s_size(K) + 8 * (int)threadIdx.x, v[j]);
        }
        for (int u = (int)threadIdx.x + kR * 256; u < units; u += 256)
            put(a_s + u * kE + 4 * ((u * kE) >> 8), reinterpret_cast<const uint4*>(a)[u]);
    }
};

template <typename TA, int LPR, bool FULL>
__global__ void __launch_bounds__(256)
q4_0_kernel(const TA* __restrict__ act, const uint8_t* __restrict__ w, float* __restrict__ y,
            int K, int N) {
    extern __shared__ float a_s[];
    const int b = blockIdx.y;
    constexpr int RPB = 256 / LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    const int nbk = K / 32;
    const int ngroups = (nbk + 7) / 8;
    float acc = 0.0f;
    if (FULL) {  // activations, then the first group's 9 loads, then the staging's stores
        F32Stage<TA> stg;
        stg.load(act + (int64_t)b * K, K);
        const uint8_t* rowp = w + (int64_t)min(row, N - 1) * nbk * 18;
        uint32_t dw[36];
        auto load_group = [&](int g) {
            const uint4* p = reinterpret_cast<const uint4*>(rowp + g * 144);
#pragma unroll
            for (int i = 0; i < 9; ++i) {
                const uint4 v = p[i];
                dw[4 * i] = v.x;
                dw[4 * i + 1] = v.y;
                dw[4 * i + 2] = v.z;
                dw[4 * i + 3] = v.w;
            }
        };
        load_group(min(sub, ngroups - 1));
        stg.store(a_s, act + (int64_t)b * K, K);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (row < N) {
            for (int g = sub; g < ngroups; g += LPR) {
                if (g != sub) load_group(g);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t dbits = byte_at(dw, 18 * i) | (byte_at(dw, 18 * i + 1) << 8);
                    const float d = half_bits_to_float((uint16_t)dbits);
                    acc = __builtin_fmaf(q4_block_dot(dw, 18 * i, a_s + (g * 8 + i) * 32 + 4 * g), d,
                                         acc);
                }
            }
        }
#pragma unroll
        for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
        if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
        return;
    }
    for (int i = threadIdx.x; i < K; i += 256) a_s[i] = to_f32<TA>(act[(int64_t)b * K + i]);
    __syncthreads();
    if (row < N) {
        const uint8_t* rowp = w + (int64_t)row * nbk * 18;
        for (int g = sub; g < ngroups; g += LPR) {
            const int b0 = g * 8;
            if (b0 + 8 <= nbk && (((uintptr_t)(rowp + b0 * 18)) & 15) == 0) {
                uint32_t dw[36];
                const uint4* p = reinterpret_cast<const uint4*>(rowp + b0 * 18);
#pragma unroll
                for (int i = 0; i < 9; ++i) {
                    const uint4 v = p[i];
                    dw[4 * i] = v.x;
                    dw[4 * i + 1] = v.y;
                    dw[4 * i + 2] = v.z;
                    dw[4 * i + 3] = v.w;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t dbits = byte_at(dw, 18 * i) | (byte_at(dw, 18 * i + 1) << 8);
                    const float d = half_bits_to_float((uint16_t)dbits);
                    acc = __builtin_fmaf(q4_block_dot(dw, 18 * i, a_s + (b0 + i) * 32), d, acc);
                }
            } else {
                for (int bb = b0; bb < nbk && bb < b0 + 8; ++bb) {
                    const uint8_t* blk = rowp + bb * 18;
                    uint32_t dw[5];
                    // 18 bytes, 2-byte aligned: assemble from halfwords
                    const uint16_t* hp = reinterpret_cast<const uint16_t*>(blk);
#pragma unroll
                    for (int i = 0; i < 4; ++i) dw[i] = hp[2 * i] | ((uint32_t)hp[2 * i + 1] << 16);
                    dw[4] = hp[8];
                    const float d = half_bits_to_float((uint16_t)(dw[0] & 0xffffu));
                    acc = __builtin_fmaf(q4_block_dot(dw, 0, a_s + bb * 32), d, acc);
                }
            }
        }
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
}

// ------------------------------------------------------------------------
// Q8_0 weights (compute_linear_gguf_q8_0, TenzoEngine.cpp:1078-1114): rows of
// K/32 blocks of 34 bytes (fp16 d, then 32 int8 codes), y_n = sum_b d_b *
// sum_j a_j q_j. Eight blocks are 272 bytes = 17 x 16, so whenever a row's
// group of 8 blocks starts 16-byte aligned (row stride 34 K/32: K % 256 == 0)
// a lane reads the group with seventeen 16-byte loads; other blocks are read
// as halfwords. LPR lanes share a row; the activation row is staged in LDS as
// fp32. A code becomes a float in one conversion of its sign-extended byte.
// ------------------------------------------------------------------------

__device__ __forceinline__ float sbyte_at(const uint32_t* dw, int o) {
    return (float)(int)(int8_t)(dw[o >> 2] >> (8 * (o & 3)));
}

// sum_j a_j q_j of the block whose fp16 scale sits at byte `off` of dw
__device__ __forceinline__ float q8_block_dot(const uint32_t* dw, int off, const float* a) {
    const float4* a4 = reinterpret_cast<const float4*>(a);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 av = a4[j];
        s = __builtin_fmaf(av.x, sbyte_at(dw, off + 2 + 4 * j), s);
        s = __builtin_fmaf(av.y, sbyte_at(dw, off + 3 + 4 * j), s);
        s = __builtin_fmaf(av.z, sbyte_at(dw, off + 4 + 4 * j), s);
        s = __builtin_fmaf(av.w, sbyte_at(dw, off + 5 + 4 * j), s);
    }
    return s;
}

template <typename TA, int LPR, bool FULL>
__global__ void __launch_bounds__(256)
q8_0_kernel(const TA* __restrict__ act, const uint8_t* __restrict__ w, float* __restrict__ y,
            int K, int N) {
    extern __shared__ float a_s[];
    const int b = blockIdx.y;
    constexpr int RPB = 256 / LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    const int nbk = K / 32;
    const int ngroups = (nbk + 7) / 8;
    float acc = 0.0f;
    if (FULL) {  // activations, then the first group's 17 loads, then the staging's stores
        F32Stage<TA> stg;
        stg.load(act + (int64_t)b * K, K);
        const uint8_t* rowp = w + (int64_t)min(row, N - 1) * nbk * 34;
        uint32_t dw[68];
        auto load_group = [&](int g) {
            const uint4* p = reinterpret_cast<const uint4*>(rowp + g * 272);
#pragma unroll
            for (int i = 0; i < 17; ++i) {
                const uint4 v = p[i];
                dw[4 * i] = v.x;
                dw[4 * i + 1] = v.y;
                dw[4 * i + 2] = v.z;
                dw[4 * i + 3] = v.w;
            }
        };
        load_group(min(sub, ngroups - 1));
        stg.store(a_s, act + (int64_t)b * K, K);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (row < N) {
            for (int g = sub; g < ngroups; g += LPR) {
                if (g != sub) load_group(g);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t dbits = (dw[(34 * i) >> 2] >> (8 * ((34 * i) & 3))) & 0xffffu;
                    const float d = half_bits_to_float((uint16_t)dbits);
                    acc = __builtin_fmaf(q8_block_dot(dw, 34 * i, a_s + (g * 8 + i) * 32 + 4 * g), d,
                                         acc);
                }
            }
        }
#pragma unroll
        for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
        if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
        return;
    }
    for (int i = threadIdx.x; i < K; i += 256) a_s[i] = to_f32<TA>(act[(int64_t)b * K + i]);
    __syncthreads();
    if (row < N) {
        const uint8_t* rowp = w + (int64_t)row * nbk * 34;
        for (int g = sub; g < ngroups; g += LPR) {
            const int b0 = g * 8;
            if (b0 + 8 <= nbk && (((uintptr_t)(rowp + b0 * 34)) & 15) == 0) {
                uint32_t dw[68];
                const uint4* p = reinterpret_cast<const uint4*>(rowp + b0 * 34);
#pragma unroll
                for (int i = 0; i < 17; ++i) {
                    const uint4 v = p[i];
                    dw[4 * i] = v.x;
                    dw[4 * i + 1] = v.y;
                    dw[4 * i + 2] = v.z;
                    dw[4 * i + 3] = v.w;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t dbits = (dw[(34 * i) >> 2] >> (8 * ((34 * i) & 3))) & 0xffffu;
                    const float d = half_bits_to_float((uint16_t)dbits);
                    acc = __builtin_fmaf(q8_block_dot(dw, 34 * i, a_s + (b0 + i) * 32), d, acc);
                }
            } else {
                for (int bb = b0; bb < nbk && bb < b0 + 8; ++bb) {
                    // 34 bytes, 2-byte aligned: assembled from halfwords
                    const uint16_t* hp = reinterpret_cast<const uint16_t*>(rowp + bb * 34);
                    uint32_t dw[9];
#pragma unroll
                    for (int i = 0; i < 8; ++i) dw[i] = hp[2 * i] | ((uint32_t)hp[2 * i + 1] << 16);
                    dw[8] = hp[16];
                    const float d = half_bits_to_float((uint16_t)(dw[0] & 0xffffu));
                    acc = __builtin_fmaf(q8_block_dot(dw, 0, a_s + bb * 32), d, acc);
                }
            }
        }
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
}

// Q8_0 with the weights staged through LDS (K % 256 == 0, 16-byte aligned
// operands). In q8_0_kernel each lane reads its own 272-byte group, so the 64
// lanes of a load instruction touch 64 cache lines and the L1 tag lookups
// (eight per line over a pass) stall the address path. Here a workgroup's
// Q8R rows (contiguous in memory) are copied into LDS by buffer loads that go
// straight to LDS, 1 KiB per wave instruction (lane l: bytes 16 l ..), so
// every line is looked up once; 32 lanes then share a row, lane s taking the
// 4-block units s, s + 32, .. (136 bytes each, read from LDS as 8-byte words:
// the 32 lanes of a row hit 64 distinct banks). Rows past N read zeros.
constexpr int kQ8R = 8;  // rows per workgroup
namespace {
typedef __attribute__((address_space(3))) void q8_lds_void;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t q8_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
}  // namespace

template <typename TA>
__global__ void __launch_bounds__(256)
q8_0_lds_kernel(const TA* __restrict__ act, const uint8_t* __restrict__ w, float* __restrict__ y,
                int K, int N) {
    extern __shared__ float a_s[];  // activations (f32s_size(K) + f32s_dump floats), then
                                    // rows (whole KiB rounds)
    const int b = blockIdx.y;
    const int nbk = K / 32;
    const int rb = nbk * 34;  // bytes per row
    const int row0 = blockIdx.x * kQ8R;
    uint8_t* w_s = reinterpret_cast<uint8_t*>(a_s + f32s_size(K) + f32s_dump<TA>(K));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    F32Stage<TA> stg;
    stg.load(act + (int64_t)b * K, K);
    {
        const uint8_t* base = w + (int64_t)row0 * rb;
        const uint32_t left = (uint32_t)(min(N - row0, kQ8R) * rb);  // this block's rows
        const __amdgpu_buffer_rsrc_t r = q8_rsrc(base, left);
        const int rounds = (kQ8R * rb + 1023) / 1024;
        for (int i = wave; i < rounds; i += 4)  // (wave-uniform)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (q8_lds_void*)(w_s + 1024 * i), 16,
                                                     (uint32_t)(1024 * i + 16 * lane), 0, 0,
                                                     2 /* nontemporal */);
    }
    stg.store(a_s, act + (int64_t)b * K, K);
    __builtin_amdgcn_s_waitcnt(0);  // (this wave's copies and loads landed)
    __syncthreads();
    const int r = tid >> 5, sub = tid & 31;
    const uint8_t* rowp = w_s + r * rb;
    float acc = 0.0f;
    for (int u = sub; u < nbk / 4; u += 32) {
        uint32_t dw[34];
        const uint2* p = reinterpret_cast<const uint2*>(rowp + 136 * u);
#pragma unroll
        for (int i = 0; i < 17; ++i) {
            const uint2 v = p[i];
            dw[2 * i] = v.x;
            dw[2 * i + 1] = v.y;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int bk = 4 * u + i;
            const uint32_t dbits = (dw[(34 * i) >> 2] >> (8 * ((34 * i) & 3))) & 0xffffu;
            const float d = half_bits_to_float((uint16_t)dbits);
            acc = __builtin_fmaf(q8_block_dot(dw, 34 * i, a_s + 32 * bk + 4 * (bk >> 3)), d, acc);
        }
    }
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) acc += __shfl_xor(acc, o, 64);
    const int row = row0 + r;
    if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
}

// Q4_0 with fp16 activations on the packed fp16 dot (v_dot2_f32_f16): the
// activations are staged in LDS as pairs (a_j, a_16+j) of each block, the
// two elements that share a weight byte; a byte becomes the pair of weights
// (lo - 8, hi - 8) in fp16 with a byte permute, an and-or that forms the fp16
// numbers 1024 + q (exponent of 1024, q in the low mantissa bits) and one
// packed subtraction of 1032, all exact; each pair then costs one dot step
// with fp32 accumulation (the products of fp16 operands are exact in fp32).
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float q4_block_h2(const uint32_t* dw, int off, const uint32_t* apb) {
    const uint4* ap4 = reinterpret_cast<const uint4*>(apb);
    const h2v bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    // the two masks in VGPRs, so the and-or is one v_and_or_b32 (a VOP3 op on
    // gfx9 takes no literal and at most one scalar operand)
    uint32_t lo4 = 0x000f000fu, one024 = 0x64006400u;
    asm volatile("" : "+v"(lo4), "+v"(one024));
    float s = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int o = off + 2 + 4 * m;  // the 4 code bytes of elements 4m..4m+3 (and +16)
        const uint32_t c = (o & 3) == 0 ? dw[o >> 2]
                                        : __builtin_amdgcn_alignbyte(dw[(o >> 2) + 1], dw[o >> 2], o & 3);
        const uint32_t hi = c >> 4;
        const uint4 A = ap4[m];
        const uint32_t a[4] = {A.x, A.y, A.z, A.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // bytes [lo nibble of byte k, 0, hi nibble of byte k, 0] as 1024 + q, fp16 pair
            const uint32_t sel = (uint32_t)k | 0x0c00u | ((uint32_t)(4 + k) << 16) | 0x0c000000u;
            const uint32_t z = (__builtin_amdgcn_perm(hi, c, sel) & lo4) | one024;
            const h2v wq = __builtin_bit_cast(h2v, z) + bias;
            s = __builtin_amdgcn_fdot2(wq, __builtin_bit_cast(h2v, a[k]), s, false);
        }
    }
    return s;
}

// With FULL (K % 256 == 0 and 16-byte aligned operands: every group of 8
// blocks is whole and aligned) the latency is arranged for one pass: each
// thread first issues its activation loads (16 bytes each, up to four in
// flight), then its row's first group of weights (nine 16-byte loads), and
// only then waits for the activations, stores them in LDS and meets the other
// waves at an s_barrier that waits for the LDS stores alone, so the weights
// stream while the activations are staged; the staged pairs get 16 bytes of
// padding per group of 8 blocks (the lanes of a row read one group apart:
// without it, all on the same LDS banks). The lane's groups are summed in the
// same order either way (bit-identical results).
template <int LPR, bool FULL>
__global__ void __launch_bounds__(256)
q4_0_f16_kernel(const uint16_t* __restrict__ act, const uint8_t* __restrict__ w,
                float* __restrict__ y, int K, int N) {
    extern __shared__ uint32_t ap[];  // K/2 words: block b, j < 16: (a_32b+j, a_32b+16+j)
    const int b = blockIdx.y;
    const uint16_t* ab = act + (int64_t)b * K;
    constexpr int RPB = 256 / LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    const int nbk = K / 32;
    const int ngroups = (nbk + 7) / 8;
    float acc = 0.0f;
    if (FULL) {
        // activations: half-blocks (a_32b+8h.., a_32b+16+8h..), 32 bytes each; thread t
        // stages half-block t first (past the last one: into its own slot of a spare area
        // behind the pairs, so the stores need no branch), the rest after the barrier's
        // weights are issued
        const int units = nbk * 2;
        const uint4* a4 = reinterpret_cast<const uint4*>(ab);
        uint4* ap4 = reinterpret_cast<uint4*>(ap);
        auto pairs = [&](uint4* dst, const uint4 lo, const uint4 hi) {
            dst[0] = uint4{(lo.x & 0xffffu) | (hi.x << 16), (lo.x >> 16) | (hi.x & 0xffff0000u),
                           (lo.y & 0xffffu) | (hi.y << 16), (lo.y >> 16) | (hi.y & 0xffff0000u)};
            dst[1] = uint4{(lo.z & 0xffffu) | (hi.z << 16), (lo.z >> 16) | (hi.z & 0xffff0000u),
                           (lo.w & 0xffffu) | (hi.w << 16), (lo.w >> 16) | (hi.w & 0xffff0000u)};
        };
        const int u0 = (int)threadIdx.x, uc = min(u0, units - 1);
        const uint4 lo0 = a4[(uc >> 1) * 4 + (uc & 1)];      // elements 32 blk + 8 h ..
        const uint4 hi0 = a4[(uc >> 1) * 4 + 2 + (uc & 1)];  // elements 32 blk + 16 + 8 h ..
        // the row's first group (rows past N read the last row, lanes past the groups the
        // last group; neither is summed)
        const uint8_t* rowp = w + (int64_t)min(row, N - 1) * nbk * 18;
        uint32_t dw[36];
        {
            const uint4* p = reinterpret_cast<const uint4*>(rowp + min(sub, ngroups - 1) * 144);
#pragma unroll
            for (int i = 0; i < 9; ++i) {
                const uint4 v = p[i];
                dw[4 * i] = v.x;
                dw[4 * i + 1] = v.y;
                dw[4 * i + 2] = v.z;
                dw[4 * i + 3] = v.w;
            }
        }
        // (pairs of block blk at uint4 4 blk + blk / 8: 16 bytes of padding per group of 8
        // blocks, so the lanes of a row, one group apart, read different banks)
        const int pad_end = 4 * nbk + ngroups;
        pairs(ap4 + (u0 < units ? 4 * (uc >> 1) + (uc >> 4) + 2 * (uc & 1) : pad_end + 2 * u0),
              lo0, hi0);
        for (int u = u0 + 256; u < units; u += 256)
            pairs(ap4 + 4 * (u >> 1) + (u >> 4) + 2 * (u & 1), a4[(u >> 1) * 4 + (u & 1)],
                  a4[(u >> 1) * 4 + 2 + (u & 1)]);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (row < N) {
            for (int g = sub; g < ngroups; g += LPR) {
                if (g != sub) {
                    const uint4* p = reinterpret_cast<const uint4*>(rowp + g * 144);
#pragma unroll
                    for (int i = 0; i < 9; ++i) {
                        const uint4 v = p[i];
                        dw[4 * i] = v.x;
                        dw[4 * i + 1] = v.y;
                        dw[4 * i + 2] = v.z;
                        dw[4 * i + 3] = v.w;
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t dbits = (dw[(18 * i) >> 2] >> (8 * ((18 * i) & 3))) & 0xffffu;
                    const float d = half_bits_to_float((uint16_t)dbits);
                    acc = __builtin_fmaf(q4_block_h2(dw, 18 * i, ap + (g * 8 + i) * 16 + 4 * g), d,
                                         acc);
                }
            }
        }
    } else {
        for (int i = threadIdx.x; i < K / 2; i += 256) {
            const int blk = i >> 4, j = i & 15;
            ap[i] = (uint32_t)ab[blk * 32 + j] | ((uint32_t)ab[blk * 32 + 16 + j] << 16);
        }
        __syncthreads();
        if (row < N) {
            const uint8_t* rowp = w + (int64_t)row * nbk * 18;
            for (int g = sub; g < ngroups; g += LPR) {
                const int b0 = g * 8;
                if (b0 + 8 <= nbk && (((uintptr_t)(rowp + b0 * 18)) & 15) == 0) {
                    uint32_t dw[36];
                    const uint4* p = reinterpret_cast<const uint4*>(rowp + b0 * 18);
#pragma unroll
                    for (int i = 0; i < 9; ++i) {
                        const uint4 v = p[i];
                        dw[4 * i] = v.x;
                        dw[4 * i + 1] = v.y;
                        dw[4 * i + 2] = v.z;
                        dw[4 * i + 3] = v.w;
                    }
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const uint32_t dbits = (dw[(18 * i) >> 2] >> (8 * ((18 * i) & 3))) & 0xffffu;
                        const float d = half_bits_to_float((uint16_t)dbits);
                        acc = __builtin_fmaf(q4_block_h2(dw, 18 * i, ap + (b0 + i) * 16), d, acc);
                    }
                } else {
                    for (int bb = b0; bb < nbk && bb < b0 + 8; ++bb) {
                        const uint16_t* hp = reinterpret_cast<const uint16_t*>(rowp + bb * 18);
                        uint32_t dw[5];
#pragma unroll
                        for (int i = 0; i < 4; ++i) dw[i] = hp[2 * i] | ((uint32_t)hp[2 * i + 1] << 16);
                        dw[4] = hp[8];
                        const float d = half_bits_to_float((uint16_t)(dw[0] & 0xffffu));
                        acc = __builtin_fmaf(q4_block_h2(dw, 0, ap + bb * 16), d, acc);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
}

// Q4_0 weights x Q8_0 activations: per block the exact int32 dot
// sum_j (q_j - 8) qa_j = dot4(q, qa) - 8 * sum_j qa_j, then an fp32 FMA with
// d_w * d_a. Activations staged in LDS as codes + fp32 scales + code sums.
template <int LPR>
__global__ void __launch_bounds__(256)
q4_0_q8_kernel(const uint8_t* __restrict__ qa, const uint8_t* __restrict__ w,
               float* __restrict__ y, int K, int N) {
    extern __shared__ int32_t smem[];
    const int nbk = K / 32;
    int32_t* codes = smem;                                    // nbk * 8 words
    float* da = reinterpret_cast<float*>(smem + nbk * 8);     // nbk
    int32_t* csum = smem + nbk * 9;                           // nbk
    const int b = blockIdx.y;
    const uint8_t* qab = qa + (int64_t)b * nbk * 34;
    for (int i = threadIdx.x; i < nbk * 8; i += 256) {
        const int blk = i >> 3, j = (i & 7) * 4;
        const uint8_t* p = qab + blk * 34 + 2 + j;
        codes[i] = (int32_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                             ((uint32_t)p[3] << 24));
    }
    for (int i = threadIdx.x; i < nbk; i += 256) {
        const uint8_t* p = qab + i * 34;
        da[i] = half_bits_to_float((uint16_t)(p[0] | (p[1] << 8)));
        int s = 0;
        for (int j = 0; j < 32; ++j) s += (int8_t)p[2 + j];
        csum[i] = s;
    }
    __syncthreads();
    constexpr int RPB = 256 / LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    float acc = 0.0f;
    if (row < N) {
        const uint8_t* rowp = w + (int64_t)row * nbk * 18;
        for (int bb = sub; bb < nbk; bb += LPR) {
            const uint16_t* hp = reinterpret_cast<const uint16_t*>(rowp + bb * 18);
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = hp[1 + 2 * i] | ((uint32_t)hp[2 + 2 * i] << 16);
            const float dw = half_bits_to_float(hp[0]);
            const int32_t* c = codes + bb * 8;
            int s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s = sdot4(q[i] & 0x0f0f0f0fu, c[i], s);          // elements 4i..4i+3
                s = sdot4((q[i] >> 4) & 0x0f0f0f0fu, c[4 + i], s);  // elements 16+4i..
            }
            s -= 8 * csum[bb];
            acc = __builtin_fmaf((float)s, __fmul_rn(dw, da[bb]), acc);
        }
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
}

// With FULL (K % 256 == 0, 16-byte aligned operands) the activation blocks
// are first copied raw into LDS with 16-byte loads, the row's first group of
// 8 weight blocks (nine 16-byte loads) is issued behind them, and the blocks
// are parsed from LDS (codes, fp32 scale, code sum) while the weights
// stream; a lane then takes whole groups of 8 blocks. The parsed codes get
// 16 bytes of padding per group and the scales and sums one word, so a row's
// lanes (one group apart) read different LDS banks.
template <int LPR>
__global__ void __launch_bounds__(256)
q4_0_q8_full_kernel(const uint8_t* __restrict__ qa, const uint8_t* __restrict__ w,
                    float* __restrict__ y, int K, int N) {
    extern __shared__ uint4 q8s[];
    const int nbk = K / 32, ngroups = nbk / 8;
    const int raw16 = nbk * 34 / 16;          // 16-byte units of the activation blocks
    uint4* raw = q8s;                          // [raw16]
    uint4* codes = q8s + raw16;                // block bb: uint4 2 bb + bb / 8 (two of them)
    float* da = reinterpret_cast<float*>(codes + 2 * nbk + ngroups);  // block bb: bb + bb / 8
    int32_t* csum = reinterpret_cast<int32_t*>(da + nbk + ngroups);
    const int b = blockIdx.y;
    const uint4* qa4 = reinterpret_cast<const uint4*>(qa + (int64_t)b * nbk * 34);
    constexpr int RPB = 256 / LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    // raw copy: two loads per thread first (past the end: stored to the thread's spare
    // slot at the end of LDS), then the row's first group
    const int t = threadIdx.x;
    const uint4 r0 = qa4[min(t, raw16 - 1)], r1 = qa4[min(t + 256, raw16 - 1)];
    const uint8_t* rowp = w + (int64_t)min(row, N - 1) * nbk * 18;
    uint32_t dw[36];
    auto load_group = [&](int g) {
        const uint4* p = reinterpret_cast<const uint4*>(rowp + g * 144);
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            const uint4 v = p[i];
            dw[4 * i] = v.x;
            dw[4 * i + 1] = v.y;
            dw[4 * i + 2] = v.z;
            dw[4 * i + 3] = v.w;
        }
    };
    load_group(min(sub, ngroups - 1));
    uint4* spare = q8s + raw16 + 2 * nbk + ngroups + ((nbk + ngroups) * 8 + 15) / 16;
    *(t < raw16 ? raw + t : spare + t) = r0;
    *(t + 256 < raw16 ? raw + t + 256 : spare + t) = r1;
    for (int u = t + 512; u < raw16; u += 256) raw[u] = qa4[u];
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // parse: block bb's 34 bytes start at byte 34 bb (word-aligned for even bb, else 2 past)
    const uint32_t* rw = reinterpret_cast<const uint32_t*>(raw);
    for (int bb = t; bb < nbk; bb += 256) {
        const int w0 = (34 * bb) >> 2, sh = (34 * bb) & 3;  // sh: 0 or 2
        uint32_t x[9];  // the block's bytes 0..33 lie in words w0 .. w0 + 8 either way
#pragma unroll
        for (int i = 0; i < 9; ++i) x[i] = rw[w0 + i];
        const uint32_t dbits = sh ? (x[0] >> 16) : (x[0] & 0xffffu);
        uint32_t c[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)  // codes: bytes 2 + 4 i .. of the block
            c[i] = sh ? x[i + 1] : __builtin_amdgcn_alignbyte(x[i + 1], x[i], 2);
        int cs = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) cs = sdot4(c[i], 0x01010101, cs);
        uint4* cd = codes + 2 * bb + bb / 8;
        cd[0] = uint4{c[0], c[1], c[2], c[3]};
        cd[1] = uint4{c[4], c[5], c[6], c[7]};
        da[bb + bb / 8] = half_bits_to_float((uint16_t)dbits);
        csum[bb + bb / 8] = cs;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float acc = 0.0f;
    if (row < N) {
        for (int g = sub; g < ngroups; g += LPR) {
            if (g != sub) load_group(g);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int bb = g * 8 + i, o = 18 * i;  // block i of the group at byte o of dw
                const uint32_t dbits = (dw[o >> 2] >> (8 * (o & 3))) & 0xffffu;
                uint32_t q[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int ob = o + 2 + 4 * m;
                    q[m] = (ob & 3) == 0 ? dw[ob >> 2]
                                         : __builtin_amdgcn_alignbyte(dw[(ob >> 2) + 1], dw[ob >> 2], ob & 3);
                }
                const uint4 c0 = codes[2 * bb + g], c1 = codes[2 * bb + g + 1];
                const int32_t cc[8] = {(int32_t)c0.x, (int32_t)c0.y, (int32_t)c0.z, (int32_t)c0.w,
                                       (int32_t)c1.x, (int32_t)c1.y, (int32_t)c1.z, (int32_t)c1.w};
                int sdot = 0;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    sdot = sdot4(q[m] & 0x0f0f0f0fu, cc[m], sdot);          // elements 4m..4m+3
                    sdot = sdot4((q[m] >> 4) & 0x0f0f0f0fu, cc[4 + m], sdot);  // elements 16+4m..
                }
                sdot -= 8 * csum[bb + g];
                acc = __builtin_fmaf((float)sdot,
                                     __fmul_rn(half_bits_to_float((uint16_t)dbits), da[bb + g]), acc);
            }
        }
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (row < N && sub == 0) y[(int64_t)b * N + row] = acc;
}

// ------------------------------------------------------------------------
// GPTQ / AWQ: qweight [K/8][N] u32, lane = output column n (coalesced 256 B
// per wave per k-octet). Split-K: block (column tile of 256, split s) covers
// k in [s*KC, (s+1)*KC), a multiple of the group size; B activation rows are
// staged in LDS as fp32 and every dequantized weight feeds all B rows.
// Partials go to scratch and the last split block of a column tile adds them
// in split order, so results are deterministic.
// ------------------------------------------------------------------------

template <bool AWQ, typename TA, typename TS, int BMAX>
__global__ void __launch_bounds__(256)
gq_kernel(const TA* __restrict__ act, const uint32_t* __restrict__ qweight,
          const TS* __restrict__ scales, const uint32_t* __restrict__ qzeros,
          float* __restrict__ y, int K, int N, int group, int B, int KC, int splits,
          float* __restrict__ part, uint32_t* __restrict__ cnt) {
    extern __shared__ float a_s[];  // [B][KC]
    __shared__ int is_last;
    const int tile = blockIdx.x;
    const int sp = blockIdx.y;
    const int k0 = sp * KC;
    const int k1 = min(K, k0 + KC);
    const int nk = k1 - k0;
    for (int i = threadIdx.x; i < B * nk; i += 256) {
        const int bb = i / nk, kk = i - bb * nk;
        a_s[bb * KC + kk] = to_f32<TA>(act[(int64_t)bb * K + k0 + kk]);
    }
    __syncthreads();
    const int n = tile * 256 + threadIdx.x;
    float acc[BMAX];
#pragma unroll
    for (int bb = 0; bb < BMAX; ++bb) acc[bb] = 0.0f;
    if (n < N) {
        for (int g0 = k0; g0 < k1; g0 += group) {
            const int g = g0 / group;
            const float s = to_f32<TS>(scales[(int64_t)g * N + n]);
            int z;
            if (AWQ) {
                z = (int)((qzeros[(int64_t)g * (N / 8) + n / 8] >> (4 * (n % 8))) & 15u);
            } else {
                z = (int)((qzeros[(int64_t)(g / 8) * N + n] >> (4 * (g % 8))) & 15u) + 1;
            }
            const int gend = min(k1, g0 + group);
            for (int k = g0; k < gend; k += 8) {
                const uint32_t qw = qweight[(int64_t)(k / 8) * N + n];
                float wd[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    wd[e] = __fmul_rn((float)((int)((qw >> (4 * e)) & 15u) - z), s);
                const int kl = k - k0;
#pragma unroll
                for (int bb = 0; bb < BMAX; ++bb) {
                    if (bb < B) {
                        const float* ab = a_s + bb * KC + kl;
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int o = AWQ ? ((e & 3) * 2 + (e >> 2)) : e;  // {0,2,4,6,1,3,5,7}
                            acc[bb] = __builtin_fmaf(ab[o], wd[e], acc[bb]);
                        }
                    }
                }
            }
        }
    }
    if (splits == 1) {
        if (n < N)
            for (int bb = 0; bb < B && bb < BMAX; ++bb) y[(int64_t)bb * N + n] = acc[bb];
        return;
    }
    if (n < N)
        for (int bb = 0; bb < B && bb < BMAX; ++bb)
            store_coherent(&part[((int64_t)sp * B + bb) * N + n], acc[bb]);
    partials_acked();
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(&cnt[tile], 1u) == (unsigned)(splits - 1);
    __syncthreads();
    if (!is_last) return;
    if (n < N) {
        for (int bb = 0; bb < B && bb < BMAX; ++bb) {
            float s = 0.0f;
            for (int q = 0; q < splits; ++q)
                s += __hip_atomic_load(&part[((int64_t)q * B + bb) * N + n], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            y[(int64_t)bb * N + n] = s;
        }
    }
    if (threadIdx.x == 0) atomicExch(&cnt[tile], 0u);
}

// GPTQ / AWQ with fp16 activations on the packed fp16 dot: per group, the
// nibble pairs of a qweight word become exact fp16 pairs (q - z) (a byte
// permute, an and-or forming 1024 + q, one packed subtraction of 1024 + z)
// and meet the activation pairs of the same two k in one v_dot2_f32_f16 step
// (exact products, fp32 accumulation); the group's sum is then scaled once,
// y += s * sum_k a_k (q_k - z). The activations are staged in LDS as pairs
// in the order of the nibble pairs: (k, k+1), (k+2, k+3), ... for GPTQ and,
// for AWQ's nibble order {0,2,4,6,1,3,5,7}, (k, k+2), (k+4, k+6), (k+1, k+3),
// (k+5, k+7). Split-K and the partial sums as gq_kernel.
template <bool AWQ, typename TS, int BMAX>
__global__ void __launch_bounds__(256)
gq_h2_kernel(const uint16_t* __restrict__ act, const uint32_t* __restrict__ qweight,
             const TS* __restrict__ scales, const uint32_t* __restrict__ qzeros,
             float* __restrict__ y, int K, int N, int group, int B, int KC, int splits,
             float* __restrict__ part, uint32_t* __restrict__ cnt) {
    extern __shared__ uint4 ap2v[];  // [BMAX][KC/2] fp16 pairs, 16-byte aligned
    uint32_t* ap2 = reinterpret_cast<uint32_t*>(ap2v);
    __shared__ int is_last;
    constexpr int kQ = 16;  // k-octets whose qweight words are loaded together
    const int tile = blockIdx.x;
    const int sp = blockIdx.y;
    const int k0 = sp * KC;
    const int k1 = min(K, k0 + KC);
    const int nk = k1 - k0;
    const int KP = KC / 2;
    // rows B..BMAX-1 are staged as zeros and computed like the others (their
    // sums are not stored), so the row loops have no branch
    for (int i = threadIdx.x; i < BMAX * (nk / 2); i += 256) {
        const int bb = i / (nk / 2), pi = i - bb * (nk / 2);  // pair pi of the split
        if (bb >= B) {
            ap2[bb * KP + pi] = 0u;
            continue;
        }
        const int oct = pi >> 2, j = pi & 3;
        int ka, kb;  // the two k of pair j of the octet
        if (AWQ) {
            ka = (j & 1) * 4 + (j >> 1);
            kb = ka + 2;
        } else {
            ka = 2 * j;
            kb = ka + 1;
        }
        const uint16_t* ab = act + (int64_t)bb * K + k0 + oct * 8;
        ap2[bb * KP + pi] = (uint32_t)ab[ka] | ((uint32_t)ab[kb] << 16);
    }
    __syncthreads();
    const int n = tile * 256 + threadIdx.x;
    float acc[BMAX];
#pragma unroll
    for (int bb = 0; bb < BMAX; ++bb) acc[bb] = 0.0f;
    uint32_t lo4 = 0x000f000fu, one024 = 0x64006400u;  // VGPR operands of v_and_or_b32
    asm volatile("" : "+v"(lo4), "+v"(one024));
    if (n < N) {
        for (int g0 = k0; g0 < k1; g0 += group) {
            const int g = g0 / group;
            const float s = to_f32<TS>(scales[(int64_t)g * N + n]);
            int z;
            if (AWQ) {
                z = (int)((qzeros[(int64_t)g * (N / 8) + n / 8] >> (4 * (n % 8))) & 15u);
            } else {
                z = (int)((qzeros[(int64_t)(g / 8) * N + n] >> (4 * (g % 8))) & 15u) + 1;
            }
            const _Float16 bz = (_Float16)(-1024.0f - (float)z);
            const h2v bias = {bz, bz};
            float gs[BMAX];
#pragma unroll
            for (int bb = 0; bb < BMAX; ++bb) gs[bb] = 0.0f;
            const int gend = min(k1, g0 + group);
            for (int kc = g0; kc < gend; kc += 8 * kQ) {
              // the chunk's qweight words first (kQ loads in flight; rows past
              // K are clamped, read and not used), then their dot steps
              uint32_t qv[kQ];
#pragma unroll
              for (int u = 0; u < kQ; ++u)
                  qv[u] = qweight[(int64_t)min(kc / 8 + u, K / 8 - 1) * N + n];
              // every octet of the chunk is computed (a use under a condition
              // would let the compiler move its load down to it): octets past
              // the group get zero weights and read pairs inside the split
#pragma unroll
              for (int u = 0; u < kQ; ++u) {
                const int k = kc + 8 * u;
                const bool live = k < gend;
                const uint32_t qw = qv[u];
                const uint32_t hi = qw >> 4;
                h2v wq[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t sel =
                        (uint32_t)i | 0x0c00u | ((uint32_t)(4 + i) << 16) | 0x0c000000u;
                    const uint32_t zz = (__builtin_amdgcn_perm(hi, qw, sel) & lo4) | one024;
                    const h2v wd = __builtin_bit_cast(h2v, zz) + bias;
                    wq[i] = live ? wd : h2v{(_Float16)0.0f, (_Float16)0.0f};
                }
                const int pk = live ? (k - k0) / 2 : 0;  // first pair of the octet
#pragma unroll
                for (int bb = 0; bb < BMAX; ++bb) {
                    // (KP and pk are multiples of 4: 16-byte LDS reads)
                    const uint4 A = ap2v[(bb * KP + pk) >> 2];
                    gs[bb] = __builtin_amdgcn_fdot2(wq[0], __builtin_bit_cast(h2v, A.x), gs[bb],
                                                    false);
                    gs[bb] = __builtin_amdgcn_fdot2(wq[1], __builtin_bit_cast(h2v, A.y), gs[bb],
                                                    false);
                    gs[bb] = __builtin_amdgcn_fdot2(wq[2], __builtin_bit_cast(h2v, A.z), gs[bb],
                                                    false);
                    gs[bb] = __builtin_amdgcn_fdot2(wq[3], __builtin_bit_cast(h2v, A.w), gs[bb],
                                                    false);
                }
              }
            }
#pragma unroll
            for (int bb = 0; bb < BMAX; ++bb) acc[bb] = __builtin_fmaf(gs[bb], s, acc[bb]);
        }
    }
    if (splits == 1) {
        if (n < N)
            for (int bb = 0; bb < B && bb < BMAX; ++bb) y[(int64_t)bb * N + n] = acc[bb];
        return;
    }
    if (n < N)
        for (int bb = 0; bb < B && bb < BMAX; ++bb)
            store_coherent(&part[((int64_t)sp * B + bb) * N + n], acc[bb]);
    partials_acked();
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(&cnt[tile], 1u) == (unsigned)(splits - 1);
    __syncthreads();
    if (!is_last) return;
    if (n < N) {
        for (int bb = 0; bb < B && bb < BMAX; ++bb) {
            float sum = 0.0f;
            for (int q = 0; q < splits; ++q)
                sum += __hip_atomic_load(&part[((int64_t)q * B + bb) * N + n], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
            y[(int64_t)bb * N + n] = sum;
        }
    }
    if (threadIdx.x == 0) atomicExch(&cnt[tile], 0u);
}

// GPTQ / AWQ with fp16 activations, batch 4..16, on fp16 MFMA
// (v_mfma_f32_16x16x16_f16): D[m][n] += sum_k A[m][k] (q - z)[k][n] over
// 16-k steps, the batch rows as M (padded to 16 with zeros) and 16 output
// columns per wave as N. A lane's B operand is 4 k of column n = lane % 16;
// lane group kq = lane / 16 takes k-octet 4 jp + kq of each step pair jp, whose
// one qweight word gives four exact fp16 pairs (q - z) of nibbles (i, i + 4)
// (a shift, an and-or forming 1024 + q, one packed subtraction of 1024 + z):
// nibbles (0,4,1,5) for the pair's first step and (2,6,3,7) for its second.
// The activations are staged in LDS with each k-octet in that order (GPTQ
// (0,4)(1,5)(2,6)(3,7); AWQ, whose nibble e holds k = {0,2,4,6,1,3,5,7}[e],
// as it is), rows padded by 8 bytes so the 16 rows of an A operand read fall
// in different banks. A group's group / 16 steps go into a fresh accumulator
// that is scaled once, y += s * sum. A workgroup owns 32 columns: waves
// (tile, part) = (w % 2, w / 2) take 16 columns and one of 4, 2 or 1 parts of
// K (whole 512-k chunks each), and the parts are added in LDS in part order.
// Each lane keeps the 16 qweight words of a chunk in flight, the first
// chunk's across the barrier that follows the activation staging. Products
// are exact and summed in fp32 (the MFMA's own order).
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef float f4m __attribute__((ext_vector_type(4)));
constexpr int kGqChunk = 512;  // k per load batch (32 words per lane)
constexpr int kGqParts = 4;    // most k parts per workgroup (2 waves each)
constexpr size_t kGqLds = 160 * 1024 - 8192;  // staged activations, beside the part sums
constexpr int kGqLR = 8;  // gq_v4_kernel: lanes per row of a workgroup's columns

template <bool AWQ, typename TS, int NG>  // NG = group / 16 steps per group
__global__ void __launch_bounds__(512)
gq_mfma_kernel(const uint16_t* __restrict__ act, const uint32_t* __restrict__ qweight,
               const TS* __restrict__ scales, const uint32_t* __restrict__ qzeros,
               float* __restrict__ y, int K, int N, int B) {
    constexpr int kSteps = kGqChunk / 16, kGroups = kSteps / NG;  // per chunk
    extern __shared__ uint2 a_lds[];  // [B][K + 4] fp16, 8-byte aligned rows
    uint16_t* ah = reinterpret_cast<uint16_t*>(a_lds);
    __shared__ f4m red[kGqParts - 1][2][64];
    const int KP = K + 4;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int parts = (int)blockDim.x >> 7;  // k parts: waves (tile, part) = (w % 2, w / 2)
    const int tile = wave & 1, part = wave >> 1;
    const int col = lane & 15, kq = lane >> 4;
    const int n = blockIdx.x * 32 + tile * 16 + col;
    const int nn = min(n, N - 1);  // columns past N read the last one, not stored
    const int kp = K / parts, ka = part * kp, kb = ka + kp;
    // this lane's 16 words of a chunk (k-octets kc/8 + 4 jp + kq: one word feeds the step
    // pair jp) and the chunk's group scales and zeros, all in flight together
    uint32_t qv[kSteps / 2];
    float sc[kGroups];
    uint32_t zw[kGroups];
    auto load_chunk = [&](int kc) {  // the group scales and zeros first: used first
#pragma unroll
        for (int gi = 0; gi < kGroups; ++gi) {
            const int g = kc / (16 * NG) + gi;
            sc[gi] = to_f32<TS>(scales[(int64_t)g * N + nn]);
            zw[gi] = AWQ ? qzeros[(int64_t)g * (N / 8) + nn / 8] : qzeros[(int64_t)(g / 8) * N + nn];
        }
#pragma unroll
        for (int jp = 0; jp < kSteps / 2; ++jp)
            qv[jp] = qweight[(int64_t)(kc / 8 + 4 * jp + kq) * N + nn];
    };
    // activations first (an L2 hit in a decode step), one k-octet (16 bytes) per thread
    // and load, four loads in flight, each octet in the order of the weight pairs (GPTQ
    // (0,4)(1,5)(2,6)(3,7); AWQ, whose nibble e holds k = {0,2,4,6,1,3,5,7}[e], as it is);
    // then the first
    // chunk's loads, which stay in flight across the barrier (s_barrier after the LDS
    // stores alone, no wait for the vector loads)
    const int K8 = K >> 3, octs = B * K8, T = (int)blockDim.x;
    const uint4* src = reinterpret_cast<const uint4*>(act);
    for (int j0 = 0; j0 * T < octs; j0 += 4) {
        uint4 v[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
            v[jj] = src[min((int)threadIdx.x + (j0 + jj) * T, octs - 1)];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int i = (int)threadIdx.x + (j0 + jj) * T;
            if (i < octs) {
                const int r = i / K8, o = i - r * K8;
                uint4 w = v[jj];
                if (!AWQ)  // halves (0,1)(2,3)(4,5)(6,7) -> (0,4)(1,5)(2,6)(3,7)
                    w = uint4{(w.x & 0xffffu) | (w.z << 16), (w.x >> 16) | (w.z & 0xffff0000u),
                              (w.y & 0xffffu) | (w.w << 16), (w.y >> 16) | (w.w & 0xffff0000u)};
                uint2* dst = reinterpret_cast<uint2*>(ah + r * KP) + 2 * o;
                dst[0] = uint2{w.x, w.y};
                dst[1] = uint2{w.z, w.w};
            }
        }
    }
    load_chunk(ka);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int m = lane & 15;  // A operand row
    const bool arow = m < B;
    const uint16_t* arp = ah + min(m, B - 1) * KP + 8 * kq;
    uint32_t lo4 = 0x000f000fu, one024 = 0x64006400u;  // VGPR operands of v_and_or_b32
    asm volatile("" : "+v"(lo4), "+v"(one024));
    f4m acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int kc = ka; kc < kb; kc += kGqChunk) {
#pragma unroll
        for (int gi = 0; gi < kGroups; ++gi) {
            const int g = kc / (16 * NG) + gi;
            const int z = AWQ ? (int)((zw[gi] >> (4 * (nn % 8))) & 15u)
                              : (int)((zw[gi] >> (4 * (g % 8))) & 15u) + 1;
            const _Float16 bz = (_Float16)(-1024.0f - (float)z);
            const h2v bias = {bz, bz};
            f4m cg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int jj = 0; jj < NG / 2; ++jj) {
                const int jp = gi * (NG / 2) + jj;  // step pair: one word, nibbles (i, i + 4)
                h2v wd[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    wd[i] = __builtin_bit_cast(h2v, ((qv[jp] >> (4 * i)) & lo4) | one024) + bias;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {  // k of the step: nibbles (0,4,1,5) / (2,6,3,7)
                    const h4v b = {wd[2 * hh].x, wd[2 * hh].y, wd[2 * hh + 1].x, wd[2 * hh + 1].y};
                    h4v a = *reinterpret_cast<const h4v*>(arp + kc + 32 * jp + 4 * hh);
                    if (!arow)
                        a = h4v{(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
                    cg = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, cg, 0, 0, 0);
                }
            }
            acc += cg * sc[gi];
        }
        if (kc + kGqChunk < kb) load_chunk(kc + kGqChunk);
    }
    // the parts' sums added in part order
    if (part > 0) red[part - 1][tile][lane] = acc;
    __syncthreads();
    if (part == 0 && n < N) {
        f4m o = acc;
        for (int p = 1; p < parts; ++p) o += red[p - 1][tile][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * kq + i;  // D: lane holds rows 4 (lane / 16) .. +3 of column n
            if (row < B) y[(int64_t)row * N + n] = o[i];
        }
    }
}

// GPTQ / AWQ at batch 1..4 with 128-bit weight loads: a lane owns 4 adjacent
// columns (one 16-byte load of a qweight row = their 4 words of one k-octet),
// LR lanes cover a workgroup's 4 LR columns and the kGqT / LR lane groups
// ("k-groups") take consecutive K ranges of SPL segments of 64 k (8 octets,
// 8 loads; the last k-groups have fewer or none when K is not a multiple of
// their total). The next segment's words, scales and zeros are in flight while a
// segment is computed, the first segment's before the activations are staged.
// Per segment and column the group's scale applies once:
// y += s * sum_k a_k (q_k - z).
//
// fp16 activations: nibbles e and e + 4 of a word become one exact fp16 pair
// (q - z) with a shift, an and-or forming 1024 + q and one packed
// subtraction of 1024 + z, and meet the activations of the same two k in
// v_dot2_f32_f16 (exact products, fp32 accumulation). The staged octet holds
// those activation pairs: GPTQ (k, k+4) for k < 4; AWQ, whose nibble e holds
// k = {0,2,4,6,1,3,5,7}[e], (0,1)(2,3)(4,5)(6,7) -- the octet as it is.
// fp32 activations: (float)q - z per nibble in fp32 FMAs, the octet staged in
// nibble order. One octet of LDS padding after each k-group's range keeps
// the k-groups of a wave on different banks. The k-groups' sums are added in
// LDS in k-group order (each output written once, by one workgroup).
constexpr int kGqT = 512;    // threads of gq_v4_kernel
constexpr int kGqStg = 8;    // 16-byte activation units staged per thread
template <typename TA>
struct GqAct;  // activations of one k-octet
template <>
struct GqAct<uint16_t> {
    static constexpr int kU4 = 1;  // 16-byte units per octet
};
template <>
struct GqAct<float> {
    static constexpr int kU4 = 2;
};

template <bool AWQ, typename TA, typename TS, int BM, int LR, int GS>  // GS: groups per segment
__global__ void __launch_bounds__(kGqT)
gq_v4_kernel(const TA* __restrict__ act, const uint32_t* __restrict__ qweight,
             const TS* __restrict__ scales, const uint32_t* __restrict__ qzeros,
             float* __restrict__ y, int K, int N, int group, int B, int SPL) {
    constexpr int KG = kGqT / LR, CW = 4 * LR, kU = GqAct<TA>::kU4;
    constexpr int kOs = 8 / GS;  // octets per group inside a segment
    constexpr int kSW = sizeof(TS) == 2 ? 2 : 4, kZW = AWQ ? 1 : 4;
    extern __shared__ uint4 av_s[];  // [B][K/8 + KG] octets of kU x 16 bytes
    __shared__ float red[KG][BM][CW];
    const int tid = threadIdx.x, cq = tid % LR, kg = tid / LR;
    const int n0 = blockIdx.x * CW + 4 * cq;
    const int nc = min(n0, N - 4);  // lanes past N read the last 4 columns, not stored
    const int K8 = K >> 3, rs = K8 + KG;  // LDS row stride in octets
    const int ob = kg * SPL * 8;          // the k-group's first octet
    const int nseg = max(0, min(SPL, (K8 - ob) >> 3));  // its segments (the last k-groups may
                                                        // have fewer or none)
    // one segment's words, with its groups' scales and zeros raw (fp16 scales as 2 words,
    // fp32 as 4; GPTQ zeros as the 4 columns' words, AWQ as the one word holding them)
    struct Seg {
        uint4 q[8];
        uint32_t s[GS][kSW];
        uint32_t z[GS][kZW];
    };
    auto load_seg = [&](Seg& d, int seg) {  // scales and zeros first: they are used first
#pragma unroll
        for (int gi = 0; gi < GS; ++gi) {
            const int g = ((ob + seg * 8) * 8) / group + gi;
            if (kSW == 2) {
                const uint2 v = *reinterpret_cast<const uint2*>(scales + (int64_t)g * N + nc);
                d.s[gi][0] = v.x;
                d.s[gi][kSW - 1] = v.y;
            } else {
                const uint4 v = *reinterpret_cast<const uint4*>(scales + (int64_t)g * N + nc);
                d.s[gi][0] = v.x;
                d.s[gi][1 % kSW] = v.y;
                d.s[gi][2 % kSW] = v.z;
                d.s[gi][kSW - 1] = v.w;
            }
            if (AWQ) {
                d.z[gi][0] = qzeros[(int64_t)g * (N / 8) + nc / 8];
            } else {
                const uint4 v = *reinterpret_cast<const uint4*>(qzeros + (int64_t)(g / 8) * N + nc);
                d.z[gi][0] = v.x;
                d.z[gi][1 % kZW] = v.y;
                d.z[gi][2 % kZW] = v.z;
                d.z[gi][kZW - 1] = v.w;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            d.q[u] = *reinterpret_cast<const uint4*>(qweight + (int64_t)(ob + seg * 8 + u) * N + nc);
    };
    // activations first (an L2 hit in a decode step: written by the step before): the octets
    // of all rows (contiguous, B * K / 8 of them), at most kGqStg 16-byte units per thread,
    // into LDS; then the first segment's loads, which stay in flight across the barrier
    // (s_barrier after the LDS stores alone, no wait for the vector loads)
    constexpr int kStg = kGqStg / kU;
    const int octs = B * K8, orng = SPL * 8;
#pragma unroll
    for (int j = 0; j < kStg; ++j) {
        const int i = tid + j * kGqT;
        if (i >= octs) break;
        const int b = i / K8, o = i - b * K8;
        uint4 v[kU];
#pragma unroll
        for (int h = 0; h < kU; ++h) v[h] = reinterpret_cast<const uint4*>(act)[i * kU + h];
        if (kU == 1 && !AWQ) {  // fp16 halves (0,1)(2,3)(4,5)(6,7) -> (0,4)(1,5)(2,6)(3,7)
            const uint4 w = v[0];
            v[0] = uint4{(w.x & 0xffffu) | (w.z << 16), (w.x >> 16) | (w.z & 0xffff0000u),
                         (w.y & 0xffffu) | (w.w << 16), (w.y >> 16) | (w.w & 0xffff0000u)};
        } else if (kU == 2 && AWQ) {  // fp32 (0..3)(4..7) -> (0,2,4,6)(1,3,5,7)
            const uint4 lo = v[0], hi = v[kU - 1];
            v[0] = uint4{lo.x, lo.z, hi.x, hi.z};
            v[kU - 1] = uint4{lo.y, lo.w, hi.y, hi.w};
        }
#pragma unroll
        for (int h = 0; h < kU; ++h) av_s[(b * rs + o + o / orng) * kU + h] = v[h];
    }
    Seg sa, sb;
    if (nseg > 0) load_seg(sa, 0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    uint32_t lo4 = 0x000f000fu, one024 = 0x64006400u;  // VGPR operands of v_and_or_b32
    asm volatile("" : "+v"(lo4), "+v"(one024));
    float acc[BM][4];
#pragma unroll
    for (int b = 0; b < BM; ++b)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[b][c] = 0.0f;
    auto compute_seg = [&](const Seg& d, int seg) {
#pragma unroll
        for (int gi = 0; gi < GS; ++gi) {
            const int g = ((ob + seg * 8) * 8) / group + gi;
            float sc[4], zf[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (kSW == 2)
                    sc[c] = half_bits_to_float((uint16_t)(d.s[gi][(c >> 1) % kSW] >> (16 * (c & 1))));
                else
                    sc[c] = __builtin_bit_cast(float, d.s[gi][c % kSW]);
                if (AWQ)
                    zf[c] = (float)((d.z[gi][0] >> (4 * (nc % 8 + c))) & 15u);
                else
                    zf[c] = (float)(((d.z[gi][c % kZW] >> (4 * (g % 8))) & 15u) + 1);
            }
            float gs[BM][4];
#pragma unroll
            for (int b = 0; b < BM; ++b)
#pragma unroll
                for (int c = 0; c < 4; ++c) gs[b][c] = 0.0f;
#pragma unroll
            for (int uu = 0; uu < kOs; ++uu) {
                const int u = gi * kOs + uu;  // octet of the segment
                const int o = ob + seg * 8 + u;
                const uint32_t qw4[4] = {d.q[u].x, d.q[u].y, d.q[u].z, d.q[u].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if (kU == 1) {
                        const _Float16 bz = (_Float16)(-1024.0f - zf[c]);
                        const h2v bias = {bz, bz};
                        h2v wd[4];  // nibbles (i, i + 4)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t zz = ((qw4[c] >> (4 * i)) & lo4) | one024;
                            wd[i] = __builtin_bit_cast(h2v, zz) + bias;
                        }
#pragma unroll
                        for (int b = 0; b < BM; ++b) {  // rows past B: row B - 1, not stored
                            const uint4 A = av_s[min(b, B - 1) * rs + o + kg];
                            float t = gs[b][c];
                            t = __builtin_amdgcn_fdot2(wd[0], __builtin_bit_cast(h2v, A.x), t, false);
                            t = __builtin_amdgcn_fdot2(wd[1], __builtin_bit_cast(h2v, A.y), t, false);
                            t = __builtin_amdgcn_fdot2(wd[2], __builtin_bit_cast(h2v, A.z), t, false);
                            t = __builtin_amdgcn_fdot2(wd[3], __builtin_bit_cast(h2v, A.w), t, false);
                            gs[b][c] = t;
                        }
                    } else {
                        const uint32_t ev = qw4[c] & 0x0f0f0f0fu, od = (qw4[c] >> 4) & 0x0f0f0f0fu;
                        float wf[8];  // nibble e = position e of the staged octet
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            wf[2 * i] = (float)((ev >> (8 * i)) & 0xffu) - zf[c];
                            wf[2 * i + 1] = (float)((od >> (8 * i)) & 0xffu) - zf[c];
                        }
#pragma unroll
                        for (int b = 0; b < BM; ++b) {
                            const int ab = (min(b, B - 1) * rs + o + kg) * 2;
                            const uint4 A0 = av_s[ab];
                            const uint4 A1 = av_s[ab + 1];
                            const uint32_t aw[8] = {A0.x, A0.y, A0.z, A0.w, A1.x, A1.y, A1.z, A1.w};
                            float t = gs[b][c];
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                t = __builtin_fmaf(__builtin_bit_cast(float, aw[e]), wf[e], t);
                            gs[b][c] = t;
                        }
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < BM; ++b)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[b][c] = __builtin_fmaf(gs[b][c], sc[c], acc[b][c]);
        }
    };
    for (int seg = 0; seg < nseg; seg += 2) {
        if (seg + 1 < nseg) load_seg(sb, seg + 1);
        compute_seg(sa, seg);
        if (seg + 1 >= nseg) break;
        if (seg + 2 < nseg) load_seg(sa, seg + 2);
        compute_seg(sb, seg + 1);
    }
#pragma unroll
    for (int b = 0; b < BM; ++b)
#pragma unroll
        for (int c = 0; c < 4; ++c) red[kg][b][4 * cq + c] = acc[b][c];
    __syncthreads();
    for (int t = tid; t < B * CW; t += kGqT) {
        const int b = t / CW, col = t - b * CW;
        const int n = blockIdx.x * CW + col;
        if (n >= N) continue;
        float sum = 0.0f;
        for (int q = 0; q < KG; ++q) sum += red[q][b][col];
        y[(int64_t)b * N + n] = sum;
    }
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

static int pick_lpr(int ngroups) {
    int l = 1;
    while (l < ngroups && l < 64) l <<= 1;
    return l;
}

template <typename TA>
static int launch_q4_0(const TA* act, const uint8_t* w, float* y, int K, int N, int B,
                       hipStream_t st) {
    const int nbk = K / 32;
    const int lpr = pick_lpr((nbk + 7) / 8);
    const bool full = K % 256 == 0 && ((uintptr_t)act & 15) == 0 && ((uintptr_t)w & 15) == 0;
    const size_t smem = full ? ((size_t)f32s_size(K) + 2048) * 4 : (size_t)K * 4;
    dim3 grid((unsigned)ceil_div(N, 256 / lpr), (unsigned)B);
#define Q4_CASE(L)                                                                      \
    case L:                                                                             \
        if (full)                                                                       \
            hipLaunchKernelGGL((q4_0_kernel<TA, L, true>), grid, dim3(256), smem, st, act, w, \
                               y, K, N);                                                \
        else                                                                            \
            hipLaunchKernelGGL((q4_0_kernel<TA, L, false>), grid, dim3(256), smem, st, act, \
                               w, y, K, N);                                             \
        break;
    switch (lpr) {
        Q4_CASE(1) Q4_CASE(2) Q4_CASE(4) Q4_CASE(8) Q4_CASE(16) Q4_CASE(32) Q4_CASE(64)
    }
#undef Q4_CASE
    return launch_status("q4_0_kernel");
}

template <typename TA>
static int launch_q8_0(const TA* act, const uint8_t* w, float* y, int K, int N, int B,
                       hipStream_t st) {
    const int nbk = K / 32;
    const int lpr = pick_lpr((nbk + 7) / 8);
    const bool full = K % 256 == 0 && ((uintptr_t)act & 15) == 0 && ((uintptr_t)w & 15) == 0;
    const size_t smem = full ? ((size_t)f32s_size(K) + 2048) * 4 : (size_t)K * 4;
    // the LDS-staged form when a workgroup's rows and activations fit 64 KiB, so at
    // least two workgroups share a CU (three at K = 4096 with fp16 activations: 51.4 KB)
    const size_t smem_lds = ((size_t)f32s_size(K) + f32s_dump<TA>(K)) * 4 +
                            (size_t)ceil_div(kQ8R * nbk * 34, 1024) * 1024;
    if (full && smem_lds <= 64 * 1024) {
        hipLaunchKernelGGL((q8_0_lds_kernel<TA>), dim3((unsigned)ceil_div(N, kQ8R), (unsigned)B),
                           dim3(256), smem_lds, st, act, w, y, K, N);
        return launch_status("q8_0_lds_kernel");
    }
    dim3 grid((unsigned)ceil_div(N, 256 / lpr), (unsigned)B);
#define Q80_CASE(L)                                                                      \
    case L:                                                                              \
        if (full)                                                                        \
            hipLaunchKernelGGL((q8_0_kernel<TA, L, true>), grid, dim3(256), smem, st, act, w, \
                               y, K, N);                                                 \
        else                                                                             \
            hipLaunchKernelGGL((q8_0_kernel<TA, L, false>), grid, dim3(256), smem, st, act,  \
                               w, y, K, N);                                              \
        break;
    switch (lpr) {
        Q80_CASE(1) Q80_CASE(2) Q80_CASE(4) Q80_CASE(8) Q80_CASE(16) Q80_CASE(32) Q80_CASE(64)
    }
#undef Q80_CASE
    return launch_status("q8_0_kernel");
}

template <bool AWQ, typename TA, typename TS>
static int launch_gq(const TA* act, const uint32_t* qweight, const TS* scales,
                     const uint32_t* qzeros, float* y, int K, int N, int group, int B,
                     hipStream_t st) {
    constexpr bool kF16 = std::is_same<TA, uint16_t>::value;
    // fp16 activations from batch 4 on: fp16 MFMA (K in whole 512-k chunks per part, groups of 16-k steps
    // dividing them, the staged activations within LDS)
    if (kF16 && B >= 4 && B <= 16 && K % kGqChunk == 0 && group % 16 == 0 &&
        kGqChunk % group == 0 && ((uintptr_t)act & 15) == 0 &&
        (size_t)B * (K + 4) * 2 <= kGqLds) {
        int parts = kGqParts;  // K split into 4, 2 or 1 parts of whole chunks
        while (K % (parts * kGqChunk) != 0) parts /= 2;
        const dim3 grid((unsigned)ceil_div(N, 32)), block((unsigned)(128 * parts));
        const size_t lds = (size_t)B * (K + 4) * 2;
        switch (group / 16) {
#define GQM_CASE(NG)                                                                          \
            case NG:                                                                          \
                hipLaunchKernelGGL((gq_mfma_kernel<AWQ, TS, NG>), grid, block, lds, st,        \
                                   (const uint16_t*)act, qweight, scales, qzeros, y, K, N, B); \
                return launch_status(AWQ ? "awq_mfma_kernel" : "gptq_mfma_kernel");
            GQM_CASE(2) GQM_CASE(4) GQM_CASE(8) GQM_CASE(16) GQM_CASE(32)
#undef GQM_CASE
            default: break;  // other group sizes: the packed fp16 dot below
        }
    }
    // batch 1..4: 128-bit weight loads, 4 columns per lane (N % 4 == 0, aligned operands,
    // K in whole 64-k segments, groups of 32 or a multiple of 64)
    {
        constexpr int LR = kGqLR, KG = kGqT / LR;
        const size_t lds = (size_t)B * (K / 8 + KG) * 16 * (kF16 ? 1 : 2);
        const bool aligned = ((uintptr_t)act & 15) == 0 && ((uintptr_t)qweight & 15) == 0 &&
                             ((uintptr_t)scales & (sizeof(TS) == 2 ? 7 : 15)) == 0 &&
                             ((uintptr_t)qzeros & (AWQ ? 3 : 15)) == 0;
        if (B <= 4 && N % 4 == 0 && K % 64 == 0 && (group == 32 || group % 64 == 0) &&
            aligned && lds <= 64 * 1024 &&
            (size_t)B * (K / 8) * (kF16 ? 1 : 2) <= (size_t)kGqStg * kGqT) {
            const int SPL = (int)ceil_div(K / 64, KG);
            const dim3 grid((unsigned)ceil_div(N, 4 * LR));
#define GQV_CASE(BM, GS)                                                                      \
            if (B <= BM && (GS == 2) == (group == 32)) {                                      \
                hipLaunchKernelGGL((gq_v4_kernel<AWQ, TA, TS, BM, LR, GS>), grid, dim3(kGqT),  \
                                   lds, st, act, qweight, scales, qzeros, y, K, N, group, B,   \
                                   SPL);                                                      \
                return launch_status(AWQ ? "awq_v4_kernel" : "gptq_v4_kernel");               \
            }
            GQV_CASE(1, 1) GQV_CASE(1, 2) GQV_CASE(2, 1) GQV_CASE(2, 2) GQV_CASE(4, 1)
            GQV_CASE(4, 2)
#undef GQV_CASE
        }
    }
    const int tiles = (int)ceil_div(N, 256);
    // split K (in whole groups) until there are ~1024 blocks
    const int ngroups = (int)ceil_div(K, group);
    int splits = (int)ceil_div(1024, tiles);
    if (splits > ngroups) splits = ngroups;
    if (splits < 1) splits = 1;
    const int gps = (int)ceil_div(ngroups, splits);
    splits = (int)ceil_div(ngroups, gps);
    const int KC = gps * group;
    float* part = nullptr;
    uint32_t* cnt = nullptr;
    if (splits > 1) {
        // counters first, at a fixed offset: they are left at zero, while the
        // partials behind them are not cleared between calls
        const size_t cnt_bytes = (size_t)ceil_div((int64_t)tiles * 4, 256) * 256;
        const size_t bytes = cnt_bytes + (size_t)splits * B * N * 4;
        char* ws = (char*)Scratch::get(kScratchTmp, bytes, st);
        if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
        cnt = (uint32_t*)ws;
        part = (float*)(ws + cnt_bytes);
    }
    const size_t smem = (size_t)B * KC * 4;
    if (smem > 64 * 1024) {
        set_error("gptq/awq: batch x group chunk too large for LDS (%zu bytes)", smem);
        return TENZO_ERROR_UNSUPPORTED;
    }
    dim3 grid((unsigned)tiles, (unsigned)splits);
#define GQ_CASE(BM)                                                                          \
    if (B <= BM) {                                                                           \
        if (kF16)                                                                            \
            hipLaunchKernelGGL((gq_h2_kernel<AWQ, TS, BM>), grid, dim3(256),                 \
                               (size_t)BM * KC * 2, st,                                      \
                               (const uint16_t*)act, qweight, scales, qzeros, y, K, N, group, \
                               B, KC, splits, part, cnt);                                    \
        else                                                                                 \
            hipLaunchKernelGGL((gq_kernel<AWQ, TA, TS, BM>), grid, dim3(256), smem, st, act,  \
                               qweight, scales, qzeros, y, K, N, group, B, KC, splits, part,  \
                               cnt);                                                         \
        return launch_status(AWQ ? "awq_kernel" : "gptq_kernel");                            \
    }
    // otherwise the packed fp16 dot (fp16 activations; the pairs need whole k-octets:
    // K % 8 == 0) or fp32 FMAs, 32-bit weight loads, split K
    GQ_CASE(1) GQ_CASE(2) GQ_CASE(4) GQ_CASE(8)
#undef GQ_CASE
    set_error("gptq/awq: batch %d > 8 needs the MFMA path (16-byte aligned fp16 activations, "
              "K %% 512 == 0, group 32..512 dividing 512, B (K + 4) fp16 within 152 KiB of LDS)",
              B);
    return TENZO_ERROR_UNSUPPORTED;
}

template <bool AWQ>
static int dispatch_gq(const void* act, int act_dtype, const uint32_t* qweight,
                       const void* scales, int scale_dtype, const uint32_t* qzeros, float* y,
                       int K, int N, int group, int B, hipStream_t st) {
    if (act_dtype == 0 && scale_dtype == 0)
        return launch_gq<AWQ>((const float*)act, qweight, (const float*)scales, qzeros, y, K, N,
                              group, B, st);
    if (act_dtype == 0 && scale_dtype == 1)
        return launch_gq<AWQ>((const float*)act, qweight, (const uint16_t*)scales, qzeros, y, K,
                              N, group, B, st);
    if (act_dtype == 1 && scale_dtype == 0)
        return launch_gq<AWQ>((const uint16_t*)act, qweight, (const float*)scales, qzeros, y, K,
                              N, group, B, st);
    return launch_gq<AWQ>((const uint16_t*)act, qweight, (const uint16_t*)scales, qzeros, y, K,
                          N, group, B, st);
}

}  // namespace tz

using namespace tz;

extern "C" {

TENZO_HIP_API int tenzo_hip_gemv_q4_0(const void* act, int act_dtype, const uint8_t* w,
                                      float* y, int K, int N, int B, void* stream) {
    TZ_CHECK(act && w && y, "gemv_q4_0: null pointer");
    TZ_CHECK(K > 0 && K % 32 == 0 && N > 0 && B > 0 && B <= 65535,
             "gemv_q4_0: need K %% 32 == 0 (K=%d)", K);
    TZ_CHECK(K <= 16384, "gemv_q4_0: K=%d above the LDS staging limit 16384", K);
    TZ_CHECK(act_dtype == 0 || act_dtype == 1, "gemv_q4_0: act_dtype must be 0 or 1");
    hipStream_t st = (hipStream_t)stream;
    if (act_dtype == 0) return launch_q4_0((const float*)act, w, y, K, N, B, st);
    // fp16 activations: the packed fp16 dot kernel
    const int nbk = K / 32;
    const int lpr = pick_lpr((nbk + 7) / 8);
    const size_t smem = (size_t)K * 2;
    dim3 grid((unsigned)ceil_div(N, 256 / lpr), (unsigned)B);
    const uint16_t* a16 = (const uint16_t*)act;
    const bool full = K % 256 == 0 && ((uintptr_t)act & 15) == 0 && ((uintptr_t)w & 15) == 0;
    const size_t smem_full = smem + (size_t)(nbk + 7) / 8 * 16 + 256 * 32;  // padding, spare slots
#define Q4H_CASE(L)                                                                        \
    case L:                                                                                \
        if (full)                                                                          \
            hipLaunchKernelGGL((q4_0_f16_kernel<L, true>), grid, dim3(256), smem_full, st,   \
                               a16, w, y, K, N);                                           \
        else                                                                               \
            hipLaunchKernelGGL((q4_0_f16_kernel<L, false>), grid, dim3(256), smem, st, a16,  \
                               w, y, K, N);                                                \
        break;
    switch (lpr) {
        Q4H_CASE(1) Q4H_CASE(2) Q4H_CASE(4) Q4H_CASE(8) Q4H_CASE(16) Q4H_CASE(32) Q4H_CASE(64)
    }
#undef Q4H_CASE
    return launch_status("q4_0_f16_kernel");
}

TENZO_HIP_API int tenzo_hip_gemv_q8_0(const void* act, int act_dtype, const uint8_t* w,
                                      float* y, int K, int N, int B, void* stream) {
    TZ_CHECK(act && w && y, "gemv_q8_0: null pointer");
    TZ_CHECK(K > 0 && K % 32 == 0 && N > 0 && B > 0 && B <= 65535,
             "gemv_q8_0: need K %% 32 == 0 (K=%d)", K);
    TZ_CHECK(K <= 16384, "gemv_q8_0: K=%d above the LDS staging limit 16384", K);
    TZ_CHECK(((uintptr_t)w & 1) == 0, "gemv_q8_0: weights must be 2-byte aligned");
    TZ_CHECK(act_dtype == 0 || act_dtype == 1, "gemv_q8_0: act_dtype must be 0 or 1");
    hipStream_t st = (hipStream_t)stream;
    if (act_dtype == 0) return launch_q8_0((const float*)act, w, y, K, N, B, st);
    return launch_q8_0((const uint16_t*)act, w, y, K, N, B, st);
}

TENZO_HIP_API int tenzo_hip_gemv_q4_0_q8_0(const uint8_t* qa, const uint8_t* w, float* y,
                                           int K, int N, int B, void* stream) {
    TZ_CHECK(qa && w && y, "gemv_q4_0_q8_0: null pointer");
    TZ_CHECK(K > 0 && K % 32 == 0 && N > 0 && B > 0 && B <= 65535,
             "gemv_q4_0_q8_0: need K %% 32 == 0");
    const int nbk = K / 32;
    const size_t smem = (size_t)nbk * 10 * 4;
    TZ_CHECK(smem <= 64 * 1024, "gemv_q4_0_q8_0: K=%d too large", K);
    hipStream_t st = (hipStream_t)stream;
    if (K % 256 == 0 && ((uintptr_t)qa & 15) == 0 && ((uintptr_t)w & 15) == 0) {
        // raw blocks, then codes (32 bytes + 16 per group), scales and sums (+ 1 per group),
        // one spare 16-byte slot per thread
        const int ng = nbk / 8;
        const size_t smem_full = (size_t)nbk * 34 + (size_t)(2 * nbk + ng) * 16 +
                                 ((size_t)(nbk + ng) * 8 + 15) / 16 * 16 + 256 * 16;
        const int lpr = pick_lpr(ng);
        dim3 grid((unsigned)ceil_div(N, 256 / lpr), (unsigned)B);
#define Q8F_CASE(L)                                                                         \
        case L:                                                                             \
            hipLaunchKernelGGL((q4_0_q8_full_kernel<L>), grid, dim3(256), smem_full, st, qa, \
                               w, y, K, N);                                                 \
            break;
        switch (lpr) {
            Q8F_CASE(1) Q8F_CASE(2) Q8F_CASE(4) Q8F_CASE(8) Q8F_CASE(16) Q8F_CASE(32) Q8F_CASE(64)
        }
#undef Q8F_CASE
        return launch_status("q4_0_q8_full_kernel");
    }
    const int lpr = pick_lpr(nbk / 4 > 0 ? nbk / 4 : 1);
    dim3 grid((unsigned)ceil_div(N, 256 / lpr), (unsigned)B);
#define Q8_CASE(L)                                                                           \
    case L:                                                                                  \
        hipLaunchKernelGGL((q4_0_q8_kernel<L>), grid, dim3(256), smem, st, qa, w, y, K, N); \
        break;
    switch (lpr) {
        Q8_CASE(1) Q8_CASE(2) Q8_CASE(4) Q8_CASE(8) Q8_CASE(16) Q8_CASE(32) Q8_CASE(64)
    }
#undef Q8_CASE
    return launch_status("q4_0_q8_kernel");
}

TENZO_HIP_API int tenzo_hip_gemv_gptq(const void* act, int act_dtype, const uint32_t* qweight,
                                      const void* scales, int scale_dtype,
                                      const uint32_t* qzeros, float* y, int K, int N,
                                      int group, int B, void* stream) {
    TZ_CHECK(act && qweight && scales && qzeros && y, "gemv_gptq: null pointer");
    TZ_CHECK(K > 0 && K % 8 == 0 && N > 0 && group > 0 && group % 8 == 0 && B >= 1 && B <= 16,
             "gemv_gptq: need K %% 8 == 0, group %% 8 == 0, 1 <= B <= 16");
    TZ_CHECK((act_dtype == 0 || act_dtype == 1) && (scale_dtype == 0 || scale_dtype == 1),
             "gemv_gptq: dtype codes must be 0 (fp32) or 1 (fp16)");
    return dispatch_gq<false>(act, act_dtype, qweight, scales, scale_dtype, qzeros, y, K, N,
                              group, B, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_gemv_awq(const void* act, int act_dtype, const uint32_t* qweight,
                                     const void* scales, int scale_dtype,
                                     const uint32_t* qzeros, float* y, int K, int N, int group,
                                     int B, void* stream) {
    TZ_CHECK(act && qweight && scales && qzeros && y, "gemv_awq: null pointer");
    TZ_CHECK(K > 0 && K % 8 == 0 && N > 0 && N % 8 == 0 && group > 0 && group % 8 == 0 &&
                 B >= 1 && B <= 16,
             "gemv_awq: need K %% 8 == 0, N %% 8 == 0, group %% 8 == 0, 1 <= B <= 16");
    TZ_CHECK((act_dtype == 0 || act_dtype == 1) && (scale_dtype == 0 || scale_dtype == 1),
             "gemv_awq: dtype codes must be 0 (fp32) or 1 (fp16)");
    return dispatch_gq<true>(act, act_dtype, qweight, scales, scale_dtype, qzeros, y, K, N,
                             group, B, (hipStream_t)stream);
}

}  // extern "C"

// Batched TL1 contraction over M tokens on int8 MFMA (multi-token prefill).
//
// The reference prefills one token at a time: prefill_token
// (src/runtime/TenzoEngine.cpp:1809-1819) runs compute_from_lut (:129-146)
// once per token and projection. Here the M tokens of a prompt share one
// pass over the weights: acc[m][n] = sum_k W[n][k] * codes[m][k] is an
// integer GEMM on v_mfma_i32_16x16x64_i8 whose int32 results are exact, so
// every output equals the per-token GEMV's bit for bit.
//
// Operands (no extra weight copy: the decode GEMV layout is read as is):
//   W  the TL1 device layout of tl1.hip: per row block b (64 rows) and
//      super-chunk s (64 columns), row r's 16 bytes hold dword q = columns
//      64s+16q+c as u = w+1 at bit 8*(c%4)+2*(c/4). (dword >> 2j) & 0x03030303
//      are the bytes of columns 16q+4j .. 16q+4j+3 in order.
//   codes  int8 [M][Kp] (Kp = 64*ceil(K/64), zero padded), with
//      q[m] = {inv_scale, sum of codes} from the activation quantizer.
// Since u = w + 1, sum_k w_k a_k = sum_k u_k a_k - sum_k a_k: the epilogue
// subtracts the code sum of the token, as the GEMV does. Every output is one
// workgroup's, so there is no cross-workgroup reduction and no scratch.
//
// v_mfma_i32_32x32x32_i8 is used rather than 16x16x64: at one wave per SIMD
// it issues one per 34 cycles (4.6 POP/s over the chip) where 16x16x64
// issues one per 32 cycles for half the work.
#include "common.h"
#include "tl1.h"

namespace tz {
namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kRawBuffer = 0x00020000;  // buffer resource word 3: raw buffer, gfx9 family
constexpr uint32_t kField = 0x03030303u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRawBuffer);
}
// 16 bytes per lane from a buffer straight into LDS (no registers): lane l's
// bytes land at dst + 16 l. Offsets past the resource's byte count read zeros.
__device__ __forceinline__ void to_lds16(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, off, 0, 0, 0);
}
// s_barrier without the workgroup fence of __syncthreads(), whose release half
// waits for every outstanding vector memory operation (vmcnt 0), which would
// drain the ring's loads at each chunk. The memory clobber keeps LDS accesses
// on their side of it; LDS-DMA completion is waited for explicitly (wait_vm).
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }
// Keeps the memory operations before it ahead of the instructions after it:
// the compiler memory clobber stops IR passes from sinking the loads to their
// first use, the scheduling barrier stops the machine scheduler.
__device__ __forceinline__ void issue_point() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}
template <int N> __device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// y = resid + float(acc - code_sum) * (inv_scale * row scale) for rows
// row .. row+3 of token m (compute_from_lut :118-126 and the residual adds of
// forward_layer_raw :1590 / :1628), one fp32 multiply and one fp32 add each.
__device__ __forceinline__ void finalize4(i4v v, const tenzo_hip_actq_t a, int m, int64_t row,
                                          int64_t N, const RowScales& rs, float* __restrict__ y,
                                          const float* __restrict__ resid,
                                          int32_t* __restrict__ acc_out) {
    int j = 0;
    while (j < rs.n - 1 && row >= rs.end[j]) ++j;  // segment ends are multiples of 64
    const float sc = __fmul_rn(a.inv_scale, rs.scale[j]);
    const int64_t o = (int64_t)m * N + row;
    const int d0 = v[0] - a.code_sum, d1 = v[1] - a.code_sum, d2 = v[2] - a.code_sum,
              d3 = v[3] - a.code_sum;
    float4 out = make_float4((float)d0 * sc, (float)d1 * sc, (float)d2 * sc, (float)d3 * sc);
    if (resid) {
        const float4 r = *reinterpret_cast<const float4*>(resid + o);
        out.x = __fadd_rn(r.x, out.x);
        out.y = __fadd_rn(r.y, out.y);
        out.z = __fadd_rn(r.z, out.z);
        out.w = __fadd_rn(r.w, out.w);
    }
    *reinterpret_cast<float4*>(y + o) = out;
    if (acc_out) *reinterpret_cast<int4*>(acc_out + o) = make_int4(d0, d1, d2, d3);
}

}  // namespace

// One workgroup = 4 waves = RW row waves x KW = 4 / RW K groups; it owns
// 64*RW rows (row blocks RW*bt .. RW*bt+RW-1) and BM = 32*CT tokens. K group
// kg takes the contiguous chunk run [kg*T, (kg+1)*T) (T = ceil(KS/KW); chunks
// past its end read zero weights). Each 64-column chunk is two 32-deep MFMA
// steps, h = 0, 1, and a wave's 64 rows are two 32-row tiles.
//
// v_mfma_i32_32x32x32_i8 operands (lane l = 32g + i):
//   A (weights): row i of the tile, k = 16g .. 16g+15 of the step: for step
//      h that is dword 2h + g of the row's 16-byte record, unpacked.
//   B (codes):   token i of the 32-token tile, the same columns: 16 bytes at
//      codes[m][64s + 16(2h + g)].
//   C:           token i, rows 8(j/4) + 4g + j%4 for registers j = 0..15.
// Per chunk and K group an LDS ring slot holds
//   codes:   2*CT fragments of 1 KiB (tile u, step h at (2u + h) KiB; lane l's
//            16 bytes at 16 l),
//   weights: RW row blocks of 1 KiB (lane l = the 16-byte record of row l),
// filled by direct-to-LDS loads issued kRing - 2 chunks ahead. Each wave loads
// its own row block's weights and 2*CT / RW of the group's code fragments.
// One block barrier per chunk both publishes the chunk and frees the slot the
// next loads overwrite. K groups then add their int32 tiles through LDS.
template <int RW, int KW, int CT>
__global__ void __launch_bounds__(64 * RW * KW)
tl1_mfma_kernel(const uint8_t* __restrict__ w, const int8_t* __restrict__ codes,
                const tenzo_hip_actq_t* __restrict__ aq, int M, int64_t N, int KS, int mtiles,
                RowScales rs, float* __restrict__ y, const float* __restrict__ resid,
                int32_t* __restrict__ acc_out) {
    constexpr int CH = 1;  // chunks per step (2 measured no faster)
    constexpr int BM = 32 * CT;
    constexpr int kFrags = 2 * CT;  // code fragments per chunk and K group
    static_assert(kFrags % RW == 0, "each row wave loads the same number of fragments");
    constexpr int kChunkBytes = (kFrags + RW) * 1024;  // one chunk of one K group
    constexpr int kGroupBytes = CH * kChunkBytes;       // one step of one K group
    constexpr int kSlotBytes = KW * kGroupBytes;
    constexpr int kLoads = CH * (1 + kFrags / RW);  // direct-to-LDS loads per wave and step
    // LDS ring of about 64 KiB, at least 4 slots: kRing - 2 steps in flight
    // ahead of the one being read (deeper rings measured no faster: the
    // per-wave issue rate, not the latency, bounds the stream)
    constexpr int kRingFit = 65536 / kSlotBytes;
    constexpr int kRing = kRingFit < 4 ? 4 : (kRingFit > 8 ? 8 : kRingFit);
    static_assert((kRing - 1) * kLoads <= 63, "vmcnt counts at most 63 loads");
    constexpr int kRingBytes = kRing * kSlotBytes;
    constexpr int kRedBytes = KW > 1 ? RW * 2 * CT * 4096 : 0;
    __shared__ __attribute__((aligned(16)))
    char lds[kRingBytes > kRedBytes ? kRingBytes : kRedBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rw = wave % RW, kg = wave / RW;
    const int G = gridDim.x, id = blockIdx.x;
    // consecutive tile ids (same row blocks: the same weights) on one XCD
    const int tid = (G & 7) == 0 ? (id & 7) * (G >> 3) + (id >> 3) : id;
    const int bt = tid / mtiles, mt = tid - bt * mtiles;
    const int b = bt * RW + rw;
    const int m0 = mt * BM;
    const int Kp = KS * 64;
    const int run = (KS + KW - 1) / KW;
    const int cb = min(KS, kg * run), ce = min(KS, cb + run);
    const int T = (run + CH - 1) / CH;  // steps

    // weights of this wave's row block, chunks [0, ce) readable
    const __amdgpu_buffer_rsrc_t rw_res = buf(w + (size_t)b * KS * 1024, (uint32_t)ce * 1024u);
    const __amdgpu_buffer_rsrc_t rc_res =
        buf(codes + (size_t)m0 * Kp, (uint32_t)min(BM, M - m0) * (uint32_t)Kp);
    const uint32_t woff = (uint32_t)lane * 16u;
    const uint32_t coff = (uint32_t)((lane & 31) * Kp + (lane >> 5) * 16);

    // step i of this K group (chunks cb + CH*i + e) into ring slot i % kRing
    auto issue = [&](int i) {
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            char* slot = lds + (i % kRing) * kSlotBytes + kg * kGroupBytes + e * kChunkBytes;
            const int c = cb + CH * i + e;
            // past the group's run: an offset past both resources (reads zeros)
            const uint32_t cw = c < ce ? (uint32_t)c * 1024u + woff : 0x80000000u;
            to_lds16(rw_res, slot + kFrags * 1024 + rw * 1024, cw);
#pragma unroll
            for (int j = 0; j < kFrags / RW; ++j) {
                const int q = rw + RW * j, u = q >> 1, h = q & 1;
                const uint32_t cc = c < ce ? (uint32_t)c * 64u + (uint32_t)(u * 32 * Kp + h * 32) + coff
                                           : 0x80000000u;
                to_lds16(rc_res, slot + q * 1024, cc);
            }
        }
    };

    // Fragments of one step in registers: packed weight dwords (chunk e, row
    // tile t, MFMA step h) and the code fragments (chunk e, tile u, step h).
    struct Frag {
        uint32_t wd[CH][2][2];
        i4v B[CH][CT][2];
    };
    auto read = [&](int i, Frag& f) {
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const char* slot = lds + (i % kRing) * kSlotBytes + kg * kGroupBytes + e * kChunkBytes;
#pragma unroll
            for (int u = 0; u < CT; ++u)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    f.B[e][u][h] =
                        *reinterpret_cast<const i4v*>(slot + (2 * u + h) * 1024 + lane * 16);
            const uint32_t* wrow = reinterpret_cast<const uint32_t*>(
                slot + kFrags * 1024 + rw * 1024 + (lane & 31) * 16 + (lane >> 5) * 4);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                f.wd[e][t][0] = wrow[t * 128];
                f.wd[e][t][1] = wrow[t * 128 + 2];
            }
        }
    };
    i16v acc[2][CT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < CT; ++u) acc[t][u] = i16v{};
    // The weight fields of the step's chunks x 2 row tiles x 2 MFMA steps,
    // then the MFMAs.
    auto unpack = [&](const Frag& f, i4v (&A)[CH][2][2]) {
#pragma unroll
        for (int e = 0; e < CH; ++e)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t wd = f.wd[e][t][h];
                    A[e][t][h] = i4v{(int)(wd & kField), (int)((wd >> 2) & kField),
                                     (int)((wd >> 4) & kField), (int)((wd >> 6) & kField)};
                }
    };
    auto mma = [&](const Frag& f, const i4v (&A)[CH][2][2]) {
#pragma unroll
        for (int e = 0; e < CH; ++e)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int u = 0; u < CT; ++u)
                        acc[t][u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[e][t][h], f.B[e][u][h],
                                                                          acc[t][u], 0, 0, 0);
    };

    // Step j computes from registers while step j+1's fragments are read from
    // LDS and step j+kRing-1 is loaded into the slot of step j-1 (read at step
    // j-2, so free once every wave has passed this step's barrier). Step j's
    // weight fields are unpacked before step j+1's reads go out, so waiting for
    // its fragments does not wait for those reads. Steps run in pairs over two
    // register sets; an odd count ends on a zero step.
#pragma unroll
    for (int i = 0; i < kRing - 1; ++i) issue(i);
    wait_vm<(kRing - 2) * kLoads>();
    block_barrier();
    Frag f0, f1;
    i4v A[CH][2][2];
    read(0, f0);
    for (int j = 0; j < T; j += 2) {
        wait_vm<(kRing - 3) * kLoads>();  // step j+1 landed (this wave's loads)
        block_barrier();                   // and everyone's
        issue(j + kRing - 1);
        unpack(f0, A);
        issue_point();
        read(j + 1, f1);
        issue_point();  // the reads go out before the MFMAs
        mma(f0, A);
        __builtin_amdgcn_sched_barrier(0);  // the MFMAs stay ahead of the next barrier
        wait_vm<(kRing - 3) * kLoads>();
        block_barrier();
        issue(j + kRing);
        unpack(f1, A);
        issue_point();
        read(j + 2, f0);
        issue_point();
        mma(f1, A);
        __builtin_amdgcn_sched_barrier(0);
    }

    // the loads issued past the end (zeros) still write the ring: let them land
    // before the ring is reused or the workgroup's LDS is released
    wait_vm<0>();
    // K groups 1 .. KW-1 hand their tiles to group 0 one at a time through
    // one LDS buffer (RW * 2 * CT tiles of 4 KiB, over the ring)
    if (KW > 1) {
        i16v* red = reinterpret_cast<i16v*>(lds);
        for (int g = 1; g < KW; ++g) {
            __syncthreads();  // the ring (g = 1) or the buffer (g > 1) is free
            if (kg == g) {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int u = 0; u < CT; ++u) red[((rw * 2 + t) * CT + u) * 64 + lane] = acc[t][u];
            }
            __syncthreads();
            if (kg == 0) {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int u = 0; u < CT; ++u) acc[t][u] += red[((rw * 2 + t) * CT + u) * 64 + lane];
            }
        }
        if (kg > 0) return;
    }

    // C lane layout: token 32u + lane % 32, rows 32t + 8q + 4(lane / 32) + 0..3
    // in registers 4q .. 4q+3
#pragma unroll
    for (int u = 0; u < CT; ++u) {
        const int m = m0 + 32 * u + (lane & 31);
        if (m >= M) continue;
        const tenzo_hip_actq_t a = aq[m];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                finalize4(i4v{acc[t][u][4 * q], acc[t][u][4 * q + 1], acc[t][u][4 * q + 2],
                              acc[t][u][4 * q + 3]},
                          a, m, (int64_t)b * 64 + 32 * t + 8 * q + 4 * (lane >> 5), N, rs, y,
                          resid, acc_out);
    }
}

// Workgroup shape for M tokens, a rule fitted to a sweep of every shape on
// MI355X (K = 2560 and 6912, N = 2560 .. 13824, M = 16 .. 512): a workgroup
// fetches about 11-13 B/cycle whatever its wave count or ring depth, so the
// time follows the bytes per workgroup and the number of workgroups that run
// at once. 128 rows x 32 tokens with two K groups (221) is best while the
// grid holds 128 .. 600 of them; fewer (small M or N) favour 64 rows x 32
// tokens with four K groups (411: four times the workgroups); more favour
// 256 rows x 64 tokens (142: a quarter of the operand bytes per output).
void tl1_mfma_plan(int64_t M, int64_t N, int64_t KS, int* KW, int* RW, int* CT) {
    (void)KS;
    const int64_t nb = N / 64;
    const int64_t wgs221 = nb % 2 == 0 ? (nb / 2) * ceil_div(M, 32) : 0;
    if (nb % 4 == 0 && (wgs221 > 600 || wgs221 == 0) && M >= 128) {
        *KW = 1, *RW = 4, *CT = 2;
    } else if (wgs221 >= 128) {
        *KW = 2, *RW = 2, *CT = 1;
    } else {
        *KW = 4, *RW = 1, *CT = 1;
    }
}

int launch_tl1_mfma(const int8_t* codes, const tenzo_hip_actq_t* q, const void* w_packed,
                    const RowScales& rs, int64_t M, int64_t N, int64_t K, float* y,
                    const float* resid, int32_t* acc_out, hipStream_t st, int tile) {
    const int64_t nb = N / 64, KS = ceil_div(K, 64);
    int KW = 4, RW = 1, CT = 1;
    tl1_mfma_plan(M, N, KS, &KW, &RW, &CT);
    if (tile > 0) {  // forced shape: 100 * KW + 10 * RW + CT
        KW = tile / 100;
        RW = tile / 10 % 10;
        CT = tile % 10;
    }
    const int64_t mtiles = ceil_div(M, 32 * CT);
    const int64_t grid = (nb / (RW > 0 ? RW : 1)) * mtiles;
    if (RW <= 0 || nb % RW || grid > INT32_MAX || M * KS * 64 > (int64_t)INT32_MAX ||
        K > (1 << 20)) {
        set_error("tl1_mfma: unsupported shape (M=%lld N=%lld K=%lld tile=%d)", (long long)M,
                  (long long)N, (long long)K, tile);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
#define TL1_MFMA_CASE(KG, R, C)                                                               \
    if (KW == KG && RW == R && CT == C) {                                                     \
        hipLaunchKernelGGL((tl1_mfma_kernel<R, KG, C>), dim3((unsigned)grid),                 \
                           dim3(64 * R * KG), 0, st, (const uint8_t*)w_packed, codes, q,      \
                           (int)M, N, (int)KS, (int)mtiles, rs, y, resid, acc_out);           \
        return launch_status("tl1_mfma_kernel");                                              \
    }
    TL1_MFMA_CASE(1, 4, 2) TL1_MFMA_CASE(2, 4, 2) TL1_MFMA_CASE(4, 4, 2)
    TL1_MFMA_CASE(2, 2, 2) TL1_MFMA_CASE(4, 2, 2) TL1_MFMA_CASE(2, 2, 1) TL1_MFMA_CASE(4, 2, 1)
    TL1_MFMA_CASE(4, 1, 2) TL1_MFMA_CASE(4, 1, 1) TL1_MFMA_CASE(8, 1, 1)
#undef TL1_MFMA_CASE
    set_error("tl1_mfma: no kernel for tile KW=%d RW=%d CT=%d", KW, RW, CT);
    return TENZO_ERROR_INVALID_ARGUMENT;
}

}  // namespace tz

using namespace tz;

extern "C" {

TENZO_HIP_API int tenzo_hip_bitlinear_tl1_batch(const int8_t* codes, const tenzo_hip_actq_t* q,
                                                const void* w_packed, float w_scale, int64_t M,
                                                int64_t N, int64_t K, float* y,
                                                int32_t* acc_out, int tile, void* stream) {
    TZ_CHECK(codes && q && w_packed && y, "bitlinear_tl1_batch: null pointer");
    TZ_CHECK(M > 0 && N > 0 && N % 64 == 0 && K > 0 && tile >= 0,
             "bitlinear_tl1_batch: need M > 0, N %% 64 == 0, K > 0 (M=%lld N=%lld K=%lld)",
             (long long)M, (long long)N, (long long)K);
    RowScales rs = RowScales::single(w_scale);
    return launch_tl1_mfma(codes, q, w_packed, rs, M, N, K, y, nullptr, acc_out,
                           (hipStream_t)stream, tile);
}

}  // extern "C"

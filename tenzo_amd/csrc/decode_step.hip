// Persistent decode-step kernel for gfx950: one cooperative launch runs the
// embedding, all layers and the LM head of one token
// (forward_layer_raw / compute_logits / the greedy sampler of the reference,
// src/runtime/TenzoEngine.cpp:1522-1755), with every CU resident for the
// whole step.
//
// Schedule. The step is a sequence of stages: per layer QKV, ATT, O, GU
// (gate|up), DOWN, then HEAD. Each stage has a list of tasks; stage s's tasks
// go to workgroups off_s, off_s+1, ... (mod nwg) with off_{s+1} = off_s +
// ntasks_s, so consecutive stages mostly use different workgroups. A GEMV
// task is one K slice of a 64-row block of a TL1 matrix: the row blocks of
// the Q|K|V, O and down projections are split along K so that every CU has a
// task, and the slices' exact int32 sums meet in an accumulator through
// integer atomics (addition of integers is exact, so the result does not
// depend on the order of arrival). An attention task is a chunk of the
// context of one kv head; an LM-head task a 64-row block.
//
// Data flow. GEMV outputs stay as int32 accumulators; the stage that reads
// them applies the epilogue y = float(acc - code_sum) * (inv_scale * w_scale)
// (the GEMV's own rounding steps) using the (inv_scale, code_sum) record the
// producing stage published, and adds the residual. Each stage input is built
// in registers (thread t owns float4 groups t, t+kT, ...), normalized and
// quantized there; the RMSNorm sum of squares runs over a copy in LDS in the
// reference build's order (eight FMA chains, common.h). Vectors later
// stages need as floats (x, h1, q|k|v, gate|up) are stored by the workgroups
// of the stage that builds them, 64-element slices spread over those
// workgroups.
//
// Latency. A workgroup issues the read-only loads of a stage (its first
// weight or KV tile, the norm weights) together with the loads of the stage
// input, so each stage costs one memory round trip before its arithmetic.
//
// Synchronisation. Data produced inside the launch is written with
// device-coherent stores / atomics (sc1: written through to the memory side);
// before arriving at a barrier every wave waits for its stores to be
// acknowledged (s_waitcnt). Every vector the stages read back (the per-layer
// x, h1, attention outputs and GEMV accumulators) lives at its own address and
// is written once per launch, before any workgroup reads it; the kernel
// starts with an L2 invalidate (agent-scope acquire) in every workgroup, so an
// XCD's L2 can hold no older copy of those lines and they are read with
// ordinary cached loads: the first workgroup of an XCD to miss fetches a line
// from memory and the other CUs of the XCD hit it in L2. Data rewritten within
// a launch (the attention partials, the sync words) is read with sc1 loads. The barrier is 16 counters on separate 256-byte
// lines polled together by one wave. The attention split-K merge is done by
// the last workgroup to finish a kv head (a per-head arrival counter). Every
// wait is bounded: on timeout a workgroup raises the error word and all
// others abort at their next poll, so the grid always drains.
//
// Arithmetic is the reference's, in the same rounding steps as the
// multi-kernel path (tl1.hip, attention.hip, lm_head.hip).
#include "attention.h"
#include "decode_step.h"
#include "tern_kv.h"

namespace tz {
namespace {

constexpr int kT = kDsThreads;   // threads per workgroup
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kPF = 40 / kW;     // tile uint4 per lane preloaded (a 2560-wide row block)
constexpr int kJ = 8192 / (4 * kT);  // float4 groups per thread: vectors up to 8192
constexpr int kNC = kDsCounters;
constexpr int kD = 128;
constexpr int kPS = kDsPartStride;  // partial record: m, l, -, -, o[128]
constexpr int kTmax = kDsMaxChunk;  // attention tokens per task (LDS V tile)
constexpr int kRT = kW * 8;      // attention tokens per round (8 per wave)
constexpr int kAR = kW >= 8 ? 2 : 4;  // attention rounds preloaded in registers
static_assert(2 * kAR <= kPF, "the attention tile uses the GEMV tile's registers");
static_assert(kW == 4 || kW == 8, "4 or 8 waves per workgroup");
constexpr float kAttnScale = 0.08838834764831845f;  // 1/sqrt(128)

// threadIdx.x behind an empty asm: values derived from it are recomputed in
// each stage instead of being hoisted out of the stage loop (which would keep
// them live, in registers, for the whole kernel).
__device__ __forceinline__ int ltid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
// The wave index, known to the compiler to be the same in every lane.
__device__ __forceinline__ int lwave() { return __builtin_amdgcn_readfirstlane(ltid() >> 6); }

enum Stage { S_QKV = 0, S_ATT = 1, S_O = 2, S_GU = 3, S_DOWN = 4, S_HEAD = 5 };

__device__ __forceinline__ float ldc(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ldci(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ldcu(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stcu(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-coherent 16-byte loads and stores through a raw buffer resource
// (cache policy sc1: served from / written through to the memory side, as the
// relaxed agent-scope atomics above). Loads past the resource's byte count
// read zeros.
typedef float f4v __attribute__((ext_vector_type(4)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, gfx9 family
constexpr int kSc1 = 16;                // cache-policy bit sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRsrcWord3);
}
__device__ __forceinline__ f4v ldc16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1));
}
__device__ __forceinline__ i4v ldc16i(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(i4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1));
}
__device__ __forceinline__ int ldc4i(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kSc1);
}
// Plain (cached) loads of read-only data through a resource: out-of-range
// lanes read zeros, so no branch is needed around them.
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
// Read-once streams (TL1 weight tiles, K/V cache rows, the LM head's rows): the
// nontemporal hint. On a pure 330 MB read it gives ~6% more bandwidth than plain loads
// (6.9 vs 6.5 TB/s); in the decode step it also shortens every grid barrier and the
// attention stage (the streams no longer displace the vectors and sync lines that every
// workgroup re-reads): 962 -> 986 tok/s.
constexpr int kNt = 2;  // cache-policy bit nt
__device__ __forceinline__ uint4 ld16nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kNt));
}
__device__ __forceinline__ int ld4int(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kNt);
}
__device__ __forceinline__ f4v ld16f(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
__device__ __forceinline__ i4v ld16i(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(i4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
__device__ __forceinline__ int ld4i(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0);
}
__device__ __forceinline__ uint32_t ld2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, byte_off, 0, 0);
}
__device__ __forceinline__ void stc16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float4 v) {
    const f4v w = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, w), r, byte_off, 0, kSc1);
}

// ---------------------------------------------------------------- layout --

// The per-layer descriptors are copied into LDS when the kernel starts (a
// scalar load of layer l's entry would otherwise miss its cache at the layer's
// first stage and stall every wave for an HBM round trip). Fields are read
// from LDS at a uniform address and moved to scalar registers.
__shared__ DsLayer s_layers[kDsMaxLayers];
// The RSQRTSS estimate table of inv_rms_ref, staged with the layer table.
__shared__ uint32_t s_rsq[kRsqrtEstWords];

template <class T>
__device__ __forceinline__ T* uni_ptr(T* q) {
    const uint64_t v = reinterpret_cast<uint64_t>(q);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

struct LayerRef {
    int l;
    __device__ const uint4* mat(int slot) const { return uni_ptr(s_layers[l].mat[slot]); }
    __device__ const float* norm(int slot) const { return uni_ptr(s_layers[l].norm[slot]); }
    __device__ float sc(int i) const {
        return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(s_layers[l].sc[i])));
    }
};
__device__ __forceinline__ LayerRef layer(const DsParams&, int l) { return LayerRef{l}; }

// Copies the layer table and the RSQRTSS table into LDS (all threads; a block
// barrier follows).
// paged_int8: the sequence's block table (blocks 0 .. pos / 16), copied into
// LDS at the start of the kernel, and the pool row of token t of (l, h):
// ((block_table[t / 16] * L + l) * Hkv + h) * 16 + t % 16 (PagedKVCache's
// layout, TenzoEngine.cpp:320-321).
__shared__ int32_t s_bt[kDsMaxBlocks];
__device__ __forceinline__ void stage_blocks(const DsParams& p) {
    for (int i = threadIdx.x; i <= p.pos / 16; i += kT) s_bt[i] = p.block_table[i];
}
__device__ __forceinline__ uint32_t page_row(const DsParams& p, int l, int h, int t) {
    return ((uint32_t)s_bt[t >> 4] * (uint32_t)(p.L * p.Hkv) + (uint32_t)(l * p.Hkv + h)) * 16u +
           (uint32_t)(t & 15);
}
// Rows of the pools (a multiple of 16 per layer and kv head).
__device__ __forceinline__ uint32_t pool_rows(const DsParams& p) {
    return (uint32_t)((p.max_seq + 15) / 16) * (uint32_t)(p.L * p.Hkv) * 16u;
}

__device__ __forceinline__ void stage_layers(const DsParams& p) {
    static_assert(sizeof(DsLayer) % 4 == 0, "copied as words");
    const uint32_t* src = reinterpret_cast<const uint32_t*>(p.layers);
    uint32_t* dst = reinterpret_cast<uint32_t*>(s_layers);
    const int words = p.L * (int)(sizeof(DsLayer) / 4);
    for (int i = threadIdx.x; i < words; i += kT) dst[i] = src[i];
    for (int i = threadIdx.x; i < kRsqrtEstWords; i += kT) s_rsq[i] = kRsqrtEstTab[i];
    __syncthreads();
}

__host__ __device__ inline size_t w_am(int, int) { return (size_t)(kNC + 1) * 64; }
__host__ __device__ inline size_t w_head(int l, int h, int Hkv) {
    return (size_t)(kNC + 2 + l * Hkv + h) * 64;
}
// (inv_scale, code_sum) of the activation codes of GEMV stage `slot` of layer
// l, each on its own 128-byte line: written once per launch, read through L2
__host__ __device__ inline size_t w_rec(int l, int slot, int L, int Hkv) {
    return (size_t)(kNC + 2 + L * Hkv) * 64 + (size_t)(l * 4 + slot) * 32;
}

// paged_int8: counter of the chunks of kv head h of layer l that have
// published their softmax statistics (one line each, after the records)
__host__ __device__ inline size_t w_stat(int l, int h, int L, int Hkv) {
    return (size_t)(kNC + 2 + L * Hkv) * 64 + (size_t)L * 4 * 32 + (size_t)(l * Hkv + h) * 64;
}

// Accumulator region of one layer: q|k|v, o, gate|up, down (int32 each).
struct AccOff {
    int o, gu, down, stride;
};
__host__ __device__ inline AccOff acc_off(int H, int F, int Hq, int Hkv) {
    AccOff a;
    a.o = (Hq + 2 * Hkv) * kD;
    a.gu = a.o + H;
    a.down = a.gu + 2 * F;
    a.stride = a.down + H;
    return a;
}

constexpr int kChainLd = (kJ * 4 * kT / 8 + 27) / 32 * 32 + 4;  // chain_ld of the longest row

struct Shared {
    int8_t codes[8192] __attribute__((aligned(16)));
    float chain[8 * kChainLd] __attribute__((aligned(16)));  // the row being normalized
    int red_i[kW][64];
    float red_a[kW], red_b[kW];
    int red_c[kW];
    int red_s[kW];
    int flag;
};

constexpr int kTpad = kTmax + 64;  // weights past the chunk are zero up to here

struct AttnShared {
    float qs[8][kD];
    float sc[8][kTpad];                                   // scores, then weights
    int8_t vt[kTpad][kD] __attribute__((aligned(16)));    // the chunk's V codes
    float vsc[kTmax];                                     // their fp16 scales
    float ow[kT * 4];                                     // cross-wave partial sums
    float mstat[8], lstat[8];
    int8_t newk[kD] __attribute__((aligned(16)));
    int8_t newv[kD] __attribute__((aligned(16)));
    float news[2];
    int last;
    // ternary modes: the new token's rotated k and its v, the query codes and
    // the appended rows (tern_kv.h)
    float xn[2][kD];
    uint32_t qw[8][32];
    int qsum[8];
    float qeff[8];
    uint32_t nrow[2][kTernRowW];
    float nsc[2];
};

union SharedAll {
    Shared s;
    AttnShared a;
};

// -------------------------------------------------------------- schedule --

// Every stage function is inlined into the kernel: a real call would pass the
// (uniform) pointers in vector registers, and each buffer load through them
// would become a loop over lanes.

// Rows of the GEMV of stage slot 0..3 (QKV, O, GU, DOWN) and its K.
__host__ __device__ inline int gemv_rows(int slot, int H, int F, int Hq, int Hkv) {
    return slot == 0 ? (Hq + 2 * Hkv) * kD : slot == 2 ? 2 * F : H;
}
__host__ __device__ inline int gemv_k(int slot, int H, int F) { return slot == 3 ? F : H; }

__device__ __forceinline__ int ntasks(const DsParams& p, int kind) {
    if (kind == S_ATT) return p.Hkv * p.C;
    if (kind == S_HEAD) return p.with_head ? (p.V + 63) / 64 : p.H / 64;
    const int slot = kind == S_QKV ? 0 : kind - 1;
    return gemv_rows(slot, p.H, p.F, p.Hq, p.Hkv) / 64 * p.split[slot];
}

// t / d and t % d for a task index t < 2^16, with m = ds_div_mul(d).
__device__ __forceinline__ int div_m(int t, unsigned m) {
    return (int)__umulhi((unsigned)t << 1, m);
}
__device__ __forceinline__ int mod_m(int t, int d, unsigned m) { return t - div_m(t, m) * d; }
// (x + nwg) % nwg for -nwg < x < nwg
__device__ __forceinline__ int wrap_wg(int x, int nwg) { return x < 0 ? x + nwg : x; }

// Stage index s = 5*layer + kind for the layers, 5*L for the head.
__device__ __forceinline__ int kind_of(const DsParams& p, int s) {
    return s >= 5 * p.L ? S_HEAD : s % 5;
}

// ------------------------------------------------------------- barrier ----

// A wait that gave up: the error word makes every workgroup abort at its next
// poll, and io[3] (not cleared with the sync area before each launch) tells
// the host, for any step of a chained decode.
__device__ __forceinline__ unsigned* err_word(const DsParams& p) { return p.bar + kNC * 64; }
__device__ __forceinline__ void raise_abort(const DsParams& p) {
    stcu(err_word(p), 1u);
    __hip_atomic_store(p.io + 3, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The kNC barrier counters (256 bytes apart) and the error word after them,
// read with scalar loads that bypass the scalar cache (glc). The region is
// uncached memory, so the reads miss in L2 as well and see every
// workgroup's arrival. Scalar loads do not queue behind the CU's vector
// loads, so a workgroup can have the next stage's weight tile in flight
// while it polls.
__device__ __forceinline__ void poll_bar(const unsigned* base, unsigned& lo, unsigned& err) {
    static_assert(kNC == 16, "16 counters polled");
    unsigned c[16];
    asm volatile(
        "s_load_dword %0, %17, 0x0 glc\n"
        "s_load_dword %1, %17, 0x100 glc\n"
        "s_load_dword %2, %17, 0x200 glc\n"
        "s_load_dword %3, %17, 0x300 glc\n"
        "s_load_dword %4, %17, 0x400 glc\n"
        "s_load_dword %5, %17, 0x500 glc\n"
        "s_load_dword %6, %17, 0x600 glc\n"
        "s_load_dword %7, %17, 0x700 glc\n"
        "s_load_dword %8, %17, 0x800 glc\n"
        "s_load_dword %9, %17, 0x900 glc\n"
        "s_load_dword %10, %17, 0xa00 glc\n"
        "s_load_dword %11, %17, 0xb00 glc\n"
        "s_load_dword %12, %17, 0xc00 glc\n"
        "s_load_dword %13, %17, 0xd00 glc\n"
        "s_load_dword %14, %17, 0xe00 glc\n"
        "s_load_dword %15, %17, 0xf00 glc\n"
        "s_load_dword %16, %17, 0x1000 glc\n"
        "s_waitcnt lgkmcnt(0)\n"
        : "=&s"(c[0]), "=&s"(c[1]), "=&s"(c[2]), "=&s"(c[3]), "=&s"(c[4]), "=&s"(c[5]),
          "=&s"(c[6]), "=&s"(c[7]), "=&s"(c[8]), "=&s"(c[9]), "=&s"(c[10]), "=&s"(c[11]),
          "=&s"(c[12]), "=&s"(c[13]), "=&s"(c[14]), "=&s"(c[15]), "=&s"(err)
        : "s"(base)
        : "memory");
    lo = c[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) lo = c[i] < lo ? c[i] : lo;
}

// Grid barrier, in two halves. bar_arrive: every wave waits for its stores'
// acknowledgements, thread 0 adds the workgroup's arrival to counter wg % kNC
// (the counters carry on across launches: generation bar_base + gen is complete
// when each holds (bar_base + gen) * nwg / kNC) and stamps the trace. bar_wait:
// `issue` starts the next stage's loads that depend on nothing of this stage
// (its weight tile) and wave 0 polls the counters with scalar loads while those
// loads are in flight. The arrival goes out before any wave's prefetch (a block
// barrier between them), so it never waits behind them in the CU's memory
// pipeline. Every wait is bounded. A workgroup whose stage work produces
// nothing that the barrier must cover (a record writer without a task) arrives
// before that work and waits after it.
// `touched` is the result of touch_norm's load: taken as an operand where
// every load of the wave has completed, it keeps the load without computing
// anything from it.
__device__ __forceinline__ void bar_arrive(const DsParams& p, int s, int touched) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are acknowledged
    asm volatile("" ::"v"(touched));
    __syncthreads();
    if (threadIdx.x == 0) {
        if (p.trace) p.trace[((size_t)s * p.nwg + blockIdx.x) * 2] = wall_clock64();
        __hip_atomic_fetch_add(p.bar + (blockIdx.x % kNC) * 64, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_barrier();
}

template <class Issue>
__device__ __forceinline__ bool bar_wait(const DsParams& p, unsigned gen, int* s_abort,
                                         Issue&& issue) {
    issue();
    if (lwave() == 0) {
        const unsigned target = (p.bar_base + gen) * (unsigned)(p.nwg / kNC);
        const unsigned* base = uni_ptr(p.bar);
        unsigned spins = 0;
        int abort = 0;
        while (true) {
            unsigned lo, err;
            poll_bar(base, lo, err);
            if (err != 0) {
                abort = 1;
                break;
            }
            if (lo >= target) break;  // (the host keeps every target below 2^31)
            if (++spins > p.spin_limit) {
                if (threadIdx.x == 0) raise_abort(p);
                abort = 1;
                break;
            }
        }
        if (threadIdx.x == 0) *s_abort = abort;
    }
    __syncthreads();
    return *s_abort == 0;
}

// Float4 groups of a K-element vector a wave holds: thread t owns groups
// t + kT j, so wave w's lanes cover groups [kT j + 64 w, kT j + 64 w + 64);
// the j with a group below K/4 (wave-uniform). Loads past that count would
// only read zeros, so they are not issued at all.
//
// The count is made opaque at each call, so each loop compares it afresh
// (s_cmp + s_cbranch per group) instead of carrying the outcome of every
// j < J from an earlier loop as a lane mask rebuilt with vector instructions.
__device__ __forceinline__ int wave_groups(int K) {
    const int K4 = K >> 2, w0 = lwave() * 64;
    int J = __builtin_amdgcn_readfirstlane(K4 > w0 ? (K4 - w0 + kT - 1) / kT : 0);
    asm volatile("" : "+s"(J));
    return J;
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] in [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt has 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Cross-wave combinations of per-wave values in LDS (lane 0 of each wave
// wrote r[wave]); the orders are fixed, and only integer sums, maxima and the
// scale estimate use them.
__device__ __forceinline__ float red_max(const float* r) {
    float m = r[0];
#pragma unroll
    for (int w = 1; w < kW; ++w) m = fmaxf(m, r[w]);
    return m;
}
__device__ __forceinline__ float red_sum(const float* r) {
    float a = r[0];
#pragma unroll
    for (int w = 1; w < kW; ++w) a += r[w];
    return a;
}
__device__ __forceinline__ int red_sum(const int* r) {
    int a = r[0];
#pragma unroll
    for (int w = 1; w < kW; ++w) a += r[w];
    return a;
}
__device__ __forceinline__ int red_or(const int* r) {
    int a = r[0];
#pragma unroll
    for (int w = 1; w < kW; ++w) a |= r[w];
    return a;
}

// -------------------------------------------------------------- tiles ----

// Loads kPF chunks per lane of K slice [c0, c1) of TL1 row block rb (KS
// super-chunks of 64 columns per row block; wave w takes chunks c0+w, c0+w+4,
// ...). Chunks past c1 read zeros, and so does every chunk when !live (the
// loads are issued all the same, with nothing to read).
__device__ __forceinline__ void load_tl1_tile(uint4 (&pf)[kPF], const uint4* __restrict__ W,
                                              int rb, int KS, int c0, int c1, bool live = true) {
    const int lane = ltid() & 63, wave = lwave();
    const __amdgpu_buffer_rsrc_t r =
        rsrc(W + (size_t)rb * KS * 64, live ? (uint32_t)c1 * 64 * 16 : 0u);
#pragma unroll
    for (int i = 0; i < kPF; ++i)
        pf[i] = ld16nt(r, (uint32_t)((c0 + wave + kW * i) * 64 + lane) * 16);
}

// Attention tile: the first kAR rounds of kRT tokens; lane (wave, l) holds 16
// bytes of token r*kRT + wave*8 + l/8 at dims (l%8)*16 of K (pf[2r]) and V
// (pf[2r+1]) and its fp16 K and V scales (pfs[2r], pfs[2r+1]). Tokens past the chunk read
// zeros; the new token's slot is read but not used. Later rounds are read in
// the loops that use them.
template <bool PAGED>
__device__ __forceinline__ void load_att_tile(uint4 (&pf)[kPF], uint32_t (&pfs)[2 * kAR],
                                              const DsParams& p, int l, int h, int c) {
    const int lane = ltid() & 63, wave = lwave();
    const int t0 = c * p.T;
    const int nt = min(p.T, p.pos + 1 - t0);
    const int d0 = (lane & 7) * 16;
    if (PAGED) {
        // each lane's token through the block table (tokens past the chunk read
        // the context's last token: finite values nothing uses)
        const uint32_t rows = pool_rows(p);
        const __amdgpu_buffer_rsrc_t rk = rsrc(p.kc, rows * kD);
        const __amdgpu_buffer_rsrc_t rv = rsrc(p.vc, rows * kD);
        const __amdgpu_buffer_rsrc_t rks = rsrc(p.pks, rows * 4);
        const __amdgpu_buffer_rsrc_t rvs = rsrc(p.pvs, rows * 4);
#pragma unroll
        for (int r = 0; r < kAR; ++r) {
            const int tl = r * kRT + wave * 8 + (lane >> 3);
            const uint32_t row = page_row(p, l, h, min(t0 + tl, p.pos));
            pf[2 * r] = ld16nt(rk, row * kD + d0);
            pfs[2 * r] = (uint32_t)ld4int(rks, row * 4);
            pf[2 * r + 1] = ld16nt(rv, row * kD + d0);
            pfs[2 * r + 1] = (uint32_t)ld4int(rvs, row * 4);
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    const size_t tok0 = ((size_t)l * p.Hkv + h) * p.max_seq + t0;
    const __amdgpu_buffer_rsrc_t rk = rsrc(p.kc + tok0 * kD, (uint32_t)nt * kD);
    const __amdgpu_buffer_rsrc_t rv = rsrc(p.vc + tok0 * kD, (uint32_t)nt * kD);
    const __amdgpu_buffer_rsrc_t rks = rsrc(p.ks + tok0, (uint32_t)nt * 2);
    const __amdgpu_buffer_rsrc_t rvs = rsrc(p.vs + tok0, (uint32_t)nt * 2);
#pragma unroll
    for (int r = 0; r < kAR; ++r) {
        const int tl = r * kRT + wave * 8 + (lane >> 3);
        pf[2 * r] = ld16nt(rk, (uint32_t)(tl * kD + d0));
        pfs[2 * r] = ld2(rks, (uint32_t)tl * 2);
        pf[2 * r + 1] = ld16nt(rv, (uint32_t)(tl * kD + d0));
        pfs[2 * r + 1] = ld2(rvs, (uint32_t)tl * 2);
        // keep the rounds in issue order: round r then waits only for its own 4 loads
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The fp16 K / V scales of load_att_tile's tokens (INT8 cache; tokens past the
// chunk read zeros), for a chunk whose rows were prefetched.
__device__ __forceinline__ void load_att_scales(uint32_t (&pfs)[2 * kAR], const DsParams& p, int l,
                                                int h, int c) {
    const int lane = ltid() & 63, wave = lwave();
    const int t0 = c * p.T;
    const int nt = min(p.T, p.pos + 1 - t0);
    const size_t tok0 = ((size_t)l * p.Hkv + h) * p.max_seq + t0;
    const __amdgpu_buffer_rsrc_t rks = rsrc(p.ks + tok0, (uint32_t)nt * 2);
    const __amdgpu_buffer_rsrc_t rvs = rsrc(p.vs + tok0, (uint32_t)nt * 2);
#pragma unroll
    for (int r = 0; r < kAR; ++r) {
        const int tl = r * kRT + wave * 8 + (lane >> 3);
        pfs[2 * r] = ld2(rks, (uint32_t)tl * 2);
        pfs[2 * r + 1] = ld2(rvs, (uint32_t)tl * 2);
    }
}

// Norm weights (thread t: float4 groups t + kT j; zeros past K) into registers.
__device__ __forceinline__ void load_norm_w(float4 (&w)[kJ], const float* nw, int K) {
    const __amdgpu_buffer_rsrc_t r = rsrc(nw, nw ? (uint32_t)K * 4 : 0u);
    const int t = ltid();
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const f4v v = __builtin_bit_cast(
            f4v, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(t + kT * j) * 16, 0, 0));
        w[j] = make_float4(v.x, v.y, v.z, v.w);
    }
}

// ------------------------------------------------------------ prologue ----

__device__ __forceinline__ void read_rec(const DsParams& p, int l, int slot, float& inv,
                                         int& csum) {
    const __amdgpu_buffer_rsrc_t r = rsrc(p.sync + w_rec(l, slot, p.L, p.Hkv), 8);
    inv = __int_as_float(ld4i(r, 0));
    csum = ld4i(r, 4);
}

// The inv_scale half of the code record (l, slot) when its writer may publish
// it after the grid barrier (the down stage's writer arrives before its work,
// bar_arrive): the bits the stage input brought (inv_bits) when already
// nonzero (records are zeroed before each launch and inv_scale >= 1e-6 / 31),
// else polled with device-coherent loads. Bounded: on a timeout the error word
// is raised and the bits returned are 0 (the step is abandoned at the next
// barrier).
__device__ __forceinline__ int wait_rec_inv(const DsParams& p, int l, int slot, int inv_bits) {
    inv_bits = __builtin_amdgcn_readfirstlane(inv_bits);
    if (inv_bits != 0) return inv_bits;
    const unsigned* r = p.sync + w_rec(l, slot, p.L, p.Hkv);
    unsigned spins = 0;
    while ((inv_bits = (int)__builtin_amdgcn_readfirstlane(ldcu(r))) == 0) {
        if (++spins > p.spin_limit) {
            raise_abort(p);
            break;
        }
        if ((spins & 63) == 0 && ldcu(err_word(p)) != 0) break;
    }
    return inv_bits;
}

// Element of a GEMV output from its accumulator (TenzoEngine.cpp:1554,
// :118-126): float(acc - code_sum) * (inv_scale * w_scale).
__device__ __forceinline__ float gemv_y(int a, int csum, float invsc) {
    return (float)(a - csum) * invsc;
}

// A stage input is read in two steps. The issue_* functions start the loads
// of all kJ float4 groups of the thread into an InRaw (groups past K read
// zeros through the resource bounds; none of these loads sits in a branch: a
// load under a condition joins a phi whose register copy waits for every
// outstanding load, the weight tile's included); the caller then issues the
// stage's weight tile and waits until only the tile is in flight (vector
// memory operations complete in issue order), and the finish_* functions
// build the input vector v (zeros past K). The issue and finish steps sit in
// separate kind branches with the tile loads between them in common code, so
// the tile's loads are pending on every path alike and waiting for the input
// never waits for the tile.
struct InRaw {
    i4v x[kJ], y[kJ];  // raw 32-bit lanes of up to two K-vectors
    int inv, csum;     // code record of the GEMV the input comes from
};

__device__ __forceinline__ void issue_rec(InRaw& in, const DsParams& p, int l, int slot) {
    const __amdgpu_buffer_rsrc_t r = rsrc(p.sync + w_rec(l, slot, p.L, p.Hkv), 8);
    in.inv = ld4i(r, 0);
    in.csum = ld4i(r, 4);
}

// Where a GEMV stage's input comes from: x = a float vector (or the gate
// half of the gate|up accumulators, or for layer 0 the token's row of the
// packed int8 embedding, 16 bytes every 1 KiB), y = the int32 accumulators
// added to it (or the up half), rec = the code record of the GEMV they come
// from. Absent parts (null) read zeros.
struct InSrc {
    const void* x;
    uint32_t xbytes;
    bool emb;
    const void* y;
    uint32_t ybytes;
    const unsigned* rec;
};

__device__ __forceinline__ void issue_in(InRaw& in, const InSrc& src) {
    const int t = ltid();
    const __amdgpu_buffer_rsrc_t rx = rsrc(src.x, src.xbytes);
    const __amdgpu_buffer_rsrc_t ry = rsrc(src.y, src.y ? src.ybytes : 0u);
    const __amdgpu_buffer_rsrc_t rr = rsrc(src.rec, src.rec ? 8u : 0u);
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const uint32_t q = (uint32_t)(t + kT * j);
        in.x[j] = ld16i(rx, src.emb ? (q >> 2) * 1024u : q * 16u);
        in.y[j] = ld16i(ry, q * 16u);
    }
    in.inv = ld4i(rr, 0);
    in.csum = ld4i(rr, 4);
}

// x = a float vector, y = int32 accumulators (each K elements; y optional)
__device__ __forceinline__ void issue_vec2(InRaw& in, const void* xs, const void* ys, int K) {
    const int t = ltid();
    const __amdgpu_buffer_rsrc_t rx = rsrc(xs, (uint32_t)K * 4);
    const __amdgpu_buffer_rsrc_t ry = rsrc(ys, ys ? (uint32_t)K * 4 : 0u);
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        in.x[j] = ld16i(rx, (uint32_t)(t + kT * j) * 16);
        in.y[j] = ld16i(ry, (uint32_t)(t + kT * j) * 16);
    }
}

// v = base + GEMV output (the residual adds :1590, :1628): x = base, y = the
// accumulators; the record is that of the GEMV, w_scale its weight scale.
__device__ __forceinline__ void finish_resid(float4 (&v)[kJ], const InRaw& in, int K, float wsc) {
    const int t = ltid(), K4 = K >> 2, Jw = wave_groups(K);
    const float invsc = __int_as_float(in.inv) * wsc;
    const int cs = in.csum;
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (j < Jw) {
            const bool ok = t + kT * j < K4;
            v[j].x = ok ? __int_as_float(in.x[j].x) + gemv_y(in.y[j].x, cs, invsc) : 0.0f;
            v[j].y = ok ? __int_as_float(in.x[j].y) + gemv_y(in.y[j].y, cs, invsc) : 0.0f;
            v[j].z = ok ? __int_as_float(in.x[j].z) + gemv_y(in.y[j].z, cs, invsc) : 0.0f;
            v[j].w = ok ? __int_as_float(in.x[j].w) + gemv_y(in.y[j].w, cs, invsc) : 0.0f;
        } else {
            v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
}

__device__ __forceinline__ void finish_plain(float4 (&v)[kJ], const InRaw& in, int K) {
    const int Jw = wave_groups(K);
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        v[j] = j < Jw ? make_float4(__int_as_float(in.x[j].x), __int_as_float(in.x[j].y),
                                    __int_as_float(in.x[j].z), __int_as_float(in.x[j].w))
                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// embedding_lookup (:1294-1316) of token io[0] from the packed int8 LM head
// (lm_head.hip layout: [V/64][H/16][64 rows][16 bytes]); x[j].x = 4 codes.
__device__ __forceinline__ int embed_token(const DsParams& p) {
    return __builtin_amdgcn_readfirstlane(p.io[0]);  // uniform: scalar descriptors
}

// Row `tok` of the packed int8 LM head (lm_head.hip layout: [V/64][H/16][64
// rows][16 bytes]): 16 bytes every 1 KiB from here.
__device__ __forceinline__ const void* embed_row(const DsParams& p, int tok) {
    const uint8_t* hb = reinterpret_cast<const uint8_t*>(p.head);
    return hb + ((size_t)(tok >> 6) * (p.H / 16) * 64 + (tok & 63)) * 16;
}

__device__ __forceinline__ void finish_embed(float4 (&v)[kJ], const InRaw& in, const DsParams& p) {
    const int t = ltid(), K4 = p.H >> 2, Jw = wave_groups(p.H);
    const float es = p.head_scales[embed_token(p)];
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const bool ok = j < Jw && t + kT * j < K4;
        // the thread's 4 bytes are word t % 4 of the 16 read
        const i4v x = in.x[j];
        const uint32_t w = (uint32_t)((t & 2) ? ((t & 1) ? x.w : x.z) : ((t & 1) ? x.y : x.x));
        v[j].x = ok ? (float)(int8_t)(w & 0xff) * es : 0.0f;
        v[j].y = ok ? (float)(int8_t)((w >> 8) & 0xff) * es : 0.0f;
        v[j].z = ok ? (float)(int8_t)((w >> 16) & 0xff) * es : 0.0f;
        v[j].w = ok ? (float)(int8_t)(w >> 24) * es : 0.0f;
    }
}

// Stores the 64-element slices of v (K elements, float4 groups as owned
// above) whose index, counted from slice0, is f modulo m, into dst.
__device__ __forceinline__ void store_slices(float* dst, const float4 (&v)[kJ], int K, int slice0,
                                             int f, int m) {
    const int t = ltid(), K4 = K >> 2;
    const __amdgpu_buffer_rsrc_t r = rsrc(dst, (uint32_t)K * 4);
    if (slice0 + K / 64 <= m) {  // every slice has a workgroup of its own: slice j is f's
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const int q = t + kT * j;
            if (q < K4 && slice0 + (q >> 4) == f) stc16(r, (uint32_t)q * 16, v[j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const int q = t + kT * j;
            if (q < K4 && (slice0 + (q >> 4)) % m == f) stc16(r, (uint32_t)q * 16, v[j]);
        }
    }
}

// relu(gate)^2 * up (:1616-1620) from the gate|up accumulators (x = gate,
// y = up, record of the GU stage); the last layer's gate and up values are
// also stored as floats (slices as in store_slices).
__device__ __forceinline__ void finish_act(float4 (&v)[kJ], const InRaw& in, const DsParams& p,
                                           int l, float wg, float wu, int f, int m) {
    const bool last = l == p.L - 1;  // only the last layer's gate|up is stored
    const int t = ltid(), F = p.F, K4 = F >> 2, Jw = wave_groups(F);
    const bool own_one = 2 * F / 64 <= m;  // every slice has a workgroup of its own
    const __amdgpu_buffer_rsrc_t rg = rsrc(p.gu, (uint32_t)F * 8);
    const float inv = __int_as_float(in.inv);
    const int csum = in.csum;
    const float sg = inv * wg, su = inv * wu;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        if (j >= Jw) {
            v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            continue;
        }
        const int q = t + kT * j;
        const bool ok = q < K4;
        const i4v g = in.x[j], u = in.y[j];
        const float4 gv = make_float4(gemv_y(g.x, csum, sg), gemv_y(g.y, csum, sg),
                                      gemv_y(g.z, csum, sg), gemv_y(g.w, csum, sg));
        const float4 uv = make_float4(gemv_y(u.x, csum, su), gemv_y(u.y, csum, su),
                                      gemv_y(u.z, csum, su), gemv_y(u.w, csum, su));
        if (last) {
            const int sg_ = q >> 4, su_ = F / 64 + (q >> 4);
            if (ok && (own_one ? sg_ == f : sg_ % m == f)) stc16(rg, (uint32_t)q * 16, gv);
            if (ok && (own_one ? su_ == f : su_ % m == f))
                stc16(rg, (uint32_t)q * 16 + (uint32_t)F * 4, uv);
        }
        float r;
        r = fmaxf(0.0f, gv.x);
        v[j].x = ok ? (r * r) * uv.x : 0.0f;
        r = fmaxf(0.0f, gv.y);
        v[j].y = ok ? (r * r) * uv.y : 0.0f;
        r = fmaxf(0.0f, gv.z);
        v[j].z = ok ? (r * r) * uv.z : 0.0f;
        r = fmaxf(0.0f, gv.w);
        v[j].w = ok ? (r * r) * uv.w : 0.0f;
    }
}

// roundf(y * scale) (half away from zero), clamped to [-128, 127] for QMAX
// 127. For |x| < 2^23, roundf(x) is the truncation of x + copysign(h, x) with
// h = 0.5 - 2^-25 (the float just below 0.5): with n = floor(|x|), a fraction
// below 0.5 leaves the sum below the float just under n + 1, and a fraction
// of at least 0.5 brings it to n + 1 or above (n + 1 - 2^-25 rounds up, to
// even, when n = 0). The conversion truncates, so a code costs a multiply, a
// sign copy, an add and a convert.
template <int QMAX>
__device__ __forceinline__ int act_code(float y, float scale) {
    const float x = y * scale;
    int r = (int)(x + __builtin_copysignf(0.49999997f, x));
    if (QMAX == 127) r = min(max(r, -128), 127);
    return r;
}

// Four codes (low bytes of c0..c3) packed into a word, c0 in the low byte.
__device__ __forceinline__ uint32_t pack4(int c0, int c1, int c2, int c3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)c1, (uint32_t)c0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)c3, (uint32_t)c2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Codes of the weighted products p (K elements, zeros past K) for the RMS
// scale inv_rms into s.codes: amax = max(floor, pmax * inv_rms), code =
// round(p * inv_rms * (QMAX / amax)) (QMAX 31: build_lut :28-42; QMAX 127:
// compute_logits :1666-1678); returns this thread's code sum.
template <int QMAX>
__device__ __forceinline__ int quant_codes(Shared& s, const float4 (&p)[kJ], int K, float inv_rms,
                                           float amax, int q_lo = 0, int q_hi = 1 << 30) {
    const int t = ltid();
    int J = wave_groups(K);
    const float scale = (float)QMAX / amax;
    int csum = 0;
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (j < J && t + kT * j >= q_lo && t + kT * j < q_hi) {
            const float4 y = make_float4(__fmul_rn(p[j].x, inv_rms), __fmul_rn(p[j].y, inv_rms),
                                         __fmul_rn(p[j].z, inv_rms), __fmul_rn(p[j].w, inv_rms));
            const int c0 = act_code<QMAX>(y.x, scale), c1 = act_code<QMAX>(y.y, scale);
            const int c2 = act_code<QMAX>(y.z, scale), c3 = act_code<QMAX>(y.w, scale);
            *reinterpret_cast<uint32_t*>(s.codes + 4 * (t + kT * j)) = pack4(c0, c1, c2, c3);
            csum += (c0 + c1) + (c2 + c3);
        }
    return csum;
}

// The products p = x * w (w only when has_w; p = x otherwise) and the
// largest |p| of this thread.
__device__ __forceinline__ float weigh(float4 (&p)[kJ], const float4 (&v)[kJ], const float4 (&w)[kJ],
                                      bool has_w, int K) {
    int J = wave_groups(K);
    float pmax = 0.0f;
    if (has_w) {  // (one branch for the stage, not one per group)
#pragma unroll
        for (int j = 0; j < kJ; ++j)
            if (j < J)
                p[j] = make_float4(__fmul_rn(v[j].x, w[j].x), __fmul_rn(v[j].y, w[j].y),
                                   __fmul_rn(v[j].z, w[j].z), __fmul_rn(v[j].w, w[j].w));
    } else {
#pragma unroll
        for (int j = 0; j < kJ; ++j)
            if (j < J) p[j] = v[j];
    }
    asm volatile("" : "+s"(J));
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (j < J)
            pmax = fmaxf(pmax, fmaxf(fmaxf(fabsf(p[j].x), fabsf(p[j].y)),
                                     fmaxf(fabsf(p[j].z), fabsf(p[j].w))));
    return pmax;
}

// The exact RMS scale of x (rms_norm_raw :148-166 in the reference build's
// arithmetic, common.h): the row goes to LDS in chain layout and wave 0 sums
// its squares in the reference build's order. Ends with the result in every
// thread (two block barriers).
__device__ __forceinline__ float exact_inv_rms(Shared& s, const float4 (&v)[kJ], int K, float eps) {
    const int t = ltid(), wave = lwave();
    int J = wave_groups(K);
    const int ld = chain_ld(K);
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (j < J) {
            const int i = 4 * (t + kT * j);
            s.chain[chain_pos(i, ld)] = v[j].x;
            s.chain[chain_pos(i + 1, ld)] = v[j].y;
            s.chain[chain_pos(i + 2, ld)] = v[j].z;
            s.chain[chain_pos(i + 3, ld)] = v[j].w;
        }
    __syncthreads();
    if (wave == 0) {
        const float inv = inv_rms_ref(chain_sumsq_wave(s.chain, ld, K), K, eps, s_rsq);
        if ((t & 63) == 0) s.red_a[0] = inv;
    }
    __syncthreads();
    return s.red_a[0];
}

// Normalizes v (K elements, zeros past K; rms_norm_raw :148-166 with weight w
// when has_w) and quantizes it into s.codes, returning the code record
// (inv_scale = amax / QMAX and the code sum). Rounding is monotonic and
// inv_rms > 0, so the absmax of the normalized row, max |p * inv_rms|, is
// max |p| * inv_rms rounded once.
template <int QMAX>
__device__ __forceinline__ void norm_quant(Shared& s, float4 (&v)[kJ], const float4 (&w)[kJ],
                                           bool has_w, int K, float eps, float& inv_out,
                                           int& csum_out) {
    const int lane = ltid() & 63, wave = lwave();
    float4 p[kJ];
    float pmax = wave_max(weigh(p, v, w, has_w, K));
    if (lane == 0) s.red_b[wave] = pmax;
    const float inv_rms = exact_inv_rms(s, v, K, eps);  // (its barriers publish red_b)
    pmax = red_max(s.red_b);
    const float amax = fmaxf(QMAX == 31 ? 1e-6f : 1e-8f, __fmul_rn(pmax, inv_rms));
    int csum = wave_sum_i32(quant_codes<QMAX>(s, p, K, inv_rms, amax));
    if (lane == 0) s.red_c[wave] = csum;
    __syncthreads();
    csum_out = red_sum(s.red_c);
    inv_out = amax * (1.0f / (float)QMAX);
}

// The inv_scale half of norm_quant<31>'s record alone (the code sum is added
// up by the workgroups that compute the codes): the exact RMS scale and the
// absmax, no codes.
__device__ __forceinline__ float norm_record_inv31(Shared& s, float4 (&v)[kJ],
                                                  const float4 (&w)[kJ], bool has_w, int K,
                                                  float eps) {
    const int lane = ltid() & 63, wave = lwave();
    float4 p[kJ];
    float pmax = wave_max(weigh(p, v, w, has_w, K));
    if (lane == 0) s.red_b[wave] = pmax;
    const float inv_rms = exact_inv_rms(s, v, K, eps);  // (its barriers publish red_b)
    pmax = red_max(s.red_b);
    return fmaxf(1e-6f, __fmul_rn(pmax, inv_rms)) * (1.0f / 31.0f);
}

// The ±31 codes of norm_quant<31> for a workgroup that needs only the codes
// (the record comes from another workgroup), without waiting for the
// sequential sum of squares in the common case. Only the float4 groups
// [q_lo, q_hi) get codes (the columns the workgroup's tasks read); the
// absmax and the estimate still cover the whole row. Returns the sum of the
// codes written (in every thread).
//
// With any positive scale r in place of inv_rms, act_code's product is
// z_i = fl(p_i r) * fl(31 / fl(pmax r)) = t_i (1 + e), t_i = 31 p_i / pmax,
// |e| <= 3.01u (u = 2^-24; three roundings, the division correctly rounded),
// as long as nothing over- or underflows and pmax r stays above the floor
// 1e-6. The code is a nondecreasing function of z_i (for a given sign) that
// steps within 2u |z| + 1.5u of each half-integer (the roundings of z and of
// z + 0.49999997, each within half an ulp). So the codes for r = an estimate
// of inv_rms (from a sum of squares in any order) and for r = inv_rms itself
// can differ only where the computed fl(z_i) lies within 9.1u |z_i| + 1.5u
// of a half-integer; the test below uses 10u |z_i| + 4u (a wider window is
// as exact and only sends more rows down the exact path). Elements that close
// are rare; if the row has one, or the estimate is not safely above the
// floor or not finite, the codes are recomputed with the exact inv_rms.
// Either way s.codes ends up holding exactly norm_quant<31>'s codes. (A
// subnormal p_i r gives |z_i| < 2^-100 for both scales: code 0 either way.)
__device__ __forceinline__ int norm_quant_codes31(Shared& s, float4 (&v)[kJ],
                                                  const float4 (&w)[kJ], bool has_w, int K,
                                                  float eps, int q_lo, int q_hi, bool need_csum) {
    const int t = ltid(), lane = t & 63, wave = lwave();
    float4 p[kJ];
    float pmax = wave_max(weigh(p, v, w, has_w, K));
    float ss = 0.0f;
    int J = wave_groups(K);
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (j < J) {
            ss = __builtin_fmaf(v[j].x, v[j].x, ss);
            ss = __builtin_fmaf(v[j].y, v[j].y, ss);
            ss = __builtin_fmaf(v[j].z, v[j].z, ss);
            ss = __builtin_fmaf(v[j].w, v[j].w, ss);
        }
    ss = wave_sum_tree(ss);
    if (lane == 0) {
        s.red_b[wave] = pmax;
        s.red_a[wave] = ss;
    }
    __syncthreads();
    pmax = red_max(s.red_b);
    ss = red_sum(s.red_a);
    // any positive scale gives the same codes up to the test below; the
    // hardware reciprocal square root is within a few ulp of 1/sqrt
    const float r = __builtin_amdgcn_rsqf(__builtin_fmaf(ss, 1.0f / (float)K, eps));
    const float amax = __fmul_rn(pmax, r);
    // estimate within 1e-3 of inv_rms (any summation order of K <= 16384
    // squares), so amax >= 2e-6 keeps the exact amax above the floor
    bool near = !(amax >= 2e-6f && amax <= 3.0e38f && ss <= 3.0e38f);
    const float scale = 31.0f / amax;
    asm volatile("" : "+s"(J));
    int csum = 0;
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (j < J && t + kT * j >= q_lo && t + kT * j < q_hi) {
            const float ys[4] = {__fmul_rn(p[j].x, r), __fmul_rn(p[j].y, r),
                                 __fmul_rn(p[j].z, r), __fmul_rn(p[j].w, r)};
            int c[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                c[e] = act_code<31>(ys[e], scale);
                const float a = fabsf(__fmul_rn(ys[e], scale));
                near |= fabsf((a - floorf(a)) - 0.5f) <= __builtin_fmaf(a, 0x1.4p-21f, 0x1p-22f);
            }
            *reinterpret_cast<uint32_t*>(s.codes + 4 * (t + kT * j)) = pack4(c[0], c[1], c[2], c[3]);
            csum += (c[0] + c[1]) + (c[2] + c[3]);
        }
    const bool wnear = __any(near);
    if (need_csum) csum = wave_sum_i32(csum);
    if (lane == 0) {
        s.red_c[wave] = wnear ? 1 : 0;
        if (need_csum) s.red_s[wave] = csum;
    }
    __syncthreads();
    if (red_or(s.red_c) != 0) {
        const float inv_rms = exact_inv_rms(s, v, K, eps);
        csum = wave_sum_i32(quant_codes<31>(s, p, K, inv_rms,
                                            fmaxf(1e-6f, __fmul_rn(pmax, inv_rms)), q_lo, q_hi));
        if (lane == 0) s.red_s[wave] = csum;
        __syncthreads();
    }
    return need_csum ? red_sum(s.red_s) : 0;
}

// ---------------------------------------------------------------- GEMV ----

// 64 columns of 2-bit codes u = w + 1 (tl1.hip layout: bits 2k..2k+1 of each
// byte of word i hold the columns paired with activation word 4i + k) against
// 64 int8 codes. Field k goes to accumulator k, masked in place rather than
// shifted down, so acc[k] collects 4^k (k = 3: 32, from a one-bit shift)
// times its exact sum; tl1_acc_total divides the factors out exactly. The
// four independent chains keep v_dot4 from waiting on its own result.
__device__ __forceinline__ void dot64(const uint4 v, const int4* c4, int (&acc)[4]) {
    const uint32_t M0 = 0x03030303u, M1 = M0 << 2, M2 = M0 << 4, M3 = M0 << 5;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    // all 16 fields first (independent of each other), then the products
    uint32_t f[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i][0] = w[i] & M0;
        f[i][1] = w[i] & M1;
        f[i][2] = w[i] & M2;
        f[i][3] = (w[i] >> 1) & M3;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int4 a = c4[i];
        acc[0] = sdot4(f[i][0], a.x, acc[0]);
        acc[1] = sdot4(f[i][1], a.y, acc[1]);
        acc[2] = sdot4(f[i][2], a.z, acc[2]);
        acc[3] = sdot4(f[i][3], a.w, acc[3]);
    }
}

__device__ __forceinline__ int tl1_acc_total(const int (&acc)[4]) {
    return (acc[0] + (acc[1] >> 2)) + ((acc[2] >> 4) + (acc[3] >> 5));
}

// K slice [c0, c1) of one TL1 row block: returns the exact int32 sum
// sum_k u_k a_k (u = w+1) over the slice in wave 0, lane = row (other waves: 0).
__device__ __forceinline__ int tl1_rowblock(Shared& s, const uint4 (&cur)[kPF],
                                            const uint4* __restrict__ W, int rb, int KS, int c0,
                                            int c1, bool more) {
    const int lane = ltid() & 63, wave = lwave();
    const int4* c4 = reinterpret_cast<const int4*>(s.codes);
    int acc4[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < kPF; ++i) {
        const int c = c0 + wave + kW * i;
        if (c < c1) dot64(cur[i], c4 + c * 4, acc4);
    }
    // K beyond the preloaded window: 8 loads in flight (past c1: zeros)
    const __amdgpu_buffer_rsrc_t r = rsrc(W + (size_t)rb * KS * 64, (uint32_t)c1 * 64 * 16);
    for (int cc = c0 + wave + kW * kPF; cc < c1; cc += 8 * kW) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ld16nt(r, (uint32_t)((cc + u * kW) * 64 + lane) * 16);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = cc + u * kW;
            if (c < c1) dot64(v[u], c4 + c * 4, acc4);
        }
    }
    const int acc = tl1_acc_total(acc4);
    s.red_i[wave][lane] = acc;
    __syncthreads();
    int tot = 0;
    if (wave == 0) {
#pragma unroll
        for (int w = 0; w < kW; ++w) tot += s.red_i[w][lane];
    }
    // before red_i is written again (a next task; without one, the block
    // barrier of the grid barrier's arrival orders it before the next stage)
    if (more) __syncthreads();
    return tot;
}

// Whether the workgroup whose first task is `first` publishes the code record
// of a GEMV stage of n tasks: the first workgroup without a task when there is
// one (it computes nothing else, so the exact sum of squares, the one
// sequential step of the stage, runs beside the other workgroups' dot
// products), else the workgroup of task 0.
__device__ __forceinline__ bool rec_writer(const DsParams& p, int first, int n) {
    return n < p.nwg ? first == n : first == 0;
}

// Whether the record writer of GEMV stage `kind` of layer l arrives at the
// grid barrier before its work (its sequential sum of squares, 864 dependent
// steps at hidden 2560 / FFN 6912, would otherwise decide when the barrier
// completes): the down stage's writer when it has no task and the next layer's
// Q|K|V stage leaves a workgroup without a task (the stage after the down
// stage is offset by one more, so that this writer is the last workgroup of
// Q|K|V and idle there while it finishes). The Q|K|V stage polls the record.
__device__ __forceinline__ bool early_writer(const DsParams& p, int kind, int l) {
    return kind == S_DOWN && l < p.L - 1 && ntasks(p, S_DOWN) < p.nwg &&
           ntasks(p, S_QKV) < p.nwg - 1;
}

// One GEMV stage (QKV, O, GU or DOWN) of layer l for a workgroup whose first
// task is `first` (< n, or the record writer): builds the stage input, stores
// the slices of it later stages read, quantizes its normalization (exactly,
// with the record, in the record writer; the codes alone elsewhere) and adds
// its tasks' K-slice sums into the accumulators.
// Returns true when the workgroup has already arrived at the grid barrier that
// follows the stage (through arrive(), early_writer).
template <class Arrive>
__device__ __forceinline__ bool tl1_stage(SharedAll& sh, const DsParams& p, int kind, int l,
                                          int first, int n, uint4 (&tile)[kPF],
                                          Arrive&& arrive) {
    Shared& s = sh.s;
    const int tid = ltid(), lane = tid & 63, wave = lwave();
    const LayerRef Lw = layer(p, l);
    const int slot = kind == S_QKV ? 0 : kind - 1;
    const int K = gemv_k(slot, p.H, p.F);
    const int m = min(n, p.nwg);
    const AccOff ao = acc_off(p.H, p.F, p.Hq, p.Hkv);
    int* accl = p.acc + (size_t)l * ao.stride;
    const int S = p.split[slot];
    const unsigned Sm = p.split_mul[slot];
    const int KS = K / 64, KSs = p.split_chunks[slot];
    const uint4* W = Lw.mat(slot);
    // The first task's weight tile is in flight already (issued during the
    // grid barrier before this stage, prefetch_tile); the stage input and the
    // norm weights go out now (the sources are chosen per kind; the loads
    // themselves are one straight sequence, none under a condition: see InRaw)
    InSrc src{nullptr, (uint32_t)K * 4, false, nullptr, (uint32_t)K * 4, nullptr};
    if (kind == S_QKV) {
        if (l == 0) {
            src.x = embed_row(p, embed_token(p));
            src.xbytes = (uint32_t)(p.H / 16) * 1024;
            src.emb = true;
        } else {
            src.x = p.h1s + (size_t)(l - 1) * p.H;
            src.y = accl - ao.stride + ao.down;
            src.rec = p.sync + w_rec(l - 1, 3, p.L, p.Hkv);
        }
    } else if (kind == S_O) {
        src.x = p.attns + (size_t)l * p.Hq * kD;
    } else if (kind == S_GU) {
        src.x = p.xs + (size_t)l * p.H;
        src.y = accl + ao.o;
        src.rec = p.sync + w_rec(l, 1, p.L, p.Hkv);
    } else {
        src.x = accl + ao.gu;
        src.y = accl + ao.gu + p.F;
        src.rec = p.sync + w_rec(l, 2, p.L, p.Hkv);
    }
    InRaw in;
    issue_in(in, src);
    float4 nwr[kJ];
    load_norm_w(nwr, Lw.norm(slot), K);
    const bool rec = rec_writer(p, first, n);
    float4 xv[kJ];
    if (kind == S_QKV) {
        if (l == 0) {
            finish_embed(xv, in, p);
        } else {
            in.inv = wait_rec_inv(p, l - 1, 3, in.inv);
            finish_resid(xv, in, K, layer(p, l - 1).sc(6));
        }
        store_slices(p.xs + (size_t)l * p.H, xv, K, 0, first, m);
    } else if (kind == S_O) {
        finish_plain(xv, in, K);
    } else if (kind == S_GU) {
        finish_resid(xv, in, K, Lw.sc(3));
        store_slices(p.h1s + (size_t)l * p.H, xv, K, 0, first, m);
        if (l == p.L - 1) store_slices(p.h1, xv, K, 0, first, m);
    } else {
        finish_act(xv, in, p, l, Lw.sc(4), Lw.sc(5), first, m);
    }
    // With fewer tasks than workgroups, every workgroup has at most one task
    // and the record writer none: the writer publishes inv_scale alone, each
    // task quantizes only the K slice it reads, and the tasks of row block 0
    // (one per slice) add their slices' code sums into the record.
    const bool single = n < p.nwg;
    unsigned* recw = p.sync + w_rec(l, slot, p.L, p.Hkv);
    if (rec && single) {
        // (the down stage's writer arrives first: its record is polled for)
        const bool early = early_writer(p, kind, l);
        if (early) arrive();
        const float inv = norm_record_inv31(s, xv, nwr, Lw.norm(slot) != nullptr, K, p.eps);
        if (tid == 0) stcu(recw, __float_as_uint(inv));
        return early;
    } else if (rec) {
        float inv;
        int csum;
        norm_quant<31>(s, xv, nwr, Lw.norm(slot) != nullptr, K, p.eps, inv, csum);
        if (tid == 0) {
            stcu(recw, __float_as_uint(inv));
            stcu(recw + 1, (unsigned)csum);
        }
    } else {
        const int c0 = mod_m(first, S, Sm) * KSs, c1 = min(KS, c0 + KSs);
        const bool contributes = single && first < S;  // adds its slice's code sum
        const int csum = norm_quant_codes31(s, xv, nwr, Lw.norm(slot) != nullptr, K, p.eps,
                                            single ? c0 * 16 : 0, single ? c1 * 16 : K / 4,
                                            contributes);
        if (contributes && tid == 0)
            __hip_atomic_fetch_add(reinterpret_cast<int*>(recw + 1), csum, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    int* out = accl + (slot == 0 ? 0 : slot == 1 ? ao.o : slot == 2 ? ao.gu : ao.down);
    for (int t = first; t < n; t += p.nwg) {
        const int rb = div_m(t, Sm), c0 = (t - rb * S) * KSs, c1 = min(KS, c0 + KSs);
        if (t != first) load_tl1_tile(tile, W, rb, KS, c0, c1);
        const int tot = tl1_rowblock(s, tile, W, rb, KS, c0, c1, t + p.nwg < n);
        if (wave == 0) {
            if (S == 1)  // the row block's only contribution
                __hip_atomic_store(out + rb * 64 + lane, tot, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            else
                __hip_atomic_fetch_add(out + rb * 64 + lane, tot, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    return false;
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

// Byte j of w as a signed integer, converted to float (one SDWA convert).
template <int J>
__device__ __forceinline__ float sbyte(uint32_t w) {
    return (float)(int8_t)(w >> (8 * J));
}

__device__ __forceinline__ void unpack16(const uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[4 * i] = sbyte<0>(w[i]);
        f[4 * i + 1] = sbyte<1>(w[i]);
        f[4 * i + 2] = sbyte<2>(w[i]);
        f[4 * i + 3] = sbyte<3>(w[i]);
    }
}

template <int G>
__device__ __forceinline__ void attn_merge(AttnShared& a, const DsParams& p, int l, int h, int g);
template <int G>
__device__ __forceinline__ void attn_merge_sum(AttnShared& a, const DsParams& p, int l, int h,
                                               int g);

// paged_int8 softmax (:395-405) for chunk c of kv head h, whose raw scores
// s_t are in a.sc: the chunk's (max m_c, sum l_c of e^{s_t - m_c}) per query
// head go into its partial records; once all C chunks of the head have
// published theirs (a counter per (layer, kv head), every chunk task of the
// stage being resident), every chunk forms M = max m_c and
// L = sum_c l_c e^{m_c - M} in the same order, and turns its scores into the
// value weights p_t s_v[t], p_t = e^{s_t - M} / (L + 1e-8), 0 where p_t < 1e-7
// (:412-414). L equals the reference's sum of e^{s_t - M} up to rounding.
// Returns false when a wait timed out (the error word is set).
template <int G>
__device__ __forceinline__ bool paged_weights(AttnShared& a, const DsParams& p, int l, int h,
                                              int c, int nt) {
    const int tid = ltid(), lane = tid & 63, wave = lwave();
    const int stride = kPS;
    for (int g = wave; g < G; g += kW) {
        float m = -1e30f;
        for (int i = lane; i < nt; i += 64) m = fmaxf(m, a.sc[g][i]);
        m = wave_max(m);
        float lsum = 0.0f;
        for (int i = lane; i < nt; i += 64) lsum += expf(a.sc[g][i] - m);
        lsum = wave_sum_tree(lsum);
        if (lane == 0) {
            a.mstat[g] = m;
            a.lstat[g] = lsum;
        }
    }
    __syncthreads();
    const float* rec = p.part + (size_t)h * p.C * G * stride;  // [C][G][stride]
    if (p.C > 1) {
        if (tid < G) {
            float* pp = p.part + (((size_t)h * p.C + c) * G + tid) * stride;
            stc(pp, a.mstat[tid]);
            stc(pp + 1, a.lstat[tid]);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            unsigned* ctr = p.sync + w_stat(l, h, p.L, p.Hkv);
            __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int ok = 1;
            unsigned spins = 0;
            while (ldcu(ctr) < (unsigned)p.C) {
                if (++spins > p.spin_limit ||
                    ((spins & 63) == 0 && ldcu(err_word(p)) != 0)) {
                    raise_abort(p);
                    ok = 0;
                    break;
                }
            }
            a.last = ok;
        }
        __syncthreads();
        if (a.last == 0) return false;
        for (int g = wave; g < G; g += kW) {
            float M = -1e30f;
            for (int q = lane; q < p.C; q += 64) M = fmaxf(M, ldc(rec + ((size_t)q * G + g) * stride));
            M = wave_max(M);
            float L = 0.0f;
            for (int q = lane; q < p.C; q += 64) {
                const float* pr = rec + ((size_t)q * G + g) * stride;
                L = __builtin_fmaf(ldc(pr + 1), expf(ldc(pr) - M), L);
            }
            L = wave_sum_tree(L);
            if (lane == 0) {
                a.mstat[g] = M;
                a.lstat[g] = __fdiv_rn(1.0f, L + 1e-8f);
            }
        }
    } else {
        if (tid < G) a.lstat[tid] = __fdiv_rn(1.0f, a.lstat[tid] + 1e-8f);
    }
    __syncthreads();
    for (int g = wave; g < G; g += kW) {
        const float M = a.mstat[g], inv = a.lstat[g];
        for (int i = lane; i < nt; i += 64) {
            const float pw = __fmul_rn(expf(a.sc[g][i] - M), inv);
            a.sc[g][i] = pw < 1e-7f ? 0.0f : __fmul_rn(pw, a.vsc[i]);
        }
        a.sc[g][nt + lane] = 0.0f;  // the value loop runs past nt by < 64
    }
    __syncthreads();
    return true;
}

// Attention of the G query heads of kv head h over context chunk c of layer
// l (attention_int8_fused, :434-864): q|k|v from the QKV accumulators, RoPE,
// the new token's K/V quantized and appended, chunk softmax and weighted
// values; with several chunks the last one to finish merges the partials.
// PAGED (paged_int8, PagedKVCache::forward_attention_raw :248-445): rows
// through the block table, fp32 scales, and the softmax normalized over the
// whole context before the values, so that weights below 1e-7 are skipped as
// the reference does: each chunk publishes its (max, sum of exponentials),
// waits until every chunk of its kv head has, and forms the normalized
// weights from the combined statistics; the partials are then plain sums.
template <int G, int KVM>
// cur: the chunk's K / V tile registers; with `pre` (INT8 cache only) they
// already hold the rows of this chunk, issued during the grid barrier before
// the stage (prefetch_next), and only their scales are loaded here.
__device__ __forceinline__ void attn_task(SharedAll& sh, const DsParams& p, int l, int h, int c,
                                          uint4 (&cur)[kPF], bool pre) {
    constexpr bool PAGED = KVM == 3, TERN = KVM == 1 || KVM == 2;
    AttnShared& a = sh.a;
    const int tid = ltid(), lane = tid & 63, wave = lwave();
    const int ctx = p.pos + 1;
    const int t0 = c * p.T;
    const int nt = min(p.T, ctx - t0);
    const int qd = p.Hq * kD, kvd = p.Hkv * kD;
    const float* rope = p.rope + (size_t)p.pos * kD;
    const size_t head = ((size_t)l * p.Hkv + h) * p.max_seq;
    const LayerRef Lw = layer(p, l);
    const __amdgpu_buffer_rsrc_t racc =
        rsrc(p.acc + (size_t)l * acc_off(p.H, p.F, p.Hq, p.Hkv).stride, (uint32_t)(qd + 2 * kvd) * 4);
    // loads first: the q (and new k / v) accumulators, the rope row, the
    // code record of the QKV stage
    constexpr int kQ = (G * 64 + kT - 1) / kT;  // query pairs per thread
    const __amdgpu_buffer_rsrc_t rr = rsrc(rope, kD * 4);
    int qa[kQ][2];
    float qc[kQ][2];
#pragma unroll
    for (int u = 0; u < kQ; ++u) {
        const int i = tid + u * kT, g = (i >> 6) % G, j = i & 63;
        const int row = (h * G + g) * kD;
        qa[u][0] = ld4i(racc, (uint32_t)(row + j) * 4);
        qa[u][1] = ld4i(racc, (uint32_t)(row + j + 64) * 4);
        qc[u][0] = __int_as_float(ldc4i(rr, (uint32_t)j * 4));
        qc[u][1] = __int_as_float(ldc4i(rr, (uint32_t)(j + 64) * 4));
    }
    const bool has_new = p.pos >= t0 && p.pos < t0 + nt;
    const int krow = qd + (wave == 0 ? 0 : kvd) + h * kD;
    const int ka0 = ld4i(racc, (uint32_t)(krow + lane) * 4);
    const int ka1 = ld4i(racc, (uint32_t)(krow + lane + 64) * 4);
    const float kc0 = __int_as_float(ldc4i(rr, (uint32_t)lane * 4));
    const float ks0 = __int_as_float(ldc4i(rr, (uint32_t)(lane + 64) * 4));
    float inv;
    int cs;
    read_rec(p, l, 0, inv, cs);
    // then, once every wave has issued those, the chunk's K / V tile (in
    // flight during the setup)
    __builtin_amdgcn_s_barrier();
    uint32_t curs[2 * kAR];
    static_assert(kPF >= 4 && 2 * kAR >= 2, "a ternary K|V row pair fits the tile registers");
    if constexpr (TERN) {
        // thread tid: the 32-byte K and V rows and fp32 scales of token t0 + tid
        // (past the head's rows: zeros)
        const __amdgpu_buffer_rsrc_t rk = rsrc(p.kc + head * 32, (uint32_t)p.max_seq * 32);
        const __amdgpu_buffer_rsrc_t rv = rsrc(p.vc + head * 32, (uint32_t)p.max_seq * 32);
        const __amdgpu_buffer_rsrc_t rks = rsrc(p.pks + head, (uint32_t)p.max_seq * 4);
        const __amdgpu_buffer_rsrc_t rvs = rsrc(p.pvs + head, (uint32_t)p.max_seq * 4);
        const uint32_t tt = (uint32_t)min(t0 + tid, p.max_seq);
        cur[0] = ld16nt(rk, tt * 32);
        cur[1] = ld16nt(rk, tt * 32 + 16);
        cur[2] = ld16nt(rv, tt * 32);
        cur[3] = ld16nt(rv, tt * 32 + 16);
        curs[0] = (uint32_t)ld4int(rks, tt * 4);
        curs[1] = (uint32_t)ld4int(rvs, tt * 4);
        wait_vm<6>();  // all but the rows
    } else {
        if (KVM == 0 && pre) {
            load_att_scales(curs, p, l, h, c);
        } else {
            load_att_tile<PAGED>(cur, curs, p, l, h, c);
            wait_vm<4 * kAR>();  // all but the tile
        }
    }
    // RoPE on the G query heads (:460-481); chunk 0 also stores q as floats
    {
        const float sq = inv * Lw.sc(0);
#pragma unroll
        for (int u = 0; u < kQ; ++u) {
            const int i = tid + u * kT;
            if (i < G * 64) {
                const int g = i >> 6, j = i & 63;
                const size_t row = (size_t)(h * G + g) * kD;
                const float x0 = gemv_y(qa[u][0], cs, sq);
                const float x1 = gemv_y(qa[u][1], cs, sq);
                if (c == 0 && l == p.L - 1) {
                    stc(p.qkv + row + j, x0);
                    stc(p.qkv + row + j + 64, x1);
                }
                const float cr = qc[u][0], sr = qc[u][1];
                a.qs[g][j] = __builtin_fmaf(x0, cr, -(x1 * sr));
                a.qs[g][j + 64] = __builtin_fmaf(x0, sr, x1 * cr);
            }
        }
    }
    // the new token: RoPE on k, quantize-append k and v (:482-533)
    if (TERN && has_new && wave < 2) {
        // ternary: rotated k and raw v to LDS; their rows are formed below
        const float sk = inv * Lw.sc(wave == 0 ? 1 : 2);
        float x0 = gemv_y(ka0, cs, sk);
        float x1 = gemv_y(ka1, cs, sk);
        if (l == p.L - 1) {
            stc(p.qkv + krow + lane, x0);
            stc(p.qkv + krow + lane + 64, x1);
        }
        if (wave == 0) {
            const float r0 = __builtin_fmaf(x0, kc0, -(x1 * ks0));
            const float r1 = __builtin_fmaf(x0, ks0, x1 * kc0);
            x0 = r0;
            x1 = r1;
        }
        a.xn[wave][lane] = x0;
        a.xn[wave][lane + 64] = x1;
    } else if (!TERN && has_new && wave < 2) {
        const float sk = inv * Lw.sc(wave == 0 ? 1 : 2);
        float x0 = gemv_y(ka0, cs, sk);
        float x1 = gemv_y(ka1, cs, sk);
        if (l == p.L - 1) {
            stc(p.qkv + krow + lane, x0);
            stc(p.qkv + krow + lane + 64, x1);
        }
        if (wave == 0) {
            const float r0 = __builtin_fmaf(x0, kc0, -(x1 * ks0));
            const float r1 = __builtin_fmaf(x0, ks0, x1 * kc0);
            x0 = r0;
            x1 = r1;
        }
        float s;
        int8_t* nb = wave == 0 ? a.newk : a.newv;
        quant_kv(x0, x1, nb, lane, &s);
        const size_t row = PAGED ? (size_t)page_row(p, l, h, p.pos) : head + p.pos;
        int8_t* dst = (wave == 0 ? p.kc : p.vc) + row * kD;
        dst[lane] = nb[lane];
        dst[lane + 64] = nb[lane + 64];
        if (lane == 0) {
            if (PAGED) {  // fp32 scales (:342-345)
                (wave == 0 ? p.pks : p.pvs)[row] = s;
                a.news[wave] = s;
            } else {
                const uint16_t sh16 = float_to_half_bits(s);
                (wave == 0 ? p.ks : p.vs)[row] = sh16;
                a.news[wave] = half_bits_to_float(sh16);
            }
        }
    }
    __syncthreads();

    if constexpr (TERN) {
        // query codes of the G heads and the new token's rows (:534-648,
        // :700-714, :766-791), one wave per job
        const int jobs = G + (has_new ? 2 : 0);
        for (int j = wave; j < jobs; j += kW) {
            if (j < G) {
                tern_query<KVM>(a.qs[j], lane, a.qw[j], &a.qsum[j], &a.qeff[j]);
            } else {
                const int kv = j - G;  // 0: k, 1: v
                float sr;
                const uint32_t w = tern_row<KVM>(a.xn[kv], kv, lane, &sr);
                if (lane < kTernRowW) {
                    a.nrow[kv][lane] = w;
                    reinterpret_cast<uint32_t*>((kv == 0 ? p.kc : p.vc) + (head + p.pos) * 32)[lane] = w;
                }
                if (lane == 0) {
                    (kv == 0 ? p.pks : p.pvs)[head + p.pos] = sr;
                    a.nsc[kv] = sr;
                }
            }
        }
        __syncthreads();
        // scores (:720-760 / :793-804): thread tid takes token t0 + tid and
        // stages its V row and scale in LDS
        if (tid < nt) {
            const int t = t0 + tid;
            uint32_t kr[kTernRowW];
            uint4 v0 = cur[2], v1 = cur[3];
            float skf = __uint_as_float(curs[0]), svf = __uint_as_float(curs[1]);
            if (t == p.pos) {
#pragma unroll
                for (int i = 0; i < kTernRowW; ++i) kr[i] = a.nrow[0][i];
                v0 = make_uint4(a.nrow[1][0], a.nrow[1][1], a.nrow[1][2], a.nrow[1][3]);
                v1 = make_uint4(a.nrow[1][4], a.nrow[1][5], a.nrow[1][6], a.nrow[1][7]);
                skf = a.nsc[0];
                svf = a.nsc[1];
            } else {
                kr[0] = cur[0].x; kr[1] = cur[0].y; kr[2] = cur[0].z; kr[3] = cur[0].w;
                kr[4] = cur[1].x; kr[5] = cur[1].y; kr[6] = cur[1].z; kr[7] = cur[1].w;
            }
            reinterpret_cast<uint4*>(&a.vt[tid][0])[0] = v0;
            reinterpret_cast<uint4*>(&a.vt[tid][0])[1] = v1;
            a.vsc[tid] = svf;
            float scv[G];
            tern_scores<G, KVM>(kr, a.qw, a.qsum, a.qeff, skf, scv);
#pragma unroll
            for (int g = 0; g < G; ++g) a.sc[g][tid] = scv[g];
        }
    } else {
    const int sub = lane >> 3, d0 = (lane & 7) * 16;
    // scores (:678-694); lane (wave, l) takes token r*kRT + wave*8 + l/8 and
    // dims (l%8)*16.. of it, and stages that token's V codes and scale in LDS
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
            uint4 kv, vv;
            float skf, svf;
            if (t == p.pos) {
                kv = *reinterpret_cast<const uint4*>(a.newk + d0);
                vv = *reinterpret_cast<const uint4*>(a.newv + d0);
                skf = a.news[0];
                svf = a.news[1];
            } else if (r < kAR) {
                kv = cur[2 * r];
                vv = cur[2 * r + 1];
                skf = PAGED ? __uint_as_float(curs[2 * r]) : half_bits_to_float((uint16_t)curs[2 * r]);
                svf = PAGED ? __uint_as_float(curs[2 * r + 1])
                            : half_bits_to_float((uint16_t)curs[2 * r + 1]);
            } else if (PAGED) {
                // past the preloaded rounds: rows through the block table
                // (tokens past the chunk read the context's last token)
                const uint32_t rows = pool_rows(p);
                const uint32_t row = page_row(p, l, h, min(t, p.pos));
                kv = ld16nt(rsrc(p.kc, rows * kD), row * kD + d0);
                vv = ld16nt(rsrc(p.vc, rows * kD), row * kD + d0);
                skf = __int_as_float(ld4int(rsrc(p.pks, rows * 4), row * 4));
                svf = __int_as_float(ld4int(rsrc(p.pvs, rows * 4), row * 4));
            } else {
                // past the preloaded rounds (long chunks): tokens past the
                // chunk read zeros through the resource bounds
                const size_t tok0 = head + t0;
                const __amdgpu_buffer_rsrc_t rk = rsrc(p.kc + tok0 * kD, (uint32_t)nt * kD);
                const __amdgpu_buffer_rsrc_t rv = rsrc(p.vc + tok0 * kD, (uint32_t)nt * kD);
                const __amdgpu_buffer_rsrc_t rks = rsrc(p.ks + tok0, (uint32_t)nt * 2);
                const __amdgpu_buffer_rsrc_t rvs = rsrc(p.vs + tok0, (uint32_t)nt * 2);
                kv = ld16nt(rk, (uint32_t)(tl * kD + d0));
                vv = ld16nt(rv, (uint32_t)(tl * kD + d0));
                skf = half_bits_to_float((uint16_t)ld2(rks, (uint32_t)tl * 2));
                svf = half_bits_to_float((uint16_t)ld2(rvs, (uint32_t)tl * 2));
            }
            float kf[16];
            unpack16(kv, kf);
            float pr[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) s = __builtin_fmaf(qr[g][j], kf[j], s);
                s += dpp_f<kDppXor1>(s);
                s += dpp_f<kDppXor2>(s);
                s += dpp_f<kDppHalfMirror>(s);
                pr[g] = s;
            }
            if (tl < nt) {
                *reinterpret_cast<uint4*>(&a.vt[tl][d0]) = vv;
                if ((lane & 7) == 0) a.vsc[tl] = svf;
                const float f = skf * kAttnScale;
#pragma unroll
                for (int g = 0; g < G; ++g)
                    if ((lane & 7) == (g & 7))  // paged: (dot * s_k) * qk_scale (:391)
                        a.sc[g][tl] = PAGED ? __fmul_rn(__fmul_rn(pr[g], skf), kAttnScale)
                                            : pr[g] * f;
            }
        }
    }
    }
    __syncthreads();
    if (PAGED) {
        if (!paged_weights<G>(a, p, l, h, c, nt)) return;
    } else {
    // chunk softmax statistics (:824-830); the weight kept for the values is
    // e^{s-m} times the token's V scale (the product the multi-kernel path
    // forms per token)
    for (int g = wave; g < G; g += kW) {
        float m = -1e30f;
        for (int i = lane; i < nt; i += 64) m = fmaxf(m, a.sc[g][i]);
        m = wave_max(m);
        float lsum = 0.0f;
        for (int i = lane; i < nt; i += 64) {
            const float e = expf(a.sc[g][i] - m);
            a.sc[g][i] = e * a.vsc[i];
            lsum += e;
        }
        a.sc[g][nt + lane] = 0.0f;  // the value loop runs past nt by < 64
        lsum = wave_sum_tree(lsum);
        if (lane == 0) {
            a.mstat[g] = m;
            a.lstat[g] = lsum;
        }
    }
    __syncthreads();
    }
    // weighted values (:842-851): lane l owns dims 4(l%32)..+3 of one head
    // (G >= 2: head 2*(wave % (G/2)) + l/32; G = 1: head 0); the kNS wave
    // (half-wave) sets that own the same outputs take every kNS-th token, and
    // their sums are added in LDS in set order
    // (ternary: thread (byte dq, head hd, token set part) of kT/32/G sets
    // decodes byte dq of each V row, dims 4 dq..4 dq+3, :852-885)
    constexpr int kWS = G >= 2 ? G / 2 : 1;          // waves per set of all heads
    constexpr int kNS = TERN ? kT / 32 / G : G >= 2 ? kW / kWS : 2 * kW;  // token sets
    static_assert(G <= 2 * kW, "at most 8 query heads per kv head");
    constexpr int kVU = 8 * kNS <= kTpad - kTmax ? 8 : (kTpad - kTmax) / kNS;  // tokens per step
    static_assert(kVU * kNS <= kTpad - kTmax, "the zero padding covers one step");
    const int dq = TERN ? tid & 31 : lane & 31, half = lane >> 5;
    const int hd = TERN ? (tid >> 5) % G : G >= 2 ? (wave % kWS) * 2 + half : 0;
    const int part = TERN ? (tid >> 5) / G : G >= 2 ? wave / kWS : wave * 2 + half;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (TERN) {
        const int word = dq >> 2, sh = 8 * (dq & 3);
        for (int t = part; t < nt; t += kNS) {
            const uint32_t* row = reinterpret_cast<const uint32_t*>(&a.vt[t][0]);
            float w[4];
            tern_value4(row[word] >> sh, w);
            const float wt = a.sc[hd][t];
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = __builtin_fmaf(w[k], wt, o[k]);
        }
    } else
    for (int tb = part; tb < nt; tb += kVU * kNS) {
        uint32_t vb[kVU];
        float wgt[kVU];
#pragma unroll
        for (int u = 0; u < kVU; ++u) {
            const int t = tb + u * kNS;  // past nt: weight 0, finite codes
            vb[u] = *reinterpret_cast<const uint32_t*>(&a.vt[t][4 * dq]);
            wgt[u] = a.sc[hd][t];
        }
#pragma unroll
        for (int u = 0; u < kVU; ++u) {
            o[0] = __builtin_fmaf(sbyte<0>(vb[u]), wgt[u], o[0]);
            o[1] = __builtin_fmaf(sbyte<1>(vb[u]), wgt[u], o[1]);
            o[2] = __builtin_fmaf(sbyte<2>(vb[u]), wgt[u], o[2]);
            o[3] = __builtin_fmaf(sbyte<3>(vb[u]), wgt[u], o[3]);
        }
    }
    if (kNS > 1) {
        float* ow = a.ow;  // [kNS][G][128]
#pragma unroll
        for (int k = 0; k < 4; ++k) ow[(part * G + hd) * kD + 4 * dq + k] = o[k];
        __syncthreads();
        if (part == 0) {
            for (int q = 1; q < kNS; ++q)
#pragma unroll
                for (int k = 0; k < 4; ++k) o[k] += ow[(q * G + hd) * kD + 4 * dq + k];
        }
    }
    const int stride = kPS;
    if (part == 0) {
        const int d = 4 * dq;
        if (p.C == 1) {
            const float L = a.lstat[hd];
            const size_t off = (size_t)(h * G + hd) * kD + d;
            const float4 r = PAGED ? make_float4(o[0], o[1], o[2], o[3])  // normalized weights
                                   : make_float4(o[0] / L, o[1] / L, o[2] / L, o[3] / L);
            stc16(rsrc(p.attns + (size_t)l * p.Hq * kD, (uint32_t)p.Hq * kD * 4),
                  (uint32_t)off * 4, r);
            if (l == p.L - 1) stc16(rsrc(p.attn, (uint32_t)p.Hq * kD * 4), (uint32_t)off * 4, r);
        } else {
            // the chunk's G records from a wave-uniform base (no per-lane descriptor)
            float* pc = p.part + ((size_t)h * p.C + c) * G * stride;
            float* pp = pc + hd * stride;
            stc16(rsrc(pc, G * stride * 4), (uint32_t)(hd * stride + 4 + d) * 4,
                  make_float4(o[0], o[1], o[2], o[3]));
            if (!PAGED && dq == 0) {  // (paged: the statistics are stored already)
                stc(pp, a.mstat[hd]);
                stc(pp + 1, a.lstat[hd]);
            }
        }
    }
    if (p.C == 1) return;
    // The last M = min(G, C) chunks of this kv head to finish merge the
    // partials, merger r taking query heads r, r+M, ...; each first waits
    // until every chunk of the head has stored its partial. When there are
    // more attention tasks than workgroups a workgroup runs several chunks in
    // turn and must not wait for one of its own later chunks: then only the
    // last chunk to finish merges (M = 1, nothing left to wait for).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int M = p.Hkv * p.C <= p.nwg ? min(G, p.C) : 1;
    unsigned* ctr = p.sync + w_head(l, h, p.Hkv);
    if (tid == 0) {
        const unsigned old =
            __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int r = (int)old - (p.C - M);
        if (r >= 0) {
            unsigned spins = 0;
            while (ldcu(ctr) < (unsigned)p.C) {
                if (++spins > p.spin_limit ||
                    ((spins & 63) == 0 && ldcu(err_word(p)) != 0)) {
                    raise_abort(p);
                    r = -1;
                    break;
                }
            }
        }
        a.last = r;
    }
    __syncthreads();
    const int r = a.last;
    for (int g = r; r >= 0 && g < G; g += M) {
        if (PAGED)
            attn_merge_sum<G>(a, p, l, h, g);
        else
            attn_merge<G>(a, p, l, h, g);
    }
}

// Merge of the C chunk partials of query head g of kv head h (same formula
// as attn_combine_kernel): out = sum_c e^{m_c-M} o_c / sum_c e^{m_c-M} l_c.
// Thread (cp, d4) = (tid / 32, tid % 32) sums dims 4 d4.. over the chunks
// c = cp, cp + kT/32, ... in order, and the kT/32 sums are added in cp order. The
// first kU chunks of each thread and every chunk statistic are loaded
// together.
template <int G>
__device__ __forceinline__ void attn_merge(AttnShared& a, const DsParams& p, int l, int h, int g) {
    const int tid = ltid(), lane = tid & 63, wave = lwave();
    const int stride = kPS;
    const float* base = p.part + (size_t)h * p.C * G * stride;
    const __amdgpu_buffer_rsrc_t r = rsrc(base, (uint32_t)(p.C * G * stride) * 4);
    float* wts = reinterpret_cast<float*>(&a.vt[0][0]);  // [C] weights (V tile no longer needed)
    float* lcs = wts + p.C;
    constexpr int kU = 8;
    constexpr int kCP = kT / 32;  // chunk sets: thread (cp, d4) takes chunks cp, cp + kCP, ...
    const int d4 = tid & 31, cp = tid >> 5;
    f4v ov[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {  // chunks past C read zeros (outside the resource)
        const int c = cp + kCP * u;
        ov[u] = ldc16(r, (uint32_t)((c * G + g) * stride + 4 + 4 * d4) * 4);
    }
    for (int c = tid; c < p.C; c += kT) {
        const f4v v = ldc16(r, (uint32_t)((c * G + g) * stride) * 4);
        wts[c] = v.x;
        lcs[c] = v.y;
    }
    __syncthreads();
    if (wave == 0) {
        float Mx = -1e30f;
        for (int c = lane; c < p.C; c += 64) Mx = fmaxf(Mx, wts[c]);
        Mx = wave_max(Mx);
        float L = 0.0f;
        for (int c = lane; c < p.C; c += 64) {
            const float e = expf(wts[c] - Mx);
            wts[c] = e;
            L = __builtin_fmaf(e, lcs[c], L);
        }
        L = wave_sum_tree(L);
        if (lane == 0) a.mstat[g] = L;
    }
    __syncthreads();
    f4v acc4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int c = cp + kCP * u;
        if (c < p.C) {
            const float e = wts[c];
            acc4.x = __builtin_fmaf(e, ov[u].x, acc4.x);
            acc4.y = __builtin_fmaf(e, ov[u].y, acc4.y);
            acc4.z = __builtin_fmaf(e, ov[u].z, acc4.z);
            acc4.w = __builtin_fmaf(e, ov[u].w, acc4.w);
        }
    }
    for (int c0 = cp + kCP * kU; c0 < p.C; c0 += kCP * kU) {
        f4v v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u)
            v[u] = ldc16(r, (uint32_t)(((c0 + kCP * u) * G + g) * stride + 4 + 4 * d4) * 4);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int c = c0 + kCP * u;
            if (c < p.C) {
                const float e = wts[c];
                acc4.x = __builtin_fmaf(e, v[u].x, acc4.x);
                acc4.y = __builtin_fmaf(e, v[u].y, acc4.y);
                acc4.z = __builtin_fmaf(e, v[u].z, acc4.z);
                acc4.w = __builtin_fmaf(e, v[u].w, acc4.w);
            }
        }
    }
    float* red = a.ow;  // [kCP][128]
    red[cp * kD + 4 * d4] = acc4.x;
    red[cp * kD + 4 * d4 + 1] = acc4.y;
    red[cp * kD + 4 * d4 + 2] = acc4.z;
    red[cp * kD + 4 * d4 + 3] = acc4.w;
    __syncthreads();
    if (tid < kD) {
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < kCP; ++q) o += red[q * kD + tid];
        const size_t off = (size_t)(h * G + g) * kD + tid;
        const float y = o / a.mstat[g];
        stc(p.attns + (size_t)l * p.Hq * kD + off, y);
        if (l == p.L - 1) stc(p.attn + off, y);
    }
    __syncthreads();
}

// paged_int8: out = the sum of the C chunk sums of query head g (their weights
// are normalized already; paged_sum_kernel's sum in another order). Thread
// (cp, d4) sums dims 4 d4.. over the chunks cp, cp + kT/32, ... and the kT/32
// sums are added in cp order.
template <int G>
__device__ __forceinline__ void attn_merge_sum(AttnShared& a, const DsParams& p, int l, int h,
                                               int g) {
    const int tid = ltid();
    const int stride = kPS;
    const float* base = p.part + (size_t)h * p.C * G * stride;
    const __amdgpu_buffer_rsrc_t r = rsrc(base, (uint32_t)(p.C * G * stride) * 4);
    constexpr int kU = 8;
    constexpr int kCP = kT / 32;
    const int d4 = tid & 31, cp = tid >> 5;
    f4v acc4 = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = cp; c0 < p.C; c0 += kCP * kU) {
        f4v v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u)  // chunks past C read zeros (outside the resource)
            v[u] = ldc16(r, (uint32_t)(((c0 + kCP * u) * G + g) * stride + 4 + 4 * d4) * 4);
#pragma unroll
        for (int u = 0; u < kU; ++u)
            if (c0 + kCP * u < p.C) acc4 += v[u];
    }
    float* red = a.ow;  // [kCP][128]
    red[cp * kD + 4 * d4] = acc4.x;
    red[cp * kD + 4 * d4 + 1] = acc4.y;
    red[cp * kD + 4 * d4 + 2] = acc4.z;
    red[cp * kD + 4 * d4 + 3] = acc4.w;
    __syncthreads();
    if (tid < kD) {
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < kCP; ++q) o += red[q * kD + tid];
        const size_t off = (size_t)(h * G + g) * kD + tid;
        stc(p.attns + (size_t)l * p.Hq * kD + off, o);
        if (l == p.L - 1) stc(p.attn + off, o);
    }
    __syncthreads();
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

// The head stage: the final hidden state x = h1 + down of the last layer
// (stored as floats), then (with_head) the final RMSNorm, +-127 codes, the
// int8 LM head over row blocks first, first+nwg, ... and the greedy argmax
// (compute_logits :1660-1700, greedy :1745-1755): a partial per workgroup,
// reduced by the last workgroup to arrive.
__device__ __forceinline__ void head_stage(SharedAll& sh, const DsParams& p, int first, int n) {
    Shared& s = sh.s;
    const int tid = ltid(), lane = tid & 63, wave = lwave(), wg = blockIdx.x;
    float best = -INFINITY;
    int besti = INT_MAX;
    if (first < n) {
        const AccOff ao = acc_off(p.H, p.F, p.Hq, p.Hkv);
        float4 nwr[kJ];
        if (p.with_head) load_norm_w(nwr, p.final_norm, p.H);
        float4 xv[kJ];
        InRaw in;
        issue_vec2(in, p.h1s + (size_t)(p.L - 1) * p.H,
                   p.acc + (size_t)(p.L - 1) * ao.stride + ao.down, p.H);
        issue_rec(in, p, p.L - 1, 3);
        // Row block t: HC chunks of 16 columns x 64 rows, 1 KiB each. When a
        // block is two rounds (HC <= 2 kHU x waves), wave w loads its chunks
        // w + kW (u + kHU r), u < kHU, of round r into one of two register
        // sets while it multiplies the other: the first round's loads go out
        // right after the stage input's (so waiting for the input does not
        // wait for them) and run under the final norm; each later round's go
        // out before the previous round's products. Loads of a block past n,
        // or past HC, read zeros (empty resource).
        const int HC = p.H / 16;
        constexpr int kHU = 10;
        const bool two_rounds = HC <= 2 * kHU * kW;
        uint4 va[kHU], vb[kHU];
        auto issue = [&](uint4 (&v)[kHU], int t, int r) {
            const bool live = p.with_head && two_rounds && t < n;
            const __amdgpu_buffer_rsrc_t rh =
                rsrc(p.head + (size_t)t * HC * 64, live ? (uint32_t)HC * 64 * 16 : 0u);
#pragma unroll
            for (int u = 0; u < kHU; ++u)
                v[u] = ld16nt(rh, (uint32_t)((wave + (u + kHU * r) * kW) * 64 + lane) * 16);
        };
        issue(va, first, 0);
        in.inv = wait_rec_inv(p, p.L - 1, 3, in.inv);
        finish_resid(xv, in, p.H, layer(p, p.L - 1).sc(6));
        float inv;
        int cs;
        store_slices(p.x, xv, p.H, 0, first, min(n, p.nwg));
        if (!p.with_head) return;
        norm_quant<127>(s, xv, nwr, p.final_norm != nullptr, p.H, p.eps, inv, cs);
        const int4* c4 = reinterpret_cast<const int4*>(s.codes);
        // the row's int32 sum (integer sums: exact in any order) -> logit, argmax
        auto finish_block = [&](int t, int part) {
            s.red_i[wave][lane] = part;
            __syncthreads();
            if (wave == 0) {
                int tot = 0;
#pragma unroll
                for (int w = 0; w < kW; ++w) tot += s.red_i[w][lane];
                const int row = t * 64 + lane;
                if (row < p.V) {
                    const float val = (float)tot * (inv * p.head_scales[row]);
                    p.logits[row] = val;
                    am_combine(best, besti, val, row);
                }
            }
            __syncthreads();
        };
        auto dot_round = [&](const uint4 (&v)[kHU], int r) {
            int acc4[4] = {0, 0, 0, 0};  // independent chains
#pragma unroll
            for (int u = 0; u < kHU; ++u) {
                const int c = min(wave + (u + kHU * r) * kW, HC - 1);  // past HC the weights read 0
                const int4 a4 = c4[c];
                acc4[0] = sdot4(v[u].x, a4.x, acc4[0]);
                acc4[1] = sdot4(v[u].y, a4.y, acc4[1]);
                acc4[2] = sdot4(v[u].z, a4.z, acc4[2]);
                acc4[3] = sdot4(v[u].w, a4.w, acc4[3]);
            }
            return (acc4[0] + acc4[1]) + (acc4[2] + acc4[3]);
        };
        if (two_rounds) {
            for (int t = first; t < n; t += p.nwg) {
                issue(vb, t, 1);
                const int part = dot_round(va, 0);
                issue(va, t + p.nwg, 0);
                finish_block(t, part + dot_round(vb, 1));
            }
        } else {
            constexpr int kHR = 8;  // 16-byte loads in flight per lane (x 8 waves)
            for (int t = first; t < n; t += p.nwg) {
                const __amdgpu_buffer_rsrc_t rh =
                    rsrc(p.head + (size_t)t * HC * 64, (uint32_t)HC * 64 * 16);
                int acc4[4] = {0, 0, 0, 0};
                for (int c0 = wave; c0 < HC; c0 += kHR * kW) {
                    uint4 v[kHR];
#pragma unroll
                    for (int u = 0; u < kHR; ++u)
                        v[u] = ld16nt(rh, (uint32_t)((c0 + u * kW) * 64 + lane) * 16);
#pragma unroll
                    for (int u = 0; u < kHR; ++u) {
                        const int c = min(c0 + u * kW, HC - 1);
                        const int4 a4 = c4[c];
                        acc4[0] = sdot4(v[u].x, a4.x, acc4[0]);
                        acc4[1] = sdot4(v[u].y, a4.y, acc4[1]);
                        acc4[2] = sdot4(v[u].z, a4.z, acc4[2]);
                        acc4[3] = sdot4(v[u].w, a4.w, acc4[3]);
                    }
                }
                finish_block(t, (acc4[0] + acc4[1]) + (acc4[2] + acc4[3]));
            }
        }
    } else if (!p.with_head) {
        return;
    }
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
        const unsigned old = __hip_atomic_fetch_add(p.sync + w_am(p.L, p.Hkv), 1u,
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s.flag = old == (unsigned)(p.nwg - 1);
    }
    __syncthreads();
    if (s.flag && wave == 0) {
        float v = -INFINITY;
        int vi = INT_MAX;
        for (int q = lane; q < p.nwg; q += 64)
            am_combine(v, vi, ldc(&p.am_part[q].x), __float_as_int(ldc(&p.am_part[q].y)));
        wave_argmax(v, vi);
        if (lane == 0) {
            p.io[2] = vi;
            p.io[0] = vi;  // the next step's input when steps are chained
            if (p.out_tokens) p.out_tokens[p.step] = vi;
        }
    }
}

// ---------------------------------------------------------------- kernel --

// Brings the norm weights of stage s (read by every workgroup, otherwise
// from HBM at that stage's start) into L2 a stage early: one dword per
// 128-byte line, lane l of wave w taking line 64 w + l (up to 8192 floats;
// past the vector, or without a norm, the load reads nothing). The value is
// only consumed after the next barrier, whose wait covers the load, so
// nothing waits for it.
__device__ __forceinline__ int touch_norm(const DsParams& p, int s) {
    const int kind = s < 5 * p.L ? s % 5 : S_HEAD;
    const int slot = kind == S_QKV ? 0 : kind - 1;
    const bool gemv = kind != S_ATT && kind != S_HEAD;
    const float* nw = kind == S_HEAD ? (p.with_head ? p.final_norm : nullptr)
                      : gemv         ? layer(p, s / 5).norm(slot)
                                     : nullptr;
    const int K = gemv ? gemv_k(slot, p.H, p.F) : p.H;
    const int line = lwave() * 64 + (ltid() & 63);
    return ld4i(rsrc(nw, nw ? (uint32_t)K * 4 : 0u), (uint32_t)line * 128);
}

// The loads of stage s that depend on nothing produced in the launch, for a
// workgroup whose first task in it is `first`, issued during the grid barrier
// before the stage: the first weight tile of its GEMV task, or, with an INT8
// cache, the K / V rows of its first attention chunk (tile[0 .. 2 kAR), the
// lane layout of load_att_tile; their fp16 scales are loaded by the task).
// Every path issues the same kPF loads, with nothing to read where there is
// nothing to load (a load under a condition would leave the registers to a
// phi whose copy waits for them); the sources are chosen with scalar selects.
template <int KVM>
__device__ __forceinline__ void prefetch_next(const DsParams& p, uint4 (&tile)[kPF], int s,
                                              int first) {
    const int lane = ltid() & 63, wave = lwave();
    const int kind = kind_of(p, s);
    const int l = min(s / 5, p.L - 1);
    const bool gemv = kind != S_ATT && kind != S_HEAD;
    const int slot = kind == S_QKV || !gemv ? 0 : kind - 1;
    const int K = gemv_k(slot, p.H, p.F), S = p.split[slot];
    const int KS = K / 64, KSs = p.split_chunks[slot];
    const int rb = div_m(first, p.split_mul[slot]), c0 = (first - rb * S) * KSs;
    const int c1 = min(KS, c0 + KSs);
    const bool live = gemv && first < ntasks(p, kind);
    const __amdgpu_buffer_rsrc_t rw =
        rsrc(layer(p, l).mat(slot) + (size_t)rb * KS * 64, live ? (uint32_t)c1 * 64 * 16 : 0u);
    // the attention chunk's rows (as load_att_tile; INT8 cache only)
    const bool att = KVM == 0 && kind == S_ATT && first < ntasks(p, S_ATT);
    const int hq = div_m(first, p.c_mul);
    const int h = att ? hq : 0, c = att ? first - hq * p.C : 0;
    const int t0 = c * p.T;
    const int nt = att ? min(p.T, p.pos + 1 - t0) : 0;
    const size_t tok0 = ((size_t)l * p.Hkv + h) * p.max_seq + t0;
    const __amdgpu_buffer_rsrc_t rk = rsrc(p.kc + tok0 * kD, (uint32_t)nt * kD);
    const __amdgpu_buffer_rsrc_t rv = rsrc(p.vc + tok0 * kD, (uint32_t)nt * kD);
    const int d0 = (lane & 7) * 16;
#pragma unroll
    for (int i = 0; i < kPF; ++i) {
        const bool a = att && i < 2 * kAR;
        const int tl = (i / 2) * kRT + wave * 8 + (lane >> 3);
        const uint32_t off = a ? (uint32_t)(tl * kD + d0)
                               : (uint32_t)((c0 + wave + kW * i) * 64 + lane) * 16;
        tile[i] = ld16nt(a ? ((i & 1) ? rv : rk) : rw, off);
    }
}

// The kernel's parameters through an opaque pointer to the kernarg segment,
// taken afresh in every stage: loads through it cannot be hoisted out of the
// stage loop, so the parameters a stage uses are reloaded (scalar loads that
// hit the scalar cache) instead of being held in scalar registers across the
// whole loop. Held, they did not fit: 156 scalar registers spilled to vector
// lanes and reloaded with v_readlane in every stage; reloaded, 14, and every
// stage runs ~0.1 us shorter.
__device__ __forceinline__ const DsParams& kparams() {
    auto k = (const __attribute__((address_space(4))) DsParams*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(k));
    return *(const DsParams*)k;
}

template <int G, int KVM>
__global__ void __launch_bounds__(kT, 1) decode_step_kernel(DsParams p) {
    __shared__ SharedAll sh;
    __shared__ int s_abort;
    const int tid = threadIdx.x;
    const int wg = blockIdx.x;
    const int nstages = 5 * p.L + 1;
    unsigned gen = 0;
    // no line of this launch's per-layer vectors may survive in L2 from an
    // earlier launch (they are read with cached loads after the first barrier):
    // one invalidation of the CU's L1 and the XCD's L2 per workgroup (the
    // caches are shared by its waves, which wait for it at the block barrier)
    if (lwave() == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // an earlier step of a chained decode aborted: this one does nothing (the
    // host reruns the chain from the step that aborted)
    if (tid == 0)
        s_abort = __hip_atomic_load(p.io + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
    if (s_abort != 0) return;
    if (KVM == 3) stage_blocks(p);  // (stage_layers' block barrier covers it)
    stage_layers(p);
    int off = 0;  // first workgroup of the current stage
    uint4 tile[kPF];  // the first weight tile of this workgroup's next GEMV task, or the
                      // K / V rows of its first attention chunk
    prefetch_next<KVM>(p, tile, 0, wg);
    // The layers' stages; the head follows the loop, so that the loop's only
    // way back to its top is through the grid barrier (a stage body exiting
    // through the loop would leave its loads pending at the top, where the
    // compiler would then wait for all of them, the prefetched tile included).
    const int nlayer_stages = nstages - 1;
    for (int s = 0; s < nlayer_stages; ++s) {
        const DsParams& p = kparams();
        const int kind = s % 5;
        const int l = s / 5;
        const int n = ntasks(p, kind);
        const int first = wrap_wg(wg - off, p.nwg);  // my first task index here
        const int touched = touch_norm(p, s + 1);
        bool arrived = false;
        if (kind == S_ATT) {
            for (int t = first; t < n; t += p.nwg) {
                const int h = div_m(t, p.c_mul);
                attn_task<G, KVM>(sh, p, l, h, t - h * p.C, tile, t == first);
                __syncthreads();
            }
        } else if (first < n || rec_writer(p, first, n)) {
            arrived = tl1_stage(sh, p, kind, l, first, n, tile, [&] {
                ++gen;
                bar_arrive(p, s, touched);
            });
        }
        // (after an early writer's stage, one more: that writer lands on the
        // last workgroup of the next stage)
        off += n + (early_writer(p, kind, l) ? 1 : 0);
        if (off >= p.nwg) off -= p.nwg;
        if (off >= p.nwg) off %= p.nwg;  // (stages of more than nwg tasks)
        if (!arrived) {
            ++gen;
            bar_arrive(p, s, touched);
        }
        const int next = wrap_wg(wg - off, p.nwg);
        if (!bar_wait(p, gen, &s_abort, [&] { prefetch_next<KVM>(p, tile, s + 1, next); }))
            return;
        if (p.trace && tid == 0) p.trace[((size_t)s * p.nwg + wg) * 2 + 1] = wall_clock64();
    }
    const int s = nlayer_stages;
    head_stage(sh, p, wrap_wg(wg - off, p.nwg), ntasks(p, S_HEAD));
    if (p.trace && tid == 0) {
        const uint64_t now = wall_clock64();
        p.trace[((size_t)s * p.nwg + wg) * 2] = now;
        p.trace[((size_t)s * p.nwg + wg) * 2 + 1] = now;
    }
}

}  // namespace

size_t ds_sync_words(int L, int Hkv) {
    const size_t w = (size_t)(kNC + 2 + L * Hkv) * 64 + (size_t)L * 4 * 32 + (size_t)L * Hkv * 64;
    return (w + 63) / 64 * 64;
}

size_t ds_vec_floats(int L, int H, int Hq) { return (size_t)L * (2 * H + Hq * kD); }

size_t ds_acc_words(int L, int H, int F, int Hq, int Hkv) {
    return (size_t)L * acc_off(H, F, Hq, Hkv).stride;
}

void ds_plan_splits(DsParams& p) {
    for (int slot = 0; slot < 4; ++slot) {
        const int nb = gemv_rows(slot, p.H, p.F, p.Hq, p.Hkv) / 64;
        const int KS = gemv_k(slot, p.H, p.F) / 64;
        int S = nb > 0 ? p.nwg / nb : 1;
        if (S > KS) S = KS;
        if (S < 1) S = 1;
        p.split[slot] = S;
        p.split_chunks[slot] = (KS + S - 1) / S;
        p.split_mul[slot] = ds_div_mul(S);
    }
    p.c_mul = ds_div_mul(p.C > 0 ? p.C : 1);
}

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
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<4, 0>, kT, 0) !=
            hipSuccess ||
        per_cu < 1)
        return 0;
    const int n = (cus / kNC) * kNC;
    return n;
}

int ds_chunk_budget(int nwg, int Hkv) { return nwg / Hkv; }

void ds_chunking(int ctx, int Hkv, int nwg, int* C, int* T) {
    int c = ds_chunk_budget(nwg, Hkv);
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
}

// The merge keeps C x G chunk statistics (2 floats each) in the V tile's
// LDS (kTmax * kD bytes).
int ds_max_context(int G) { return kTmax * kD / 8 / G * kTmax; }

int launch_decode_step(const DsParams& p, int G, bool coop, hipStream_t st) {
    void* args[] = {const_cast<DsParams*>(&p)};
    void* fn = nullptr;
    const bool paged = p.kv_mode == 3;
    if (p.kv_mode < 0 || p.kv_mode > 3 || (paged != (p.block_table != nullptr))) {
        set_error("decode step: kv mode %d", p.kv_mode);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    switch (G * 4 + p.kv_mode) {
#define TZ_DS_CASE(g, m) \
        case g * 4 + m: fn = (void*)decode_step_kernel<g, m>; break;
        TZ_DS_CASE(1, 0) TZ_DS_CASE(1, 1) TZ_DS_CASE(1, 2) TZ_DS_CASE(1, 3)
        TZ_DS_CASE(2, 0) TZ_DS_CASE(2, 1) TZ_DS_CASE(2, 2) TZ_DS_CASE(2, 3)
        TZ_DS_CASE(4, 0) TZ_DS_CASE(4, 1) TZ_DS_CASE(4, 2) TZ_DS_CASE(4, 3)
        TZ_DS_CASE(8, 0) TZ_DS_CASE(8, 1) TZ_DS_CASE(8, 2) TZ_DS_CASE(8, 3)
#undef TZ_DS_CASE
        default:
            set_error("decode step: query heads per kv head must be 1, 2, 4 or 8");
            return TENZO_ERROR_UNSUPPORTED;
    }
    if (p.L > kDsMaxLayers) {
        set_error("decode step: at most %d layers", kDsMaxLayers);
        return TENZO_ERROR_UNSUPPORTED;
    }
    // paged: the block table fits in LDS, and every chunk task of the
    // attention stage is resident (their softmax waits for all of them)
    if (paged && (p.pos / 16 >= kDsMaxBlocks || p.C * p.Hkv > p.nwg ||
                  (size_t)(p.max_seq + 15) / 16 * 16 * p.L * p.Hkv * kD >= (1ull << 32))) {
        set_error("decode step (paged): context %d needs %d attention tasks for %d workgroups",
                  p.pos + 1, p.C * p.Hkv, p.nwg);
        return TENZO_ERROR_UNSUPPORTED;
    }
    if (p.H % 64 || p.F % 64 || p.H > kJ * 4 * kT || p.F > kJ * 4 * kT) {
        set_error("decode step: hidden and ffn sizes must be multiples of 64, at most %d",
                  kJ * 4 * kT);
        return TENZO_ERROR_UNSUPPORTED;
    }
    // The kernel needs all nwg workgroups resident at once: one per CU
    // (ds_grid_size checked the occupancy), which an ordinary launch of this
    // grid gives on a device with no other work resident. The cooperative
    // launch guarantees it but costs ~19 us more per step (1.1795 vs 1.1994 ms
    // per BitNet-2B token), so the engine launches ordinarily and reruns a step
    // that aborted under the cooperative launch: every wait in the kernel is
    // bounded, so a grid that is not fully resident ends the step with the
    // abort flag set instead of hanging. The runtime refuses a cooperative
    // launch while another process holds the device's cooperative-launch
    // resources; that is reported (kDsCoopRefused) rather than replaced by
    // another ordinary launch, so the engine can take its graph path instead.
    hipError_t e;
    if (coop) {
        e = hipLaunchCooperativeKernel(fn, dim3(p.nwg), dim3(kT), args, 0, st);
        if (e == hipErrorIllegalState || e == hipErrorNotSupported ||
            e == hipErrorCooperativeLaunchTooLarge) {
            (void)hipGetLastError();
            return kDsCoopRefused;
        }
    } else {
        e = hipLaunchKernel(fn, dim3(p.nwg), dim3(kT), args, 0, st);
    }
    if (e != hipSuccess) return hip_fail(e, "launch of decode_step_kernel");
    return TENZO_SUCCESS;
}

}  // namespace tz

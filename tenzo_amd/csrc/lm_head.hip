// int8 LM head, greedy argmax and embedding lookup on gfx950
// (reference src/runtime/TenzoEngine.cpp:1294-1316 embedding_lookup,
// :1634-1720 compute_logits, :1735-1755 repetition penalty + greedy branch of
// sample_top_k_top_p).
//
// Device layout of the int8 [V][H] table: for row block b (64 rows) and
// column chunk c (16 columns) there are 64 x 16 bytes, row r's 16 bytes at
// offset r*16. A wave reads one chunk of its row block as 1 KiB contiguous
// (lane = row) and takes the matching 16 activation codes as 4 wave-uniform
// dwords, so each lane issues four v_dot4_i32_i8 per 16-byte load. Rows past
// V are zero.
#include "lm_head.h"
#include "tl1.h"

namespace tz {

// ------------------------------------------------------------------ repack --

__global__ void i8_repack_kernel(const int8_t* __restrict__ src, uint32_t* __restrict__ dst,
                                 int64_t V, int64_t H, int64_t nb) {
    // one dword of the packed layout per thread
    const int64_t HC = H / 16;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nb * HC * 256) return;
    const int q = (int)(idx & 3);
    const int r = (int)((idx >> 2) & 63);
    const int64_t bc = idx >> 8;
    const int64_t c = bc % HC;
    const int64_t b = bc / HC;
    const int64_t row = b * 64 + r;
    uint32_t v = 0;
    if (row < V) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(src) + row * H + c * 16 + q * 4;
        v = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
            ((uint32_t)p[3] << 24);
    }
    dst[idx] = v;
}

// ------------------------------------------------------------------ argmax --

// First maximum: the larger value wins, equal values go to the smaller index
// (the sequential scan at :1745-1755 keeps the first of equal maxima).
__device__ __forceinline__ void am_combine(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const int oi = __shfl_xor(i, o, kWave);
        am_combine(v, i, ov, oi);
    }
}

// Called by every thread of a 256-thread block once the block's partial is in
// am.part[blockIdx.x]. The last block to arrive reduces all nparts partials
// into *am.out_idx and re-arms the counter.
__device__ void argmax_finish(const ArgmaxWs& am, int nparts) {
    __shared__ int is_last;
    __shared__ float rv[4];
    __shared__ int ri[4];
    partials_acked();
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(am.counter, 1u) == (unsigned)(nparts - 1);
    __syncthreads();
    if (!is_last) return;
    float v = -INFINITY;
    int i = INT_MAX;
    for (int p = threadIdx.x; p < nparts; p += 256) {
        const float pv = __hip_atomic_load(&am.part[p].x, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        const float pi = __hip_atomic_load(&am.part[p].y, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        am_combine(v, i, pv, __float_as_int(pi));
    }
    wave_argmax(v, i);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        rv[wave] = v;
        ri[wave] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) am_combine(rv[0], ri[0], rv[w], ri[w]);
        *am.out_idx = ri[0];
        atomicExch(am.counter, 0u);
    }
}

constexpr int kArgmaxPerBlock = 4096;

__global__ void __launch_bounds__(256)
argmax_kernel(const float* __restrict__ logits, int64_t V, ArgmaxWs am) {
    const int64_t base = (int64_t)blockIdx.x * kArgmaxPerBlock;
    const int64_t end = base + kArgmaxPerBlock < V ? base + kArgmaxPerBlock : V;
    float v = -INFINITY;
    int i = INT_MAX;
    for (int64_t k = base + threadIdx.x; k < end; k += 256) am_combine(v, i, logits[k], (int)k);
    wave_argmax(v, i);
    __shared__ float rv[4];
    __shared__ int ri[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        rv[wave] = v;
        ri[wave] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) am_combine(rv[0], ri[0], rv[w], ri[w]);
        store_coherent(&am.part[blockIdx.x].x, rv[0]);
        store_coherent(&am.part[blockIdx.x].y, __int_as_float(ri[0]));
    }
    argmax_finish(am, (int)gridDim.x);
}

// ----------------------------------------------------------------- LM head --

// One block per 64-row block; its 4 waves split the H/16 chunks and reduce
// through LDS. int32 sums are exact; logit = float(acc) * (s_x * s_v) (:1718).
__global__ void __launch_bounds__(256)
lm_head_i8_kernel(const uint4* __restrict__ w, const int32_t* __restrict__ codes,
                  const tenzo_hip_actq_t* __restrict__ aq, const float* __restrict__ scales,
                  float* __restrict__ logits, int64_t V, int64_t HC, ArgmaxWs am) {
    __shared__ int red[4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t b = blockIdx.x;
    const uint4* wb = w + b * HC * 64 + lane;
    int acc0 = 0, acc1 = 0;
    int64_t c = wave;
    for (; c + 12 < HC; c += 16) {
        const uint4 v0 = ld_nt16(&wb[c * 64]);
        const uint4 v1 = ld_nt16(&wb[(c + 4) * 64]);
        const uint4 v2 = ld_nt16(&wb[(c + 8) * 64]);
        const uint4 v3 = ld_nt16(&wb[(c + 12) * 64]);
        const int32_t* a0 = codes + c * 4;
        acc0 = sdot4(v0.x, a0[0], acc0);
        acc0 = sdot4(v0.y, a0[1], acc0);
        acc0 = sdot4(v0.z, a0[2], acc0);
        acc0 = sdot4(v0.w, a0[3], acc0);
        acc1 = sdot4(v1.x, a0[16], acc1);
        acc1 = sdot4(v1.y, a0[17], acc1);
        acc1 = sdot4(v1.z, a0[18], acc1);
        acc1 = sdot4(v1.w, a0[19], acc1);
        acc0 = sdot4(v2.x, a0[32], acc0);
        acc0 = sdot4(v2.y, a0[33], acc0);
        acc0 = sdot4(v2.z, a0[34], acc0);
        acc0 = sdot4(v2.w, a0[35], acc0);
        acc1 = sdot4(v3.x, a0[48], acc1);
        acc1 = sdot4(v3.y, a0[49], acc1);
        acc1 = sdot4(v3.z, a0[50], acc1);
        acc1 = sdot4(v3.w, a0[51], acc1);
    }
    for (; c < HC; c += 4) {
        const uint4 v0 = ld_nt16(&wb[c * 64]);
        const int32_t* a0 = codes + c * 4;
        acc0 = sdot4(v0.x, a0[0], acc0);
        acc0 = sdot4(v0.y, a0[1], acc0);
        acc0 = sdot4(v0.z, a0[2], acc0);
        acc0 = sdot4(v0.w, a0[3], acc0);
    }
    red[wave][lane] = acc0 + acc1;
    __syncthreads();
    if (wave == 0) {
        const int tot = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
        const int64_t row = b * 64 + lane;
        float val = -INFINITY;
        if (row < V) {
            val = (float)tot * __fmul_rn(aq->inv_scale, scales[row]);
            logits[row] = val;
        }
        if (am.out_idx) {
            int idx = (int)row;
            wave_argmax(val, idx);
            if (lane == 0) {
                store_coherent(&am.part[b].x, val);
                store_coherent(&am.part[b].y, __int_as_float(idx));
            }
        }
    }
    if (am.out_idx) argmax_finish(am, (int)gridDim.x);
}

// fp32 table: one wave per row, float4 loads along H, fp32 FMA and a wave sum.
__global__ void __launch_bounds__(256)
lm_head_f32_kernel(const float* __restrict__ xn, const float* __restrict__ E,
                   float* __restrict__ logits, int64_t V, int64_t H) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= V) return;
    const float* er = E + row * H;
    float s = 0.0f;
    if ((H & 3) == 0) {
        const float4* e4 = reinterpret_cast<const float4*>(er);
        const float4* x4 = reinterpret_cast<const float4*>(xn);
        for (int64_t i = lane; i < H / 4; i += 64) {
            const float4 e = e4[i], x = x4[i];
            s = __builtin_fmaf(x.x, e.x, s);
            s = __builtin_fmaf(x.y, e.y, s);
            s = __builtin_fmaf(x.z, e.z, s);
            s = __builtin_fmaf(x.w, e.w, s);
        }
    } else {
        for (int64_t i = lane; i < H; i += 64) s = __builtin_fmaf(xn[i], er[i], s);
    }
    s = wave_sum_tree(s);
    if (lane == 0) logits[row] = s;
}

// --------------------------------------------------------------- embedding --

__global__ void embed_i8_kernel(const uint8_t* __restrict__ w, const float* __restrict__ scales,
                                const int32_t* __restrict__ token_dev, int64_t V, int64_t H,
                                float* __restrict__ x) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    const int tok = token_dev[blockIdx.y];  // row blockIdx.y of x
    x += (int64_t)blockIdx.y * H;
    if (tok < 0 || (int64_t)tok >= V) {
        x[i] = 0.0f;
        return;
    }
    const int64_t b = tok >> 6, r = tok & 63, c = i >> 4;
    const int8_t e = (int8_t)w[((b * (H / 16) + c) * 64 + r) * 16 + (i & 15)];
    x[i] = __fmul_rn((float)e, scales[tok]);  // :1300-1315
}

__global__ void embed_f32_kernel(const float* __restrict__ E, const int32_t* __restrict__ token_dev,
                                 int64_t V, int64_t H, float* __restrict__ x) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    const int tok = token_dev[blockIdx.y];
    x += (int64_t)blockIdx.y * H;
    x[i] = (tok < 0 || (int64_t)tok >= V) ? 0.0f : E[(int64_t)tok * H + i];
}

// :1735-1743, sequential so that repeated tokens compound as in the reference.
// The reference build (-ffast-math) hoists the division out of the loop: it
// computes 1 / penalty once (vdivss) and multiplies each positive logit by it.
__global__ void rep_penalty_kernel(float* __restrict__ logits, int64_t V,
                                   const int32_t* __restrict__ tokens, int n, float penalty) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const float inv = __fdiv_rn(1.0f, penalty);
    for (int k = 0; k < n; ++k) {
        const int t = tokens[k];
        if (t >= 0 && (int64_t)t < V) {
            const float l = logits[t];
            logits[t] = l > 0.0f ? __fmul_rn(l, inv) : __fmul_rn(l, penalty);
        }
    }
}

// --------------------------------------------------------- table loading --
// The loader's LM-head quantization (load_model_from_files,
// TenzoEngine.cpp:1925-1941) as the reference is built (-ffast-math): per row
// amax (floor 1e-8), stored scale = amax * (1/127) (the divide by the
// constant folded into a multiply), codes = clamp(round(x * (127 / amax)),
// -127, 127) (1 / (amax * (1/127)) re-associated; x * (1 / scale) differs at
// exact .5 ties). One block per row.
__global__ void __launch_bounds__(256) quant_rows_i8_kernel(const float* __restrict__ E,
                                                            int64_t H, int8_t* __restrict__ codes,
                                                            float* __restrict__ scales) {
    __shared__ float red[4];
    const int64_t v = blockIdx.x;
    const float* row = E + v * H;
    float amax = 1e-8f;
    for (int64_t i = threadIdx.x; i < H; i += 256) amax = fmaxf(amax, fabsf(row[i]));
    amax = block256_max(amax, red);
    const float scale = __fmul_rn(amax, 1.0f / 127.0f);
    const float inv_s = 127.0f / amax;
    for (int64_t i = threadIdx.x; i < H; i += 256) {
        const float c = fminf(fmaxf(roundf(__fmul_rn(row[i], inv_s)), -127.0f), 127.0f);
        codes[v * H + i] = (int8_t)c;
    }
    if (threadIdx.x == 0) scales[v] = scale;
}

int launch_quant_rows_i8(const float* E, int64_t V, int64_t H, int8_t* codes, float* scales,
                         hipStream_t st) {
    hipLaunchKernelGGL(quant_rows_i8_kernel, dim3((unsigned)V), dim3(256), 0, st, E, H, codes,
                       scales);
    return launch_status("quant_rows_i8_kernel");
}

// ------------------------------------------------------------- sampling --
// sample_top_k_top_p (:1722-1807) for temperature > 0: the top-k (k <= 64)
// logits, a softmax at the temperature over them, the top-p cutoff and one
// draw r in [0, 1]. Stage 1: each workgroup sorts a slice of kSampleSlice
// logits in LDS (bitonic, order "a before b" = larger value, or equal value
// and lower index) and keeps its first 64; stage 2: one workgroup sorts the
// slices' candidates the same way, takes the first k, orders them as the
// reference's heap hands them out (descending (value, index)), and one lane
// replays the reference's probability, cutoff and draw loops in its order.

template <int N, int THREADS>
__device__ __forceinline__ void bitonic_sort_desc(float* v, int* idx) {
    for (int size = 2; size <= N; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < N / 2; t += THREADS) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;  // this run sorts "before" first
                const float a = v[lo], b = v[hi];
                const int ia = idx[lo], ib = idx[hi];
                const bool b_first = b > a || (b == a && ib < ia);
                if (b_first == up) {
                    v[lo] = b;
                    v[hi] = a;
                    idx[lo] = ib;
                    idx[hi] = ia;
                }
            }
            __syncthreads();
        }
    }
}

__global__ void __launch_bounds__(256) sample_slice_kernel(const float* __restrict__ logits,
                                                           int64_t V, float2* __restrict__ cand) {
    __shared__ float v[kSampleSlice];
    __shared__ int idx[kSampleSlice];
    const int64_t base = (int64_t)blockIdx.x * kSampleSlice;
    for (int t = threadIdx.x; t < kSampleSlice; t += 256) {
        const int64_t i = base + t;
        v[t] = i < V ? logits[i] : -INFINITY;
        idx[t] = i < V ? (int)i : INT_MAX;
    }
    __syncthreads();
    bitonic_sort_desc<kSampleSlice, 256>(v, idx);
    if (threadIdx.x < kSampleK)
        cand[(int64_t)blockIdx.x * kSampleK + threadIdx.x] =
            make_float2(v[threadIdx.x], __int_as_float(idx[threadIdx.x]));
}

__global__ void __launch_bounds__(1024)
sample_pick_kernel(const float2* __restrict__ cand, int nslices, int k, float top_p,
                   float temperature, float r, int32_t* __restrict__ out) {
    __shared__ float v[kSampleSlice * 4];
    __shared__ int idx[kSampleSlice * 4];
    const int n = nslices * kSampleK;
    for (int t = threadIdx.x; t < kSampleSlice * 4; t += 1024) {
        const float2 c = t < n ? cand[t] : make_float2(-INFINITY, __int_as_float(INT_MAX));
        v[t] = c.x;
        idx[t] = __float_as_int(c.y);
    }
    __syncthreads();
    bitonic_sort_desc<kSampleSlice * 4, 1024>(v, idx);
    if (threadIdx.x != 0) return;
    // candidates as the heap hands them out: descending (value, index) (:1769-1774)
    float cv[kSampleK];
    int ci[kSampleK];
    int m = 0;
    for (int j = 0; j < k; ++j)
        if (idx[j] != INT_MAX) {
            cv[m] = v[j];
            ci[m] = idx[j];
            ++m;
        }
    for (int a = 1; a < m; ++a) {  // equal values: higher index first
        const float x = cv[a];
        const int xi = ci[a];
        int b = a - 1;
        while (b >= 0 && cv[b] == x && ci[b] < xi) {
            cv[b + 1] = cv[b];
            ci[b + 1] = ci[b];
            --b;
        }
        cv[b + 1] = x;
        ci[b + 1] = xi;
    }
    float probs[kSampleK];
    const float max_l = cv[0];
    float sum_exp = 0.0f;
    for (int i = 0; i < m; ++i) {  // :1776-1782
        probs[i] = expf((cv[i] - max_l) / temperature);
        sum_exp += probs[i];
    }
    for (int i = 0; i < m; ++i) probs[i] /= sum_exp;
    float cum_p = 0.0f;
    int cutoff = m;
    for (int i = 0; i < m; ++i) {  // :1784-1792
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
    int pick = ci[0];
    for (int i = 0; i < cutoff; ++i) {  // :1798-1804
        acc += probs[i];
        if (r <= acc) {
            pick = ci[i];
            break;
        }
    }
    *out = pick;
}

// -------------------------------------------------------------------- host --

static int64_t head_blocks(int64_t V) { return ceil_div(V, 64); }
static int64_t argmax_blocks(int64_t V) { return ceil_div(V, kArgmaxPerBlock); }

// Workspace: the counter at offset 0 (the same place whatever V is, so a
// region reused across calls of different V keeps a zero counter), then the
// partials from offset 256.
size_t argmax_ws_bytes(int64_t V) {
    int64_t n = head_blocks(V);
    if (argmax_blocks(V) > n) n = argmax_blocks(V);
    return 256 + (size_t)ceil_div(n * 8, 256) * 256;
}

ArgmaxWs argmax_ws_at(void* base, int64_t V, int32_t* out_idx) {
    (void)V;
    ArgmaxWs am;
    am.counter = reinterpret_cast<uint32_t*>(base);
    am.part = reinterpret_cast<float2*>(reinterpret_cast<char*>(base) + 256);
    am.out_idx = out_idx;
    return am;
}

int launch_i8_repack(const int8_t* w, void* w_packed, int64_t V, int64_t H, hipStream_t st) {
    const int64_t nb = head_blocks(V);
    const int64_t total = nb * (H / 16) * 256;
    hipLaunchKernelGGL(i8_repack_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                       w, (uint32_t*)w_packed, V, H, nb);
    return launch_status("i8_repack_kernel");
}

int launch_lm_head_i8(const int8_t* codes, const tenzo_hip_actq_t* aq, const void* w_packed,
                      const float* scales, float* logits, int64_t V, int64_t H,
                      const ArgmaxWs& am, hipStream_t st) {
    hipLaunchKernelGGL(lm_head_i8_kernel, dim3((unsigned)head_blocks(V)), dim3(256), 0, st,
                       (const uint4*)w_packed, (const int32_t*)codes, aq, scales, logits, V,
                       H / 16, am);
    return launch_status("lm_head_i8_kernel");
}

int launch_lm_head_f32(const float* xn, const float* E, float* logits, int64_t V, int64_t H,
                       hipStream_t st) {
    hipLaunchKernelGGL(lm_head_f32_kernel, dim3((unsigned)ceil_div(V, 4)), dim3(256), 0, st, xn,
                       E, logits, V, H);
    return launch_status("lm_head_f32_kernel");
}

int launch_argmax(const float* logits, int64_t V, const ArgmaxWs& am, hipStream_t st) {
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)argmax_blocks(V)), dim3(256), 0, st, logits,
                       V, am);
    return launch_status("argmax_kernel");
}

int launch_embed_i8(const void* w_packed, const float* scales, const int32_t* token_dev,
                    int64_t V, int64_t H, float* x, hipStream_t st, int n) {
    hipLaunchKernelGGL(embed_i8_kernel, dim3((unsigned)ceil_div(H, 256), (unsigned)n), dim3(256),
                       0, st, (const uint8_t*)w_packed, scales, token_dev, V, H, x);
    return launch_status("embed_i8_kernel");
}

int launch_embed_f32(const float* E, const int32_t* token_dev, int64_t V, int64_t H, float* x,
                     hipStream_t st, int n) {
    hipLaunchKernelGGL(embed_f32_kernel, dim3((unsigned)ceil_div(H, 256), (unsigned)n), dim3(256),
                       0, st, E, token_dev, V, H, x);
    return launch_status("embed_f32_kernel");
}

size_t sample_ws_bytes(int64_t V) { return (size_t)ceil_div(V, kSampleSlice) * kSampleK * 8; }

int launch_sample(const float* logits, int64_t V, int top_k, float top_p, float temperature,
                  float r, void* ws, int32_t* out_token, hipStream_t st) {
    const int64_t nslices = ceil_div(V, kSampleSlice);
    if (nslices * kSampleK > kSampleSlice * 4) {
        set_error("sampler: vocab %lld above %d", (long long)V, kSampleSlice * kSampleSlice * 4 / kSampleK);
        return TENZO_ERROR_UNSUPPORTED;
    }
    const int k = top_k < 1 ? 1 : (top_k > kSampleK ? kSampleK : top_k);  // :1731
    hipLaunchKernelGGL(sample_slice_kernel, dim3((unsigned)nslices), dim3(256), 0, st, logits, V,
                       (float2*)ws);
    int rc = launch_status("sample_slice_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(sample_pick_kernel, dim3(1), dim3(1024), 0, st, (const float2*)ws,
                       (int)nslices, k, top_p, temperature, r, out_token);
    return launch_status("sample_pick_kernel");
}

int launch_rep_penalty(float* logits, int64_t V, const int32_t* tokens, int n, float penalty,
                       hipStream_t st) {
    hipLaunchKernelGGL(rep_penalty_kernel, dim3(1), dim3(64), 0, st, logits, V, tokens, n,
                       penalty);
    return launch_status("rep_penalty_kernel");
}

}  // namespace tz

using namespace tz;

extern "C" {

TENZO_HIP_API size_t tenzo_hip_i8_packed_bytes(int64_t V, int64_t H) {
    return (size_t)ceil_div(V, 64) * (size_t)(H / 16) * 1024;
}

TENZO_HIP_API int tenzo_hip_i8_rows_repack(const int8_t* w, void* w_packed, int64_t V,
                                           int64_t H, void* stream) {
    TZ_CHECK(w && w_packed, "i8_rows_repack: null pointer");
    TZ_CHECK(V > 0 && H > 0 && H % 16 == 0, "i8_rows_repack: need H %% 16 == 0 (H=%lld)",
             (long long)H);
    return launch_i8_repack(w, w_packed, V, H, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_lm_head_i8(const float* x, const float* norm_w, float eps,
                                       const void* w_packed, const float* scales,
                                       float* logits, int64_t V, int64_t H, void* stream) {
    TZ_CHECK(x && w_packed && scales && logits, "lm_head_i8: null pointer");
    TZ_CHECK(V > 0 && V <= INT32_MAX && H > 0 && H % 16 == 0,
             "lm_head_i8: need H %% 16 == 0 (H=%lld)", (long long)H);
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)Scratch::get(kScratchAct, (size_t)H + 256, st);
    if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
    tenzo_hip_actq_t* q = (tenzo_hip_actq_t*)ws;
    int8_t* codes = (int8_t*)(ws + 256);
    // final rms_norm_raw (:1638) then the int8 activation quantization (:1666-1678)
    int rc = launch_actquant(1, 127, x, norm_w, eps, 1, H, H, codes, q, nullptr, st);
    if (rc) return rc;
    return launch_lm_head_i8(codes, q, w_packed, scales, logits, V, H, ArgmaxWs{}, st);
}

TENZO_HIP_API int tenzo_hip_rmsnorm_quant127(const float* x, const float* norm_w, int do_norm,
                                             float eps, int64_t M, int64_t K, int8_t* codes,
                                             tenzo_hip_actq_t* q, void* stream) {
    TZ_CHECK(x && codes && q, "rmsnorm_quant127: null pointer");
    TZ_CHECK(M > 0 && M <= 65535 && K > 0 && K % 16 == 0,
             "rmsnorm_quant127: need K %% 16 == 0 (K=%lld)", (long long)K);
    return launch_actquant(do_norm || norm_w ? 1 : 0, 127, x, norm_w, eps, M, K, K, codes, q,
                           nullptr, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_lm_head_i8_codes(const int8_t* codes, const tenzo_hip_actq_t* q,
                                             const void* w_packed, const float* scales,
                                             float* logits, int64_t V, int64_t H,
                                             int32_t* out_idx, void* stream) {
    TZ_CHECK(codes && q && w_packed && scales && logits, "lm_head_i8_codes: null pointer");
    TZ_CHECK(V > 0 && V <= INT32_MAX && H > 0 && H % 16 == 0,
             "lm_head_i8_codes: need H %% 16 == 0 (H=%lld)", (long long)H);
    TZ_CHECK(((uintptr_t)codes & 3) == 0, "lm_head_i8_codes: codes must be 4-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    ArgmaxWs am{};
    if (out_idx) {
        void* ws = Scratch::get(kScratchHead, argmax_ws_bytes(V), st);
        if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
        am = argmax_ws_at(ws, V, out_idx);
    }
    return launch_lm_head_i8(codes, q, w_packed, scales, logits, V, H, am, st);
}

TENZO_HIP_API int tenzo_hip_argmax(const float* logits, int64_t V, int32_t* out_idx,
                                   void* stream) {
    TZ_CHECK(logits && out_idx && V > 0 && V <= INT32_MAX, "argmax: bad arguments");
    hipStream_t st = (hipStream_t)stream;
    void* ws = Scratch::get(kScratchHead, argmax_ws_bytes(V), st);
    if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
    return launch_argmax(logits, V, argmax_ws_at(ws, V, out_idx), st);
}

TENZO_HIP_API int tenzo_hip_quant_rows_i8(const float* E, int64_t V, int64_t H, int8_t* codes,
                                          float* scales, void* stream) {
    TZ_CHECK(E && codes && scales && V > 0 && H > 0 && V <= INT32_MAX,
             "quant_rows_i8: bad arguments");
    return launch_quant_rows_i8(E, V, H, codes, scales, (hipStream_t)stream);
}

TENZO_HIP_API int tenzo_hip_sample_top_k_top_p(const float* logits, int64_t V, int top_k,
                                               float top_p, float temperature, float r,
                                               int32_t* out_token, void* stream) {
    TZ_CHECK(logits && out_token && V > 0, "sample_top_k_top_p: bad arguments");
    TZ_CHECK(temperature > 0.0f, "sample_top_k_top_p: temperature must be > 0 (got %g)",
             (double)temperature);
    hipStream_t st = (hipStream_t)stream;
    void* ws = Scratch::get(kScratchTmp, sample_ws_bytes(V), st);
    if (!ws) return TENZO_ERROR_OUT_OF_MEMORY;
    return launch_sample(logits, V, top_k, top_p, temperature, r, ws, out_token, st);
}

TENZO_HIP_API int tenzo_hip_embed_i8(const void* w_packed, const float* scales,
                                     const int32_t* token_dev, int64_t V, int64_t H, float* x,
                                     void* stream) {
    TZ_CHECK(w_packed && scales && token_dev && x, "embed_i8: null pointer");
    TZ_CHECK(V > 0 && H > 0 && H % 16 == 0, "embed_i8: need H %% 16 == 0");
    return launch_embed_i8(w_packed, scales, token_dev, V, H, x, (hipStream_t)stream);
}

}  // extern "C"

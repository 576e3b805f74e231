// The engine behind include/tenzo.h on an MI355X: the reference's
// TenzoEngineImpl (src/runtime/TenzoEngine.h:195-262, TenzoEngine.cpp:1215-1838
// and the C API at :2086-2204) with every stage of the decode step on the GPU.
//
// All state is device resident: TL1 weights in the GEMV layout (Q|K|V and
// gate|up concatenated along rows so each pair is one launch), norm vectors,
// the int8 LM head, the INT8 KV cache [L][Hkv][max_seq][128] with fp16
// scales, a RoPE cos/sin table per position, and the activation buffers. One
// decode step is
//   embed ; per layer:
//     actquant(in_norm)        -> codes           (rms_norm_raw + build_lut)
//     TL1 GEMV Q|K|V           -> qkv             (:1547-1572)
//     attention chunks+combine -> attn            (:1578, RoPE/append/softmax)
//     actquant(attn_sub_norm)  -> codes           (:1582-1585)
//     TL1 GEMV O + residual    -> h1 = x + o      (:1586-1590)
//     actquant(post_norm)      -> codes           (:1594-1596)
//     TL1 GEMV gate|up         -> gu              (:1598-1614)
//     actquant(relu^2*up, ffn_sub_norm) -> codes  (:1616-1624)
//     TL1 GEMV down + residual -> x = h1 + down   (:1625-1628)
//   actquant(final_norm, +-127) ; LM head + fused greedy argmax (:1634-1755)
// By default the whole step runs as ONE persistent cooperative kernel
// (decode_step.hip) with in-kernel barriers between the stages above; the
// same stages as separate kernels, replayed from a captured HIP graph
// (position and token read from device memory, one graph per attention chunk
// size) or launched eagerly, remain selectable (tenzo_hip_engine_set_mode).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "attention.h"
#include "common.h"
#include "decode_step.h"
#include "lm_head.h"
#include "model_file.h"
#include "tl1.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

using namespace tz;

namespace {

constexpr int kD = 128;

struct DevLayer {
    void* qkv = nullptr;   // TL1 GEMV layout, rows Q | K | V
    void* o = nullptr;
    void* gu = nullptr;    // rows gate | up
    void* down = nullptr;
    float sc[7] = {};      // q, k, v, o, gate, up, down
    float* norm[4] = {};   // in, attn_sub, post, ffn_sub (null = no weight)
    bool mlp = false;
    bool set = false;
};

}  // namespace

struct tenzo_engine_opaque {
    tenzo_config_t cfg{};
    std::string kv_mode, device;
    int dev = 0;
    hipStream_t st = nullptr;
    int H = 0, Hq = 0, Hkv = 0, L = 0, F = 0, V = 0, max_seq = 0, qd = 0, kvd = 0;
    float eps = 1e-5f;
    float theta = 10000.0f;  // the reference hard-codes 10000 (TenzoEngine.cpp:456,466)

    std::vector<DevLayer> layers;
    std::vector<void*> allocs;  // everything to free at destroy
    float* final_norm = nullptr;
    int head_kind = 0;          // 0 none, 1 int8, 2 fp32
    void* head_i8 = nullptr;
    float* head_scales = nullptr;
    float* head_f32 = nullptr;

    // KV cache: kv_kind 0 int8_fused (rows of 128 int8 codes, fp16 scales),
    // 1 tl1_fused / 2 popcount_fused (rows of 32 bytes, fp32 scales)
    int kv_kind = 0;
    int kv_row = 128;  // bytes per (layer, kv head, token) row
    int kv_sb = 2;     // bytes per scale
    // paged_int8 (kv_kind 3): kc / vc / ks / vs are block pools
    // [blocks][L][Hkv][16][...]; the block manager mirrors PagedBlockManager
    // (TenzoEngine.h:120-152: free list filled high to low, taken from the back)
    int pg_blocks = 0;
    std::vector<int32_t> pg_free, pg_table;
    int32_t* pg_bt = nullptr;  // device copy of pg_table
    float* pg_ws = nullptr;    // scores, chunk maxima and chunk sums
    int8_t* kc = nullptr;
    int8_t* vc = nullptr;
    uint16_t* ks = nullptr;
    uint16_t* vs = nullptr;

    float* x = nullptr;
    float* qkv = nullptr;
    float* attn = nullptr;
    float* h1 = nullptr;
    float* gu = nullptr;
    float* xn = nullptr;
    float* logits = nullptr;
    int8_t* codes = nullptr;
    tenzo_hip_actq_t* aq = nullptr;
    void* gemv_ws = nullptr;
    float* attn_part = nullptr;
    void* am_ws = nullptr;
    void* sample_ws = nullptr;   // top-k candidates of the sampler
    int32_t* io_dev = nullptr;   // [0] token, [1] position, [2] result token, [3] abort flag
    int32_t* io_host = nullptr;  // pinned mirror
    int32_t* pen_dev = nullptr;  // past tokens for the repetition penalty
    int pen_cap = 0;
    float* rope = nullptr;       // [max_seq][128]

    int seq_len = 0;
    int mode = 2;                // 0 eager kernels, 1 HIP graph, 2 persistent kernel
    std::map<std::pair<int, int>, hipGraphExec_t> graphs;  // (T, with head)

    // persistent decode kernel
    int ds_nwg = 0;              // 0: not available on this device
    DsLayer* ds_layers = nullptr;  // device array [L]
    bool ds_layers_dirty = true;
    unsigned* ds_sync = nullptr;   // sync words, then the int32 GEMV accumulators
    float* ds_vec = nullptr;       // per-layer x, h1, attention outputs
    float* ds_part = nullptr;
    float2* ds_am = nullptr;
    size_t ds_sync_bytes = 0;
    int32_t* dec_out = nullptr;  // device tokens of tenzo_hip_engine_decode
    int dec_cap = 0;
    uint64_t* ds_trace = nullptr;  // step trace (tenzo_hip_engine_trace), null when off
    bool ds_state_valid = false;   // the last step ran the persistent kernel
    bool ds_coop = false;          // cooperative launches (after an ordinary one aborted)
    unsigned* ds_bar = nullptr;    // grid-barrier counters + error word (uncached, bar_pool)
    unsigned ds_bar_base = 0;      // barrier generations completed by earlier launches
    bool ds_bar_reset = true;      // zero the counters before the next launch
    // polls before a wait gives up, under an ordinary launch (TENZO_HIP_SPIN_LIMIT)
    // and under the cooperative one (TENZO_HIP_SPIN_LIMIT_COOP)
    unsigned ds_spin = kDsSpinLimit;
    unsigned ds_spin_coop = kDsSpinLimit;

    // batched prefill (tenzo_hip_engine_prefill): rows of up to pf_cap tokens
    int pf_cap = 0;
    float* pf_x = nullptr;
    float* pf_h1 = nullptr;
    float* pf_qkv = nullptr;
    float* pf_attn = nullptr;
    float* pf_gu = nullptr;
    int8_t* pf_codes = nullptr;
    tenzo_hip_actq_t* pf_aq = nullptr;
    int32_t* pf_tok = nullptr;

};

namespace {

// Grid-barrier regions of the persistent kernel: uncached device memory (the
// kernel polls it with scalar loads, which must miss every cache). Uncached
// memory that a kernel has read is never freed here: a region returns to this
// pool when its engine is destroyed and is handed to the next engine made on
// the same device; the pool lives until the process ends.
struct BarPool {
    std::mutex mu;
    std::vector<std::pair<int, unsigned*>> free;  // (device, region)
};
BarPool& bar_pool() {
    static BarPool* pool = new BarPool();  // never destroyed (outlives every engine)
    return *pool;
}
constexpr size_t kBarBytes = (size_t)kDsBarWords * 4;

int bar_take(int dev, unsigned** out) {
    BarPool& bp = bar_pool();
    {
        std::lock_guard<std::mutex> g(bp.mu);
        for (size_t i = 0; i < bp.free.size(); ++i)
            if (bp.free[i].first == dev) {
                *out = bp.free[i].second;
                bp.free.erase(bp.free.begin() + (long)i);
                return TENZO_SUCCESS;
            }
    }
    void* v = nullptr;
    TZ_HIP(hipExtMallocWithFlags(&v, kBarBytes, hipDeviceMallocUncached));
    TZ_HIP(hipMemset(v, 0, kBarBytes));
    *out = static_cast<unsigned*>(v);
    return TENZO_SUCCESS;
}

void bar_give(int dev, unsigned* region) {
    if (!region) return;
    BarPool& bp = bar_pool();
    std::lock_guard<std::mutex> g(bp.mu);
    bp.free.emplace_back(dev, region);
}

int alloc_tracked(tenzo_engine_t e, void** p, size_t bytes, bool zero) {
    void* v = nullptr;
    TZ_HIP(hipMalloc(&v, bytes < 256 ? 256 : bytes));
    e->allocs.push_back(v);
    if (zero) TZ_HIP(hipMemset(v, 0, bytes < 256 ? 256 : bytes));
    *p = v;
    return TENZO_SUCCESS;
}

template <typename T>
int alloc_t(tenzo_engine_t e, T** p, size_t bytes, bool zero = false) {
    void* v = nullptr;
    int rc = alloc_tracked(e, &v, bytes, zero);
    *p = static_cast<T*>(v);
    return rc;
}

void drop_graphs(tenzo_engine_t e) {
    for (auto& kv : e->graphs) (void)hipGraphExecDestroy(kv.second);
    e->graphs.clear();
}

int upload_rope(tenzo_engine_t e) {
    std::vector<float> cs((size_t)e->max_seq * kD);
    tenzo_hip_rope_table(e->theta, kD, 0, e->max_seq, cs.data());
    TZ_HIP(hipMemcpy(e->rope, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    return TENZO_SUCCESS;
}

// Uploads `rows` TL1 rows [N/64][K/2][32] and repacks them into `dst` at row
// block offset `row0` (row0 % 64 == 0) of a matrix with K columns.
int upload_tl1(tenzo_engine_t e, const int8_t* host, int64_t N, int64_t K, void* dst,
               int64_t row0) {
    void* staging = nullptr;
    const size_t raw = (size_t)N * K / 4;
    TZ_HIP(hipMalloc(&staging, raw));
    int rc = TENZO_SUCCESS;
    if (hipMemcpy(staging, host, raw, hipMemcpyDefault) != hipSuccess) {
        set_error("set_layer_weights: copy to device failed");
        rc = TENZO_ERROR_OUT_OF_MEMORY;
    }
    if (!rc) {
        char* out = (char*)dst + (size_t)(row0 / 64) * ceil_div(K, 64) * 1024;
        rc = launch_tl1_repack((const uint8_t*)staging, out, N, K, e->st);
    }
    if (hipStreamSynchronize(e->st) != hipSuccess && !rc) rc = TENZO_ERROR_UNSUPPORTED;
    (void)hipFree(staging);
    return rc;
}

int upload_vec(tenzo_engine_t e, const float* host, int64_t n, float** dst) {
    if (!host) {
        *dst = nullptr;
        return TENZO_SUCCESS;
    }
    if (!*dst) {
        int rc = alloc_t(e, dst, (size_t)n * 4);
        if (rc) return rc;
    }
    TZ_HIP(hipMemcpy(*dst, host, (size_t)n * 4, hipMemcpyDefault));
    return TENZO_SUCCESS;
}

bool ready(tenzo_engine_t e, bool need_head) {
    for (int l = 0; l < e->L; ++l)
        if (!e->layers[l].set) {
            set_error("layer %d has no weights (tenzo_set_layer_weights)", l);
            return false;
        }
    if (need_head && e->head_kind == 0) {
        set_error("no LM head (tenzo_set_lm_head_i8 / _f32)");
        return false;
    }
    if (e->head_kind == 0) {
        set_error("no embedding table (the LM head is the tied embedding)");
        return false;
    }
    return true;
}

// Between chained steps: the greedy token becomes the next input, the
// position advances.
__global__ void chain_kernel(int32_t* io, int32_t* out) {
    if (threadIdx.x == 0) {
        const int t = io[2];
        io[0] = t;
        io[1] += 1;
        *out = t;
    }
}

__global__ void copy_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// Paged pools <-> the contiguous export layout [L][Hkv][seq][128] through the block
// table: export row (l*Hkv + h)*seq + t is pool row ((table[t/16]*L + l)*Hkv + h)*16 +
// t%16 (PagedKVCache's block layout, TenzoEngine.cpp:308-322). One thread per 16-byte
// piece of a K and a V row; the piece-0 thread also moves the row's two scales.
__global__ void kv_page_copy_kernel(int8_t* __restrict__ pk, int8_t* __restrict__ pv,
                                    float* __restrict__ pks, float* __restrict__ pvs,
                                    int8_t* __restrict__ xk, int8_t* __restrict__ xv,
                                    float* __restrict__ xks, float* __restrict__ xvs,
                                    const int32_t* __restrict__ table, int lh_rows, int seq,
                                    int to_pool) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)lh_rows * seq * 8) return;
    const int64_t r = i >> 3;
    const int piece = (int)(i & 7);
    const int t = (int)(r % seq);
    const int64_t lh = r / seq;
    const int64_t p = ((int64_t)table[t >> 4] * lh_rows + lh) * 16 + (t & 15);
    uint4* pk4 = (uint4*)(pk + p * kD) + piece;
    uint4* pv4 = (uint4*)(pv + p * kD) + piece;
    uint4* xk4 = (uint4*)(xk + r * kD) + piece;
    uint4* xv4 = (uint4*)(xv + r * kD) + piece;
    if (to_pool) {
        *pk4 = *xk4;
        *pv4 = *xv4;
        if (piece == 0) pks[p] = xks[r], pvs[p] = xvs[r];
    } else {
        *xk4 = *pk4;
        *xv4 = *pv4;
        if (piece == 0) xks[r] = pks[p], xvs[r] = pvs[p];
    }
}

// Moves seq_len tokens of every (layer, kv head) between the paged pools and the
// contiguous layout through one staging buffer: the four arrays in one copy each and
// one table-driven kernel, instead of four copies per 16-token block per row.
int pg_transfer(tenzo_engine_t e, int8_t* kc, int8_t* vc, float* ks, float* vs, int seq_len,
                hipMemcpyKind kind, bool to_pool) {
    const int lh = e->L * e->Hkv;
    const size_t rows = (size_t)lh * seq_len;
    void* stage = nullptr;
    if (hipMalloc(&stage, rows * (2 * kD + 8)) != hipSuccess) {
        set_error("paged KV transfer: cannot allocate %zu bytes of staging",
                  rows * (2 * kD + 8));
        return TENZO_ERROR_OUT_OF_MEMORY;
    }
    int8_t* xk = (int8_t*)stage;
    int8_t* xv = xk + rows * kD;
    float* xks = (float*)(xv + rows * kD);
    float* xvs = xks + rows;
    hipError_t err = hipSuccess;
    auto copy = [&](void* d, const void* s, size_t n) {
        if (err == hipSuccess) err = hipMemcpyAsync(d, s, n, kind, e->st);
    };
    if (to_pool) {
        copy(xk, kc, rows * kD), copy(xv, vc, rows * kD);
        copy(xks, ks, rows * 4), copy(xvs, vs, rows * 4);
    }
    if (err == hipSuccess) {
        hipLaunchKernelGGL(kv_page_copy_kernel, dim3((unsigned)ceil_div((int64_t)rows * 8, 256)),
                           dim3(256), 0, e->st, e->kc, e->vc, (float*)e->ks, (float*)e->vs, xk,
                           xv, xks, xvs, e->pg_bt, lh, seq_len, (int)to_pool);
        err = hipGetLastError();
    }
    if (!to_pool) {
        copy(kc, xk, rows * kD), copy(vc, xv, rows * kD);
        copy(ks, xks, rows * 4), copy(vs, xvs, rows * 4);
    }
    const hipError_t serr = hipStreamSynchronize(e->st);
    (void)hipFree(stage);
    if (err == hipSuccess) err = serr;
    if (err != hipSuccess) {
        set_error("paged KV transfer: %s", hipGetErrorString(err));
        return TENZO_ERROR_UNSUPPORTED;
    }
    return TENZO_SUCCESS;
}

// One layer (forward_layer_raw, TenzoEngine.cpp:1522-1632).
int enqueue_layer(tenzo_engine_t e, int l, int T, int max_chunks) {
    const DevLayer& w = e->layers[l];
    hipStream_t st = e->st;
    const int64_t KpH = ceil_div(e->H, 64) * 64;
    int rc;
    // 1-3: in-norm, activation quantization, fused Q|K|V
    if ((rc = launch_actquant(1, 31, e->x, w.norm[0], e->eps, 1, e->H, KpH, e->codes, e->aq,
                              nullptr, st)))
        return rc;
    RowScales rs{};
    rs.n = 3;
    rs.end[0] = e->qd;
    rs.end[1] = e->qd + e->kvd;
    rs.end[2] = INT64_MAX;
    rs.scale[0] = w.sc[0];
    rs.scale[1] = w.sc[1];
    rs.scale[2] = w.sc[2];
    if ((rc = launch_tl1_gemv(e->codes, e->aq, w.qkv, rs, 1, e->qd + 2 * e->kvd, e->H, e->qkv,
                              nullptr, nullptr, st, 0, e->gemv_ws)))
        return rc;
    // 4: RoPE, KV append at the device-held position, attention
    if (e->kv_kind == 3) {
        AttnPagedLaunch p{};
        p.q = e->qkv;
        p.k_new = e->qkv + e->qd;
        p.v_new = e->qkv + e->qd + e->kvd;
        p.pk = e->kc;
        p.pv = e->vc;
        p.pks = reinterpret_cast<float*>(e->ks);
        p.pvs = reinterpret_cast<float*>(e->vs);
        p.block_table = e->pg_bt;
        p.rope = e->rope;
        p.rope_indexed = 1;
        p.pos_dev = e->io_dev + 1;
        p.n_layers = e->L;
        p.layer = l;
        p.Hq = e->Hq;
        p.Hkv = e->Hkv;
        p.T = T;
        p.max_chunks = max_chunks;
        p.ws = e->pg_ws;
        p.out = e->attn;
        if ((rc = launch_attn_paged(p, st))) return rc;
    } else if (e->kv_kind != 0) {
        const size_t rows = (size_t)l * e->Hkv * e->max_seq;
        AttnTernLaunch t{};
        t.mode = e->kv_kind;
        t.q = e->qkv;
        t.k_new = e->qkv + e->qd;
        t.v_new = e->qkv + e->qd + e->kvd;
        t.kb = reinterpret_cast<uint8_t*>(e->kc) + rows * 32;
        t.vb = reinterpret_cast<uint8_t*>(e->vc) + rows * 32;
        t.ks = reinterpret_cast<float*>(e->ks) + rows;
        t.vs = reinterpret_cast<float*>(e->vs) + rows;
        t.rope = e->rope;
        t.rope_indexed = 1;
        t.pos_dev = e->io_dev + 1;
        t.Hq = e->Hq;
        t.Hkv = e->Hkv;
        t.max_seq = e->max_seq;
        t.T = T;
        t.max_chunks = max_chunks;
        t.out = e->attn;
        t.part = e->attn_part;
        if ((rc = launch_attn_tern(t, st))) return rc;
    } else {
        AttnLaunch a{};
        a.q = e->qkv;
        a.k_new = e->qkv + e->qd;
        a.v_new = e->qkv + e->qd + e->kvd;
        const size_t head_off = (size_t)l * e->Hkv * e->max_seq;
        a.kc = e->kc + head_off * kD;
        a.vc = e->vc + head_off * kD;
        a.ks = e->ks + head_off;
        a.vs = e->vs + head_off;
        a.rope = e->rope;
        a.rope_indexed = 1;
        a.pos_dev = e->io_dev + 1;
        a.B = 1;
        a.Hq = e->Hq;
        a.Hkv = e->Hkv;
        a.max_seq = e->max_seq;
        a.T = T;
        a.max_chunks = max_chunks;
        a.out = e->attn;
        a.part = e->attn_part;
        if ((rc = launch_attn(a, st))) return rc;
    }
    // 5-7: attn sub-norm, O projection, residual 1
    if ((rc = launch_actquant(1, 31, e->attn, w.norm[1], e->eps, 1, e->H, KpH, e->codes, e->aq,
                              nullptr, st)))
        return rc;
    if ((rc = launch_tl1_gemv(e->codes, e->aq, w.o, RowScales::single(w.sc[3]), 1, e->H, e->H,
                              e->h1, e->x, nullptr, st, 0, e->gemv_ws)))
        return rc;
    if (!w.mlp) {  // :1629-1631
        hipLaunchKernelGGL(copy_kernel, dim3((unsigned)ceil_div(e->H, 256)), dim3(256), 0, st,
                           e->h1, e->x, (int64_t)e->H);
        return launch_status("copy_kernel");
    }
    // 8: post-norm, fused gate|up, relu^2 * up, ffn sub-norm, down, residual 2
    if ((rc = launch_actquant(1, 31, e->h1, w.norm[2], e->eps, 1, e->H, KpH, e->codes, e->aq,
                              nullptr, st)))
        return rc;
    RowScales gs{};
    gs.n = 2;
    gs.end[0] = e->F;
    gs.end[1] = INT64_MAX;
    gs.scale[0] = w.sc[4];
    gs.scale[1] = w.sc[5];
    if ((rc = launch_tl1_gemv(e->codes, e->aq, w.gu, gs, 1, 2 * e->F, e->H, e->gu, nullptr,
                              nullptr, st, 0, e->gemv_ws)))
        return rc;
    const int64_t KpF = ceil_div(e->F, 64) * 64;
    if ((rc = launch_actquant(3, 31, e->gu, w.norm[3], e->eps, 1, e->F, KpF, e->codes, e->aq,
                              nullptr, st)))
        return rc;
    return launch_tl1_gemv(e->codes, e->aq, w.down, RowScales::single(w.sc[6]), 1, e->H, e->F,
                           e->x, e->h1, nullptr, st, 0, e->gemv_ws);
}

// compute_logits (:1634-1720) + the greedy branch of the sampler (:1745-1755).
int enqueue_head(tenzo_engine_t e) {
    hipStream_t st = e->st;
    ArgmaxWs am = argmax_ws_at(e->am_ws, e->V, e->io_dev + 2);
    int rc;
    if (e->head_kind == 1) {
        if ((rc = launch_actquant(1, 127, e->x, e->final_norm, e->eps, 1, e->H, e->H, e->codes,
                                  e->aq, nullptr, st)))
            return rc;
        return launch_lm_head_i8(e->codes, e->aq, e->head_i8, e->head_scales, e->logits, e->V,
                                 e->H, am, st);
    }
    if ((rc = launch_rmsnorm(e->x, e->final_norm, e->xn, e->H, e->eps, st))) return rc;
    if ((rc = launch_lm_head_f32(e->xn, e->head_f32, e->logits, e->V, e->H, st))) return rc;
    return launch_argmax(e->logits, e->V, am, st);
}

int enqueue_step(tenzo_engine_t e, bool head, int T, int max_chunks) {
    int rc = e->head_kind == 1
                 ? launch_embed_i8(e->head_i8, e->head_scales, e->io_dev, e->V, e->H, e->x, e->st)
                 : launch_embed_f32(e->head_f32, e->io_dev, e->V, e->H, e->x, e->st);
    if (rc) return rc;
    for (int l = 0; l < e->L; ++l)
        if ((rc = enqueue_layer(e, l, T, max_chunks))) return rc;
    return head ? enqueue_head(e) : TENZO_SUCCESS;
}

// ---- tenzo_load_model (load_model_from_files, TenzoEngine.cpp:1887-2078) ----

// weights.bin mapped read-only for the duration of a load.
struct MappedFile {
    const uint8_t* p = nullptr;
    size_t n = 0;
    int fd = -1;
    ~MappedFile() {
        if (p && n) munmap(const_cast<uint8_t*>(p), n);
        if (fd >= 0) close(fd);
    }
    bool open_ro(const char* path) {
        fd = ::open(path, O_RDONLY);
        if (fd < 0) return false;
        struct stat st {};
        if (fstat(fd, &st) != 0) return false;
        n = (size_t)st.st_size;
        if (n == 0) return true;
        void* m = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) return false;
        p = static_cast<const uint8_t*>(m);
        return true;
    }
};

// The next tensor's offset: the next memref view of the MLIR, else the
// running sequential offset (get_offset, :1991-2001); the running offset
// advances by the tensor's size either way.
struct OffsetCursor {
    const std::vector<uint64_t>& views;
    size_t v = 1;  // view 0 is the embedding table
    uint64_t seq;
    uint64_t next(uint64_t bytes) {
        const uint64_t off = v < views.size() ? views[v++] : seq;
        seq += bytes;
        return off;
    }
};

// A ternary projection of N rows x K columns from the raw [N/4][K] bytes at
// off into rows row0.. of a device matrix; past the end of the file the
// projection is all zeros (raw byte 0x55, as safe_pack_ternary's 0x55 TL1
// fill, :1975-1983).
int load_raw_projection(tenzo_engine_t e, const MappedFile& f, uint64_t off, int64_t N,
                        int64_t K, void* dst, int64_t row0, uint8_t* staging) {
    const size_t bytes = (size_t)N * (size_t)(K / 4);
    if (off + bytes <= f.n) {
        TZ_HIP(hipMemcpy(staging, f.p + off, bytes, hipMemcpyHostToDevice));
    } else {
        TZ_HIP(hipMemsetAsync(staging, 0x55, bytes, e->st));
    }
    char* out = (char*)dst + (size_t)(row0 / 64) * ceil_div(K, 64) * 1024;
    int rc = launch_tl1_repack_raw(staging, out, N, K, e->st);
    if (rc) return rc;
    TZ_HIP(hipStreamSynchronize(e->st));
    return TENZO_SUCCESS;
}

// An fp32 vector of n at off (norm weights); past the end of the file ones
// (safe_slice_f32, :1966-1973).
int load_vec(tenzo_engine_t e, const MappedFile& f, uint64_t off, int64_t n, float** dst) {
    std::vector<float> v((size_t)n, 1.0f);
    if (off + (uint64_t)n * 4 <= f.n) std::memcpy(v.data(), f.p + off, (size_t)n * 4);
    return upload_vec(e, v.data(), n, dst);
}

int load_model_files(tenzo_engine_t e, const char* weights_path, const char* mlir_path) {
    std::string text;
    {
        FILE* mf = std::fopen(mlir_path, "rb");
        if (!mf) {
            set_error("load_model: cannot open %s", mlir_path);
            return TENZO_ERROR_IO;
        }
        char buf[1 << 16];
        size_t got;
        while ((got = std::fread(buf, 1, sizeof(buf), mf)) > 0) text.append(buf, got);
        std::fclose(mf);
    }
    MappedFile f;
    if (!f.open_ro(weights_path)) {
        set_error("load_model: cannot open %s", weights_path);
        return TENZO_ERROR_IO;
    }
    const int64_t H = e->H, F = e->F, V = e->V, qd = e->qd, kvd = e->kvd;
    const uint64_t embed_bytes = (uint64_t)V * H * 4;
    if (f.n < embed_bytes) {  // the reference reads the table without a bound (:1913)
        set_error("load_model: %s holds %zu bytes, less than the %dx%d fp32 embedding table",
                  weights_path, f.n, (int)V, (int)H);
        return TENZO_ERROR_MODEL_PARSE;
    }
    ModelFileIndex ix;
    parse_model_mlir(text.data(), text.size(), &ix);

    // staging for the largest raw projection
    const size_t stage_bytes = (size_t)std::max({qd * (H / 4), kvd * (H / 4), H * (qd / 4),
                                                  F * (H / 4), H * (F / 4)});
    uint8_t* staging = nullptr;
    TZ_HIP(hipMalloc(&staging, stage_bytes));
    OffsetCursor oc{ix.views, 1, embed_bytes};
    size_t si = 0;
    auto scale = [&]() { return si < ix.scales.size() ? ix.scales[si++] : 1.0f; };  // :2003-2008
    const int64_t KSH = ceil_div(H, 64), KSF = ceil_div(F, 64), KSQ = ceil_div(qd, 64);
    int rc = TENZO_SUCCESS;
    for (int l = 0; l < e->L && !rc; ++l) {
        DevLayer& d = e->layers[l];
        if (!d.qkv) rc = alloc_tracked(e, &d.qkv, (size_t)((qd + 2 * kvd) / 64) * KSH * 1024, false);
        if (!rc && !d.o) rc = alloc_tracked(e, &d.o, (size_t)(H / 64) * KSQ * 1024, false);
        if (!rc && !d.gu) rc = alloc_tracked(e, &d.gu, (size_t)(2 * F / 64) * KSH * 1024, false);
        if (!rc && !d.down) rc = alloc_tracked(e, &d.down, (size_t)(H / 64) * KSF * 1024, false);
        if (rc) break;
        // the order of :2010-2070: in_norm, q, k, v, attn_sub_norm, out, post_norm, gate,
        // up, ffn_sub_norm, down
        if (!rc) rc = load_vec(e, f, oc.next(H * 4), H, &d.norm[0]);
        if (!rc) rc = load_raw_projection(e, f, oc.next(qd * (H / 4)), qd, H, d.qkv, 0, staging);
        d.sc[0] = scale();
        if (!rc) rc = load_raw_projection(e, f, oc.next(kvd * (H / 4)), kvd, H, d.qkv, qd, staging);
        d.sc[1] = scale();
        if (!rc)
            rc = load_raw_projection(e, f, oc.next(kvd * (H / 4)), kvd, H, d.qkv, qd + kvd,
                                     staging);
        d.sc[2] = scale();
        if (!rc) rc = load_vec(e, f, oc.next(H * 4), H, &d.norm[1]);
        if (!rc) rc = load_raw_projection(e, f, oc.next(H * (qd / 4)), H, qd, d.o, 0, staging);
        d.sc[3] = scale();
        if (!rc) rc = load_vec(e, f, oc.next(H * 4), H, &d.norm[2]);
        if (!rc) rc = load_raw_projection(e, f, oc.next(F * (H / 4)), F, H, d.gu, 0, staging);
        d.sc[4] = scale();
        if (!rc) rc = load_raw_projection(e, f, oc.next(F * (H / 4)), F, H, d.gu, F, staging);
        d.sc[5] = scale();
        if (!rc) rc = load_vec(e, f, oc.next(F * 4), F, &d.norm[3]);
        if (!rc) rc = load_raw_projection(e, f, oc.next(H * (F / 4)), H, F, d.down, 0, staging);
        d.sc[6] = scale();
        d.mlp = true;
        d.set = !rc;
    }
    (void)hipFree(staging);
    if (rc) return rc;
    // final norm: the next view, else the running offset (:2073-2075)
    const uint64_t foff = oc.v < ix.views.size() ? ix.views[oc.v] : oc.seq;
    if ((rc = load_vec(e, f, foff, H, &e->final_norm))) return rc;

    // int8 LM head / tied embedding from the fp32 table at offset 0 (:1925-1941),
    // quantized on the device in chunks of rows
    if (!e->head_i8 &&
        (rc = alloc_tracked(e, &e->head_i8, tenzo_hip_i8_packed_bytes(V, H), false)))
        return rc;
    if (!e->head_scales && (rc = alloc_t(e, &e->head_scales, (size_t)V * 4))) return rc;
    int8_t* codes = nullptr;
    float* rows = nullptr;
    const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(V, (256 << 20) / (H * 4)));
    bool ok = hipMalloc(&codes, (size_t)V * H) == hipSuccess &&
              hipMalloc(&rows, (size_t)chunk * H * 4) == hipSuccess;
    for (int64_t v0 = 0; ok && v0 < V; v0 += chunk) {
        const int64_t n = std::min(chunk, V - v0);
        ok = hipMemcpy(rows, f.p + (size_t)v0 * H * 4, (size_t)n * H * 4, hipMemcpyHostToDevice) ==
                 hipSuccess &&
             launch_quant_rows_i8(rows, n, H, codes + v0 * H, e->head_scales + v0, e->st) == 0 &&
             hipStreamSynchronize(e->st) == hipSuccess;
    }
    ok = ok && launch_i8_repack(codes, e->head_i8, V, H, e->st) == 0 &&
         hipStreamSynchronize(e->st) == hipSuccess;
    if (rows) (void)hipFree(rows);
    if (codes) (void)hipFree(codes);
    if (!ok) {
        set_error("load_model: uploading the LM head failed");
        return TENZO_ERROR_OUT_OF_MEMORY;
    }
    e->head_kind = 1;
    e->ds_layers_dirty = true;
    drop_graphs(e);
    return TENZO_SUCCESS;
}

// Tokens per batched-prefill pass: longer prompts go through in passes of
// this many rows (every activation buffer holds that many rows).
constexpr int kPrefillRows = 512;

int prefill_buffers(tenzo_engine_t e) {
    if (e->pf_cap) return TENZO_SUCCESS;
    const size_t R = kPrefillRows;
    const int64_t Kp = std::max(ceil_div(e->F, 64), ceil_div(e->H, 64)) * 64;
    int rc;
    if ((rc = alloc_t(e, &e->pf_x, R * e->H * 4)) || (rc = alloc_t(e, &e->pf_h1, R * e->H * 4)) ||
        (rc = alloc_t(e, &e->pf_qkv, R * (e->qd + 2 * e->kvd) * 4)) ||
        (rc = alloc_t(e, &e->pf_attn, R * e->qd * 4)) ||
        (rc = alloc_t(e, &e->pf_gu, R * 2 * e->F * 4)) ||
        (rc = alloc_t(e, &e->pf_codes, R * Kp, true)) ||
        (rc = alloc_t(e, &e->pf_aq, R * sizeof(tenzo_hip_actq_t))) ||
        (rc = alloc_t(e, &e->pf_tok, R * 4)))
        return rc;
    e->pf_cap = kPrefillRows;
    return TENZO_SUCCESS;
}

// One layer for the m prompt tokens at positions pos0 .. pos0+m-1 (the m
// forward_layer_raw calls of m prefill_token steps, TenzoEngine.cpp:1522-1632
// and :1809-1819): the same stages as enqueue_layer with M = m rows, the TL1
// contractions on int8 MFMA and the attention of every token over its own
// prefix.
int enqueue_prefill_layer(tenzo_engine_t e, int l, int pos0, int m, bool exact) {
    const DevLayer& w = e->layers[l];
    hipStream_t st = e->st;
    const int64_t KpH = ceil_div(e->H, 64) * 64;
    const int64_t nqkv = e->qd + 2 * e->kvd;
    int rc;
    if ((rc = launch_actquant(1, 31, e->pf_x, w.norm[0], e->eps, m, e->H, KpH, e->pf_codes,
                              e->pf_aq, nullptr, st)))
        return rc;
    RowScales rs{};
    rs.n = 3;
    rs.end[0] = e->qd;
    rs.end[1] = e->qd + e->kvd;
    rs.end[2] = INT64_MAX;
    rs.scale[0] = w.sc[0];
    rs.scale[1] = w.sc[1];
    rs.scale[2] = w.sc[2];
    if ((rc = launch_tl1_mfma(e->pf_codes, e->pf_aq, w.qkv, rs, m, nqkv, e->H, e->pf_qkv,
                              nullptr, nullptr, st, 0)))
        return rc;
    AttnPrefill a{};
    a.q = e->pf_qkv;
    a.k_new = e->pf_qkv + e->qd;
    a.v_new = e->pf_qkv + e->qd + e->kvd;
    a.row_stride = nqkv;
    const size_t head_off = (size_t)l * e->Hkv * e->max_seq;
    a.kc = e->kc + head_off * kD;
    a.vc = e->vc + head_off * kD;
    a.ks = e->ks + head_off;
    a.vs = e->vs + head_off;
    a.rope = e->rope;
    a.pos0 = pos0;
    a.n = m;
    a.Hq = e->Hq;
    a.Hkv = e->Hkv;
    a.max_seq = e->max_seq;
    a.out = e->pf_attn;
    a.out_stride = e->qd;
    a.exact = exact ? 1 : 0;
    if ((rc = launch_attn_prefill(a, st))) return rc;
    if ((rc = launch_actquant(1, 31, e->pf_attn, w.norm[1], e->eps, m, e->H, KpH, e->pf_codes,
                              e->pf_aq, nullptr, st)))
        return rc;
    if ((rc = launch_tl1_mfma(e->pf_codes, e->pf_aq, w.o, RowScales::single(w.sc[3]), m, e->H,
                              e->H, e->pf_h1, e->pf_x, nullptr, st, 0)))
        return rc;
    if (!w.mlp) {  // :1629-1631
        const int64_t n = (int64_t)m * e->H;
        hipLaunchKernelGGL(copy_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st,
                           e->pf_h1, e->pf_x, n);
        return launch_status("copy_kernel");
    }
    if ((rc = launch_actquant(1, 31, e->pf_h1, w.norm[2], e->eps, m, e->H, KpH, e->pf_codes,
                              e->pf_aq, nullptr, st)))
        return rc;
    RowScales gs{};
    gs.n = 2;
    gs.end[0] = e->F;
    gs.end[1] = INT64_MAX;
    gs.scale[0] = w.sc[4];
    gs.scale[1] = w.sc[5];
    if ((rc = launch_tl1_mfma(e->pf_codes, e->pf_aq, w.gu, gs, m, 2 * e->F, e->H, e->pf_gu,
                              nullptr, nullptr, st, 0)))
        return rc;
    const int64_t KpF = ceil_div(e->F, 64) * 64;
    if ((rc = launch_actquant(3, 31, e->pf_gu, w.norm[3], e->eps, m, e->F, KpF, e->pf_codes,
                              e->pf_aq, nullptr, st)))
        return rc;
    return launch_tl1_mfma(e->pf_codes, e->pf_aq, w.down, RowScales::single(w.sc[6]), m, e->H,
                           e->F, e->pf_x, e->pf_h1, nullptr, st, 0);
}

// n prompt tokens from position seq_len on, in passes of kPrefillRows; the
// engine's x ends as the last token's hidden state, as after n prefill_token
// calls (bit for bit when exact, else up to the streaming attention's
// softmax rounding).
int run_step(tenzo_engine_t e, int token, bool head);
int run_step_sync(tenzo_engine_t e, int token, bool head);

// PagedBlockManager::reset (TenzoEngine.h:127-133) and the table's reset.
void pg_reset(tenzo_engine_t e) {
    e->pg_free.clear();
    for (int i = e->pg_blocks - 1; i >= 0; --i) e->pg_free.push_back(i);
    e->pg_table.clear();
}

// Blocks for the first n tokens, allocated as PagedKVCache does on reaching a
// new block (:318-324: the last free block); the new entries are copied to
// the device table before anything reads them.
int pg_ensure(tenzo_engine_t e, int n) {
    const size_t had = e->pg_table.size();
    while ((int)e->pg_table.size() * 16 < n) {
        if (e->pg_free.empty()) {
            set_error("paged KV: no free block for %d tokens", n);
            return TENZO_ERROR_OUT_OF_MEMORY;
        }
        e->pg_table.push_back(e->pg_free.back());
        e->pg_free.pop_back();
    }
    if (e->pg_table.size() > had) {
        TZ_HIP(hipMemcpyAsync(e->pg_bt + had, e->pg_table.data() + had,
                              (e->pg_table.size() - had) * 4, hipMemcpyHostToDevice, e->st));
        TZ_HIP(hipStreamSynchronize(e->st));
    }
    return TENZO_SUCCESS;
}

int run_prefill(tenzo_engine_t e, const int32_t* tokens, int n, bool exact) {
    if (!ready(e, false)) return TENZO_ERROR_INVALID_ARGUMENT;
    if (n <= 0 || !tokens) {
        set_error("prefill: need n > 0 tokens (n=%d)", n);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= e->V) {
            set_error("token %d outside [0, %d)", tokens[i], e->V);
            return TENZO_ERROR_INVALID_ARGUMENT;
        }
    if ((int64_t)e->seq_len + n > e->max_seq) {
        set_error("KV cache full (%d + %d positions > %d)", e->seq_len, n, e->max_seq);
        return TENZO_ERROR_OUT_OF_MEMORY;
    }
    TZ_HIP(hipSetDevice(e->dev));
    int rc;
    if (e->kv_kind != 0) {
        // the batched pass appends INT8 rows; a ternary cache is filled by
        // decode steps without the LM head (tenzo_prefill_token per token)
        for (int i = 0; i < n; ++i) {
            if ((rc = run_step_sync(e, tokens[i], false))) return rc;
            e->seq_len += 1;
        }
        return TENZO_SUCCESS;
    }
    if ((rc = prefill_buffers(e))) return rc;
    int m = 0;
    for (int i0 = 0; i0 < n; i0 += m) {
        m = std::min(e->pf_cap, n - i0);
        TZ_HIP(hipMemcpyAsync(e->pf_tok, tokens + i0, (size_t)m * 4, hipMemcpyHostToDevice, e->st));
        rc = e->head_kind == 1 ? launch_embed_i8(e->head_i8, e->head_scales, e->pf_tok, e->V, e->H,
                                                 e->pf_x, e->st, m)
                               : launch_embed_f32(e->head_f32, e->pf_tok, e->V, e->H, e->pf_x,
                                                  e->st, m);
        if (rc) return rc;
        for (int l = 0; l < e->L; ++l)
            if ((rc = enqueue_prefill_layer(e, l, e->seq_len, m, exact))) return rc;
        // the copy of the tokens and the next pass's buffers are reused
        TZ_HIP(hipStreamSynchronize(e->st));
        e->seq_len += m;
    }
    TZ_HIP(hipMemcpyAsync(e->x, e->pf_x + (int64_t)(m - 1) * e->H, (size_t)e->H * 4,
                          hipMemcpyDeviceToDevice, e->st));
    TZ_HIP(hipStreamSynchronize(e->st));
    return TENZO_SUCCESS;
}

// Whether the persistent kernel can run this model as loaded.
bool ds_usable(tenzo_engine_t e) {
    if (e->ds_nwg <= 0 || e->kv_kind < 0 || e->kv_kind > 3 || e->head_kind != 1 ||
        e->H > 8192 || e->F > 8192 || e->H % 64 || e->F % 64 || e->L > kDsMaxLayers ||
        e->max_seq > ds_max_context(e->Hq / e->Hkv))
        return false;
    if (e->kv_kind == 3) {
        // paged: the block table in LDS, every attention chunk task resident
        // (chunks of at most kDsMaxChunk tokens, ds_chunk_budget of them per
        // kv head), the pools addressable with 32-bit offsets
        if (e->max_seq > kDsMaxBlocks * 16 ||
            e->max_seq > kDsMaxChunk * ds_chunk_budget(e->ds_nwg, e->Hkv) ||
            (size_t)e->pg_blocks * 16 * e->L * e->Hkv * kD >= (1ull << 32))
            return false;
    }
    for (const DevLayer& d : e->layers)
        if (!d.mlp) return false;
    return true;
}

int ds_sync_layers(tenzo_engine_t e) {
    if (!e->ds_layers_dirty) return TENZO_SUCCESS;
    std::vector<DsLayer> h(e->L);
    for (int l = 0; l < e->L; ++l) {
        const DevLayer& d = e->layers[l];
        h[l].mat[0] = (const uint4*)d.qkv;
        h[l].mat[1] = (const uint4*)d.o;
        h[l].mat[2] = (const uint4*)d.gu;
        h[l].mat[3] = (const uint4*)d.down;
        for (int i = 0; i < 4; ++i) h[l].norm[i] = d.norm[i];
        for (int i = 0; i < 7; ++i) h[l].sc[i] = d.sc[i];
    }
    TZ_HIP(hipMemcpy(e->ds_layers, h.data(), h.size() * sizeof(DsLayer), hipMemcpyHostToDevice));
    e->ds_layers_dirty = false;
    return TENZO_SUCCESS;
}

int run_persistent(tenzo_engine_t e, bool head, int pos, int32_t* out_tokens = nullptr,
                   int step = 0) {
    int rc = ds_sync_layers(e);
    if (rc) return rc;
    DsParams p{};
    p.layers = e->ds_layers;
    p.final_norm = e->final_norm;
    p.head = (const uint4*)e->head_i8;
    p.head_scales = e->head_scales;
    p.rope = e->rope;
    p.kc = e->kc;
    p.vc = e->vc;
    p.kv_mode = e->kv_kind;
    if (e->kv_kind != 0) {  // fp32 scales (paged pools or ternary rows)
        p.block_table = e->kv_kind == 3 ? e->pg_bt : nullptr;
        p.pks = (float*)e->ks;
        p.pvs = (float*)e->vs;
    } else {
        p.ks = (uint16_t*)e->ks;
        p.vs = (uint16_t*)e->vs;
    }
    p.x = e->x;
    p.qkv = e->qkv;
    p.attn = e->attn;
    p.h1 = e->h1;
    p.gu = e->gu;
    p.logits = e->logits;
    p.part = e->ds_part;
    p.am_part = e->ds_am;
    p.sync = e->ds_sync;
    p.acc = reinterpret_cast<int*>(e->ds_sync + ds_sync_words(e->L, e->Hkv));
    p.xs = e->ds_vec;
    p.h1s = p.xs + (size_t)e->L * e->H;
    p.attns = p.h1s + (size_t)e->L * e->H;
    p.io = e->io_dev;
    p.H = e->H;
    p.F = e->F;
    p.Hq = e->Hq;
    p.Hkv = e->Hkv;
    p.L = e->L;
    p.V = e->V;
    p.max_seq = e->max_seq;
    p.pos = pos;
    ds_chunking(pos + 1, e->Hkv, e->ds_nwg, &p.C, &p.T);
    p.nwg = e->ds_nwg;
    ds_plan_splits(p);
    p.with_head = head ? 1 : 0;
    p.eps = e->eps;
    p.trace = e->ds_trace;
    p.spin_limit = e->ds_coop ? e->ds_spin_coop : e->ds_spin;
    p.out_tokens = out_tokens;
    p.step = step;
    // barrier targets stay below 2^31: (base + barriers) * workgroups per counter
    const uint64_t per = (uint64_t)(e->ds_nwg / kDsCounters);
    if (e->ds_bar_reset || ((uint64_t)e->ds_bar_base + ds_barriers(e->L)) * per >= (1ull << 31)) {
        TZ_HIP(hipMemsetAsync(e->ds_bar, 0, (size_t)kDsBarWords * 4, e->st));
        e->ds_bar_base = 0;
        e->ds_bar_reset = false;
    }
    p.bar = e->ds_bar;
    p.bar_base = e->ds_bar_base;
    TZ_HIP(hipMemsetAsync(e->ds_sync, 0, e->ds_sync_bytes, e->st));
    rc = launch_decode_step(p, e->Hq / e->Hkv, e->ds_coop, e->st);
    e->ds_state_valid = rc == TENZO_SUCCESS;
    if (rc == TENZO_SUCCESS) e->ds_bar_base += ds_barriers(e->L);
    return rc;
}

// After persistent steps: the kernel's abort flag (io[3], set when a wait
// timed out and a step was abandoned; cleared by the host before the steps),
// copied next to the result token. An abort under an ordinary launch can mean
// that the grid was not all resident (other work on the device). An aborted
// step leaves nothing behind that a rerun does not rewrite: the sequence
// length is advanced by the host only after a good step, the step's KV rows
// at its position are appended again, its input token (io[0]) is written only
// by a step that completed, and the sync area and accumulators are cleared
// before every launch. So ds_retry, called after such an abort, moves the
// engine to the cooperative launch (all workgroups resident, guaranteed) and
// says whether the caller should rerun the step(s) once; ds_check then reports
// an abort that remains.
bool ds_retry(tenzo_engine_t e) {
    if (e->io_host[3] != 0) e->ds_bar_reset = true;  // the counters stopped part-way
    if (e->io_host[3] == 0 || e->ds_coop) return false;
    e->ds_coop = true;
    e->io_host[3] = 0;
    return true;
}

int ds_check(tenzo_engine_t e) {
    if (e->io_host[3] != 0) {
        e->ds_state_valid = false;
        e->ds_bar_reset = true;
        set_error("decode step aborted: an in-kernel wait timed out under the cooperative "
                  "launch (engine state is invalid: reset or re-prefill)");
        return TENZO_ERROR_UNSUPPORTED;
    }
    return TENZO_SUCCESS;
}

// Runs one token through the layers (and the head) at position seq_len.
int run_step(tenzo_engine_t e, int token, bool head) {
    if (!ready(e, head)) return TENZO_ERROR_INVALID_ARGUMENT;
    if (token < 0 || token >= e->V) {
        set_error("token %d outside [0, %d)", token, e->V);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    if (e->seq_len >= e->max_seq) {
        set_error("KV cache full (%d positions)", e->max_seq);
        return TENZO_ERROR_OUT_OF_MEMORY;
    }
    TZ_HIP(hipSetDevice(e->dev));
    const int pos = e->seq_len;
    const int T = attn_pick_chunk(pos + 1, e->Hkv, 1);
    if (e->kv_kind == 3) {
        const int prc = pg_ensure(e, pos + 1);
        if (prc) return prc;
    }
    e->io_host[0] = token;
    e->io_host[1] = pos;
    e->io_host[2] = 0;
    e->io_host[3] = 0;  // the abort flag
    TZ_HIP(hipMemcpyAsync(e->io_dev, e->io_host, 16, hipMemcpyHostToDevice, e->st));
    int rc;
    e->ds_state_valid = false;
    bool graph = e->mode == 1;
    if (e->mode == 2 && ds_usable(e)) {
        rc = run_persistent(e, head, pos);
        if (rc == kDsCoopRefused) {
            graph = true;  // this step on the stage kernels instead
        } else {
            if (rc) return rc;
            TZ_HIP(hipMemcpyAsync(e->io_host + 3, e->io_dev + 3, 4, hipMemcpyDeviceToHost,
                                  e->st));
        }
    } else if (e->mode >= 1) {
        graph = true;
    }
    if (graph) {
        const int max_chunks = (int)ceil_div(e->max_seq, T);
        auto key = std::make_pair(T, head ? 1 : 0);
        auto it = e->graphs.find(key);
        if (it == e->graphs.end()) {
            hipGraph_t g = nullptr;
            TZ_HIP(hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal));
            rc = enqueue_step(e, head, T, max_chunks);
            hipError_t ce = hipStreamEndCapture(e->st, &g);
            if (rc) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            if (ce != hipSuccess) return hip_fail(ce, "hipStreamEndCapture");
            hipGraphExec_t ex = nullptr;
            hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ie != hipSuccess) return hip_fail(ie, "hipGraphInstantiate");
            it = e->graphs.emplace(key, ex).first;
        }
        TZ_HIP(hipGraphLaunch(it->second, e->st));
    } else if (e->mode == 0) {
        if ((rc = enqueue_step(e, head, T, (int)ceil_div(pos + 1, T)))) return rc;
    }
    return TENZO_SUCCESS;
}

// run_step, synchronized, rerun once under the cooperative launch when the
// persistent kernel aborted under an ordinary one (ds_retry).
int run_step_sync(tenzo_engine_t e, int token, bool head) {
    for (int attempt = 0;; ++attempt) {
        int rc = run_step(e, token, head);
        if (rc) return rc;
        TZ_HIP(hipStreamSynchronize(e->st));
        if (attempt > 0 || !ds_retry(e)) break;
    }
    return ds_check(e);
}

}  // namespace

extern "C" {

TENZO_API const char* tenzo_get_version(void) { return TENZO_VERSION_STRING; }

TENZO_API tenzo_config_t tenzo_default_config(void) {
    // TenzoEngine.cpp:2092-2105
    tenzo_config_t c;
    c.hidden_size = 2560;
    c.num_q_heads = 20;
    c.num_kv_heads = 5;
    c.head_dim = 128;
    c.num_layers = 30;
    c.ffn_dim = 6912;
    c.vocab_size = 128256;
    c.max_seq_len = 8192;
    c.kv_mode = "int8_fused";
    c.device = "rocm";
    return c;
}

TENZO_API tenzo_sampling_params_t tenzo_default_sampling_params(void) {
    // TenzoEngine.cpp:2107-2114
    tenzo_sampling_params_t p;
    p.temperature = 0.7f;
    p.top_p = 0.9f;
    p.top_k = 40;
    p.repetition_penalty = 1.15f;
    return p;
}

TENZO_API void tenzo_destroy_engine(tenzo_engine_t e);

TENZO_API tenzo_engine_t tenzo_create_engine(const tenzo_config_t* config) {
    tenzo_config_t c = config ? *config : tenzo_default_config();
    const std::string kv = c.kv_mode ? c.kv_mode : "int8_fused";
    const int kv_kind = kv == "int8_fused" ? 0 : kv == "tl1_fused" ? 1 : kv == "popcount_fused" ? 2
                        : kv == "paged_int8" ? 3 : -1;
    if (kv_kind < 0) {
        set_error("kv_mode \"%s\" is not provided on the GPU (int8_fused, tl1_fused, "
                  "popcount_fused, paged_int8)", kv.c_str());
        return nullptr;
    }
    const int H = c.hidden_size, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    if (c.head_dim != kD || H <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv ||
        (Hq / Hkv != 1 && Hq / Hkv != 2 && Hq / Hkv != 4 && Hq / Hkv != 8) || Hq * kD != H ||
        H % 64 || c.ffn_dim <= 0 || c.ffn_dim % 64 || c.num_layers <= 0 || c.vocab_size <= 0 ||
        c.max_seq_len <= 0) {
        set_error("unsupported config: need head_dim 128, hidden = q_heads*128, hidden and "
                  "ffn multiples of 64, q_heads/kv_heads in {1,2,4,8}");
        return nullptr;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        set_error("no HIP device");
        return nullptr;
    }
    auto* e = new tenzo_engine_opaque();
    e->cfg = c;
    // a smaller in-kernel poll budget (tests force the abort path with it)
    auto spin_env = [](const char* name, unsigned* out) {
        if (const char* sl = std::getenv(name)) {
            char* end = nullptr;
            const unsigned long v = std::strtoul(sl, &end, 10);
            if (end != sl && v <= kDsSpinLimit) *out = (unsigned)v;
        }
    };
    spin_env("TENZO_HIP_SPIN_LIMIT", &e->ds_spin);
    spin_env("TENZO_HIP_SPIN_LIMIT_COOP", &e->ds_spin_coop);
    e->kv_mode = kv;
    e->kv_kind = kv_kind;
    e->kv_row = kv_kind == 0 || kv_kind == 3 ? kD : 32;
    e->kv_sb = kv_kind == 0 ? 2 : 4;
    e->device = c.device ? c.device : "rocm";
    e->cfg.kv_mode = e->kv_mode.c_str();
    e->cfg.device = e->device.c_str();
    e->H = H;
    e->Hq = Hq;
    e->Hkv = Hkv;
    e->L = c.num_layers;
    e->F = c.ffn_dim;
    e->V = c.vocab_size;
    e->max_seq = c.max_seq_len;
    e->qd = Hq * kD;
    e->kvd = Hkv * kD;
    e->layers.resize(e->L);
    bool ok = hipGetDevice(&e->dev) == hipSuccess && hipStreamCreate(&e->st) == hipSuccess;
    // paged_int8: the reference sizes its pool at ceil(max_seq / 16) blocks (:1218)
    e->pg_blocks = kv_kind == 3 ? (int)ceil_div(e->max_seq, 16) : 0;
    const size_t cache = (size_t)e->L * Hkv * (kv_kind == 3 ? (size_t)e->pg_blocks * 16 : e->max_seq);
    const int Tmin = 32;
    const size_t parts = (size_t)Hq * ceil_div(e->max_seq, Tmin) * kPartStride * 4;
    const int64_t Fp = ceil_div(e->F, 64) * 64;
    const size_t ws = tl1_ws_bytes(1, 2 * e->F > e->qd + 2 * e->kvd ? 2 * e->F
                                                                    : e->qd + 2 * e->kvd);
    const size_t row = (size_t)e->kv_row, sb = (size_t)e->kv_sb;
    ok = ok && !alloc_t(e, &e->kc, cache * row, true) && !alloc_t(e, &e->vc, cache * row, true) &&
         !alloc_t(e, &e->ks, cache * sb, true) && !alloc_t(e, &e->vs, cache * sb, true) &&
         !alloc_t(e, &e->x, (size_t)H * 4) && !alloc_t(e, &e->qkv, (size_t)(e->qd + 2 * e->kvd) * 4) &&
         !alloc_t(e, &e->attn, (size_t)e->qd * 4) && !alloc_t(e, &e->h1, (size_t)H * 4) &&
         !alloc_t(e, &e->gu, (size_t)2 * e->F * 4) && !alloc_t(e, &e->xn, (size_t)H * 4) &&
         !alloc_t(e, &e->logits, (size_t)e->V * 4) &&
         !alloc_t(e, &e->codes, (size_t)(Fp > H ? Fp : ceil_div(H, 64) * 64), true) &&
         !alloc_t(e, &e->aq, 256) && !alloc_t(e, &e->gemv_ws, ws, true) &&
         !alloc_t(e, &e->attn_part, parts) &&
         !alloc_t(e, &e->am_ws, argmax_ws_bytes(e->V), true) &&
         !alloc_t(e, &e->sample_ws, sample_ws_bytes(e->V)) &&
         !alloc_t(e, &e->io_dev, 256, true) &&
         !alloc_t(e, &e->rope, (size_t)e->max_seq * kD * 4);
    if (ok && kv_kind == 3) {
        const int mc = (int)ceil_div(e->max_seq, 32);
        ok = !alloc_t(e, &e->pg_bt, (size_t)e->pg_blocks * 4, true) &&
             !alloc_t(e, &e->pg_ws, (size_t)Hq * ((size_t)e->max_seq + 256 + (size_t)mc * (kD + 1)) * 4);
        pg_reset(e);
    }
    if (ok) {
        void* h = nullptr;
        ok = hipHostMalloc(&h, 256, hipHostMallocDefault) == hipSuccess;
        e->io_host = static_cast<int32_t*>(h);
    }
    ok = ok && !upload_rope(e);
    if (ok) {
        e->ds_nwg = ds_grid_size();
        if (e->ds_nwg > 0) {
            const int G = Hq / Hkv;
            int cmax = ds_chunk_budget(e->ds_nwg, Hkv);
            const int cseq = (int)ceil_div(e->max_seq, kDsMaxChunk);
            if (cseq > cmax) cmax = cseq;
            if (cmax < 1) cmax = 1;
            e->ds_sync_bytes =
                (ds_sync_words(e->L, Hkv) + ds_acc_words(e->L, e->H, e->F, Hq, Hkv)) * 4;
            ok = !alloc_t(e, &e->ds_layers, sizeof(DsLayer) * e->L) &&
                 !alloc_t(e, &e->ds_sync, e->ds_sync_bytes, true) &&
                 !alloc_t(e, &e->ds_vec, ds_vec_floats(e->L, e->H, Hq) * 4) &&
                 !alloc_t(e, &e->ds_part, (size_t)Hkv * cmax * G * kDsPartStride * 4) &&
                 !alloc_t(e, &e->ds_am, (size_t)e->ds_nwg * sizeof(float2)) &&
                 !bar_take(e->dev, &e->ds_bar);
        }
    }
    if (!ok) {
        tenzo_destroy_engine(e);
        return nullptr;
    }
    return e;
}

TENZO_API void tenzo_destroy_engine(tenzo_engine_t e) {
    if (!e) return;
    (void)hipSetDevice(e->dev);
    if (e->st) (void)hipStreamSynchronize(e->st);
    drop_graphs(e);
    for (void* p : e->allocs) (void)hipFree(p);
    bar_give(e->dev, e->ds_bar);
    if (e->ds_trace) (void)hipFree(e->ds_trace);
    if (e->dec_out) (void)hipFree(e->dec_out);
    if (e->io_host) (void)hipHostFree(e->io_host);
    if (e->st) (void)hipStreamDestroy(e->st);
    delete e;
}

TENZO_API void tenzo_reset(tenzo_engine_t e) {
    // TenzoEngine.cpp:1249-1255 / :213-215: only the sequence length
    if (e) {
        e->seq_len = 0;
        if (e->kv_kind == 3) pg_reset(e);  // PagedKVCache::reset (:246-250)
    }
}

TENZO_API int tenzo_get_seq_len(tenzo_engine_t e) { return e ? e->seq_len : 0; }

TENZO_API tenzo_status_t tenzo_set_layer_weights(tenzo_engine_t e, int l,
                                                 const tenzo_layer_weights_t* w) {
    if (!e || !w) return TENZO_ERROR_INVALID_ARGUMENT;
    if (l < 0 || l >= e->L) return TENZO_SUCCESS;  // ignored, as TenzoEngine.cpp:1258
    if (!w->q_w || !w->k_w || !w->v_w || !w->out_w) {
        set_error("set_layer_weights: q/k/v/out weights are required");
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    if (hipSetDevice(e->dev) != hipSuccess) return TENZO_ERROR_UNSUPPORTED;
    DevLayer& d = e->layers[l];
    const int64_t H = e->H, F = e->F, qd = e->qd, kvd = e->kvd;
    const int64_t KSH = ceil_div(H, 64), KSF = ceil_div(F, 64);
    int rc = TENZO_SUCCESS;
    if (!d.qkv) rc = alloc_tracked(e, &d.qkv, (size_t)((qd + 2 * kvd) / 64) * KSH * 1024, false);
    if (!rc && !d.o) rc = alloc_tracked(e, &d.o, (size_t)(H / 64) * KSH * 1024, false);
    if (!rc) rc = upload_tl1(e, w->q_w, qd, H, d.qkv, 0);
    if (!rc) rc = upload_tl1(e, w->k_w, kvd, H, d.qkv, qd);
    if (!rc) rc = upload_tl1(e, w->v_w, kvd, H, d.qkv, qd + kvd);
    if (!rc) rc = upload_tl1(e, w->out_w, H, H, d.o, 0);
    d.mlp = w->gate_w && w->up_w && w->down_w;
    if (!rc && d.mlp) {
        if (!d.gu) rc = alloc_tracked(e, &d.gu, (size_t)(2 * F / 64) * KSH * 1024, false);
        if (!rc && !d.down) rc = alloc_tracked(e, &d.down, (size_t)(H / 64) * KSF * 1024, false);
        if (!rc) rc = upload_tl1(e, w->gate_w, F, H, d.gu, 0);
        if (!rc) rc = upload_tl1(e, w->up_w, F, H, d.gu, F);
        if (!rc) rc = upload_tl1(e, w->down_w, H, F, d.down, 0);
    }
    const float* nv[4] = {w->in_norm, w->attn_sub_norm, w->post_norm, w->ffn_sub_norm};
    const int64_t nd[4] = {H, H, H, F};
    for (int i = 0; i < 4 && !rc; ++i) rc = upload_vec(e, nv[i], nd[i], &d.norm[i]);
    if (rc) return (tenzo_status_t)rc;
    const float sc[7] = {w->q_scale, w->k_scale, w->v_scale, w->out_scale,
                         w->gate_scale, w->up_scale, w->down_scale};
    std::memcpy(d.sc, sc, sizeof(sc));
    d.set = true;
    e->ds_layers_dirty = true;
    drop_graphs(e);  // scales are captured in the graph's kernel arguments
    return TENZO_SUCCESS;
}

TENZO_API tenzo_status_t tenzo_set_final_norm(tenzo_engine_t e, const float* norm_w) {
    if (!e || !norm_w) return TENZO_ERROR_INVALID_ARGUMENT;
    if (hipSetDevice(e->dev) != hipSuccess) return TENZO_ERROR_UNSUPPORTED;
    float* before = e->final_norm;
    int rc = upload_vec(e, norm_w, e->H, &e->final_norm);
    if (before != e->final_norm) drop_graphs(e);
    return (tenzo_status_t)rc;
}

TENZO_API tenzo_status_t tenzo_set_lm_head_i8(tenzo_engine_t e, const int8_t* w,
                                              const float* scales, int vocab, int hidden) {
    if (!e || !w || !scales) return TENZO_ERROR_INVALID_ARGUMENT;
    if (vocab != e->V || hidden != e->H) {
        set_error("set_lm_head_i8: table %dx%d does not match the config %dx%d", vocab, hidden,
                  e->V, e->H);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    if (hipSetDevice(e->dev) != hipSuccess) return TENZO_ERROR_UNSUPPORTED;
    int rc = TENZO_SUCCESS;
    if (!e->head_i8)
        rc = alloc_tracked(e, &e->head_i8, tenzo_hip_i8_packed_bytes(e->V, e->H), false);
    if (!rc && !e->head_scales) rc = alloc_t(e, &e->head_scales, (size_t)e->V * 4);
    if (rc) return (tenzo_status_t)rc;
    void* staging = nullptr;
    const size_t bytes = (size_t)e->V * e->H;
    if (hipMalloc(&staging, bytes) != hipSuccess) return TENZO_ERROR_OUT_OF_MEMORY;
    bool ok = hipMemcpy(staging, w, bytes, hipMemcpyDefault) == hipSuccess &&
              launch_i8_repack((const int8_t*)staging, e->head_i8, e->V, e->H, e->st) == 0 &&
              hipStreamSynchronize(e->st) == hipSuccess &&
              hipMemcpy(e->head_scales, scales, (size_t)e->V * 4, hipMemcpyDefault) ==
                  hipSuccess;
    (void)hipFree(staging);
    if (!ok) return TENZO_ERROR_OUT_OF_MEMORY;
    e->head_kind = 1;
    drop_graphs(e);
    return TENZO_SUCCESS;
}

TENZO_API tenzo_status_t tenzo_set_lm_head_f32(tenzo_engine_t e, const float* w, int vocab,
                                               int hidden) {
    if (!e || !w) return TENZO_ERROR_INVALID_ARGUMENT;
    if (vocab != e->V || hidden != e->H) {
        set_error("set_lm_head_f32: table %dx%d does not match the config %dx%d", vocab, hidden,
                  e->V, e->H);
        return TENZO_ERROR_INVALID_ARGUMENT;
    }
    if (hipSetDevice(e->dev) != hipSuccess) return TENZO_ERROR_UNSUPPORTED;
    int rc = TENZO_SUCCESS;
    if (!e->head_f32) rc = alloc_t(e, &e->head_f32, (size_t)e->V * e->H * 4);
    if (rc) return (tenzo_status_t)rc;
    if (hipMemcpy(e->head_f32, w, (size_t)e->V * e->H * 4, hipMemcpyDefault) != hipSuccess)
        return TENZO_ERROR_OUT_OF_MEMORY;
    e->head_kind = 2;
    drop_graphs(e);
    return TENZO_SUCCESS;
}

TENZO_API tenzo_status_t tenzo_load_model(tenzo_engine_t e, const char* weights_path,
                                          const char* mlir_path) {
    if (!e || !weights_path || !mlir_path) return TENZO_ERROR_INVALID_ARGUMENT;
    if (hipSetDevice(e->dev) != hipSuccess) return TENZO_ERROR_UNSUPPORTED;
    return (tenzo_status_t)load_model_files(e, weights_path, mlir_path);
}

TENZO_API tenzo_status_t tenzo_prefill_token(tenzo_engine_t e, int token) {
    if (!e) return TENZO_ERROR_INVALID_ARGUMENT;
    const int rc = run_step_sync(e, token, false);
    if (rc) return (tenzo_status_t)rc;
    e->seq_len += 1;  // :1816-1818
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_prefill(tenzo_engine_t e, const int32_t* tokens, int n,
                                           int exact) {
    if (!e) return TENZO_ERROR_INVALID_ARGUMENT;
    return run_prefill(e, tokens, n, exact != 0);
}

static int generate_once(tenzo_engine_t e, int cur_token, float temperature, float top_p,
                         int top_k, float penalty, const int* past, int past_len, float draw);

TENZO_API int tenzo_generate_step(tenzo_engine_t e, int cur_token,
                                  const tenzo_sampling_params_t* params, const int* past,
                                  int past_len) {
    if (!e) return -1;
    // sample_top_k_top_p's defaults (:1728-1731)
    const float temperature = params ? params->temperature : 0.7f;
    const float top_p = params ? params->top_p : 0.9f;
    const int top_k = params ? params->top_k : 40;
    const float penalty = params ? params->repetition_penalty : 1.15f;
    if (temperature > 0.0f && e->V > 262144) {
        set_error("generate_step: sampling supports vocabularies up to 262144");
        return -1;
    }
    // the draw of :1797, from the process's rand() as in the reference (taken
    // once, so a step rerun after an abort uses the same draw)
    const float draw = temperature > 0.0f
                           ? static_cast<float>(rand()) / static_cast<float>(RAND_MAX)
                           : 0.0f;
    for (int attempt = 0;; ++attempt) {
        if (generate_once(e, cur_token, temperature, top_p, top_k, penalty, past, past_len,
                          draw))
            return -1;
        if (attempt > 0 || !ds_retry(e)) break;
    }
    if (ds_check(e)) return -1;
    e->seq_len += 1;  // :1833-1835
    return e->io_host[2];
}

// One decode step of tenzo_generate_step with its penalty and sampling,
// synchronized (0, or -1 with the error set).
static int generate_once(tenzo_engine_t e, int cur_token, float temperature, float top_p,
                         int top_k, float penalty, const int* past, int past_len, float draw) {
    if (run_step(e, cur_token, true)) return -1;
    if (penalty != 1.0f && past && past_len > 0) {
        // :1735-1743 on the device, then the greedy argmax again
        hipStream_t st = e->st;
        if (past_len > e->pen_cap) {
            if (e->pen_dev) {
                (void)hipStreamSynchronize(st);
                (void)hipFree(e->pen_dev);
            }
            if (hipMalloc(&e->pen_dev, (size_t)past_len * 4) != hipSuccess) {
                e->pen_dev = nullptr;
                e->pen_cap = 0;
                set_error("generate_step: out of memory for past tokens");
                return -1;
            }
            e->pen_cap = past_len;
        }
        ArgmaxWs am = argmax_ws_at(e->am_ws, e->V, e->io_dev + 2);
        if (hipMemcpyAsync(e->pen_dev, past, (size_t)past_len * 4, hipMemcpyHostToDevice, st) !=
                hipSuccess ||
            launch_rep_penalty(e->logits, e->V, e->pen_dev, past_len, penalty, st) ||
            (temperature <= 0.0f && launch_argmax(e->logits, e->V, am, st)))
            return -1;
    }
    if (temperature > 0.0f &&
        launch_sample(e->logits, e->V, top_k, top_p, temperature, draw, e->sample_ws,
                      e->io_dev + 2, e->st))
        return -1;
    if (hipMemcpyAsync(e->io_host + 2, e->io_dev + 2, 4, hipMemcpyDeviceToHost, e->st) !=
            hipSuccess ||
        hipStreamSynchronize(e->st) != hipSuccess) {
        set_error("generate_step: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    return 0;
}

// ---- engine extensions (include/tenzo_hip.h) ----

// Enqueues steps i0 .. n-1 of a chained decode (step i at position seq_len + i,
// the first step's token in io[0]), the persistent kernel when `persistent`;
// a cooperative launch the runtime refuses moves the rest of the chain to the
// stage kernels.
static int enqueue_chain(tenzo_engine_t e, int i0, int n, bool persistent) {
    bool pos_set = false;
    for (int i = i0; i < n; ++i) {
        const int pos = e->seq_len + i;
        int rc;
        if (persistent) {
            rc = run_persistent(e, true, pos, e->dec_out, i);
            if (rc != kDsCoopRefused) {
                if (rc) return rc;
                continue;
            }
            persistent = false;
        }
        // stage kernels: token and position chained on the device
        const int T = attn_pick_chunk(pos + 1, e->Hkv, 1);
        if (!pos_set) {
            e->io_host[1] = pos;
            TZ_HIP(hipMemcpyAsync(e->io_dev + 1, e->io_host + 1, 4, hipMemcpyHostToDevice,
                                  e->st));
            pos_set = true;
        }
        if ((rc = enqueue_step(e, true, T, (int)ceil_div(pos + 1, T)))) return rc;
        hipLaunchKernelGGL(chain_kernel, dim3(1), dim3(64), 0, e->st, e->io_dev,
                           e->dec_out + i);
        if ((rc = launch_status("chain_kernel"))) return rc;
    }
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_decode(tenzo_engine_t e, int token, int n, int32_t* out,
                                          float* ms) {
    TZ_CHECK(e && out && n > 0, "engine_decode: bad arguments");
    if (!ready(e, true)) return TENZO_ERROR_INVALID_ARGUMENT;
    TZ_CHECK(token >= 0 && token < e->V, "engine_decode: token %d outside [0, %d)", token, e->V);
    TZ_CHECK(e->seq_len + n <= e->max_seq, "engine_decode: %d steps from position %d exceed "
             "max_seq %d", n, e->seq_len, e->max_seq);
    TZ_HIP(hipSetDevice(e->dev));
    if (e->kv_kind == 3) {
        const int prc = pg_ensure(e, e->seq_len + n);
        if (prc) return prc;
    }
    if (n > e->dec_cap) {
        if (e->dec_out) {
            TZ_HIP(hipStreamSynchronize(e->st));
            TZ_HIP(hipFree(e->dec_out));
            e->dec_out = nullptr;
            e->dec_cap = 0;
        }
        TZ_HIP(hipMalloc(&e->dec_out, (size_t)n * 4));
        e->dec_cap = n;
    }
    const bool persistent = e->mode == 2 && ds_usable(e);
    hipEvent_t t0 = nullptr, t1 = nullptr;
    TZ_HIP(hipEventCreate(&t0));
    TZ_HIP(hipEventCreate(&t1));
    // Every step that completes stores its token in dec_out; a persistent step
    // that aborts stores none and the steps after it return at once (io[3]),
    // so the first -1 marks where a rerun starts.
    auto attempt = [&](int i0, int tok, bool first) -> int {
        e->io_host[0] = tok;
        e->io_host[3] = 0;
        if (hipMemcpyAsync(e->io_dev, e->io_host, 4, hipMemcpyHostToDevice, e->st) != hipSuccess ||
            hipMemcpyAsync(e->io_dev + 3, e->io_host + 3, 4, hipMemcpyHostToDevice, e->st) !=
                hipSuccess ||
            (persistent && hipMemsetAsync(e->dec_out + i0, 0xff, (size_t)(n - i0) * 4, e->st) !=
                               hipSuccess) ||
            (first && hipEventRecord(t0, e->st) != hipSuccess))
            return TENZO_ERROR_UNSUPPORTED;
        int rc = enqueue_chain(e, i0, n, persistent);
        if (rc) return rc;
        if (hipEventRecord(t1, e->st) != hipSuccess ||
            (persistent && hipMemcpyAsync(e->io_host + 3, e->io_dev + 3, 4,
                                          hipMemcpyDeviceToHost, e->st) != hipSuccess) ||
            hipMemcpyAsync(out + i0, e->dec_out + i0, (size_t)(n - i0) * 4,
                           hipMemcpyDeviceToHost, e->st) != hipSuccess ||
            hipStreamSynchronize(e->st) != hipSuccess)
            return TENZO_ERROR_UNSUPPORTED;
        return TENZO_SUCCESS;
    };
    int rc = attempt(0, token, true);
    if (!rc && persistent && ds_retry(e)) {
        int k = 0;
        while (k < n && out[k] >= 0) ++k;
        rc = k < n ? attempt(k, k == 0 ? token : out[k - 1], false) : TENZO_SUCCESS;
    }
    if (!rc && ms) (void)hipEventElapsedTime(ms, t0, t1);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    if (rc) {
        if (rc == TENZO_ERROR_UNSUPPORTED) set_error("engine_decode: %s", hipGetErrorString(hipGetLastError()));
        return rc;
    }
    if ((rc = ds_check(e))) return rc;
    e->seq_len += n;
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_set_kv(tenzo_engine_t e, const void* kc, const void* vc,
                                          const void* ks, const void* vs, int seq_len,
                                          int is_device) {
    TZ_CHECK(e && kc && vc && ks && vs, "engine_set_kv: null pointer");
    TZ_CHECK(seq_len >= 0 && seq_len <= e->max_seq, "engine_set_kv: seq_len %d outside [0, %d]",
             seq_len, e->max_seq);
    TZ_HIP(hipSetDevice(e->dev));
    if (e->kv_kind == 3) {  // logical rows scattered into fresh blocks
        TZ_HIP(hipStreamSynchronize(e->st));
        pg_reset(e);
        const int prc = pg_ensure(e, seq_len);
        if (prc) return prc;
        if (seq_len > 0) {
            const int trc = pg_transfer(e, (int8_t*)kc, (int8_t*)vc, (float*)ks, (float*)vs,
                                        seq_len, is_device ? hipMemcpyDeviceToDevice
                                                           : hipMemcpyHostToDevice, true);
            if (trc) return trc;
        }
        e->seq_len = seq_len;
        return TENZO_SUCCESS;
    }
    if (seq_len > 0) {
        const hipMemcpyKind k = is_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
        const size_t rows = (size_t)e->L * e->Hkv;
        const size_t R = (size_t)e->kv_row, S = (size_t)e->kv_sb;
        TZ_HIP(hipMemcpy2DAsync(e->kc, R * e->max_seq, kc, R * seq_len,
                                R * seq_len, rows, k, e->st));
        TZ_HIP(hipMemcpy2DAsync(e->vc, R * e->max_seq, vc, R * seq_len,
                                R * seq_len, rows, k, e->st));
        TZ_HIP(hipMemcpy2DAsync(e->ks, S * e->max_seq, ks, S * seq_len,
                                S * seq_len, rows, k, e->st));
        TZ_HIP(hipMemcpy2DAsync(e->vs, S * e->max_seq, vs, S * seq_len,
                                S * seq_len, rows, k, e->st));
        TZ_HIP(hipStreamSynchronize(e->st));
    }
    e->seq_len = seq_len;
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_get_kv(tenzo_engine_t e, void* kc, void* vc, void* ks,
                                          void* vs, int seq_len) {
    TZ_CHECK(e && kc && vc && ks && vs, "engine_get_kv: null pointer");
    TZ_CHECK(seq_len > 0 && seq_len <= e->max_seq, "engine_get_kv: bad seq_len %d", seq_len);
    TZ_HIP(hipSetDevice(e->dev));
    if (e->kv_kind == 3) {  // gathered from the blocks in table order
        TZ_CHECK((int)e->pg_table.size() * 16 >= seq_len, "engine_get_kv: %d tokens but %d "
                 "blocks", seq_len, (int)e->pg_table.size());
        TZ_HIP(hipStreamSynchronize(e->st));
        return pg_transfer(e, (int8_t*)kc, (int8_t*)vc, (float*)ks, (float*)vs, seq_len,
                           hipMemcpyDeviceToHost, false);
    }
    const size_t rows = (size_t)e->L * e->Hkv;
    const size_t R = (size_t)e->kv_row, S = (size_t)e->kv_sb;
    TZ_HIP(hipStreamSynchronize(e->st));
    TZ_HIP(hipMemcpy2D(kc, R * seq_len, e->kc, R * e->max_seq,
                       R * seq_len, rows, hipMemcpyDeviceToHost));
    TZ_HIP(hipMemcpy2D(vc, R * seq_len, e->vc, R * e->max_seq,
                       R * seq_len, rows, hipMemcpyDeviceToHost));
    TZ_HIP(hipMemcpy2D(ks, S * seq_len, e->ks, S * e->max_seq,
                       S * seq_len, rows, hipMemcpyDeviceToHost));
    TZ_HIP(hipMemcpy2D(vs, S * seq_len, e->vs, S * e->max_seq,
                       S * seq_len, rows, hipMemcpyDeviceToHost));
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_block_table(tenzo_engine_t e, int32_t* out, int cap) {
    TZ_CHECK(e && (out || cap == 0), "engine_block_table: null pointer");
    TZ_CHECK(e->kv_kind == 3, "engine_block_table: kv_mode is not paged_int8");
    const int n = (int)e->pg_table.size();
    for (int i = 0; i < n && i < cap; ++i) out[i] = e->pg_table[i];
    return n;
}

TENZO_HIP_API int tenzo_hip_engine_set_seq_len(tenzo_engine_t e, int seq_len) {
    TZ_CHECK(e, "engine_set_seq_len: null engine");
    TZ_CHECK(seq_len >= 0 && seq_len <= e->seq_len,
             "engine_set_seq_len: %d outside [0, %d] (only rewinding is allowed)", seq_len,
             e->seq_len);
    e->seq_len = seq_len;
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_set_rope_theta(tenzo_engine_t e, float theta) {
    TZ_CHECK(e && theta > 0.0f, "engine_set_rope_theta: bad arguments");
    TZ_HIP(hipSetDevice(e->dev));
    TZ_HIP(hipStreamSynchronize(e->st));
    e->theta = theta;
    return upload_rope(e);
}

TENZO_HIP_API int tenzo_hip_engine_get_logits(tenzo_engine_t e, float* logits) {
    TZ_CHECK(e && logits, "engine_get_logits: null pointer");
    TZ_HIP(hipSetDevice(e->dev));
    TZ_HIP(hipStreamSynchronize(e->st));
    TZ_HIP(hipMemcpy(logits, e->logits, (size_t)e->V * 4, hipMemcpyDeviceToHost));
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_get_buffer(tenzo_engine_t e, const char* name, float* out,
                                              int64_t n) {
    TZ_CHECK(e && name && out, "engine_get_buffer: null pointer");
    struct B {
        const char* n;
        const float* p;
        int64_t len;
    } bufs[] = {{"x", e->x, e->H},
                {"qkv", e->qkv, e->qd + 2 * e->kvd},
                {"attn_out", e->attn, e->qd},
                {"h1", e->h1, e->H},
                {"gate_up", e->gu, 2 * (int64_t)e->F},
                {"logits", e->logits, e->V}};
    for (const B& b : bufs) {
        if (std::strcmp(b.n, name) == 0) {
            TZ_CHECK(n >= b.len, "engine_get_buffer: %s needs %lld floats", name,
                     (long long)b.len);
            TZ_HIP(hipSetDevice(e->dev));
            TZ_HIP(hipStreamSynchronize(e->st));
            TZ_HIP(hipMemcpy(out, b.p, (size_t)b.len * 4, hipMemcpyDeviceToHost));
            return TENZO_SUCCESS;
        }
    }
    set_error("engine_get_buffer: unknown buffer \"%s\"", name);
    return TENZO_ERROR_INVALID_ARGUMENT;
}

TENZO_HIP_API int tenzo_hip_engine_get_layer_state(tenzo_engine_t e, int layer, int which,
                                                   void* out, int64_t n) {
    TZ_CHECK(e && out, "engine_get_layer_state: null pointer");
    TZ_CHECK(layer >= 0 && layer < e->L, "engine_get_layer_state: layer %d out of range", layer);
    TZ_CHECK(e->ds_state_valid,
             "engine_get_layer_state: the last step did not run the persistent kernel");
    const int* acc = reinterpret_cast<const int*>(e->ds_sync + ds_sync_words(e->L, e->Hkv));
    const int64_t qkv = e->qd + 2 * (int64_t)e->kvd;
    const int64_t stride = qkv + 2 * (int64_t)e->H + 2 * (int64_t)e->F;  // q|k|v, o, gate|up, down
    const int* al = acc + layer * stride;
    const float* xs = e->ds_vec;
    const float* h1s = xs + (size_t)e->L * e->H;
    const float* attns = h1s + (size_t)e->L * e->H;
    const void* src = nullptr;
    int64_t len = 0;
    switch (which) {
        case 0: src = xs + (size_t)layer * e->H; len = e->H; break;
        case 1: src = h1s + (size_t)layer * e->H; len = e->H; break;
        case 2: src = attns + (size_t)layer * e->qd; len = e->qd; break;
        case 3: src = al; len = qkv; break;
        case 4: src = al + qkv; len = e->H; break;
        case 5: src = al + qkv + e->H; len = 2 * (int64_t)e->F; break;
        case 6: src = al + qkv + e->H + 2 * (int64_t)e->F; len = e->H; break;
        default:
            set_error("engine_get_layer_state: unknown buffer %d", which);
            return TENZO_ERROR_INVALID_ARGUMENT;
    }
    TZ_CHECK(n >= len, "engine_get_layer_state: buffer %d needs %lld words", which,
             (long long)len);
    TZ_HIP(hipSetDevice(e->dev));
    TZ_HIP(hipStreamSynchronize(e->st));
    TZ_HIP(hipMemcpy(out, src, (size_t)len * 4, hipMemcpyDeviceToHost));
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_use_graph(tenzo_engine_t e, int on) {
    TZ_CHECK(e, "engine_use_graph: null engine");
    e->mode = on ? 1 : 0;
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_set_mode(tenzo_engine_t e, int mode) {
    TZ_CHECK(e, "engine_set_mode: null engine");
    TZ_CHECK(mode >= 0 && mode <= 2, "engine_set_mode: mode %d not in {0, 1, 2}", mode);
    e->mode = mode;
    return TENZO_SUCCESS;
}

TENZO_HIP_API int tenzo_hip_engine_get_mode(tenzo_engine_t e) {
    if (!e) return -1;
    return e->mode == 2 && !ds_usable(e) ? 1 : e->mode;
}

TENZO_HIP_API void* tenzo_hip_engine_stream(tenzo_engine_t e) { return e ? e->st : nullptr; }

static size_t trace_words(tenzo_engine_t e) {
    return (size_t)(5 * e->L + 1) * (size_t)(e->ds_nwg > 0 ? e->ds_nwg : 1) * 2;
}

TENZO_HIP_API int tenzo_hip_engine_trace(tenzo_engine_t e, int on) {
    TZ_CHECK(e, "engine_trace: null engine");
    TZ_HIP(hipSetDevice(e->dev));
    if (on && !e->ds_trace) {
        TZ_CHECK(e->ds_nwg > 0, "engine_trace: the persistent decode kernel is not available");
        void* p = nullptr;
        TZ_HIP(hipMalloc(&p, trace_words(e) * 8));
        TZ_HIP(hipMemset(p, 0, trace_words(e) * 8));
        e->ds_trace = static_cast<uint64_t*>(p);
    } else if (!on && e->ds_trace) {
        TZ_HIP(hipStreamSynchronize(e->st));
        TZ_HIP(hipFree(e->ds_trace));
        e->ds_trace = nullptr;
    }
    return TENZO_SUCCESS;
}

TENZO_HIP_API int64_t tenzo_hip_engine_get_trace(tenzo_engine_t e, uint64_t* out, int64_t n) {
    if (!e || !e->ds_trace) return -1;
    const int64_t words = (int64_t)trace_words(e);
    if (!out) return words;
    if (n < words || hipStreamSynchronize(e->st) != hipSuccess ||
        hipMemcpy(out, e->ds_trace, (size_t)words * 8, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    return words;
}

}  // extern "C"

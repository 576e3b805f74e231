// Test infrastructure only: a harness that compiles the reference's own CPU
// engine (TenzoEngine.cpp, read in place from the reference checkout) and
// exposes its hot-path functions through a flat C ABI, so tests can produce
// golden vectors and bench.py can time the reference CPU path as a baseline.
// Nothing in the product (tenzo_amd/) links or loads this library.
//
// The include below pulls the reference translation unit into this one, which
// makes its anonymous-namespace helpers (build_lut, compute_from_lut,
// rms_norm_raw, pack_ternary_weights_raw) callable from here.
#include "runtime/TenzoEngine.cpp"

#include <chrono>
#include <cstdint>
#include <cstring>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

using tenzo::FusedKVCache;
using tenzo::TenzoEngineImpl;
using tenzo::Vec256i;

extern "C" {

// build_lut (TenzoEngine.cpp:22-62): returns absmax/31 and the 32-byte LUT
// record per k-pair (K/2 * 32 bytes).
float ref_build_lut(const float* x, int64_t K, int8_t* lut_out) {
    std::vector<Vec256i> lut(K / 2);
    float inv = tenzo::build_lut(x, K, reinterpret_cast<__m256i*>(lut.data()));
    std::memcpy(lut_out, lut.data(), static_cast<size_t>(K / 2) * 32);
    return inv;
}

// build_lut + compute_from_lut (TenzoEngine.cpp:22-146, as called at :1585-1586).
void ref_tl1_gemv(const float* x, const int8_t* w, int64_t K, int64_t N,
                  float w_scale, float* y) {
    std::vector<Vec256i> lut(K / 2);
    float inv = tenzo::build_lut(x, K, reinterpret_cast<__m256i*>(lut.data()));
    tenzo::compute_from_lut(reinterpret_cast<const __m256i*>(lut.data()), w, N / 64,
                            K / 2, y, inv * w_scale);
}

// Same, with total scale 1.0 so y = float(acc) exactly; returns the int32
// accumulators (|acc| <= 31*K < 2^24, so the float round trip is exact).
float ref_tl1_gemv_acc(const float* x, const int8_t* w, int64_t K, int64_t N,
                       int32_t* acc) {
    std::vector<Vec256i> lut(K / 2);
    std::vector<float> y(N);
    float inv = tenzo::build_lut(x, K, reinterpret_cast<__m256i*>(lut.data()));
    tenzo::compute_from_lut(reinterpret_cast<const __m256i*>(lut.data()), w, N / 64,
                            K / 2, y.data(), 1.0f);
    for (int64_t n = 0; n < N; ++n) acc[n] = static_cast<int32_t>(y[n]);
    return inv;
}

// rms_norm_raw (TenzoEngine.cpp:148-166).
void ref_rms_norm(const float* x, const float* w, float* y, int dim, float eps) {
    tenzo::rms_norm_raw(x, w, y, dim, eps);
}

// pack_ternary_weights_raw (TenzoEngine.cpp:1842-1884): HF [N/4][K] 2-bit -> TL1.
void ref_pack_raw(const uint8_t* raw, int64_t N, int64_t K, int8_t* out) {
    std::vector<int8_t> p = tenzo::pack_ternary_weights_raw(raw, N, K);
    std::memcpy(out, p.data(), p.size());
}

// FusedKVCache::forward_attention_raw (TenzoEngine.cpp:447-919), int8_fused mode,
// one layer. The caller's cache arrays ([Hkv][max_seq][128] codes, [Hkv][max_seq]
// fp32 scales) are copied in, the call appends at position pos, and the cache
// (with the appended token), the rotated q/k and the output are copied back.
void ref_attention_int8(int Hq, int Hkv, int max_seq, int pos,
                        float* q, float* k, float* v,
                        int8_t* kc, int8_t* vc, float* ks, float* vs,
                        float* out) {
    FusedKVCache c(1, Hq, Hkv, 128, max_seq, "int8_fused");
    size_t n_el = static_cast<size_t>(Hkv) * max_seq * 128;
    size_t n_sc = static_cast<size_t>(Hkv) * max_seq;
    std::memcpy(c.int8_k.data(), kc, n_el);
    std::memcpy(c.int8_v.data(), vc, n_el);
    std::memcpy(c.int8_k_scales.data(), ks, n_sc * 4);
    std::memcpy(c.int8_v_scales.data(), vs, n_sc * 4);
    c.cur_seq_len = pos;
    c.forward_attention_raw(0, q, k, v, out);
    std::memcpy(kc, c.int8_k.data(), n_el);
    std::memcpy(vc, c.int8_v.data(), n_el);
    std::memcpy(ks, c.int8_k_scales.data(), n_sc * 4);
    std::memcpy(vs, c.int8_v_scales.data(), n_sc * 4);
}

// Timing of the same call without the copies: one cache of `batch` sequences
// ([batch][Hkv][max_seq] rows) filled once from the arrays, then `reps` rounds
// of forward_attention_raw at position pos for every sequence (the reference
// serves a batch as one call per sequence). Returns the mean seconds per round.
double ref_attention_int8_time(int batch, int Hq, int Hkv, int max_seq, int pos,
                               const int8_t* kc, const int8_t* vc, const float* ks,
                               const float* vs, const float* q, const float* k, const float* v,
                               int reps) {
    const size_t n_el = static_cast<size_t>(Hkv) * max_seq * 128;
    const size_t n_sc = static_cast<size_t>(Hkv) * max_seq;
    std::vector<FusedKVCache*> cs;
    for (int b = 0; b < batch; ++b) {
        FusedKVCache* c = new FusedKVCache(1, Hq, Hkv, 128, max_seq, "int8_fused");
        std::memcpy(c->int8_k.data(), kc + b * n_el, n_el);
        std::memcpy(c->int8_v.data(), vc + b * n_el, n_el);
        std::memcpy(c->int8_k_scales.data(), ks + b * n_sc, n_sc * 4);
        std::memcpy(c->int8_v_scales.data(), vs + b * n_sc, n_sc * 4);
        cs.push_back(c);
    }
    std::vector<float> qq(Hq * 128), kk(Hkv * 128), vv(Hkv * 128), out(Hq * 128);
    double total = 0.0;
    for (int r = 0; r <= reps; ++r) {  // round 0 warms up
        const auto t0 = std::chrono::steady_clock::now();
        for (int b = 0; b < batch; ++b) {
            std::memcpy(qq.data(), q + (size_t)b * Hq * 128, qq.size() * 4);  // RoPE is in place
            std::memcpy(kk.data(), k + (size_t)b * Hkv * 128, kk.size() * 4);
            std::memcpy(vv.data(), v + (size_t)b * Hkv * 128, vv.size() * 4);
            cs[b]->cur_seq_len = pos;
            cs[b]->forward_attention_raw(0, qq.data(), kk.data(), vv.data(), out.data());
        }
        const double dt =
            std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        if (r > 0) total += dt;
    }
    for (FusedKVCache* c : cs) delete c;
    return total / reps;
}

// The ternary KV modes (TenzoEngine.cpp:534-648, :695-885): mode 1 tl1_fused,
// 2 popcount_fused. kb / vb [Hkv][max_seq][32] bytes (popcount K: the
// PopcountBitplanes structs), ks / vs fp32; updated in place.
void ref_attention_tern(int mode, int Hq, int Hkv, int max_seq, int pos, float* q, float* k,
                        float* v, uint8_t* kb, uint8_t* vb, float* ks, float* vs, float* out) {
    FusedKVCache c(1, Hq, Hkv, 128, max_seq, mode == 1 ? "tl1_fused" : "popcount_fused");
    const size_t n_b = static_cast<size_t>(Hkv) * max_seq * 32;
    const size_t n_sc = static_cast<size_t>(Hkv) * max_seq * 4;
    uint8_t* ck = mode == 1 ? c.tl1_k.data() : reinterpret_cast<uint8_t*>(c.popcount_k.data());
    uint8_t* cv = mode == 1 ? c.tl1_v.data() : c.popcount_v.data();
    float* cks = mode == 1 ? c.tl1_k_scales.data() : c.popcount_k_scales.data();
    float* cvs = mode == 1 ? c.tl1_v_scales.data() : c.popcount_v_scales.data();
    std::memcpy(ck, kb, n_b);
    std::memcpy(cv, vb, n_b);
    std::memcpy(cks, ks, n_sc);
    std::memcpy(cvs, vs, n_sc);
    c.cur_seq_len = pos;
    c.forward_attention_raw(0, q, k, v, out);
    std::memcpy(kb, ck, n_b);
    std::memcpy(vb, cv, n_b);
    std::memcpy(ks, cks, n_sc);
    std::memcpy(vs, cvs, n_sc);
}

// PagedKVCache::forward_attention_raw (TenzoEngine.cpp:269-445) on caller-held
// pools ([total_blocks][n_layers][Hkv][16][128] codes, fp32 scales) and block
// table (n_bt entries, their blocks taken out of the free list); the call may
// allocate one block. Pools and table are copied back; returns the table size.
int ref_attention_paged(int Hq, int Hkv, int n_layers, int layer, int total_blocks, int pos,
                        float* q, float* k, float* v, int8_t* pk, int8_t* pv, float* pks,
                        float* pvs, int32_t* block_table, int n_bt, float* out) {
    tenzo::PagedKVCache c(n_layers, Hq, Hkv, 128, total_blocks);
    std::memcpy(c.paged_k_pool.data(), pk, c.paged_k_pool.size());
    std::memcpy(c.paged_v_pool.data(), pv, c.paged_v_pool.size());
    std::memcpy(c.paged_k_scales.data(), pks, c.paged_k_scales.size() * 4);
    std::memcpy(c.paged_v_scales.data(), pvs, c.paged_v_scales.size() * 4);
    c.block_table.assign(block_table, block_table + n_bt);
    for (int i = 0; i < n_bt; ++i) {
        auto& f = c.block_mgr.free_blocks;
        for (size_t j = 0; j < f.size(); ++j)
            if (f[j] == block_table[i]) { f.erase(f.begin() + j); break; }
    }
    c.cur_seq_len = pos;
    c.forward_attention_raw(layer, q, k, v, out);
    std::memcpy(pk, c.paged_k_pool.data(), c.paged_k_pool.size());
    std::memcpy(pv, c.paged_v_pool.data(), c.paged_v_pool.size());
    std::memcpy(pks, c.paged_k_scales.data(), c.paged_k_scales.size() * 4);
    std::memcpy(pvs, c.paged_v_scales.data(), c.paged_v_scales.size() * 4);
    for (size_t i = 0; i < c.block_table.size(); ++i) block_table[i] = c.block_table[i];
    return (int)c.block_table.size();
}

// The paged pools and block table of an engine created with kv_mode paged_int8.
int ref_engine_get_kv_paged(void* e, int8_t* pk, int8_t* pv, float* pks, float* pvs,
                            int32_t* block_table) {
    tenzo::PagedKVCache& c = static_cast<tenzo_engine_t>(e)->impl->paged_kv_cache;
    std::memcpy(pk, c.paged_k_pool.data(), c.paged_k_pool.size());
    std::memcpy(pv, c.paged_v_pool.data(), c.paged_v_pool.size());
    std::memcpy(pks, c.paged_k_scales.data(), c.paged_k_scales.size() * 4);
    std::memcpy(pvs, c.paged_v_scales.data(), c.paged_v_scales.size() * 4);
    for (size_t i = 0; i < c.block_table.size(); ++i) block_table[i] = c.block_table[i];
    return (int)c.block_table.size();
}

// Quantized GEMV free functions (TenzoEngine.cpp:1022-1175).
void ref_q4_0(const float* a, const uint8_t* w, float* y, int K, int N) {
    tenzo::compute_linear_gguf_q4_0(a, w, y, K, N);
}
void ref_q8_0(const float* a, const uint8_t* w, float* y, int K, int N) {
    tenzo::compute_linear_gguf_q8_0(a, w, y, K, N);
}
void ref_gptq(const float* a, const uint32_t* qw, const float* s, const uint32_t* qz,
              float* y, int K, int N, int group) {
    tenzo::compute_linear_gptq(a, qw, s, qz, y, K, N, group);
}
void ref_awq(const float* a, const uint32_t* qw, const float* s, const uint32_t* qz,
             float* y, int K, int N, int group) {
    tenzo::compute_linear_awq(a, qw, s, qz, y, K, N, group);
}

// ---- Whole engine (TenzoEngine.cpp:1215-1838) through the reference's C API ----

// kv_mode is borrowed by the engine and re-read every layer, hence literals.
void* ref_engine_create_mode(int H, int Hq, int Hkv, int L, int F, int V, int max_seq, int mode) {
    tenzo_config_t cfg = tenzo_default_config();
    cfg.hidden_size = H;
    cfg.num_q_heads = Hq;
    cfg.num_kv_heads = Hkv;
    cfg.head_dim = 128;
    cfg.num_layers = L;
    cfg.ffn_dim = F;
    cfg.vocab_size = V;
    cfg.max_seq_len = max_seq;
    cfg.kv_mode = mode == 1 ? "tl1_fused" : mode == 2 ? "popcount_fused"
                : mode == 3 ? "paged_int8" : "int8_fused";
    cfg.device = "cpu";
    return tenzo_create_engine(&cfg);
}

void* ref_engine_create(int H, int Hq, int Hkv, int L, int F, int V, int max_seq) {
    tenzo_config_t cfg = tenzo_default_config();
    cfg.hidden_size = H;
    cfg.num_q_heads = Hq;
    cfg.num_kv_heads = Hkv;
    cfg.head_dim = 128;
    cfg.num_layers = L;
    cfg.ffn_dim = F;
    cfg.vocab_size = V;
    cfg.max_seq_len = max_seq;
    cfg.kv_mode = "int8_fused";
    cfg.device = "cpu";
    return tenzo_create_engine(&cfg);
}

void ref_engine_destroy(void* e) { tenzo_destroy_engine(static_cast<tenzo_engine_t>(e)); }

int ref_engine_set_layer(void* e, int l, const tenzo_layer_weights_t* w) {
    return tenzo_set_layer_weights(static_cast<tenzo_engine_t>(e), l, w);
}

int ref_engine_set_head(void* e, const int8_t* W, const float* s, const float* final_norm,
                        int V, int H) {
    auto* eng = static_cast<tenzo_engine_t>(e);
    int st = tenzo_set_lm_head_i8(eng, W, s, V, H);
    if (st) return st;
    return tenzo_set_final_norm(eng, final_norm);
}

// Prefill the int8 cache directly (public FusedKVCache state) instead of running
// seq_len prefill steps. Arrays are [L][Hkv][max_seq][128] / [L][Hkv][max_seq].
void ref_engine_set_kv(void* e, const int8_t* kc, const int8_t* vc, const float* ks,
                       const float* vs, int seq_len) {
    FusedKVCache& c = static_cast<tenzo_engine_t>(e)->impl->kv_cache;
    std::memcpy(c.int8_k.data(), kc, c.int8_k.size());
    std::memcpy(c.int8_v.data(), vc, c.int8_v.size());
    std::memcpy(c.int8_k_scales.data(), ks, c.int8_k_scales.size() * 4);
    std::memcpy(c.int8_v_scales.data(), vs, c.int8_v_scales.size() * 4);
    c.cur_seq_len = seq_len;
}

void ref_engine_get_kv(void* e, int8_t* kc, int8_t* vc, float* ks, float* vs) {
    FusedKVCache& c = static_cast<tenzo_engine_t>(e)->impl->kv_cache;
    std::memcpy(kc, c.int8_k.data(), c.int8_k.size());
    std::memcpy(vc, c.int8_v.data(), c.int8_v.size());
    std::memcpy(ks, c.int8_k_scales.data(), c.int8_k_scales.size() * 4);
    std::memcpy(vs, c.int8_v_scales.data(), c.int8_v_scales.size() * 4);
}

// Writes the ternary caches (full [L][Hkv][max_seq] layout) and the length.
void ref_engine_set_kv_tern(void* e, int mode, const uint8_t* kb, const uint8_t* vb,
                            const float* ks, const float* vs, int seq_len) {
    FusedKVCache& c = static_cast<tenzo_engine_t>(e)->impl->kv_cache;
    if (mode == 1) {
        std::memcpy(c.tl1_k.data(), kb, c.tl1_k.size());
        std::memcpy(c.tl1_v.data(), vb, c.tl1_v.size());
        std::memcpy(c.tl1_k_scales.data(), ks, c.tl1_k_scales.size() * 4);
        std::memcpy(c.tl1_v_scales.data(), vs, c.tl1_v_scales.size() * 4);
    } else {
        std::memcpy(c.popcount_k.data(), kb, c.popcount_k.size() * 32);
        std::memcpy(c.popcount_v.data(), vb, c.popcount_v.size());
        std::memcpy(c.popcount_k_scales.data(), ks, c.popcount_k_scales.size() * 4);
        std::memcpy(c.popcount_v_scales.data(), vs, c.popcount_v_scales.size() * 4);
    }
    c.cur_seq_len = seq_len;
}

// The ternary caches of an engine created with mode 1 / 2 (rows of 32 bytes).
void ref_engine_get_kv_tern(void* e, int mode, uint8_t* kb, uint8_t* vb, float* ks, float* vs) {
    FusedKVCache& c = static_cast<tenzo_engine_t>(e)->impl->kv_cache;
    if (mode == 1) {
        std::memcpy(kb, c.tl1_k.data(), c.tl1_k.size());
        std::memcpy(vb, c.tl1_v.data(), c.tl1_v.size());
        std::memcpy(ks, c.tl1_k_scales.data(), c.tl1_k_scales.size() * 4);
        std::memcpy(vs, c.tl1_v_scales.data(), c.tl1_v_scales.size() * 4);
    } else {
        std::memcpy(kb, c.popcount_k.data(), c.popcount_k.size() * 32);
        std::memcpy(vb, c.popcount_v.data(), c.popcount_v.size());
        std::memcpy(ks, c.popcount_k_scales.data(), c.popcount_k_scales.size() * 4);
        std::memcpy(vs, c.popcount_v_scales.data(), c.popcount_v_scales.size() * 4);
    }
}

int ref_engine_seq_len(void* e) { return tenzo_get_seq_len(static_cast<tenzo_engine_t>(e)); }

// One greedy decode step (temperature 0, penalty 1.0); copies the logits out
// when logits is non-null and returns the token.
int ref_engine_step(void* e, int token, float* logits) {
    auto* eng = static_cast<tenzo_engine_t>(e);
    tenzo_sampling_params_t p = tenzo_default_sampling_params();
    p.temperature = 0.0f;
    p.repetition_penalty = 1.0f;
    int tok = tenzo_generate_step(eng, token, &p, nullptr, 0);
    if (logits) {
        const auto& ls = eng->impl->logits_scratch;
        std::memcpy(logits, ls.data(), ls.size() * 4);
    }
    return tok;
}

int ref_engine_prefill(void* e, int token) {
    return tenzo_prefill_token(static_cast<tenzo_engine_t>(e), token);
}

// Hidden state after the layers of the last step (buf_x), for stage checks.
void ref_engine_hidden(void* e, float* x) {
    auto* eng = static_cast<tenzo_engine_t>(e);
    std::memcpy(x, eng->impl->buf_x.data(), eng->impl->config.hidden_size * 4);
}

// Stage-level access for tracing one step: embedding, one layer, and the
// engine's scratch buffers by index (TenzoEngine.h:216-230 order).
void ref_engine_embed(void* e, int token) {
    static_cast<tenzo_engine_t>(e)->impl->embedding_lookup(token);
}
void ref_engine_layer(void* e, int l) {
    static_cast<tenzo_engine_t>(e)->impl->forward_layer_raw(l);
}
void ref_engine_finish(void* e) {
    auto* impl = static_cast<tenzo_engine_t>(e)->impl.get();
    impl->kv_cache.increment_seq_len(1);
    impl->compute_logits();
}
int ref_engine_buf(void* e, int which, float* out) {
    auto* impl = static_cast<tenzo_engine_t>(e)->impl.get();
    std::vector<float>* bufs[] = {
        &impl->buf_x, &impl->buf_norm_x, &impl->buf_q, &impl->buf_k, &impl->buf_v,
        &impl->buf_attn_out, &impl->buf_attn_sub, &impl->buf_out, &impl->buf_h1,
        &impl->buf_post_norm, &impl->buf_gate, &impl->buf_up, &impl->buf_act,
        &impl->buf_ffn_norm, &impl->buf_down, &impl->logits_scratch};
    if (which < 0 || which >= 16) return -1;
    std::vector<float>& b = *bufs[which];
    std::memcpy(out, b.data(), b.size() * 4);
    return static_cast<int>(b.size());
}

// sample_top_k_top_p (TenzoEngine.cpp:1722-1807) of the engine on the given
// logits (copied into its logits scratch): the reference's own sampler,
// drawing from the process's rand().
int ref_engine_sample(void* e, const float* logits, float temperature, float top_p, int top_k,
                      float penalty, const int* past, int past_len) {
    auto* impl = static_cast<tenzo_engine_t>(e)->impl.get();
    std::memcpy(impl->logits_scratch.data(), logits, impl->logits_scratch.size() * 4);
    tenzo_sampling_params_t p = tenzo_default_sampling_params();
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.repetition_penalty = penalty;
    return impl->sample_top_k_top_p(&p, past, past_len);
}

// load_model_from_files (TenzoEngine.cpp:1887-2078) through the C API.
int ref_engine_load(void* e, const char* weights, const char* mlir) {
    return tenzo_load_model(static_cast<tenzo_engine_t>(e), weights, mlir);
}

// What the loader put in layer l: which 0..6 = q, k, v, out, gate, up, down
// TL1 bytes (returns the byte count and writes the scale), 7..10 = in_norm,
// attn_sub_norm, post_norm, ffn_sub_norm (returns the float count).
long ref_engine_layer_data(void* e, int l, int which, void* out, float* scale) {
    auto& lw = static_cast<tenzo_engine_t>(e)->impl->layers[l];
    const std::vector<int8_t>* w[7] = {&lw.q_w, &lw.k_w, &lw.v_w, &lw.out_w,
                                       &lw.gate_w, &lw.up_w, &lw.down_w};
    const float sc[7] = {lw.q_scale, lw.k_scale, lw.v_scale, lw.out_scale,
                         lw.gate_scale, lw.up_scale, lw.down_scale};
    const std::vector<float>* nv[4] = {&lw.in_norm, &lw.attn_sub_norm, &lw.post_norm,
                                       &lw.ffn_sub_norm};
    if (which >= 0 && which < 7) {
        if (out) std::memcpy(out, w[which]->data(), w[which]->size());
        if (scale) *scale = sc[which];
        return (long)w[which]->size();
    }
    if (which >= 7 && which < 11) {
        const std::vector<float>& v = *nv[which - 7];
        if (out) std::memcpy(out, v.data(), v.size() * 4);
        return (long)v.size();
    }
    return -1;
}

// The loader's int8 LM head (codes [V][H], scales [V]) and final norm [H].
void ref_engine_head_data(void* e, int8_t* codes, float* scales, float* final_norm) {
    auto* impl = static_cast<tenzo_engine_t>(e)->impl.get();
    if (codes) std::memcpy(codes, impl->embed_w_i8.data(), impl->embed_w_i8.size());
    if (scales) std::memcpy(scales, impl->embed_scales.data(), impl->embed_scales.size() * 4);
    if (final_norm)
        std::memcpy(final_norm, impl->final_norm_w.data(), impl->final_norm_w.size() * 4);
}

int ref_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}  // extern "C"

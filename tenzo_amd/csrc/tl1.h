// Internal interface of the TL1 kernels (used by the C ABI and the engine).
#pragma once

#include "common.h"

namespace tz {

// Per-row output scales of a GEMV over row-concatenated matrices (fused
// Q|K|V or gate|up): rows [end[j-1], end[j]) use scale[j].
struct RowScales {
    int64_t end[4];
    float scale[4];
    int n;
    static RowScales single(float s) {
        RowScales r{};
        r.end[0] = INT64_MAX;
        r.scale[0] = s;
        r.n = 1;
        return r;
    }
};

int launch_tl1_repack(const uint8_t* w_tl1, void* w_packed, int64_t N, int64_t K,
                      hipStream_t st);
// From the loader's raw [N/4][K] 2-bit layout (pack_ternary_weights_raw's input).
int launch_tl1_repack_raw(const uint8_t* raw, void* w_packed, int64_t N, int64_t K,
                          hipStream_t st);
// mode 0: codes of x; 1: codes of rms_norm_raw(x, norm_w); 3: x is gate|up
// ([M][2K]) and the row is relu(gate)^2 * up before the norm. qmax 31 (TL1
// activations) or 127 (LM head). Codes are written with row stride Kp.
int launch_actquant(int mode, int qmax, const float* x, const float* norm_w, float eps,
                    int64_t M, int64_t K, int64_t Kp, int8_t* codes, tenzo_hip_actq_t* q,
                    float* y_out, hipStream_t st);
// rms_norm_raw (TenzoEngine.cpp:148-166) of one vector, w may be null.
int launch_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps,
                   hipStream_t st);
int launch_quant31(const float* x, const float* norm_w, bool do_norm, float eps, int64_t M,
                   int64_t K, int8_t* codes, tenzo_hip_actq_t* q, float* y_out, hipStream_t st);
// Split-K workspace: M*N int32 accumulators + M*N/64 counters, zero on entry
// and left zero on exit.
size_t tl1_ws_bytes(int64_t M, int64_t N);
// y = resid + float(acc) * (q.inv_scale * row scale); resid may be null, acc_out
// may be null; splits <= 0 picks a split count; ws null uses library scratch.
int launch_tl1_gemv(const int8_t* codes, const tenzo_hip_actq_t* q, const void* w_packed,
                    const RowScales& rs, int64_t M, int64_t N, int64_t K, float* y,
                    const float* resid, int32_t* acc_out, hipStream_t st, int splits,
                    void* ws);
int tl1_pick_splits(int64_t nb, int64_t KS, int64_t M);
// The same contraction for M tokens at once on int8 MFMA (tl1_gemm.hip); the
// arguments and results are those of launch_tl1_gemv. tile 0 picks the
// workgroup shape, else 100 * K groups + 10 * row waves + 32-token tiles.
int launch_tl1_mfma(const int8_t* codes, const tenzo_hip_actq_t* q, const void* w_packed,
                    const RowScales& rs, int64_t M, int64_t N, int64_t K, float* y,
                    const float* resid, int32_t* acc_out, hipStream_t st, int tile);
void tl1_mfma_plan(int64_t M, int64_t N, int64_t KS, int* KW, int* RW, int* CT);

}  // namespace tz

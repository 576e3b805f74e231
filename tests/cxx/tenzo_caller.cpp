// A C++ caller of the engine SDK written against include/ only (tenzo.hpp /
// tenzo.h), in the manner of the reference's examples/basic_inference.cpp:
// load a model from weights.bin + model.mlir, prefill a prompt token by token,
// then decode greedily. Test infrastructure: tests/test_gpu_cxx_caller.py
// builds it with g++ against libtenzo_hip.so and compares its tokens with the
// CPU oracle.
//
//   tenzo_caller weights.bin model.mlir H Hq Hkv L F V max_seq n_gen tok0 tok1 ...
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "tenzo.hpp"
#include "tenzo_hip.h"  // tenzo_hip_last_error, for the failure message

int main(int argc, char** argv) {
    if (argc < 13) {
        std::fprintf(stderr, "usage: %s weights mlir H Hq Hkv L F V max_seq n_gen prompt...\n",
                     argv[0]);
        return 2;
    }
    tenzo_config_t cfg = tenzo_default_config();
    cfg.hidden_size = std::atoi(argv[3]);
    cfg.num_q_heads = std::atoi(argv[4]);
    cfg.num_kv_heads = std::atoi(argv[5]);
    cfg.num_layers = std::atoi(argv[6]);
    cfg.ffn_dim = std::atoi(argv[7]);
    cfg.vocab_size = std::atoi(argv[8]);
    cfg.max_seq_len = std::atoi(argv[9]);
    cfg.device = "rocm";
    const int n_gen = std::atoi(argv[10]);
    std::vector<int> prompt;
    for (int i = 11; i < argc; ++i) prompt.push_back(std::atoi(argv[i]));
    try {
        tenzo::Engine engine(cfg);
        engine.load_model(argv[1], argv[2]);
        for (size_t i = 0; i + 1 < prompt.size(); ++i) engine.prefill_token(prompt[i]);
        tenzo_sampling_params_t params = tenzo_default_sampling_params();
        params.temperature = 0.0f;
        params.repetition_penalty = 1.0f;
        std::vector<int> past(prompt.begin(), prompt.end());
        int tok = prompt.back();
        for (int i = 0; i < n_gen; ++i) {
            tok = engine.generate_step(tok, params, past);
            past.push_back(tok);
            std::printf("%d\n", tok);
        }
        std::fprintf(stderr, "seq_len %d\n", engine.get_seq_len());
        tenzo::Engine moved(std::move(engine));  // move-only ownership
        if (engine.get_raw_handle() != nullptr || moved.get_raw_handle() == nullptr) return 3;
    } catch (const std::exception& ex) {
        std::fprintf(stderr, "error: %s (%s)\n", ex.what(), tenzo_hip_last_error());
        return 1;
    }
    return 0;
}

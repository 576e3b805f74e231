/*
 * tenzo.hpp - C++ RAII wrapper over the engine C API of include/tenzo.h, with
 * the public interface of the reference's wrapper (reference
 * include/tenzo.hpp:18-94: class tenzo::Engine - construction from a
 * tenzo_config_t, move-only ownership of the handle, load_model, reset,
 * get_seq_len, prefill_token, generate_step, get_raw_handle; failures throw
 * std::runtime_error), so callers written against the reference SDK
 * (e.g. examples/basic_inference.cpp, src/main_inference.cpp) compile and
 * link against libtenzo_hip.so unchanged. Header-only; it calls nothing but
 * the C API.
 */
#ifndef TENZO_HPP
#define TENZO_HPP

#include <stdexcept>
#include <string>
#include <vector>

#include "tenzo.h"

namespace tenzo {

class Engine {
public:
    explicit Engine(const tenzo_config_t& config = tenzo_default_config())
        : engine_(tenzo_create_engine(&config)) {
        if (!engine_) throw std::runtime_error("tenzo: tenzo_create_engine failed");
    }

    ~Engine() { release(); }

    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;

    Engine(Engine&& other) noexcept : engine_(other.engine_) { other.engine_ = nullptr; }

    Engine& operator=(Engine&& other) noexcept {
        if (this != &other) {
            release();
            engine_ = other.engine_;
            other.engine_ = nullptr;
        }
        return *this;
    }

    // weights.bin + model.mlir as the reference's exporter writes them.
    void load_model(const std::string& weights_path, const std::string& mlir_path) {
        check(tenzo_load_model(engine_, weights_path.c_str(), mlir_path.c_str()),
              "load_model(" + weights_path + ")");
    }

    void reset() { tenzo_reset(engine_); }

    int get_seq_len() const { return tenzo_get_seq_len(engine_); }

    void prefill_token(int token_id) { check(tenzo_prefill_token(engine_, token_id), "prefill_token"); }

    // One decode step from cur_token; returns the sampled next token.
    int generate_step(int cur_token, const tenzo_sampling_params_t& params,
                      const std::vector<int>& past_tokens) {
        const int next = tenzo_generate_step(engine_, cur_token, &params, past_tokens.data(),
                                             static_cast<int>(past_tokens.size()));
        if (next < 0) throw std::runtime_error("tenzo: generate_step failed");
        return next;
    }

    tenzo_engine_t get_raw_handle() const { return engine_; }

private:
    static void check(tenzo_status_t st, const std::string& what) {
        if (st != TENZO_SUCCESS)
            throw std::runtime_error("tenzo: " + what + " failed (status " + std::to_string(st) +
                                     ")");
    }

    void release() noexcept {
        if (engine_) tenzo_destroy_engine(engine_);
        engine_ = nullptr;
    }

    tenzo_engine_t engine_ = nullptr;
};

}  // namespace tenzo

#endif /* TENZO_HPP */

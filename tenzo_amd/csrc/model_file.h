// Internal interface of the model-file reader (model_file.hip).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

namespace tz {

// Byte offsets of the memref views and the bitlinear scales of a model.mlir,
// in order of appearance (load_model_from_files, TenzoEngine.cpp:1943-1959).
struct ModelFileIndex {
    std::vector<uint64_t> views;
    std::vector<float> scales;
};
void parse_model_mlir(const char* text, size_t len, ModelFileIndex* out);

}  // namespace tz

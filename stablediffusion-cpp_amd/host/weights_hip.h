// weights_hip.h - named model weights on the MI355X: the reference's Weights
// (src/safetensors.h:23-55) over sdh::Tensor, loaded from .safetensors files
// straight into device memory, or filled with seeded random values of a given
// model's shapes (for benchmarks, where no checkpoint is available).
//
// The .safetensors format: an 8-byte little-endian header length N, N bytes
// of JSON ({"name": {"dtype", "shape", "data_offsets": [begin, end]}, ...,
// "__metadata__": {...}}), then the raw tensor bytes. F32, F16 and BF16
// tensors are read; other dtypes are skipped with a message on stderr, as
// the reference does (safetensors.cpp:105-108).
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>

#include "tensor_hip.h"

namespace sdh {

struct Weights {
    std::unordered_map<std::string, Tensor> tensors;  // device tensors

    // safetensors.h:37-39: every float tensor of the file, on the device. With
    // keep_bf16, tensors of at least bf16_min_numel elements are stored as
    // BF16 (rounded from F16/F32 if needed) and the rest as F32.
    void load_safetensors(const std::string& path, bool keep_bf16 = false, int64_t bf16_min_numel = 1 << 20);

    // A device tensor of `shape` drawn from N(mean, std) with the library's
    // seeded generator; BF16 (rounded on the device) when keep_bf16 and it
    // has at least bf16_min_numel elements.
    void add_random(const std::string& name, std::vector<int64_t> shape, uint64_t seed, float mean, float std,
                    bool keep_bf16 = false, int64_t bf16_min_numel = 1 << 20);

    // safetensors.h:48-53
    const Tensor& get(const std::string& name) const;  // throws "missing weight: <name>"
    const Tensor* try_get(const std::string& name) const;
    bool has(const std::string& name) const { return tensors.count(name) != 0; }
    size_t total_params() const;
};

}  // namespace sdh

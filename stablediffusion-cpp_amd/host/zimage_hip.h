// zimage_hip.h - one denoising step of Z-Image's single-stream diffusion
// transformer, run entirely on the MI355X through backend_hip.
//
// Interface: the reference's ZImageTransformer (src/zimage.h:40-79) --
// constructed from the checkpoint's named weights and the config.json
// hyper-parameters, forward(latent [1, C, H, W], t, text [1, L, cap_dim])
// returning the model output of the latent's shape (ZImageTransformer::forward,
// src/zimage.cpp:138-228). Everything behind the interface is this library's
// own design (zimage_hip.cpp):
//   * the step works on one token buffer [image rows, image pad rows, text
//     rows, text pad rows] x dim, allocated once per call: the embedders
//     write their rows into it, the two refiner stacks update its image and
//     text row ranges in place, and the main stack runs on the whole buffer,
//     so the joint sequence is never assembled by copies;
//   * the rotary tables of a token layout are built once (from per-pair
//     frequencies precomputed at construction) and kept for later calls; the
//     refiners read row ranges of the joint table;
//   * block weights are bound by role from a table of the checkpoint's name
//     suffixes, and each block's path (the fused BF16 ops, or the fp32 ops)
//     is fixed when it is bound.
#pragma once

#include <cstdint>
#include <memory>
#include <string>

#include "tensor_hip.h"
#include "weights_hip.h"

namespace sdh {

class ZImageTransformer {
public:
    // Hyper-parameters the weights do not determine (zimage.h:44-51); the
    // defaults are the released model's.
    struct Config {
        int patch = 2;
        int heads = 30;
        float norm_eps = 1e-5f;
        float rope_theta = 256.0f;
        float t_scale = 1000.0f;
        int axes_dims[3] = {32, 48, 48};
        // Opt-in, no counterpart in the reference: attention from block-scaled
        // fp16 operands (sdh_attention_fp16), a third of the MFMA work, for a
        // step whose tolerance allows it; off gives the reference's fp32
        // attention numerics.
        bool fp16_attention = false;
    };
    // Tensor shapes of a model, for filling Weights with random values.
    struct Shapes {
        int64_t dim = 3840, ffn = 10240, in_channels = 16, cap_dim = 2560, t_freq = 256, t_hidden = 1024,
                adaln_dim = 256;
        int heads = 30, patch = 2, noise_refiners = 2, context_refiners = 2, layers = 30;
    };
    // Adds every tensor of a model of shapes `s` under the checkpoint's names
    // to w: linears N(0, 1/sqrt(fan-in)), norm weights N(1, 0.05), biases
    // N(0, 0.02), pad tokens N(0, 1); BF16 from bf16_min_numel elements, as
    // the pipeline loads the checkpoint (pipeline.cpp:113).
    static void random_weights(Weights& w, const Shapes& s, uint64_t seed, int64_t bf16_min_numel = 1 << 20);

    explicit ZImageTransformer(const Weights& w);
    ZImageTransformer(const Weights& w, const Config& cfg);
    ~ZImageTransformer();
    ZImageTransformer(const ZImageTransformer&) = delete;
    ZImageTransformer& operator=(const ZImageTransformer&) = delete;

    // latent: [1, C, H, W] device tensor, H and W multiples of the patch; t in
    // [0, 1]; text: [1, L, cap_dim] device tensor of text hidden states.
    // Returns a [1, C, H, W] device tensor. Safe to call from several threads.
    Tensor forward(const Tensor& latent, float t, const Tensor& text) const;

    // Switches the attention numerics of later forward calls (Config::fp16_attention).
    void set_fp16_attention(bool on);

    int in_channels() const;
    int64_t dim() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace sdh

// C entry points for callers without C++ (Python tests and benchmarks).
// Inputs and outputs are host float32 buffers; every call returns 0 or -1
// with sdhm_last_error() set.
extern "C" {
const char* sdhm_last_error(void);
// Loads a Z-Image transformer from a .safetensors file (BF16 from
// bf16_min_numel elements when keep_bf16) with `heads` attention heads.
int sdhm_zimage_load(const char* path, int keep_bf16, int64_t bf16_min_numel, int heads, void** model);
// A model of the given shapes with seeded random weights (BF16 from 2^20 elements).
int sdhm_zimage_random(int64_t dim, int heads, int64_t ffn, int64_t in_channels, int64_t cap_dim, int64_t t_hidden,
                       int64_t adaln_dim, int noise_refiners, int context_refiners, int layers, uint64_t seed,
                       void** model);
// out [1, C, H, W] = forward(x [1, C, H, W], t, cap [1, L, cap_dim]).
int sdhm_zimage_forward(void* model, const float* x, int64_t C, int64_t H, int64_t W, float t, const float* cap,
                        int64_t L, int64_t cap_dim, float* out);
// Times `steps` forwards (after `warmup`) on seeded inputs already on the
// device; *ms = mean milliseconds per forward (host clock around
// synchronised steps).
int sdhm_zimage_time(void* model, int64_t H, int64_t W, int64_t L, int64_t cap_dim, int steps, int warmup,
                     double* ms);
// Opt-in attention from block-scaled fp16 operands for later forwards (on != 0).
int sdhm_zimage_set_fp16_attention(void* model, int on);
int64_t sdhm_zimage_params(void* model);
void sdhm_zimage_free(void* model);
}

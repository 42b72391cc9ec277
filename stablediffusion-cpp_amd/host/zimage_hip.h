// zimage_hip.h - the Z-Image single-stream diffusion transformer (S3-DiT) on
// the MI355X: one denoising step, ZImageTransformer::forward of the reference
// (src/zimage.h:40-79, src/zimage.cpp:138-228), computed entirely on the
// device through backend_hip.
//
// The step (zimage.h:5-21): timestep embedding -> adaLN vector; image latent
// -> 2x2 patches -> tokens (padded to a multiple of 32 with x_pad_token), 2
// modulated noise-refiner blocks; text hidden states -> RMSNorm -> tokens
// (padded with cap_pad_token), 2 context-refiner blocks; the joint [image,
// text] sequence through the main blocks (30 heads of 128, RMS QK-norm,
// 3-axis rotary positions, SwiGLU); final LayerNorm * (1 + scale) -> linear
// -> unpatchify. Weights keep the checkpoint's names.
//
// Each block runs on backend_hip as the reference's run_block
// (zimage.cpp:90-136) with fused ops that give the same values: the four
// QK-norm / RoPE passes are one sdh_qknorm_rope launch; attention is the
// fused kernel; with BF16 weights RMSNorm * (1 + scale) emits the GEMMs' bf16
// A directly (one rounding for to_q, to_k, to_v), swiglu emits w2's bf16 A,
// and RMSNorm + gated residual is one pass over x.
#pragma once

#include <array>
#include <cstdint>
#include <string>
#include <vector>

#include "tensor_hip.h"
#include "weights_hip.h"

namespace sdh {

class ZImageTransformer {
public:
    // zimage.h:44-51: hyper-parameters not derivable from the weights.
    struct Config {
        int patch = 2;
        int heads = 30;
        float norm_eps = 1e-5f;
        float rope_theta = 256.0f;
        float t_scale = 1000.0f;
        int axes_dims[3] = {32, 48, 48};
    };
    // Shapes of a model, for Weights filled with random values (benchmarks).
    struct Shapes {
        int64_t dim = 3840, ffn = 10240, in_channels = 16, cap_dim = 2560, t_freq = 256, t_hidden = 1024,
                adaln_dim = 256;
        int heads = 30, patch = 2, noise_refiners = 2, context_refiners = 2, layers = 30;
    };
    // Adds every tensor of a model of `s` to w (N(0, 1/sqrt(fan-in)) linears,
    // N(1, 0.05) norm weights), BF16 from bf16_min_numel elements as the
    // pipeline loads Z-Image (pipeline.cpp:113).
    static void random_weights(Weights& w, const Shapes& s, uint64_t seed, int64_t bf16_min_numel = 1 << 20);

    explicit ZImageTransformer(const Weights& w);
    ZImageTransformer(const Weights& w, const Config& cfg);

    // x: [1, C, H, W] latent (H, W even); t in [0, 1]; cap: [1, L, cap_dim]
    // text hidden states; device tensors. Returns [1, C, H, W] on the device.
    Tensor forward(const Tensor& x, float t, const Tensor& cap) const;

    int in_channels() const { return in_channels_; }
    int64_t dim() const { return dim_; }

    // modules.h:23-30: a bound linear layer (weight [out, in], optional bias).
    struct Linear {
        const Tensor* W = nullptr;
        const Tensor* b = nullptr;
        Linear() = default;
        Linear(const Weights& w, const std::string& prefix);
        Tensor operator()(const Tensor& x) const { return linear(x, *W, b); }
        bool valid() const { return W != nullptr; }
    };

private:
    struct Block {
        const Tensor *attn_norm1, *attn_norm2, *ffn_norm1, *ffn_norm2, *norm_q, *norm_k;
        Linear to_q, to_k, to_v, to_out, w1, w2, w3;
        Linear adaln;  // modulated blocks only
    };
    Block load_block(const Weights& w, const std::string& prefix, bool modulated) const;
    void run_block(const Block& b, Tensor& x, const Tensor& cos, const Tensor& sin, const Tensor* adaln) const;
    // interleaved rotary tables [S, head_dim] for (axis0, h, w) positions, on the device
    void rope_tables(const std::vector<std::array<int, 3>>& pos, Tensor& cos, Tensor& sin) const;

    Config cfg_;
    int64_t dim_ = 0, head_dim_ = 0;
    int in_channels_ = 0;
    Linear x_embed_, cap_embed_, t_mlp0_, t_mlp2_, final_linear_, final_adaln_;
    const Tensor *cap_norm_ = nullptr, *x_pad_ = nullptr, *cap_pad_ = nullptr;
    std::vector<Block> noise_refiner_, context_refiner_, layers_;
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
int64_t sdhm_zimage_params(void* model);
void sdhm_zimage_free(void* model);
}

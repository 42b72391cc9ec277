// zimage_reference_timing.cpp - the reference's own Z-Image transformer
// (src/zimage.cpp, ZImageTransformer::forward, zimage.cpp:138-228) on
// backend_hip through the reference's backend interface
// (reference_backend_binding.cpp): what a user of the reference gets by
// linking this library in place of its CUDA backend, op by op, with none of
// this library's fused block ops.
//
// Built by oracle/Makefile (target suite) with the reference's zimage.cpp,
// modules.cpp, safetensors.cpp, json.cpp and tensor.cpp where they lie. The
// weights are random, in the checkpoint's names and shapes, generated in
// memory: linears of variance 1/fan-in as BF16 from 2^20 elements (as
// pipeline.cpp:113 keeps them), norms near 1, biases small.
//
//   zimage_reference_timing <device> <latent H> <latent W> <text tokens>
//                           <layers> <refiners> <steps>
//
// Times <steps> forwards after one warm-up, each ending with the output's
// download (the pipeline downloads every step's output, pipeline.cpp:234-237),
// and prints "ms per step" and the output's finiteness.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "safetensors.h"
#include "tensor.h"
#include "zimage.h"

namespace {

// A normal deviate from a counter (splitmix64 -> Box-Muller).
uint64_t mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
float normal(uint64_t seed, uint64_t i) {
    const uint64_t a = mix(seed * 0x100000001B3ull + 2 * i), b = mix(seed * 0x100000001B3ull + 2 * i + 1);
    const double u1 = ((a >> 11) + 1.0) * (1.0 / 9007199254740993.0), u2 = (b >> 11) * (1.0 / 9007199254740992.0);
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

// A uniform deviate of mean 0 and variance 1 from a counter: the weights'
// values (a timing run needs their scale, not their distribution).
float unit_uniform(uint64_t seed, uint64_t i) {
    return (float)((double)(mix(seed * 0x100000001B3ull + i) >> 40) * (1.0 / 16777216.0) * 3.4641016151377544 -
                   1.7320508075688772);
}

// Parallel fill of n values.
template <class F>
void fill(int64_t n, F&& put) {
    const int nt = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t)
        th.emplace_back([&, t] {
            for (int64_t i = n * t / nt; i < n * (t + 1) / nt; ++i) put(i);
        });
    for (auto& x : th) x.join();
}

void add(sd::Weights& w, const std::string& name, std::vector<int64_t> shape, uint64_t seed, float mean, float stdv,
         bool bf16_ok) {
    sd::Tensor t;
    t.shape = std::move(shape);
    const int64_t n = sd::Tensor::numel_of(t.shape);
    if (bf16_ok && n >= (int64_t(1) << 20)) {
        t.dtype = sd::DType::BF16;
        t.data16.resize((size_t)n);
        fill(n, [&](int64_t i) {
            const float f = mean + stdv * unit_uniform(seed, (uint64_t)i);
            uint32_t u;
            std::memcpy(&u, &f, 4);
            t.data16[(size_t)i] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);  // round to nearest even
        });
    } else {
        t.data.resize((size_t)n);
        fill(n, [&](int64_t i) { t.data[(size_t)i] = mean + stdv * unit_uniform(seed, (uint64_t)i); });
    }
    w.tensors[name] = std::move(t);
}

}  // namespace

int main(int argc, char** argv) {
    using namespace std::chrono;
    if (argc < 8) {
        std::fprintf(stderr, "usage: %s <cpu|cuda> <H> <W> <L> <layers> <refiners> <steps>\n", argv[0]);
        return 2;
    }
    const sd::Device dev = sd::parse_device(argv[1]);
    const int64_t H = std::atoll(argv[2]), W = std::atoll(argv[3]), L = std::atoll(argv[4]);
    const int layers = std::atoi(argv[5]), refiners = std::atoi(argv[6]), steps = std::atoi(argv[7]);
    // Z-Image's shapes; test_zimage.cpp builds the default Config (30 heads, axes 32 + 48 + 48)
    const int64_t D = 3840, F = 10240, C = 16, cap_dim = 2560, t_freq = 256, t_hidden = 1024, adaln = 256, hd = 128;
    auto t0 = steady_clock::now();
    sd::Weights w;
    uint64_t seed = 11;
    auto proj = [&](const std::string& p, int64_t out, int64_t in, bool bias) {
        add(w, p + ".weight", {out, in}, seed++, 0.0f, 1.0f / std::sqrt((float)in), true);
        if (bias) add(w, p + ".bias", {out}, seed++, 0.0f, 0.02f, false);
    };
    auto norm = [&](const std::string& p, int64_t n) { add(w, p, {n}, seed++, 1.0f, 0.05f, false); };
    proj("all_x_embedder.2-1", D, 4 * C, true);
    norm("cap_embedder.0.weight", cap_dim);
    proj("cap_embedder.1", D, cap_dim, true);
    proj("t_embedder.mlp.0", t_hidden, t_freq, true);
    proj("t_embedder.mlp.2", adaln, t_hidden, true);
    proj("all_final_layer.2-1.linear", 4 * C, D, true);
    proj("all_final_layer.2-1.adaLN_modulation.1", D, adaln, true);
    add(w, "x_pad_token", {1, D}, seed++, 0.0f, 1.0f, false);
    add(w, "cap_pad_token", {1, D}, seed++, 0.0f, 1.0f, false);
    auto block = [&](const std::string& p, bool modulated) {
        for (const char* n : {"attention_norm1", "attention_norm2", "ffn_norm1", "ffn_norm2"})
            norm(p + "." + n + ".weight", D);
        norm(p + ".attention.norm_q.weight", hd);
        norm(p + ".attention.norm_k.weight", hd);
        for (const char* n : {"to_q", "to_k", "to_v", "to_out.0"}) proj(p + ".attention." + n, D, D, false);
        proj(p + ".feed_forward.w1", F, D, false);
        proj(p + ".feed_forward.w2", D, F, false);
        proj(p + ".feed_forward.w3", F, D, false);
        if (modulated) proj(p + ".adaLN_modulation.0", 4 * D, adaln, true);
    };
    for (int i = 0; i < refiners; ++i) block("noise_refiner." + std::to_string(i), true);
    for (int i = 0; i < refiners; ++i) block("context_refiner." + std::to_string(i), false);
    for (int i = 0; i < layers; ++i) block("layers." + std::to_string(i), true);
    int64_t params = 0;
    for (const auto& kv : w.tensors) params += sd::Tensor::numel_of(kv.second.shape);
    w.to_device(dev);
    sd::ZImageTransformer tr(w);
    std::printf("%lld parameters built and placed on %s in %.1f s\n", (long long)params, sd::device_name(dev),
                duration<double>(steady_clock::now() - t0).count());

    sd::Tensor x({1, C, H, W}), cap({1, L, cap_dim});
    fill(x.numel(), [&](int64_t i) { x.data[(size_t)i] = normal(901, (uint64_t)i); });
    fill(cap.numel(), [&](int64_t i) { cap.data[(size_t)i] = normal(902, (uint64_t)i); });
    const sd::Tensor xd = x.to(dev), capd = cap.to(dev);
    sd::Tensor out = tr.forward(xd, 0.5f, capd).to(sd::Device::CPU);  // warm-up
    t0 = steady_clock::now();
    for (int s = 0; s < steps; ++s) out = tr.forward(xd, 0.5f, capd).to(sd::Device::CPU);
    const double ms = duration<double, std::milli>(steady_clock::now() - t0).count() / steps;
    bool finite = true;
    double asum = 0.0;
    for (int64_t i = 0; i < out.numel(); ++i) {
        finite = finite && std::isfinite(out.data[(size_t)i]);
        asum += std::fabs(out.data[(size_t)i]);
    }
    std::printf("forward %s, %lld text tokens, %d layers, %d refiners of each kind on %s: %.2f ms per step "
                "(%d steps); output mean |y| %.4g, %s\n",
                x.shape_str().c_str(), (long long)L, layers, refiners, sd::device_name(dev), ms, steps,
                asum / (double)out.numel(), finite ? "finite" : "NOT FINITE");
    return finite ? 0 : 1;
}

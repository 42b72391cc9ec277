// zimage_hip.cpp - see zimage_hip.h. The order of operations follows
// src/zimage.cpp (lines cited per step); the arithmetic is backend_hip's.
#include "zimage_hip.h"

#include <chrono>
#include <cmath>
#include <memory>
#include <stdexcept>
#include <string>

#include "sd_hip.hpp"

namespace sdh {
namespace {

constexpr int64_t kSeqMultiple = 32;  // zimage.cpp:28: sequences are padded to a multiple of 32
int64_t pad_to(int64_t n) { return (n + kSeqMultiple - 1) / kSeqMultiple * kSeqMultiple; }

// rows [n, D] followed by n_pad copies of the [1, D] pad token (zimage.cpp:31-35)
Tensor pad_rows(const Tensor& rows, const Tensor& pad, int64_t n_pad) {
    if (n_pad <= 0) return rows;
    return concat_batch(rows, repeat_batch(pad, n_pad));
}

}  // namespace

ZImageTransformer::Linear::Linear(const Weights& w, const std::string& prefix)
    : W(&w.get(prefix + ".weight")), b(w.try_get(prefix + ".bias")) {}

// zimage.cpp:38-47: the checkpoint's tensor names of one block
ZImageTransformer::Block ZImageTransformer::load_block(const Weights& w, const std::string& p, bool modulated) const {
    Block b{&w.get(p + ".attention_norm1.weight"),
            &w.get(p + ".attention_norm2.weight"),
            &w.get(p + ".ffn_norm1.weight"),
            &w.get(p + ".ffn_norm2.weight"),
            &w.get(p + ".attention.norm_q.weight"),
            &w.get(p + ".attention.norm_k.weight"),
            Linear(w, p + ".attention.to_q"),
            Linear(w, p + ".attention.to_k"),
            Linear(w, p + ".attention.to_v"),
            Linear(w, p + ".attention.to_out.0"),
            Linear(w, p + ".feed_forward.w1"),
            Linear(w, p + ".feed_forward.w2"),
            Linear(w, p + ".feed_forward.w3"),
            Linear()};
    if (modulated) b.adaln = Linear(w, p + ".adaLN_modulation.0");
    return b;
}

ZImageTransformer::ZImageTransformer(const Weights& w) : ZImageTransformer(w, Config()) {}

// zimage.cpp:51-68
ZImageTransformer::ZImageTransformer(const Weights& w, const Config& cfg)
    : cfg_(cfg),
      x_embed_(w, "all_x_embedder.2-1"),
      cap_embed_(w, "cap_embedder.1"),
      t_mlp0_(w, "t_embedder.mlp.0"),
      t_mlp2_(w, "t_embedder.mlp.2"),
      final_linear_(w, "all_final_layer.2-1.linear"),
      final_adaln_(w, "all_final_layer.2-1.adaLN_modulation.1"),
      cap_norm_(&w.get("cap_embedder.0.weight")),
      x_pad_(&w.get("x_pad_token")),
      cap_pad_(&w.get("cap_pad_token")) {
    dim_ = x_embed_.W->dim(0);
    head_dim_ = dim_ / cfg_.heads;
    in_channels_ = (int)(x_embed_.W->dim(1) / (cfg_.patch * cfg_.patch));
    if (cfg_.axes_dims[0] + cfg_.axes_dims[1] + cfg_.axes_dims[2] != head_dim_)
        throw std::runtime_error("Z-Image: axes_dims must sum to the head dim");
    for (int i = 0; w.has("noise_refiner." + std::to_string(i) + ".attention_norm1.weight"); ++i)
        noise_refiner_.push_back(load_block(w, "noise_refiner." + std::to_string(i), true));
    for (int i = 0; w.has("context_refiner." + std::to_string(i) + ".attention_norm1.weight"); ++i)
        context_refiner_.push_back(load_block(w, "context_refiner." + std::to_string(i), false));
    for (int i = 0; w.has("layers." + std::to_string(i) + ".attention_norm1.weight"); ++i)
        layers_.push_back(load_block(w, "layers." + std::to_string(i), true));
    if (layers_.empty()) throw std::runtime_error("Z-Image: no transformer layers found");
}

// zimage.cpp:71-88: per axis a, freq_k = theta^(-2k/d_a) in double, angle =
// (float)(position * freq_k); pair (2k, 2k+1) of the concatenated axes holds
// cos and sin of the angle twice (interleaved layout).
void ZImageTransformer::rope_tables(const std::vector<std::array<int, 3>>& pos, Tensor& cos, Tensor& sin) const {
    const int64_t S = (int64_t)pos.size(), d = head_dim_;
    Tensor c({S, d}), s({S, d});
    for (int64_t i = 0; i < S; ++i) {
        int64_t off = 0;
        for (int a = 0; a < 3; ++a) {
            const int da = cfg_.axes_dims[a];
            for (int k = 0; k < da / 2; ++k) {
                const double freq = 1.0 / std::pow((double)cfg_.rope_theta, (double)(2 * k) / (double)da);
                const float ang = (float)((double)pos[i][a] * freq);
                c.data[i * d + off + 2 * k] = c.data[i * d + off + 2 * k + 1] = std::cos(ang);
                s.data[i * d + off + 2 * k] = s.data[i * d + off + 2 * k + 1] = std::sin(ang);
            }
            off += da;
        }
    }
    cos = c.to(Device::HIP);
    sin = s.to(Device::HIP);
}

// zimage.cpp:90-136
void ZImageTransformer::run_block(const Block& b, Tensor& x, const Tensor& cos, const Tensor& sin,
                                  const Tensor* adaln) const {
    const int64_t D = dim_;
    // modulation: mod [1, 4D] = scale_msa | gate_msa | scale_mlp | gate_mlp,
    // scales as 1 + s and gates as tanh(g) (zimage.cpp:96-113)
    Tensor scale_msa, gate_msa, scale_mlp, gate_mlp;
    const bool mod = b.adaln.valid();
    if (mod) {
        Tensor m = b.adaln(*adaln);
        m.reshape({4, D});
        // views, not copies: each row only feeds the in-place op that follows
        scale_msa = rows_view(m, 0, 1);
        gate_msa = rows_view(m, 1, 2);
        scale_mlp = rows_view(m, 2, 3);
        gate_mlp = rows_view(m, 3, 4);
        affine_(scale_msa, 1.0f, 1.0f);
        affine_(scale_mlp, 1.0f, 1.0f);
        tanh_(gate_msa);
        tanh_(gate_mlp);
        scale_msa.reshape({D});
        gate_msa.reshape({D});
        scale_mlp.reshape({D});
        gate_mlp.reshape({D});
    }
    const bool all_bf16 = b.to_q.W->is_bf16() && b.to_k.W->is_bf16() && b.to_v.W->is_bf16() &&
                          b.to_out.W->is_bf16() && b.w1.W->is_bf16() && b.w2.W->is_bf16() && b.w3.W->is_bf16();
    if (all_bf16) {
        // BF16 weights: the same values through the fused ops, each equal to the
        // sequence it replaces bit for bit. The normalised, modulated rows are
        // emitted as the GEMMs' bf16 A once for to_q, to_k and to_v (and once
        // for w1, w3), attention and swiglu emit the bf16 A of to_out and w2,
        // and the norm + gated residual after to_out and w2 is one pass over x.
        Tensor h16 = rms_norm_modulate_bf16(x, b.attn_norm1, mod ? &scale_msa : nullptr, cfg_.norm_eps);
        Tensor q = b.to_q(h16), k = b.to_k(h16), v = b.to_v(h16);
        qknorm_rope_(q, k, head_dim_, b.norm_q, b.norm_k, 1e-5f, cos, sin, true);
        Tensor a = b.to_out(attention_bf16(q, k, v, cfg_.heads, false));
        rms_norm_gated_add_(x, a, b.attn_norm2, mod ? &gate_msa : nullptr, cfg_.norm_eps);
        h16 = rms_norm_modulate_bf16(x, b.ffn_norm1, mod ? &scale_mlp : nullptr, cfg_.norm_eps);
        Tensor f = b.w2(swiglu_bf16(b.w1(h16), b.w3(h16)));
        rms_norm_gated_add_(x, f, b.ffn_norm2, mod ? &gate_mlp : nullptr, cfg_.norm_eps);
        return;
    }
    // attention (zimage.cpp:115-127)
    Tensor h = rms_norm(x, b.attn_norm1, cfg_.norm_eps);
    if (mod) mul_rows_(h, scale_msa);
    Tensor q = b.to_q(h), k = b.to_k(h), v = b.to_v(h);
    // rms_norm_heads_(q), rms_norm_heads_(k), rope_(q), rope_(k) in one launch
    qknorm_rope_(q, k, head_dim_, b.norm_q, b.norm_k, 1e-5f, cos, sin, true);
    Tensor a = b.to_out(attention(q, k, v, cfg_.heads, false));
    a = rms_norm(a, b.attn_norm2, cfg_.norm_eps);
    if (mod)
        add_rows_scaled_(x, a, gate_msa);
    else
        add_(x, a);
    // feed-forward (zimage.cpp:128-135)
    h = rms_norm(x, b.ffn_norm1, cfg_.norm_eps);
    if (mod) mul_rows_(h, scale_mlp);
    Tensor g = (b.w1.W->is_bf16() && b.w3.W->is_bf16() && !b.w1.b && !b.w3.b) ? linear_swiglu(h, *b.w1.W, *b.w3.W)
                                                                                : swiglu(b.w1(h), b.w3(h));
    Tensor f = b.w2(g);
    f = rms_norm(f, b.ffn_norm2, cfg_.norm_eps);
    if (mod)
        add_rows_scaled_(x, f, gate_mlp);
    else
        add_(x, f);
}

// zimage.cpp:138-228
Tensor ZImageTransformer::forward(const Tensor& x_in, float t, const Tensor& cap_in) const {
    const int64_t C = x_in.dim(1), H = x_in.dim(2), W = x_in.dim(3), p = cfg_.patch, D = dim_;
    if (x_in.dim(0) != 1 || cap_in.dim(0) != 1) throw std::runtime_error("Z-Image: batch size must be 1");
    if (C != in_channels_ || H % p || W % p) throw std::runtime_error("Z-Image: bad latent shape " + x_in.shape_str());
    if (!x_in.is_hip() || !cap_in.is_hip()) throw std::runtime_error("Z-Image: latent and text must be device tensors");
    const int64_t Ht = H / p, Wt = W / p, n_img = Ht * Wt, n_img_pad = pad_to(n_img);
    const int64_t n_cap = cap_in.dim(1), n_cap_pad = pad_to(n_cap);

    // 1. timestep embedding -> adaln (zimage.cpp:148-163): sinusoid in float, MLP with SiLU
    Tensor adaln;
    {
        const int64_t F = t_mlp0_.W->dim(1), half = F / 2;
        Tensor freq({1, F});
        const float tt = t * cfg_.t_scale;
        for (int64_t i = 0; i < half; ++i) {
            const float f = std::exp(-std::log(10000.0f) * (float)i / (float)half);
            freq.data[i] = std::cos(tt * f);
            freq.data[half + i] = std::sin(tt * f);
        }
        adaln = t_mlp0_(freq.to(Device::HIP));
        silu_(adaln);
        adaln = t_mlp2_(adaln);
    }

    // 2. image tokens: patchify (features ordered ph, pw, c), embed, pad (zimage.cpp:166-169)
    Tensor img = x_embed_(patchify2d(x_in, (int)p));
    Tensor img_seq = pad_rows(img, *x_pad_, n_img_pad - n_img);
    img_seq.reshape({1, n_img_pad, D});

    // 3. text tokens: RMSNorm, embed, pad (zimage.cpp:172-175)
    Tensor cap = cap_embed_(rms_norm(cap_in, cap_norm_, cfg_.norm_eps));
    cap.reshape({n_cap, D});
    Tensor cap_seq = pad_rows(cap, *cap_pad_, n_cap_pad - n_cap);
    cap_seq.reshape({1, n_cap_pad, D});

    // rotary positions (zimage.cpp:177-191): text (1 + i, 0, 0) for every row
    // including its pad; image (n_cap_pad + 1, h, w); image pad rows (0, 0, 0)
    std::vector<std::array<int, 3>> cap_pos(n_cap_pad, {0, 0, 0}), img_pos(n_img_pad, {0, 0, 0});
    for (int64_t i = 0; i < n_cap_pad; ++i) cap_pos[i] = {(int)(1 + i), 0, 0};
    for (int64_t hh = 0; hh < Ht; ++hh)
        for (int64_t ww = 0; ww < Wt; ++ww) img_pos[hh * Wt + ww] = {(int)(n_cap_pad + 1), (int)hh, (int)ww};
    Tensor img_cos, img_sin, cap_cos, cap_sin;
    rope_tables(img_pos, img_cos, img_sin);
    rope_tables(cap_pos, cap_cos, cap_sin);

    // refiners (zimage.cpp:194-201)
    for (const Block& b : noise_refiner_) run_block(b, img_seq, img_cos, img_sin, &adaln);
    for (const Block& b : context_refiner_) run_block(b, cap_seq, cap_cos, cap_sin, nullptr);

    // 4. the unified sequence [image, text] through the main stack (zimage.cpp:204-215)
    Tensor uni = concat_batch(img_seq.reshape({n_img_pad, D}), cap_seq.reshape({n_cap_pad, D}));
    uni.reshape({1, n_img_pad + n_cap_pad, D});
    std::vector<std::array<int, 3>> uni_pos = img_pos;
    uni_pos.insert(uni_pos.end(), cap_pos.begin(), cap_pos.end());
    Tensor uni_cos, uni_sin;
    rope_tables(uni_pos, uni_cos, uni_sin);
    for (const Block& b : layers_) run_block(b, uni, uni_cos, uni_sin, &adaln);

    // 5. final layer on the image tokens, unpatchify (zimage.cpp:218-227)
    Tensor img_out = slice_rows(uni, 0, n_img);
    Tensor c = adaln;
    silu_(c);
    Tensor scale = final_adaln_(c);
    affine_(scale, 1.0f, 1.0f);
    scale.reshape({D});
    img_out = layer_norm(img_out, nullptr, nullptr, 1e-6f);
    mul_rows_(img_out, scale);
    Tensor out_tok = final_linear_(img_out);
    return unpatchify2d(out_tok, C, H, W, (int)p);
}

void ZImageTransformer::random_weights(Weights& w, const Shapes& s, uint64_t seed, int64_t mn) {
    uint64_t k = seed;
    auto lin = [&](const std::string& p, int64_t out, int64_t in, bool bias) {
        w.add_random(p + ".weight", {out, in}, k++, 0.0f, 1.0f / std::sqrt((float)in), true, mn);
        if (bias) w.add_random(p + ".bias", {out}, k++, 0.0f, 0.02f);
    };
    auto norm = [&](const std::string& name, int64_t n) { w.add_random(name, {n}, k++, 1.0f, 0.05f); };
    const int64_t D = s.dim, hd = s.dim / s.heads, pp = (int64_t)s.patch * s.patch;
    lin("all_x_embedder.2-1", D, pp * s.in_channels, true);
    norm("cap_embedder.0.weight", s.cap_dim);
    lin("cap_embedder.1", D, s.cap_dim, true);
    lin("t_embedder.mlp.0", s.t_hidden, s.t_freq, true);
    lin("t_embedder.mlp.2", s.adaln_dim, s.t_hidden, true);
    lin("all_final_layer.2-1.linear", pp * s.in_channels, D, true);
    lin("all_final_layer.2-1.adaLN_modulation.1", D, s.adaln_dim, true);
    w.add_random("x_pad_token", {1, D}, k++, 0.0f, 1.0f);
    w.add_random("cap_pad_token", {1, D}, k++, 0.0f, 1.0f);
    auto block = [&](const std::string& p, bool modulated) {
        norm(p + ".attention_norm1.weight", D);
        norm(p + ".attention_norm2.weight", D);
        norm(p + ".ffn_norm1.weight", D);
        norm(p + ".ffn_norm2.weight", D);
        norm(p + ".attention.norm_q.weight", hd);
        norm(p + ".attention.norm_k.weight", hd);
        lin(p + ".attention.to_q", D, D, false);
        lin(p + ".attention.to_k", D, D, false);
        lin(p + ".attention.to_v", D, D, false);
        lin(p + ".attention.to_out.0", D, D, false);
        lin(p + ".feed_forward.w1", s.ffn, D, false);
        lin(p + ".feed_forward.w2", D, s.ffn, false);
        lin(p + ".feed_forward.w3", s.ffn, D, false);
        if (modulated) lin(p + ".adaLN_modulation.0", 4 * D, s.adaln_dim, true);
    };
    for (int i = 0; i < s.noise_refiners; ++i) block("noise_refiner." + std::to_string(i), true);
    for (int i = 0; i < s.context_refiners; ++i) block("context_refiner." + std::to_string(i), false);
    for (int i = 0; i < s.layers; ++i) block("layers." + std::to_string(i), true);
}

}  // namespace sdh

// ---- C entry points -----------------------------------------------------------
namespace {
thread_local std::string g_err;
struct Model {
    sdh::Weights w;
    std::unique_ptr<sdh::ZImageTransformer> m;
};
template <class F>
int guard(F&& f) {
    try {
        g_err.clear();
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}
}  // namespace

extern "C" {

const char* sdhm_last_error(void) { return g_err.c_str(); }

int sdhm_zimage_load(const char* path, int keep_bf16, int64_t bf16_min_numel, int heads, void** model) {
    return guard([&] {
        auto md = std::make_unique<Model>();
        md->w.load_safetensors(path, keep_bf16 != 0, bf16_min_numel);
        sdh::ZImageTransformer::Config cfg;
        cfg.heads = heads;
        md->m = std::make_unique<sdh::ZImageTransformer>(md->w, cfg);
        *model = md.release();
    });
}

int sdhm_zimage_random(int64_t dim, int heads, int64_t ffn, int64_t in_channels, int64_t cap_dim, int64_t t_hidden,
                       int64_t adaln_dim, int noise_refiners, int context_refiners, int layers, uint64_t seed,
                       void** model) {
    return guard([&] {
        sdh::ZImageTransformer::Shapes s;
        s.dim = dim;
        s.heads = heads;
        s.ffn = ffn;
        s.in_channels = in_channels;
        s.cap_dim = cap_dim;
        s.t_hidden = t_hidden;
        s.adaln_dim = adaln_dim;
        s.noise_refiners = noise_refiners;
        s.context_refiners = context_refiners;
        s.layers = layers;
        auto md = std::make_unique<Model>();
        sdh::ZImageTransformer::random_weights(md->w, s, seed);
        sdh::ZImageTransformer::Config cfg;
        cfg.heads = heads;
        md->m = std::make_unique<sdh::ZImageTransformer>(md->w, cfg);
        *model = md.release();
    });
}

int sdhm_zimage_forward(void* model, const float* x, int64_t C, int64_t H, int64_t W, float t, const float* cap,
                        int64_t L, int64_t cap_dim, float* out) {
    return guard([&] {
        const Model* md = static_cast<const Model*>(model);
        sdh::Tensor xh({1, C, H, W}), ch({1, L, cap_dim});
        std::copy(x, x + xh.numel(), xh.data.begin());
        std::copy(cap, cap + ch.numel(), ch.data.begin());
        sdh::Tensor y = md->m->forward(xh.to(sdh::Device::HIP), t, ch.to(sdh::Device::HIP)).to(sdh::Device::CPU);
        std::copy(y.data.begin(), y.data.end(), out);
    });
}

int sdhm_zimage_time(void* model, int64_t H, int64_t W, int64_t L, int64_t cap_dim, int steps, int warmup,
                     double* ms) {
    return guard([&] {
        const Model* md = static_cast<const Model*>(model);
        sdh::Tensor x = sdh::Tensor::empty({1, md->m->in_channels(), H, W}, sdh::Device::HIP);
        sdh::Tensor cap = sdh::Tensor::empty({1, L, cap_dim}, sdh::Device::HIP);
        sd::hip::fill_normal(x.dptr(), x.numel(), 91, 0.0f, 1.0f);
        sd::hip::fill_normal(cap.dptr(), cap.numel(), 92, 0.0f, 1.0f);
        for (int i = 0; i < warmup; ++i) md->m->forward(x, 0.5f, cap);
        sd::hip::synchronize();
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; ++i) md->m->forward(x, 0.5f, cap);
        sd::hip::synchronize();
        *ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() /
              (steps > 0 ? steps : 1);
    });
}

int64_t sdhm_zimage_params(void* model) { return (int64_t) static_cast<Model*>(model)->w.total_params(); }

void sdhm_zimage_free(void* model) { delete static_cast<Model*>(model); }

}  // extern "C"

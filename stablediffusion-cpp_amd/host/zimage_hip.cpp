// zimage_hip.cpp - one Z-Image denoising step on the device (see
// zimage_hip.h for the design). The function computed is the reference's
// ZImageTransformer::forward (src/zimage.cpp:138-228): the same checkpoint
// tensors, the same order of operations and the same rotary positions; the
// code below is organised around this library's token buffer, cached rotary
// tables and fused block ops.
#include "zimage_hip.h"

#include <algorithm>
#include <atomic>
#include <cctype>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <fstream>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "sd_hip.hpp"

namespace sdh {
namespace {

// ---- the checkpoint's layout ---------------------------------------------------
// A block's tensors by role. The strings are the checkpoint's module names
// (the file format; zimage.cpp:38-47 reads the same ones).
enum NormRole { kNormAttnIn, kNormAttnOut, kNormFfnIn, kNormFfnOut, kNormQ, kNormK, kNormRoles };
enum ProjRole { kProjQ, kProjK, kProjV, kProjOut, kProjGate, kProjDown, kProjUp, kProjMod, kProjRoles };
const char* const kNormName[kNormRoles] = {"attention_norm1", "attention_norm2", "ffn_norm1",
                                           "ffn_norm2",       "attention.norm_q", "attention.norm_k"};
const char* const kProjName[kProjRoles] = {"attention.to_q",  "attention.to_k",  "attention.to_v",
                                           "attention.to_out.0", "feed_forward.w1", "feed_forward.w2",
                                           "feed_forward.w3", "adaLN_modulation.0"};

// The block stacks in the order a step runs them. The noise refiner (image
// tokens) and the main stack are modulated by the timestep; the context
// refiner (text tokens) is not.
enum Stack { kNoiseRefiner, kContextRefiner, kMainStack, kStacks };
const char* const kStackName[kStacks] = {"noise_refiner", "context_refiner", "layers"};
const bool kStackModulated[kStacks] = {true, false, true};

// Token counts are padded up to a multiple of 32 with the pad tokens
// (transformer_z_image.py's SEQ_MULTI_OF, zimage.cpp:28).
constexpr int64_t kTokenGranule = 32;
int64_t padded(int64_t n) { return (n + kTokenGranule - 1) / kTokenGranule * kTokenGranule; }

// QK-norm's eps is a literal in the model, not config.json's norm_eps
// (zimage.cpp:117-118).
constexpr float kQkNormEps = 1e-5f;
// The final LayerNorm: no affine, eps 1e-6 (zimage.cpp:223).
constexpr float kHeadNormEps = 1e-6f;

struct Proj {
    const Tensor* W = nullptr;
    const Tensor* b = nullptr;
};

struct BlockBinding {
    const Tensor* norm[kNormRoles] = {};
    Proj proj[kProjRoles];
    bool modulated = false;
    // Every projection but the modulation is BF16: the block runs the fused
    // ops (the normalised rows emitted as the GEMMs' bf16 A, attention and
    // SwiGLU emitting the next GEMM's bf16 A), which give the values of the
    // op sequence they replace.
    bool fused_bf16 = false;
};

// Rows of one step's token buffer: image tokens, image pads, text tokens,
// text pads.
struct TokenLayout {
    int64_t grid_h = 0, grid_w = 0;  // patches down and across
    int64_t img = 0, img_rows = 0;   // image tokens, and with their pads
    int64_t txt = 0, txt_rows = 0;   // text tokens, and with their pads
    int64_t rows() const { return img_rows + txt_rows; }
};

// Blocks in a stack: one past the largest "<stack>.<index>." any weight name has.
int64_t stack_depth(const Weights& w, const std::string& stack) {
    const std::string head = stack + ".";
    int64_t depth = 0;
    for (const auto& kv : w.tensors) {
        const std::string& name = kv.first;
        if (name.compare(0, head.size(), head) != 0) continue;
        size_t i = head.size();
        int64_t idx = 0;
        while (i < name.size() && std::isdigit((unsigned char)name[i]) && idx < (int64_t(1) << 40))
            idx = idx * 10 + (name[i++] - '0');
        if (i > head.size() && i < name.size() && name[i] == '.') depth = std::max(depth, idx + 1);
    }
    return depth;
}

// y = x W^T (+ b) written into `out`, which already has x's rows and W's
// outputs (a row range of a bigger device tensor): the embedders fill their
// rows of the token buffer without an intermediate tensor.
void project_into(const Tensor& x, const Proj& p, Tensor& out, const char* what) {
    const int64_t in = x.dim(-1), n = p.W->dim(0), rows = x.numel() / (in > 0 ? in : 1);
    if (p.W->dim(1) != in || out.numel() != rows * n)
        throw std::runtime_error(std::string("ZImageTransformer: ") + what + " takes " + std::to_string(p.W->dim(1)) +
                                 " features per token, the input has " + x.shape_str());
    const float* bias = p.b ? p.b->dptr() : nullptr;
    if (p.W->is_bf16())
        sd::hip::gemm_nt_bf16(rows, n, in, x.dptr(), in, p.W->dptr16(), in, out.dptr(), n, bias, false);
    else
        sd::hip::gemm_nt_f32(rows, n, in, x.dptr(), in, p.W->dptr(), in, out.dptr(), n, bias, false);
}

// Rows [from, to) of a [rows, D] device tensor set to a [1, D] token: one
// copy of the token, then copies of the rows written so far, doubling.
// With ZIMAGE_TRACE=<prefix> set, named intermediates of a forward are
// written as <prefix>_trace_<name>.bin (float32 rows) and .json ({"shape":
// [rows, cols]}), at the points and under the names the reference's
// forward uses (zimage.cpp:15-26), so the two can be compared stage by
// stage. Tensors are downloaded only when the variable is set.
void trace(const char* name, const Tensor& t) {
    const char* prefix = std::getenv("ZIMAGE_TRACE");
    if (!prefix || !*prefix) return;
    const Tensor h = t.is_hip() ? t.to(Device::CPU) : t;
    const std::string base = std::string(prefix) + "_trace_" + name;
    std::ofstream bin(base + ".bin", std::ios::binary);
    bin.write(reinterpret_cast<const char*>(h.ptr()), (std::streamsize)(h.numel() * (int64_t)sizeof(float)));
    std::ofstream js(base + ".json");
    const int64_t cols = h.ndim() ? h.dim(-1) : 1;
    js << "{\"shape\": [" << (cols ? h.numel() / cols : 0) << ", " << cols << "]}";
    if (!bin || !js) throw std::runtime_error("ZIMAGE_TRACE: cannot write " + base);
}

void fill_rows(Tensor& buf, int64_t from, int64_t to, const Tensor& token) {
    const int64_t D = buf.dim(-1), n = to - from;
    if (n <= 0) return;
    if (token.numel() != D) throw std::runtime_error("ZImageTransformer: a pad token must have dim features");
    float* base = buf.dptr() + from * D;
    sd::hip::copy(base, token.dptr(), (size_t)D * sizeof(float));
    for (int64_t done = 1; done < n; done *= 2)
        sd::hip::copy(base + done * D, base, (size_t)(std::min(done, n - done) * D) * sizeof(float));
}

Tensor as_sequence(Tensor rows) {
    rows.reshape({1, rows.dim(0), rows.dim(1)});
    return rows;
}

}  // namespace

struct ZImageTransformer::Impl {
    Config cfg;
    std::atomic<bool> fp16_attention{false};  // opt-in: attention from block-scaled fp16 operands
    int64_t dim = 0, head_dim = 0;
    int channels = 0;
    Proj patch_embed, text_embed, t_in, t_out, head_mod, head_out;
    const Tensor *text_norm = nullptr, *img_pad = nullptr, *txt_pad = nullptr;
    std::vector<BlockBinding> stacks[kStacks];
    std::vector<float> t_freq;         // timestep sinusoid: frequency i of F/2
    std::vector<double> pair_freq;     // rotary pair k: theta^(-2j/d_a) for its axis a and index j in it
    std::vector<int> pair_axis;        // rotary pair k: the position axis it turns with
    mutable std::mutex rotary_mu;      // the cache below is filled by const forward calls
    mutable std::map<std::tuple<int64_t, int64_t, int64_t>, std::pair<Tensor, Tensor>> rotary_cache;

    explicit Impl(const Config& c) : cfg(c), fp16_attention(c.fp16_attention) {}

    Proj bind_proj(const Weights& w, const std::string& name) const {
        return Proj{&w.get(name + ".weight"), w.try_get(name + ".bias")};
    }

    BlockBinding bind_block(const Weights& w, const std::string& prefix, bool modulated) const {
        BlockBinding b;
        b.modulated = modulated;
        for (int r = 0; r < kNormRoles; ++r) b.norm[r] = &w.get(prefix + "." + kNormName[r] + ".weight");
        for (int r = 0; r < kProjRoles; ++r)
            if (r != kProjMod || modulated) b.proj[r] = bind_proj(w, prefix + "." + kProjName[r]);
        b.fused_bf16 = true;
        for (int r = 0; r < kProjMod; ++r) b.fused_bf16 = b.fused_bf16 && b.proj[r].W->is_bf16();
        return b;
    }

    void bind(const Weights& w) {
        patch_embed = bind_proj(w, "all_x_embedder.2-1");
        text_norm = &w.get("cap_embedder.0.weight");
        text_embed = bind_proj(w, "cap_embedder.1");
        t_in = bind_proj(w, "t_embedder.mlp.0");
        t_out = bind_proj(w, "t_embedder.mlp.2");
        head_out = bind_proj(w, "all_final_layer.2-1.linear");
        head_mod = bind_proj(w, "all_final_layer.2-1.adaLN_modulation.1");
        img_pad = &w.get("x_pad_token");
        txt_pad = &w.get("cap_pad_token");
        const int64_t pp = (int64_t)cfg.patch * cfg.patch;
        dim = patch_embed.W->dim(0);
        if (cfg.heads <= 0 || dim % cfg.heads)
            throw std::runtime_error("ZImageTransformer: model width " + std::to_string(dim) + " is not a multiple of " +
                                     std::to_string(cfg.heads) + " heads");
        head_dim = dim / cfg.heads;
        channels = (int)(patch_embed.W->dim(1) / pp);
        const int64_t axes = (int64_t)cfg.axes_dims[0] + cfg.axes_dims[1] + cfg.axes_dims[2];
        if (axes != head_dim)
            throw std::runtime_error("ZImageTransformer: rotary axes of " + std::to_string(axes) +
                                     " channels for heads of " + std::to_string(head_dim));
        for (int s = 0; s < kStacks; ++s) {
            const int64_t n = stack_depth(w, kStackName[s]);
            for (int64_t i = 0; i < n; ++i)
                stacks[s].push_back(bind_block(w, std::string(kStackName[s]) + "." + std::to_string(i), kStackModulated[s]));
        }
        if (stacks[kMainStack].empty())
            throw std::runtime_error("ZImageTransformer: the weights hold no main-stack block (layers.<i>.*)");

        // timestep sinusoid frequencies, in float as the model forms them (zimage.cpp:152-153)
        const int64_t half = t_in.W->dim(1) / 2;
        for (int64_t i = 0; i < half; ++i) t_freq.push_back(std::exp(-std::log(10000.0f) * (float)i / (float)half));
        // rotary pair frequencies per axis in double (zimage.cpp:80)
        for (int a = 0; a < 3; ++a)
            for (int j = 0; j < cfg.axes_dims[a] / 2; ++j) {
                pair_freq.push_back(1.0 / std::pow((double)cfg.rope_theta, (double)(2 * j) / (double)cfg.axes_dims[a]));
                pair_axis.push_back(a);
            }
    }

    TokenLayout layout(const Tensor& latent, const Tensor& text) const {
        if (!latent.is_hip() || !text.is_hip())
            throw std::runtime_error("ZImageTransformer::forward: latent and text must be device tensors");
        if (latent.ndim() != 4 || latent.dim(0) != 1 || text.ndim() != 3 || text.dim(0) != 1)
            throw std::runtime_error("ZImageTransformer::forward: one sample at a time: latent [1, C, H, W] and text "
                                     "[1, L, features], got " + latent.shape_str() + " and " + text.shape_str());
        const int64_t p = cfg.patch;
        if (latent.dim(1) != channels || latent.dim(2) % p || latent.dim(3) % p)
            throw std::runtime_error("ZImageTransformer::forward: the latent needs " + std::to_string(channels) +
                                     " channels and sides that are multiples of " + std::to_string(p) + ", got " +
                                     latent.shape_str());
        TokenLayout g;
        g.grid_h = latent.dim(2) / p;
        g.grid_w = latent.dim(3) / p;
        g.img = g.grid_h * g.grid_w;
        g.img_rows = padded(g.img);
        g.txt = text.dim(1);
        g.txt_rows = padded(g.txt);
        return g;
    }

    // The adaLN conditioning vector [1, adaln_dim] of timestep t (zimage.cpp:148-163).
    Tensor condition(float t) const {
        const int64_t half = (int64_t)t_freq.size();
        Tensor v({1, 2 * half});
        const float tt = t * cfg.t_scale;
        for (int64_t i = 0; i < half; ++i) {
            v.data[i] = std::cos(tt * t_freq[i]);
            v.data[half + i] = std::sin(tt * t_freq[i]);
        }
        Tensor h = linear(v.to(Device::HIP), *t_in.W, t_in.b);
        silu_(h);
        return linear(h, *t_out.W, t_out.b);
    }

    // Interleaved rotary tables [rows, head_dim] of a token layout, built on
    // the first call with that layout. Row positions (axis 0, 1, 2)
    // (zimage.cpp:177-191): image token (txt_rows + 1, row, column) of the
    // patch grid; image pad (0, 0, 0); text row j, pads included, (1 + j, 0, 0).
    // Pair k of a row turns by the float angle position[axis(k)] * freq(k)
    // formed in double, cos and sin stored twice (zimage.cpp:81-83).
    const std::pair<Tensor, Tensor>& rotary(const TokenLayout& g) const {
        std::lock_guard<std::mutex> lk(rotary_mu);
        const auto key = std::make_tuple(g.grid_h, g.grid_w, g.txt_rows);
        auto it = rotary_cache.find(key);
        if (it != rotary_cache.end()) return it->second;
        const int64_t rows = g.rows(), hd = head_dim, pairs = (int64_t)pair_freq.size();
        Tensor c({rows, hd}), s({rows, hd});
        for (int64_t r = 0; r < rows; ++r) {
            int64_t pos[3] = {0, 0, 0};
            if (r < g.img) {
                pos[0] = g.txt_rows + 1;
                pos[1] = r / g.grid_w;
                pos[2] = r % g.grid_w;
            } else if (r >= g.img_rows) {
                pos[0] = 1 + (r - g.img_rows);
            }
            float* cr = c.data.data() + r * hd;
            float* sr = s.data.data() + r * hd;
            for (int64_t k = 0; k < pairs; ++k) {
                const float ang = (float)((double)pos[pair_axis[k]] * pair_freq[k]);
                cr[2 * k] = cr[2 * k + 1] = std::cos(ang);
                sr[2 * k] = sr[2 * k + 1] = std::sin(ang);
            }
        }
        return rotary_cache.emplace(key, std::make_pair(c.to(Device::HIP), s.to(Device::HIP))).first->second;
    }

    // The token buffer's rows: patch embeddings, image pads, embedded
    // (RMS-normalised) text, text pads (zimage.cpp:165-175).
    void embed(const Tensor& latent, const Tensor& text, const TokenLayout& g, Tensor& seq) const {
        Tensor img = rows_view(seq, 0, g.img);
        project_into(patchify2d(latent, cfg.patch), patch_embed, img, "the patch embedder");
        trace("x_embed", img);
        fill_rows(seq, g.img, g.img_rows, *img_pad);
        Tensor txt = rows_view(seq, g.img_rows, g.img_rows + g.txt);
        project_into(rms_norm(text, text_norm, cfg.norm_eps), text_embed, txt, "the text embedder");
        trace("cap_embed", txt);
        fill_rows(seq, g.img_rows + g.txt, g.rows(), *txt_pad);
    }

    // The input of a sublayer: rms_norm(x) * (1 + scale), as the BF16 GEMM
    // operand on the fused path.
    Tensor sublayer_input(const BlockBinding& b, const Tensor& x, NormRole n, const Tensor* scale) const {
        if (b.fused_bf16) return rms_norm_modulate_bf16(x, b.norm[n], scale, cfg.norm_eps);
        Tensor h = rms_norm(x, b.norm[n], cfg.norm_eps);
        if (scale) mul_rows_(h, *scale);
        return h;
    }

    Tensor project(const Tensor& x, const BlockBinding& b, ProjRole r) const {
        return linear(x, *b.proj[r].W, b.proj[r].b);
    }

    // Self-attention with QK-norm and rotary positions, then to_out (zimage.cpp:116-122).
    Tensor attend(const BlockBinding& b, const Tensor& in, const Tensor& cos, const Tensor& sin) const {
        Tensor q = project(in, b, kProjQ), k = project(in, b, kProjK), v = project(in, b, kProjV);
        // QK-norm, rotary and attention in one entry point (k's normalised
        // rows go straight into the attention's packed tiles); the output is
        // to_out's bf16 A on the fused path
        const Tensor o = qknorm_rope_attention_(q, k, v, cfg.heads, head_dim, b.norm[kNormQ], b.norm[kNormK],
                                                kQkNormEps, cos, sin, b.fused_bf16,
                                                fp16_attention.load(std::memory_order_relaxed));
        return project(o, b, kProjOut);
    }

    // w2(silu(w1 x) * w3 x) (zimage.cpp:130).
    Tensor feed_forward(const BlockBinding& b, const Tensor& in) const {
        const Proj &gate = b.proj[kProjGate], &up = b.proj[kProjUp];
        Tensor hidden;
        if (b.fused_bf16)
            hidden = swiglu_bf16(project(in, b, kProjGate), project(in, b, kProjUp));
        else if (gate.W->is_bf16() && up.W->is_bf16() && !gate.b && !up.b)
            hidden = linear_swiglu(in, *gate.W, *up.W);
        else
            hidden = swiglu(project(in, b, kProjGate), project(in, b, kProjUp));
        return project(hidden, b, kProjDown);
    }

    // A block's modulation rows (zimage.cpp:104-107): 1 + scale and tanh(gate)
    // for the attention and the FFN sublayer; none for unmodulated blocks.
    struct Modulation {
        Tensor mod;  // [4, dim]: attention scale, attention gate, FFN scale, FFN gate
        Tensor scale[2], gate[2];
        bool on = false;
        const Tensor* scale_of(int s) const { return on ? &scale[s] : nullptr; }
        const Tensor* gate_of(int s) const { return on ? &gate[s] : nullptr; }
    };

    Modulation modulation(const BlockBinding& b, const Tensor* cond) const {
        Modulation m;
        if (!b.modulated) return m;
        m.on = true;
        m.mod = project(*cond, b, kProjMod);
        m.mod.reshape({4, dim});
        modulation_rows_(m.mod);  // 1 + scale, tanh(gate): one launch
        for (int s = 0; s < 2; ++s) {
            m.scale[s] = rows_view(m.mod, 2 * s, 2 * s + 1);
            m.gate[s] = rows_view(m.mod, 2 * s + 1, 2 * s + 2);
            m.scale[s].reshape({dim});
            m.gate[s].reshape({dim});
        }
        return m;
    }

    // Closes a sublayer of block b: x += gate * rms_norm(out). With next, also
    // returns the input of the sublayer that follows (next's norm role nn,
    // modulated by scale); in one pass over x when both blocks run fused.
    Tensor close_sublayer(const BlockBinding& b, Tensor& x, const Tensor& out, NormRole n, const Tensor* gate,
                          const BlockBinding* next, NormRole nn, const Tensor* scale) const {
        if (next && b.fused_bf16 && next->fused_bf16)
            return rms_norm_gated_add_modulate_bf16_(x, out, b.norm[n], gate, next->norm[nn], scale, cfg.norm_eps);
        rms_norm_gated_add_(x, out, b.norm[n], gate, cfg.norm_eps);
        return next ? sublayer_input(*next, x, nn, scale) : Tensor();
    }

    // A stack of blocks on rows x ([1, S, dim], a range of the token buffer,
    // updated in place), rotary rows cos/sin [S, head_dim], conditioning
    // vector cond (modulated stacks). Each block's two sublayers add
    // gate * rms_norm(sublayer(rms_norm(x) * (1 + scale))) to x, attention
    // first, then the FFN; unmodulated blocks have no scale and gate
    // (zimage.cpp:90-136). A sublayer's input is formed where the previous
    // sublayer closes, the next block's modulation computed one block ahead.
    // first_trace: the trace name of x after the first block (or null).
    void run_stack(const std::vector<BlockBinding>& blocks, Tensor& x, const Tensor& cos, const Tensor& sin,
                   const Tensor* cond, const char* first_trace = nullptr) const {
        if (blocks.empty()) return;
        Modulation cur = modulation(blocks[0], cond);
        Tensor in = sublayer_input(blocks[0], x, kNormAttnIn, cur.scale_of(0));
        for (size_t i = 0; i < blocks.size(); ++i) {
            const BlockBinding& b = blocks[i];
            const BlockBinding* nb = i + 1 < blocks.size() ? &blocks[i + 1] : nullptr;
            Modulation nxt = nb ? modulation(*nb, cond) : Modulation();
            Tensor out = attend(b, in, cos, sin);
            in = close_sublayer(b, x, out, kNormAttnOut, cur.gate_of(0), &b, kNormFfnIn, cur.scale_of(1));
            out = feed_forward(b, in);
            in = close_sublayer(b, x, out, kNormFfnOut, cur.gate_of(1), nb, kNormAttnIn, nxt.scale_of(0));
            if (i == 0 && first_trace) trace(first_trace, x);
            cur = std::move(nxt);
        }
    }

    // The final layer on the image tokens (zimage.cpp:218-227): LayerNorm
    // without affine, times (1 + scale(silu(cond))), projection to patches,
    // patches back to the latent's layout. cond is not used afterwards, so
    // its SiLU is taken in place.
    Tensor head(const Tensor& seq, Tensor& cond, const TokenLayout& g, int64_t H, int64_t W) const {
        silu_(cond);
        Tensor scale = linear(cond, *head_mod.W, head_mod.b);
        affine_(scale, 1.0f, 1.0f);
        scale.reshape({dim});
        Tensor y = layer_norm(rows_view(seq, 0, g.img), nullptr, nullptr, kHeadNormEps);
        mul_rows_(y, scale);
        const Tensor tokens = linear(y, *head_out.W, head_out.b);
        trace("final", tokens);
        return unpatchify2d(tokens, channels, H, W, cfg.patch);
    }
};

ZImageTransformer::ZImageTransformer(const Weights& w) : ZImageTransformer(w, Config()) {}

ZImageTransformer::ZImageTransformer(const Weights& w, const Config& cfg) : impl_(new Impl(cfg)) { impl_->bind(w); }

ZImageTransformer::~ZImageTransformer() = default;

int ZImageTransformer::in_channels() const { return impl_->channels; }
void ZImageTransformer::set_fp16_attention(bool on) { impl_->fp16_attention.store(on, std::memory_order_relaxed); }
int64_t ZImageTransformer::dim() const { return impl_->dim; }

Tensor ZImageTransformer::forward(const Tensor& latent, float t, const Tensor& text) const {
    const Impl& m = *impl_;
    const TokenLayout g = m.layout(latent, text);
    Tensor cond = m.condition(t);
    trace("adaln", cond);
    Tensor seq = Tensor::empty({g.rows(), m.dim}, Device::HIP);
    m.embed(latent, text, g, seq);
    const auto& rot = m.rotary(g);
    // the refiners update the image and the text rows in place, each with
    // its rows of the joint rotary tables
    const int64_t split[3] = {0, g.img_rows, g.rows()};
    for (int part = 0; part < 2; ++part) {
        const Stack st = part == 0 ? kNoiseRefiner : kContextRefiner;
        Tensor x = as_sequence(rows_view(seq, split[part], split[part + 1]));
        const Tensor c = rows_view(rot.first, split[part], split[part + 1]);
        const Tensor s = rows_view(rot.second, split[part], split[part + 1]);
        m.run_stack(m.stacks[st], x, c, s, kStackModulated[st] ? &cond : nullptr,
                    part == 0 ? "noise_refiner0" : nullptr);
        trace(part == 0 ? "noise_refined" : "cap_refined", x);
    }
    Tensor all = as_sequence(rows_view(seq, 0, g.rows()));
    m.run_stack(m.stacks[kMainStack], all, rot.first, rot.second, &cond, "layer0");
    trace("layers_out", all);
    return m.head(seq, cond, g, latent.dim(2), latent.dim(3));
}

void ZImageTransformer::random_weights(Weights& w, const Shapes& s, uint64_t seed, int64_t bf16_min_numel) {
    uint64_t next = seed;
    auto proj = [&](const std::string& name, int64_t out, int64_t in, bool bias) {
        w.add_random(name + ".weight", {out, in}, next++, 0.0f, 1.0f / std::sqrt((float)in), true, bf16_min_numel);
        if (bias) w.add_random(name + ".bias", {out}, next++, 0.0f, 0.02f);
    };
    auto norm = [&](const std::string& name, int64_t n) { w.add_random(name + ".weight", {n}, next++, 1.0f, 0.05f); };
    const int64_t D = s.dim, hd = s.dim / s.heads, pp = (int64_t)s.patch * s.patch;
    proj("all_x_embedder.2-1", D, pp * s.in_channels, true);
    norm("cap_embedder.0", s.cap_dim);
    proj("cap_embedder.1", D, s.cap_dim, true);
    proj("t_embedder.mlp.0", s.t_hidden, s.t_freq, true);
    proj("t_embedder.mlp.2", s.adaln_dim, s.t_hidden, true);
    proj("all_final_layer.2-1.linear", pp * s.in_channels, D, true);
    proj("all_final_layer.2-1.adaLN_modulation.1", D, s.adaln_dim, true);
    w.add_random("x_pad_token", {1, D}, next++, 0.0f, 1.0f);
    w.add_random("cap_pad_token", {1, D}, next++, 0.0f, 1.0f);
    const int depth[kStacks] = {s.noise_refiners, s.context_refiners, s.layers};
    for (int st = 0; st < kStacks; ++st)
        for (int i = 0; i < depth[st]; ++i) {
            const std::string p = std::string(kStackName[st]) + "." + std::to_string(i) + ".";
            for (int r = 0; r < kNormRoles; ++r) norm(p + kNormName[r], r == kNormQ || r == kNormK ? hd : D);
            for (int r = 0; r < kProjRoles; ++r) {
                // (out, in) of each projection; only the modulation has a bias
                const int64_t out = r == kProjGate || r == kProjUp ? s.ffn : r == kProjMod ? 4 * D : D;
                const int64_t in = r == kProjDown ? s.ffn : r == kProjMod ? s.adaln_dim : D;
                if (r != kProjMod || kStackModulated[st]) proj(p + kProjName[r], out, in, r == kProjMod);
            }
        }
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

int sdhm_zimage_set_fp16_attention(void* model, int on) {
    return guard([&] { static_cast<Model*>(model)->m->set_fp16_attention(on != 0); });
}

int64_t sdhm_zimage_params(void* model) { return (int64_t) static_cast<Model*>(model)->w.total_params(); }

void sdhm_zimage_free(void* model) { delete static_cast<Model*>(model); }

}  // extern "C"

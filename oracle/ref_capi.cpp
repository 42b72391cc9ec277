// ref_capi.cpp - C entry points over the REFERENCE's own tensor library, for
// use as a checker and CPU baseline. TEST INFRASTRUCTURE ONLY.
//
// Built by oracle/Makefile together with /root/reference/src/tensor.cpp and
// /root/reference/src/backend_cuda_stub.cpp, compiled where they lie (nothing
// of the reference is copied into this repository), into oracle/_ref/.
//
// The API is handle based so that a caller can time an op exactly as the
// reference calls it (output allocation included, tensor.h:58) without the
// cost of copying inputs into sd::Tensor objects inside the timed region.
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

#include "tensor.h"
#include "vae.h"
#include "zimage.h"

using sd::Tensor;

namespace {
thread_local std::string g_err;

template <class F>
void* guard_ptr(F&& f) {
    try {
        g_err.clear();
        return f();
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}
template <class F>
int guard(F&& f) {
    try {
        g_err.clear();
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}
Tensor* T(void* h) { return static_cast<Tensor*>(h); }
const Tensor* opt(void* h) { return h ? static_cast<Tensor*>(h) : nullptr; }
void* wrap(Tensor&& t) { return new Tensor(std::move(t)); }
}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_err.c_str(); }
void ref_set_threads(int n) { sd::set_num_threads(n); }
int ref_num_threads(void) { return sd::num_threads(); }

void* ref_tensor_new(const int64_t* shape, int ndim) {
    return guard_ptr([&] { return wrap(Tensor(std::vector<int64_t>(shape, shape + ndim))); });
}
float* ref_tensor_data(void* h) { return T(h)->ptr(); }
int64_t ref_tensor_numel(void* h) { return T(h)->numel(); }
void ref_tensor_free(void* h) { delete T(h); }

// ---- ops returning a new tensor ----
void* ref_group_norm(void* x, int groups, void* g, void* b, float eps) {
    return guard_ptr([&] { return wrap(sd::group_norm(*T(x), groups, *T(g), *T(b), eps)); });
}
void* ref_layer_norm(void* x, void* g, void* b, float eps) {
    return guard_ptr([&] { return wrap(sd::layer_norm(*T(x), opt(g), opt(b), eps)); });
}
void* ref_rms_norm(void* x, void* g, float eps) {
    return guard_ptr([&] { return wrap(sd::rms_norm(*T(x), opt(g), eps)); });
}
void* ref_swiglu(void* g, void* u) {
    return guard_ptr([&] { return wrap(sd::swiglu(*T(g), *T(u))); });
}
void* ref_geglu(void* x) {
    return guard_ptr([&] { return wrap(sd::geglu(*T(x))); });
}

// ---- in-place ops ----
int ref_rms_norm_heads_(void* x, int64_t dim, void* g, float eps) {
    return guard([&] { sd::rms_norm_heads_(*T(x), dim, opt(g), eps); });
}
int ref_rope_(void* x, int64_t dim, void* c, void* s, int interleaved) {
    return guard([&] { sd::rope_(*T(x), dim, *T(c), *T(s), interleaved != 0); });
}
int ref_softmax_rows_(void* x, int64_t rows, int64_t cols, float scale, int causal) {
    return guard([&] { sd::softmax_rows_(T(x)->ptr(), rows, cols, scale, causal != 0); });
}
int ref_silu_(void* x) { return guard([&] { sd::silu_(*T(x)); }); }
int ref_tanh_(void* x) { return guard([&] { sd::tanh_(*T(x)); }); }
int ref_gelu_(void* x) { return guard([&] { sd::gelu_(*T(x)); }); }
int ref_quick_gelu_(void* x) { return guard([&] { sd::quick_gelu_(*T(x)); }); }
int ref_add_(void* a, void* b) { return guard([&] { sd::add_(*T(a), *T(b)); }); }
int ref_scale_(void* x, float s) { return guard([&] { sd::scale_(*T(x), s); }); }
int ref_affine_(void* x, float a, float b) { return guard([&] { sd::affine_(*T(x), a, b); }); }
int ref_mul_rows_(void* x, void* v) { return guard([&] { sd::mul_rows_(*T(x), *T(v)); }); }
int ref_add_rows_scaled_(void* x, void* y, void* g) { return guard([&] { sd::add_rows_scaled_(*T(x), *T(y), *T(g)); }); }
int ref_add_channel_bias_(void* x, void* b) { return guard([&] { sd::add_channel_bias_(*T(x), *T(b)); }); }

// ---- bf16 weights and linear ----
int ref_tensor_to_bf16(void* h) { return guard([&] { T(h)->to_bf16(); }); }
const uint16_t* ref_tensor_data16(void* h) { return T(h)->ptr16(); }
void* ref_linear(void* x, void* W, void* b) { return guard_ptr([&] { return wrap(sd::linear(*T(x), *T(W), opt(b))); }); }

// ---- conv2d (new tensor, tensor.cpp:520-560) ----
void* ref_conv2d(void* x, void* w, void* b, int stride, int pad) {
    return guard_ptr([&] { return wrap(sd::conv2d(*T(x), *T(w), opt(b), stride, pad)); });
}

// ---- attention (new tensor) ----
void* ref_attention(void* q, void* k, void* v, int heads, int causal, int kv_heads) {
    return guard_ptr([&] { return wrap(sd::attention(*T(q), *T(k), *T(v), heads, causal != 0, kv_heads)); });
}

// ---- the Z-Image transformer, one forward on the CPU (zimage.cpp:138-228) ----
// Weights from a .safetensors file as Weights::load_safetensors(path, keep_bf16,
// bf16_min_numel) loads them; x [1, C, H, W], cap [1, L, cap_dim]; out [1, C, H, W].
int ref_zimage_forward(const char* path, int keep_bf16, int64_t bf16_min_numel, int heads, const float* x, int64_t C,
                       int64_t H, int64_t W, float t, const float* cap, int64_t L, int64_t cap_dim, float* out) {
    return guard([&] {
        sd::Weights w;
        w.load_safetensors(path, keep_bf16 != 0, bf16_min_numel);
        sd::ZImageTransformer::Config cfg;
        cfg.heads = heads;
        sd::ZImageTransformer m(w, cfg);
        Tensor xt({1, C, H, W}), ct({1, L, cap_dim});
        std::memcpy(xt.ptr(), x, (size_t)xt.numel() * sizeof(float));
        std::memcpy(ct.ptr(), cap, (size_t)ct.numel() * sizeof(float));
        Tensor y = m.forward(xt, t, ct);
        std::memcpy(out, y.ptr(), (size_t)y.numel() * sizeof(float));
    });
}

// ---- the VAE decoder, one decode on the CPU (vae.cpp:35-51) ----
// Weights from a .safetensors file as Weights::load_safetensors(path) loads
// them (F32); z [1, C, H, W]. Writes the image into out (capacity out_cap
// floats) and its shape into shape4; returns 0, or -1 with the error.
int ref_vae_decode(const char* path, float scaling, float shift, const float* z, int64_t C, int64_t H, int64_t W,
                   float* out, int64_t out_cap, int64_t* shape4) {
    return guard([&] {
        sd::Weights w;
        w.load_safetensors(path);
        sd::VAEDecoder vae(w, scaling, shift);
        Tensor zt({1, C, H, W});
        std::memcpy(zt.ptr(), z, (size_t)zt.numel() * sizeof(float));
        Tensor y = vae.decode(zt);
        if (y.ndim() != 4 || y.numel() > out_cap) throw std::runtime_error("ref_vae_decode: output larger than out_cap");
        for (int i = 0; i < 4; ++i) shape4[i] = y.dim(i);
        std::memcpy(out, y.ptr(), (size_t)y.numel() * sizeof(float));
    });
}

// ---- layout ops (new tensors) ----
void* ref_patchify2d(void* x, int p) { return guard_ptr([&] { return wrap(sd::patchify2d(*T(x), p)); }); }
void* ref_unpatchify2d(void* t, int64_t C, int64_t H, int64_t W, int p) {
    return guard_ptr([&] { return wrap(sd::unpatchify2d(*T(t), C, H, W, p)); });
}
void* ref_slice_rows(void* x, int64_t from, int64_t to) {
    return guard_ptr([&] { return wrap(sd::slice_rows(*T(x), from, to)); });
}
void* ref_upsample_nearest2x(void* x) { return guard_ptr([&] { return wrap(sd::upsample_nearest2x(*T(x))); }); }
void* ref_concat_channels(void* a, void* b) {
    return guard_ptr([&] { return wrap(sd::concat_channels(*T(a), *T(b))); });
}
void* ref_concat_batch(void* a, void* b) { return guard_ptr([&] { return wrap(sd::concat_batch(*T(a), *T(b))); }); }
void* ref_nchw_to_nlc(void* x) { return guard_ptr([&] { return wrap(sd::nchw_to_nlc(*T(x))); }); }
void* ref_nlc_to_nchw(void* x, int64_t H, int64_t W) {
    return guard_ptr([&] { return wrap(sd::nlc_to_nchw(*T(x), H, W)); });
}
void* ref_slice_batch(void* x, int64_t b) { return guard_ptr([&] { return wrap(sd::slice_batch(*T(x), b)); }); }
void* ref_repeat_batch(void* x, int64_t times) {
    return guard_ptr([&] { return wrap(sd::repeat_batch(*T(x), times)); });
}

}  // extern "C"

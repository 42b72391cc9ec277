// sd_hip.hpp - C++17 face of backend_hip for the reference's tensor library.
//
// This header is the drop-in for the elementwise / reduction / broadcast half
// of src/backend_cuda.h: namespace sd::hip has the functions of namespace
// sd::cuda (backend_cuda.h:23-80) with the same parameter lists, so
// tensor.cpp's `if (x.is_cuda()) cuda::op(...)` branches become
// `if (x.is_hip()) hip::op(...)` with no other change. Each function calls the
// C ABI (include/sdh_backend.h) and turns a non-zero status into
// std::runtime_error carrying sdh_last_error(), which is how the reference's
// backend reports failures (check()/launched(), backend_cuda.cu:41-48, and the
// stub's throw, backend_cuda_stub.cpp:14).
//
// Every function of backend_cuda.h has its counterpart here, conv2d, the
// GEMMs (gemm_nt_bf16, gemm_nt_f32) and attention included.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "sdh_backend.h"

namespace sd {
namespace hip {

namespace detail {
inline void check(int status, const char* what) {
    if (status != SDH_OK) throw std::runtime_error(std::string(what) + ": " + sdh_last_error());
}
}  // namespace detail

// backend_cuda.h:24-27
inline bool available() { return sdh_available() != 0; }
inline const char* device_name() { return sdh_device_name(); }
inline size_t device_memory() { return sdh_device_memory(); }

// backend_cuda.h:30-36
inline void* malloc(size_t bytes) {
    void* p = nullptr;
    detail::check(sdh_malloc(bytes, &p), "hip::malloc");
    return p;
}
inline void free(void* p) { detail::check(sdh_free(p), "hip::free"); }
inline void upload(void* dst, const void* src, size_t bytes) { detail::check(sdh_upload(dst, src, bytes), "hip::upload"); }
inline void download(void* dst, const void* src, size_t bytes) {
    detail::check(sdh_download(dst, src, bytes), "hip::download");
}
inline void copy(void* dst, const void* src, size_t bytes) { detail::check(sdh_copy(dst, src, bytes), "hip::copy"); }
inline void zero(void* dst, size_t bytes) { detail::check(sdh_zero(dst, bytes), "hip::zero"); }
// Additive: seeded N(mean, std) fill of device memory (the library's generator).
inline void fill_normal(float* x, int64_t n, uint64_t seed, float mean, float std) {
    detail::check(sdh_fill_normal(x, n, seed, mean, std), "hip::fill_normal");
}
inline void synchronize() { detail::check(sdh_synchronize(), "hip::synchronize"); }

// backend_cuda.h:41-43
inline void gemm_nt_bf16(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const uint16_t* B, int64_t ldb,
                         float* C, int64_t ldc, const float* bias, bool accumulate) {
    detail::check(sdh_gemm_nt_bf16(M, N, K, A, lda, B, ldb, C, ldc, bias, accumulate ? 1 : 0), "hip::gemm_nt_bf16");
}

// backend_cuda.h:48-52
inline void group_norm(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                       const float* beta, float eps) {
    detail::check(sdh_group_norm(x, y, N, C, HW, groups, gamma, beta, eps), "hip::group_norm");
}
inline void layer_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, const float* beta,
                       float eps) {
    detail::check(sdh_layer_norm(x, y, rows, C, gamma, beta, eps), "hip::layer_norm");
}
inline void rms_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, float eps) {
    detail::check(sdh_rms_norm(x, y, rows, C, gamma, eps), "hip::rms_norm");
}
inline void rms_norm_heads(float* x, int64_t groups, int64_t dim, const float* gamma, float eps) {
    detail::check(sdh_rms_norm_heads(x, groups, dim, gamma, eps), "hip::rms_norm_heads");
}
// backend_cuda.h:54-56
inline void rope(float* x, int64_t N, int64_t S, int64_t inner, int64_t dim, const float* cos, const float* sin,
                 bool interleaved) {
    detail::check(sdh_rope(x, N, S, inner, dim, cos, sin, interleaved ? 1 : 0), "hip::rope");
}
inline void softmax_rows(float* x, int64_t rows, int64_t cols, float scale, bool causal) {
    detail::check(sdh_softmax_rows(x, rows, cols, scale, causal ? 1 : 0), "hip::softmax_rows");
}
// backend_cuda.h:57-59: q [N, Sq, heads*d]; k, v [N, Skv, kv_heads*d]; out [N, Sq, heads*d]
// zimage.cpp:104-107 in one launch: x [2 pairs, dim], rows 2p -> 1 + x, rows 2p + 1 -> tanh(x)
inline void modulation_rows(float* x, int64_t pairs, int64_t dim) {
    detail::check(sdh_modulation_rows(x, pairs, dim), "hip::modulation_rows");
}
inline void attention(const float* q, const float* k, const float* v, float* out, int64_t N, int64_t Sq, int64_t Skv,
                      int heads, int kv_heads, int64_t d, bool causal) {
    detail::check(sdh_attention(q, k, v, out, N, Sq, Skv, heads, kv_heads, d, causal ? 1 : 0), "hip::attention");
}
// attention with out as the bf16 bits gemm_nt_bf16 would round it to (the next projection's A)
inline void attention_bf16(const float* q, const float* k, const float* v, uint16_t* out, int64_t N, int64_t Sq,
                           int64_t Skv, int heads, int kv_heads, int64_t d, bool causal) {
    detail::check(sdh_attention_bf16(q, k, v, out, N, Sq, Skv, heads, kv_heads, d, causal ? 1 : 0),
                  "hip::attention_bf16");
}
// opt-in: attention from block-scaled fp16 operands (no reference counterpart); out fp32 or bf16 bits
inline void attention_fp16(const float* q, const float* k, const float* v, void* out, bool out_bf16, int64_t N,
                           int64_t Sq, int64_t Skv, int heads, int kv_heads, int64_t d, bool causal) {
    detail::check(sdh_attention_fp16(q, k, v, out, out_bf16 ? 1 : 0, N, Sq, Skv, heads, kv_heads, d, causal ? 1 : 0),
                  "hip::attention_fp16");
}
// fused: qknorm_rope of q and k, then attention; q updated in place, k and v read only
inline void qknorm_rope_attention(float* q, const float* k, const float* v, void* out, bool out_bf16, int64_t N,
                                  int64_t S, int heads, int64_t dim, const float* gamma_q, const float* gamma_k,
                                  float eps, const float* cos, const float* sin, bool fp16) {
    detail::check(sdh_qknorm_rope_attention(q, k, v, out, out_bf16 ? 1 : 0, N, S, heads, dim, gamma_q, gamma_k, eps,
                                            cos, sin, fp16 ? 1 : 0),
                  "hip::qknorm_rope_attention");
}
// backend_cuda.h:60-61
inline void geglu(const float* x, float* y, int64_t rows, int64_t D) {
    detail::check(sdh_geglu(x, y, rows, D), "hip::geglu");
}
inline void swiglu(const float* gate, const float* up, float* y, int64_t n) {
    detail::check(sdh_swiglu(gate, up, y, n), "hip::swiglu");
}
// backend_cuda.h:64-73
inline void silu(float* x, int64_t n) { detail::check(sdh_silu(x, n), "hip::silu"); }
inline void tanh(float* x, int64_t n) { detail::check(sdh_tanh(x, n), "hip::tanh"); }
inline void gelu(float* x, int64_t n) { detail::check(sdh_gelu(x, n), "hip::gelu"); }
inline void quick_gelu(float* x, int64_t n) { detail::check(sdh_quick_gelu(x, n), "hip::quick_gelu"); }
inline void add(float* a, const float* b, int64_t n) { detail::check(sdh_add(a, b, n), "hip::add"); }
inline void scale(float* x, float s, int64_t n) { detail::check(sdh_scale(x, s, n), "hip::scale"); }
inline void affine(float* x, float a, float b, int64_t n) { detail::check(sdh_affine(x, a, b, n), "hip::affine"); }
inline void mul_rows(float* x, const float* v, int64_t rows, int64_t dim) {
    detail::check(sdh_mul_rows(x, v, rows, dim), "hip::mul_rows");
}
inline void add_rows_scaled(float* x, const float* y, const float* g, int64_t rows, int64_t dim) {
    detail::check(sdh_add_rows_scaled(x, y, g, rows, dim), "hip::add_rows_scaled");
}
inline void add_channel_bias(float* x, const float* b, int64_t N, int64_t C, int64_t HW) {
    detail::check(sdh_add_channel_bias(x, b, N, C, HW), "hip::add_channel_bias");
}
// backend_cuda.h:74-80 layout ops
inline void upsample_nearest2x(const float* x, float* y, int64_t NC, int64_t H, int64_t W) {
    detail::check(sdh_upsample_nearest2x(x, y, NC, H, W), "hip::upsample_nearest2x");
}
inline void concat_channels(const float* a, const float* b, float* y, int64_t N, int64_t Ca, int64_t Cb, int64_t HW) {
    detail::check(sdh_concat_channels(a, b, y, N, Ca, Cb, HW), "hip::concat_channels");
}
inline void nchw_to_nlc(const float* x, float* y, int64_t N, int64_t C, int64_t HW) {
    detail::check(sdh_nchw_to_nlc(x, y, N, C, HW), "hip::nchw_to_nlc");
}
inline void nlc_to_nchw(const float* x, float* y, int64_t N, int64_t C, int64_t HW) {
    detail::check(sdh_nlc_to_nchw(x, y, N, C, HW), "hip::nlc_to_nchw");
}
inline void patchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p) {
    detail::check(sdh_patchify(x, y, C, H, W, p), "hip::patchify");
}
inline void unpatchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p) {
    detail::check(sdh_unpatchify(x, y, C, H, W, p), "hip::unpatchify");
}

// Additive entry points (no single backend_cuda.h counterpart).
inline void add_rows(float* x, const float* v, int64_t rows, int64_t dim) {
    detail::check(sdh_add_rows(x, v, rows, dim), "hip::add_rows");
}
inline void softmax_rows_batched(float* x, int64_t rows, int64_t cols, float scale, bool causal, int64_t period) {
    detail::check(sdh_softmax_rows_batched(x, rows, cols, scale, causal ? 1 : 0, period), "hip::softmax_rows_batched");
}
inline void rope_qk(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                    const float* cos, const float* sin, bool interleaved) {
    detail::check(sdh_rope_qk(q, inner_q, k, inner_k, N, S, dim, cos, sin, interleaved ? 1 : 0), "hip::rope_qk");
}
inline void qknorm_rope(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                        const float* gamma_q, const float* gamma_k, float eps, const float* cos, const float* sin,
                        bool interleaved) {
    detail::check(sdh_qknorm_rope(q, inner_q, k, inner_k, N, S, dim, gamma_q, gamma_k, eps, cos, sin, interleaved ? 1 : 0),
                  "hip::qknorm_rope");
}
inline void gemm_nt_f32(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B, int64_t ldb,
                        float* C, int64_t ldc, const float* bias, bool accumulate) {
    detail::check(sdh_gemm_nt_f32(M, N, K, A, lda, B, ldb, C, ldc, bias, accumulate ? 1 : 0), "hip::gemm_nt_f32");
}
inline void to_bf16(const float* x, uint16_t* y, int64_t n) { detail::check(sdh_to_bf16(x, y, n), "hip::to_bf16"); }
// backend_cuda.h:45-47
inline void conv2d(const float* x, int64_t N, int64_t Cin, int64_t H, int64_t W, const float* w, int64_t Cout,
                   int64_t kh, int64_t kw, const float* bias, int stride, int pad, float* out, int64_t Ho, int64_t Wo) {
    detail::check(sdh_conv2d(x, N, Cin, H, W, w, Cout, kh, kw, bias, stride, pad, out, Ho, Wo), "hip::conv2d");
}
inline void gemm_nt_bf16_packed(int64_t M, int64_t N, int64_t K, const uint16_t* A, int64_t lda, const uint16_t* B,
                                int64_t ldb, float* C, int64_t ldc, const float* bias, bool accumulate) {
    detail::check(sdh_gemm_nt_bf16_packed(M, N, K, A, lda, B, ldb, C, ldc, bias, accumulate ? 1 : 0),
                  "hip::gemm_nt_bf16_packed");
}
inline void rms_norm_modulate_bf16(const float* x, uint16_t* y, int64_t rows, int64_t C, const float* gamma,
                                   const float* scale, float eps) {
    detail::check(sdh_rms_norm_modulate_bf16(x, y, rows, C, gamma, scale, eps), "hip::rms_norm_modulate_bf16");
}
inline void rms_norm_gated_add(float* x, const float* a, int64_t rows, int64_t C, const float* gamma,
                               const float* gate, float eps) {
    detail::check(sdh_rms_norm_gated_add(x, a, rows, C, gamma, gate, eps), "hip::rms_norm_gated_add");
}
inline void rms_norm_gated_add_modulate_bf16(float* x, const float* a, uint16_t* y, int64_t rows, int64_t C,
                                            const float* gamma_out, const float* gate, const float* gamma_in,
                                            const float* scale, float eps_out, float eps_in) {
    detail::check(sdh_rms_norm_gated_add_modulate_bf16(x, a, y, rows, C, gamma_out, gate, gamma_in, scale, eps_out,
                                                       eps_in),
                  "hip::rms_norm_gated_add_modulate_bf16");
}
inline void swiglu_bf16(const float* gate, const float* up, uint16_t* y, int64_t n) {
    detail::check(sdh_swiglu_bf16(gate, up, y, n), "hip::swiglu_bf16");
}
inline void linear_swiglu(const float* x, const uint16_t* w1, const uint16_t* w3, float* y, int64_t rows, int64_t in,
                          int64_t hidden) {
    detail::check(sdh_linear_swiglu(x, w1, w3, y, rows, in, hidden), "hip::linear_swiglu");
}
inline void add_rms_norm(float* x, const float* r, float* y, int64_t rows, int64_t C, const float* gamma, float eps) {
    detail::check(sdh_add_rms_norm(x, r, y, rows, C, gamma, eps), "hip::add_rms_norm");
}
inline void group_norm_silu(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups,
                            const float* gamma, const float* beta, float eps) {
    detail::check(sdh_group_norm_silu(x, y, N, C, HW, groups, gamma, beta, eps), "hip::group_norm_silu");
}
inline void ln_modulate_gate(const float* x, float* res, const float* scale, const float* shift, const float* gate,
                             float* y_out, int64_t rows, int64_t C, float eps) {
    detail::check(sdh_ln_modulate_gate(x, res, scale, shift, gate, y_out, rows, C, eps), "hip::ln_modulate_gate");
}

}  // namespace hip
}  // namespace sd

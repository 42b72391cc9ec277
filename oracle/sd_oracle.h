/*
 * sd_oracle.h - CPU restatement of the reference tensor library's
 * elementwise / reduction / broadcast ops (wolfatthegate/StableDiffusion-cpp,
 * src/tensor.cpp), used as the parity ORACLE.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libsdh, the C++ host
 * shim, the Python bindings' op path) links, loads or calls this code. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it,
 * and only as the checker.
 *
 * Every function takes host pointers and plain sizes with the meaning of the
 * reference GPU boundary (src/backend_cuda.h:48-80) and computes what the
 * reference CPU branch of the matching tensor.h op computes, with the same
 * arithmetic: same precision of every intermediate (double statistics where
 * the reference uses double), same operation order, same libm calls. The
 * per-function comment cites the tensor.cpp lines it follows.
 *
 * Threading: results do not depend on the thread count (every output element
 * is computed by exactly one serial loop). Work is split like the reference's
 * parallel_chunks (tensor.cpp:255-265) with OpenMP.
 */
#ifndef SD_ORACLE_H
#define SD_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Thread count for the chunked loops (0 = OpenMP default). */
void orc_set_threads(int n);
int orc_num_threads(void);

/* Portable seeded N(mean, std) generator: counter-based splitmix64 feeding
 * Box-Muller in double, rounded to float. Element i depends only on (seed, i). */
void orc_fill_normal(float* out, int64_t n, uint64_t seed, double mean, double std);

/* ---- norms ---- */
void orc_group_norm(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                    const float* beta, float eps);
void orc_layer_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, const float* beta,
                    float eps);
void orc_rms_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, float eps);
void orc_rms_norm_heads(float* x, int64_t groups, int64_t dim, const float* gamma, float eps);

/* ---- rotary ---- */
void orc_rope(float* x, int64_t N, int64_t S, int64_t inner, int64_t dim, const float* cos_t, const float* sin_t,
              int interleaved);
/* Z-Image 3-axis interleaved tables [S, dim] (zimage.cpp:71-88). pos is [S, 3]. */
void orc_rope_tables_3axis(const int32_t* pos, int64_t S, const int32_t* axes_dims, int64_t dim, double theta,
                           float* cos_t, float* sin_t);
/* Qwen3 rotate_half tables [S, dim] (qwen3.cpp:46-53), positions 0..S-1. */
void orc_rope_tables_half(int64_t S, int64_t dim, double theta, float* cos_t, float* sin_t);

/* ---- activations ---- */
void orc_swiglu(const float* gate, const float* up, float* y, int64_t n);
void orc_geglu(const float* x, float* y, int64_t rows, int64_t D);
void orc_silu(float* x, int64_t n);
void orc_tanh(float* x, int64_t n);
void orc_gelu(float* x, int64_t n);
void orc_quick_gelu(float* x, int64_t n);

/* ---- softmax ---- */
/* tensor.h:236 semantics: the causal row index is the row index in the call. */
void orc_softmax_rows(float* x, int64_t rows, int64_t cols, float scale, int causal);
/* Causal row index taken modulo `period` (a stack of score matrices). */
void orc_softmax_rows_period(float* x, int64_t rows, int64_t cols, float scale, int causal, int64_t period);

/* ---- broadcasts / residual ---- */
void orc_add(float* a, const float* b, int64_t n);
void orc_scale(float* x, float s, int64_t n);
void orc_affine(float* x, float a, float b, int64_t n);
void orc_mul_rows(float* x, const float* v, int64_t rows, int64_t dim);
void orc_add_rows_scaled(float* x, const float* y, const float* g, int64_t rows, int64_t dim);
void orc_add_channel_bias(float* x, const float* b, int64_t N, int64_t C, int64_t HW);

/* ---- reference compositions of the fused entry points ---- */
/* add_(x, r) then y = rms_norm(x, gamma, eps)  (zimage.cpp:123-128 order). */
void orc_add_rms_norm(float* x, const float* r, float* y, int64_t rows, int64_t C, const float* gamma, float eps);
/* y = group_norm(x); silu_(y)  (modules.cpp:34-35, vae.cpp:48-49). */
void orc_group_norm_silu(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                         const float* beta, float eps);
/* y = layer_norm(x, no affine, eps); s1 = affine_(scale,1,1); tg = tanh_(gate);
 * mul_rows_(y, s1); add_rows_scaled_(y, ones, shift) [if shift]; add_rows_scaled_(res, y, tg).
 * y_out may be NULL. */
void orc_ln_modulate_gate(const float* x, float* res, const float* scale, const float* shift, const float* gate,
                          float* y_out, int64_t rows, int64_t C, float eps);

/* rms_norm_heads_(q), rms_norm_heads_(k), rope_(q), rope_(k): zimage.cpp:117-120,
 * qwen3.cpp:59-62 (composition of the functions above). */
void orc_qknorm_rope(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                     const float* gamma_q, const float* gamma_k, float eps, const float* cos_t, const float* sin_t,
                     int interleaved);

/* ---- layout (tensor.cpp:931-1099); y never overlaps the inputs ---- */
/* tensor.cpp:982-1004: x [NC, H, W] -> y [NC, 2H, 2W]. */
void orc_upsample_nearest2x(const float* x, float* y, int64_t NC, int64_t H, int64_t W);
/* tensor.cpp:1006-1023: a [N, Ca, HW], b [N, Cb, HW] -> y [N, Ca + Cb, HW]. */
void orc_concat_channels(const float* a, const float* b, float* y, int64_t N, int64_t Ca, int64_t Cb, int64_t HW);
/* tensor.cpp:1041-1056: x [N, C, HW] -> y [N, HW, C]. */
void orc_nchw_to_nlc(const float* x, float* y, int64_t N, int64_t C, int64_t HW);
/* tensor.cpp:1058-1074: x [N, HW, C] -> y [N, C, HW]. */
void orc_nlc_to_nchw(const float* x, float* y, int64_t N, int64_t C, int64_t HW);
/* tensor.cpp:931-949: x [C, H, W] -> y [(H/p)(W/p), p*p*C], features (ph, pw, c). */
void orc_patchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p);
/* tensor.cpp:951-968: tokens [(H/p)(W/p), p*p*C] -> y [C, H, W]; rows/columns
 * beyond (H/p)p, (W/p)p are left untouched (the reference zero-allocates y). */
void orc_unpatchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p);

/* Planted-mistake switch for the oracle's own pin tests (0 = none). The pins
 * must fail when a mistake is planted; see tests/test_oracle_pins.py. */
void orc_plant_mistake(int which);

#ifdef __cplusplus
}
#endif

#endif

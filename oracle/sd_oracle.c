/*
 * sd_oracle.c - CPU restatement of the reference's elementwise / reduction /
 * broadcast ops. TEST INFRASTRUCTURE ONLY (see sd_oracle.h): the product never
 * links or calls this file.
 *
 * Each function cites the lines of wolfatthegate/StableDiffusion-cpp
 * src/tensor.cpp (or zimage.cpp / qwen3.cpp for the rotary tables) whose
 * arithmetic it restates. Intermediates keep the reference's precision
 * (double statistics, float data), its operation order and its libm calls
 * (expf, tanhf, erff, cosf, sinf, sqrt, pow, cos, sin), so that with the
 * same compiler flags the results agree bit for bit with the compiled
 * reference; tests/test_oracle_vs_ref.py checks exactly that.
 */
#include "sd_oracle.h"

#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;
static int g_plant = 0;

void orc_set_threads(int n) { g_threads = n; }
int orc_num_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}
void orc_plant_mistake(int which) { g_plant = which; }

/* The reference's parallel_chunks split (tensor.cpp:255-265): at most 4
 * ranges per thread and none shorter than min_chunk. Each range [b, e) is
 * handed to body(ctx, b, e). */
typedef void (*range_fn)(void* ctx, int64_t b, int64_t e);

static void chunks(int64_t n, int64_t min_chunk, range_fn body, void* ctx) {
    if (n <= 0) return;
    int64_t mc = min_chunk > 1 ? min_chunk : 1;
    int64_t by_size = n / mc;
    if (by_size < 1) by_size = 1;
    int64_t nch = (int64_t)orc_num_threads() * 4;
    if (nch > by_size) nch = by_size;
    const int64_t chunk = (n + nch - 1) / nch;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(orc_num_threads())
#endif
    for (int64_t t = 0; t < nch; ++t) {
        int64_t b = t * chunk, e = b + chunk;
        if (e > n) e = n;
        if (b < e) body(ctx, b, e);
    }
}

/* parallel_for (tensor.cpp:253): one task per item. */
static void items(int64_t n, range_fn body, void* ctx) {
    if (n <= 0) return;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(orc_num_threads())
#endif
    for (int64_t t = 0; t < n; ++t) body(ctx, t, t + 1);
}

/* ------------------------------------------------------------------------ */
/* Generator                                                                 */
/* ------------------------------------------------------------------------ */
#define GOLDEN 0x9E3779B97F4A7C15ULL

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

void orc_fill_normal(float* out, int64_t n, uint64_t seed, double mean, double std) {
    const uint64_t key = mix64(seed + GOLDEN);
    const double two_pi = 6.283185307179586476925286766559;
    const double inv53 = 1.0 / 9007199254740992.0; /* 2^-53 */
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_num_threads())
#endif
    for (int64_t j = 0; j < (n + 1) / 2; ++j) {
        const uint64_t h1 = mix64(key + (uint64_t)(2 * j + 1) * GOLDEN);
        const uint64_t h2 = mix64(key + (uint64_t)(2 * j + 2) * GOLDEN);
        const double u1 = (double)((h1 >> 11) + 1) * inv53; /* (0, 1] */
        const double u2 = (double)(h2 >> 11) * inv53;       /* [0, 1) */
        const double r = sqrt(-2.0 * log(u1));
        const double th = two_pi * u2;
        out[2 * j] = (float)(mean + std * (r * cos(th)));
        if (2 * j + 1 < n) out[2 * j + 1] = (float)(mean + std * (r * sin(th)));
    }
}

/* ------------------------------------------------------------------------ */
/* GroupNorm  (tensor.cpp:592-625)                                           */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *x, *gamma, *beta;
    float* y;
    int64_t C, HW, groups, cg;
    float eps;
    int silu;
} gn_ctx;

static void gn_body(void* vctx, int64_t t, int64_t te) {
    gn_ctx* c = (gn_ctx*)vctx;
    (void)te;
    const int64_t n = t / c->groups, g = t % c->groups;
    const int64_t len = c->cg * c->HW;
    const float* p = c->x + (n * c->C + g * c->cg) * c->HW;
    float* q = c->y + (n * c->C + g * c->cg) * c->HW;
    double sum = 0;
    for (int64_t i = 0; i < len; ++i) sum += p[i];
    const double mean = sum / len;
    double var = 0;
    for (int64_t i = 0; i < len; ++i) {
        double d = p[i] - mean;
        var += d * d;
    }
    const float rstd = (float)(1.0 / sqrt(var / len + c->eps));
    for (int64_t ci = 0; ci < c->cg; ++ci) {
        const int64_t ch = (g_plant == 4) ? g : g * c->cg + ci; /* plant 4: wrong gamma index */
        const float a = rstd * c->gamma[ch];
        const float bb = c->beta[ch] - (float)mean * a;
        const float* pc = p + ci * c->HW;
        float* qc = q + ci * c->HW;
        for (int64_t i = 0; i < c->HW; ++i) qc[i] = pc[i] * a + bb;
        if (c->silu) /* silu_ (tensor.cpp:843-849) applied to the finished channel */
            for (int64_t i = 0; i < c->HW; ++i) qc[i] = qc[i] / (1.0f + expf(-qc[i]));
    }
}

static void group_norm_impl(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups,
                            const float* gamma, const float* beta, float eps, int silu) {
    gn_ctx c = {x, gamma, beta, y, C, HW, groups, C / groups, eps, silu};
    items(N * groups, gn_body, &c);
}

void orc_group_norm(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                    const float* beta, float eps) {
    group_norm_impl(x, y, N, C, HW, groups, gamma, beta, eps, 0);
}

/* group_norm followed by silu_ on its output: silu of each element only
 * depends on that element, so applying it per finished channel gives the
 * same floats as a separate full pass. */
void orc_group_norm_silu(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                         const float* beta, float eps) {
    group_norm_impl(x, y, N, C, HW, groups, gamma, beta, eps, 1);
}

/* ------------------------------------------------------------------------ */
/* LayerNorm  (tensor.cpp:628-658)                                           */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *x, *gamma, *beta;
    float* y;
    int64_t C;
    float eps;
} ln_ctx;

/* The compiled reference rounds (x-mean)*rstd*gamma and +beta separately here
 * (no fused multiply-add), so contraction is switched off for this body. */
__attribute__((optimize("fp-contract=off"))) static void ln_body(void* vctx, int64_t rb, int64_t re) {
    ln_ctx* c = (ln_ctx*)vctx;
    const int64_t C = c->C;
    for (int64_t r = rb; r < re; ++r) {
        const float* p = c->x + r * C;
        float* q = c->y + r * C;
        double sum = 0;
        for (int64_t i = 0; i < C; ++i) sum += p[i];
        const float mean = (float)(sum / C);
        double var = 0;
        for (int64_t i = 0; i < C; ++i) {
            float d = p[i] - mean;
            var += (double)d * d;
        }
        const float rstd = (float)(1.0 / sqrt(var / C + c->eps));
        for (int64_t i = 0; i < C; ++i) {
            float v = (p[i] - mean) * rstd;
            if (c->gamma) v *= c->gamma[i];
            if (c->beta) v += c->beta[i];
            q[i] = v;
        }
    }
}

void orc_layer_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, const float* beta,
                    float eps) {
    ln_ctx c = {x, gamma, beta, y, C, eps};
    chunks(rows, 8, ln_body, &c);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm  (tensor.cpp:660-679) and per-head RMSNorm (tensor.cpp:681-696)   */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float* x;
    float* y;
    const float* gamma;
    int64_t C;
    float eps;
} rms_ctx;

static void rms_body(void* vctx, int64_t rb, int64_t re) {
    rms_ctx* c = (rms_ctx*)vctx;
    const int64_t C = c->C;
    for (int64_t r = rb; r < re; ++r) {
        const float* p = c->x + r * C;
        float* q = c->y + r * C;
        double ss = 0;
        for (int64_t i = 0; i < C; ++i) ss += (double)p[i] * p[i];
        const double e = (g_plant == 2) ? 0.0 : (double)c->eps; /* plant 2: eps dropped */
        const float rstd = (float)(1.0 / sqrt(ss / C + e));
        for (int64_t i = 0; i < C; ++i) q[i] = p[i] * rstd * (c->gamma ? c->gamma[i] : 1.0f);
    }
}

void orc_rms_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, float eps) {
    rms_ctx c = {x, y, gamma, C, eps};
    chunks(rows, 8, rms_body, &c);
}

void orc_rms_norm_heads(float* x, int64_t groups, int64_t dim, const float* gamma, float eps) {
    /* Same per-group arithmetic as rms_norm, in place (tensor.cpp:687-695). */
    rms_ctx c = {x, x, gamma, dim, eps};
    chunks(groups, 64, rms_body, &c);
}

/* ------------------------------------------------------------------------ */
/* Rotary  (tensor.cpp:698-730); tables zimage.cpp:71-88, qwen3.cpp:46-53    */
/* ------------------------------------------------------------------------ */
typedef struct {
    float* x;
    const float *cs, *sn;
    int64_t S, inner, dim;
    int interleaved;
} rope_ctx;

static void rope_body(void* vctx, int64_t b, int64_t e) {
    rope_ctx* c = (rope_ctx*)vctx;
    const int64_t dim = c->dim, half = dim / 2, heads = c->inner / dim;
    for (int64_t ns = b; ns < e; ++ns) {
        const int64_t s = ns % c->S;
        const float* cc = c->cs + s * dim;
        const float* sv = c->sn + s * dim;
        for (int64_t h = 0; h < heads; ++h) {
            float* p = c->x + ns * c->inner + h * dim;
            if (c->interleaved) {
                for (int64_t i = 0; i < dim; i += 2) {
                    const float a = p[i], bb = p[i + 1];
                    if (g_plant == 1) { /* plant 1: sign of the sine term flipped */
                        p[i] = a * cc[i] + bb * sv[i];
                        p[i + 1] = bb * cc[i] - a * sv[i];
                    } else {
                        p[i] = a * cc[i] - bb * sv[i];
                        p[i + 1] = bb * cc[i] + a * sv[i];
                    }
                }
            } else {
                for (int64_t i = 0; i < half; ++i) {
                    const float a = p[i], bb = p[i + half];
                    p[i] = a * cc[i] - bb * sv[i];
                    p[i + half] = bb * cc[i + half] + a * sv[i + half];
                }
            }
        }
    }
}

void orc_rope(float* x, int64_t N, int64_t S, int64_t inner, int64_t dim, const float* cos_t, const float* sin_t,
              int interleaved) {
    rope_ctx c = {x, cos_t, sin_t, S, inner, dim, interleaved};
    chunks(N * S, 16, rope_body, &c);
}

void orc_rope_tables_3axis(const int32_t* pos, int64_t S, const int32_t* axes_dims, int64_t dim, double theta,
                           float* cos_t, float* sin_t) {
    for (int64_t s = 0; s < S; ++s) {
        int64_t off = 0;
        for (int a = 0; a < 3; ++a) {
            const int da = axes_dims[a];
            for (int k = 0; k < da / 2; ++k) {
                const double freq = 1.0 / pow(theta, (double)(2 * k) / (double)da);
                const float ang = (float)((double)pos[s * 3 + a] * freq);
                const float cv = cosf(ang), sv = sinf(ang);
                cos_t[s * dim + off + 2 * k] = cv;
                cos_t[s * dim + off + 2 * k + 1] = cv;
                sin_t[s * dim + off + 2 * k] = sv;
                sin_t[s * dim + off + 2 * k + 1] = sv;
            }
            off += da;
        }
    }
}

void orc_rope_tables_half(int64_t S, int64_t dim, double theta, float* cos_t, float* sin_t) {
    for (int64_t s = 0; s < S; ++s)
        for (int64_t i = 0; i < dim / 2; ++i) {
            const double inv_freq = pow(theta, -2.0 * (double)i / (double)dim);
            const double a = (double)s * inv_freq;
            cos_t[s * dim + i] = cos_t[s * dim + i + dim / 2] = (float)cos(a);
            sin_t[s * dim + i] = sin_t[s * dim + i + dim / 2] = (float)sin(a);
        }
}

/* ------------------------------------------------------------------------ */
/* Activations  (tensor.cpp:732-748, 812-868)                                */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *a, *b;
    float* y;
    float s0, s1;
    int64_t D;
} ew_ctx;

static void swiglu_body(void* vctx, int64_t b, int64_t e) {
    ew_ctx* c = (ew_ctx*)vctx;
    const float *g = c->a, *u = c->b;
    float* o = c->y;
    if (g_plant == 5) { /* plant 5: exp(+g) instead of exp(-g) */
        for (int64_t i = b; i < e; ++i) o[i] = g[i] / (1.0f + expf(g[i])) * u[i];
        return;
    }
    for (int64_t i = b; i < e; ++i) o[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

void orc_swiglu(const float* gate, const float* up, float* y, int64_t n) {
    ew_ctx c = {gate, up, y, 0, 0, 0};
    chunks(n, 16384, swiglu_body, &c);
}

static void geglu_body(void* vctx, int64_t rb, int64_t re) {
    ew_ctx* c = (ew_ctx*)vctx;
    const int64_t D = c->D;
    for (int64_t r = rb; r < re; ++r) {
        const float* a = c->a + r * 2 * D;
        const float* g = a + D;
        float* o = c->y + r * D;
        for (int64_t i = 0; i < D; ++i) {
            float gg = g[i];
            o[i] = a[i] * 0.5f * gg * (1.0f + erff(gg * 0.70710678118654752f));
        }
    }
}

void orc_geglu(const float* x, float* y, int64_t rows, int64_t D) {
    ew_ctx c = {x, NULL, y, 0, 0, D};
    chunks(rows, 8, geglu_body, &c);
}

static void silu_body(void* vctx, int64_t b, int64_t e) {
    float* p = ((ew_ctx*)vctx)->y;
    for (int64_t i = b; i < e; ++i) p[i] = p[i] / (1.0f + expf(-p[i]));
}
static void gelu_body(void* vctx, int64_t b, int64_t e) {
    float* p = ((ew_ctx*)vctx)->y;
    for (int64_t i = b; i < e; ++i) p[i] = 0.5f * p[i] * (1.0f + erff(p[i] * 0.70710678118654752f));
}
static void qgelu_body(void* vctx, int64_t b, int64_t e) {
    float* p = ((ew_ctx*)vctx)->y;
    for (int64_t i = b; i < e; ++i) p[i] = p[i] / (1.0f + expf(-1.702f * p[i]));
}

void orc_silu(float* x, int64_t n) {
    ew_ctx c = {NULL, NULL, x, 0, 0, 0};
    chunks(n, 16384, silu_body, &c);
}
void orc_gelu(float* x, int64_t n) {
    ew_ctx c = {NULL, NULL, x, 0, 0, 0};
    chunks(n, 16384, gelu_body, &c);
}
void orc_quick_gelu(float* x, int64_t n) {
    ew_ctx c = {NULL, NULL, x, 0, 0, 0};
    chunks(n, 16384, qgelu_body, &c);
}
/* tanh_ is a serial loop in the reference (tensor.cpp:850-853). */
void orc_tanh(float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = tanhf(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Softmax  (tensor.cpp:752-769; period as backend_cuda.cu:351-367)          */
/* ------------------------------------------------------------------------ */
typedef struct {
    float* x;
    int64_t cols, period;
    float scale;
    int causal;
} sm_ctx;

static void softmax_body(void* vctx, int64_t rb, int64_t re) {
    sm_ctx* c = (sm_ctx*)vctx;
    const int64_t cols = c->cols;
    const float scale = c->scale;
    for (int64_t r = rb; r < re; ++r) {
        float* p = c->x + r * cols;
        const int64_t rr = r % c->period;
        const int64_t valid = c->causal ? (cols < rr + 1 ? cols : rr + 1) : cols;
        float m = -INFINITY;
        for (int64_t j = 0; j < valid; ++j) m = fmaxf(m, p[j] * scale);
        if (g_plant == 3) m = 0.0f; /* plant 3: max not subtracted (overflows on large logits) */
        float sum = 0.0f;
        for (int64_t j = 0; j < valid; ++j) {
            p[j] = expf(p[j] * scale - m);
            sum += p[j];
        }
        const float inv = 1.0f / sum;
        for (int64_t j = 0; j < valid; ++j) p[j] *= inv;
        for (int64_t j = valid; j < cols; ++j) p[j] = 0.0f;
    }
}

void orc_softmax_rows_period(float* x, int64_t rows, int64_t cols, float scale, int causal, int64_t period) {
    sm_ctx c = {x, cols, period > 0 ? period : rows, scale, causal};
    if (c.period <= 0) c.period = 1;
    chunks(rows, 4, softmax_body, &c);
}

void orc_softmax_rows(float* x, int64_t rows, int64_t cols, float scale, int causal) {
    orc_softmax_rows_period(x, rows, cols, scale, causal, rows);
}

/* ------------------------------------------------------------------------ */
/* Broadcasts / residual  (tensor.cpp:869-929)                               */
/* ------------------------------------------------------------------------ */
static void add_body(void* vctx, int64_t s, int64_t e) {
    ew_ctx* c = (ew_ctx*)vctx;
    float* p = c->y;
    const float* q = c->a;
    for (int64_t i = s; i < e; ++i) p[i] += q[i];
}

void orc_add(float* a, const float* b, int64_t n) {
    ew_ctx c = {b, NULL, a, 0, 0, 0};
    chunks(n, 16384, add_body, &c);
}

/* scale_ and affine_ are serial loops in the reference (tensor.cpp:879-887). */
void orc_scale(float* x, float s, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] *= s;
}
void orc_affine(float* x, float a, float b, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] * a + b;
}

static void mul_rows_body(void* vctx, int64_t rb, int64_t re) {
    ew_ctx* c = (ew_ctx*)vctx;
    const int64_t dim = c->D;
    const float* vv = c->a;
    for (int64_t r = rb; r < re; ++r) {
        float* p = c->y + r * dim;
        for (int64_t i = 0; i < dim; ++i) p[i] *= vv[i];
    }
}

void orc_mul_rows(float* x, const float* v, int64_t rows, int64_t dim) {
    ew_ctx c = {v, NULL, x, 0, 0, dim};
    chunks(rows, 16, mul_rows_body, &c);
}

static void add_rows_scaled_body(void* vctx, int64_t rb, int64_t re) {
    ew_ctx* c = (ew_ctx*)vctx;
    const int64_t dim = c->D;
    const float* gg = c->b;
    for (int64_t r = rb; r < re; ++r) {
        float* p = c->y + r * dim;
        const float* q = c->a + r * dim;
        for (int64_t i = 0; i < dim; ++i) p[i] += gg[i] * q[i];
    }
}

void orc_add_rows_scaled(float* x, const float* y, const float* g, int64_t rows, int64_t dim) {
    ew_ctx c = {y, g, x, 0, 0, dim};
    chunks(rows, 16, add_rows_scaled_body, &c);
}

static void add_channel_bias_body(void* vctx, int64_t nc, int64_t nce) {
    ew_ctx* c = (ew_ctx*)vctx;
    (void)nce;
    const int64_t HW = c->D;
    const float add = c->a[nc];
    float* p = c->y + nc * HW;
    for (int64_t i = 0; i < HW; ++i) p[i] += add;
}

void orc_add_channel_bias(float* x, const float* b, int64_t N, int64_t C, int64_t HW) {
    ew_ctx c = {b, NULL, x, 0, 0, HW};
    items(N * C, add_channel_bias_body, &c);
}

void orc_qknorm_rope(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                     const float* gamma_q, const float* gamma_k, float eps, const float* cos_t, const float* sin_t,
                     int interleaved) {
    orc_rms_norm_heads(q, N * S * inner_q / dim, dim, gamma_q, eps);
    orc_rms_norm_heads(k, N * S * inner_k / dim, dim, gamma_k, eps);
    orc_rope(q, N, S, inner_q, dim, cos_t, sin_t, interleaved);
    orc_rope(k, N, S, inner_k, dim, cos_t, sin_t, interleaved);
}

/* ------------------------------------------------------------------------ */
/* Layout (tensor.cpp:931-1099): copies, in the reference's loop order       */
/* ------------------------------------------------------------------------ */
void orc_upsample_nearest2x(const float* x, float* y, int64_t NC, int64_t H, int64_t W) {
    for (int64_t nc = 0; nc < NC; ++nc) {
        const float* p = x + nc * H * W;
        float* q = y + nc * 4 * H * W;
        for (int64_t i = 0; i < H; ++i) {
            float* r0 = q + (2 * i) * 2 * W;
            float* r1 = r0 + 2 * W;
            for (int64_t j = 0; j < W; ++j) {
                const float v = p[i * W + j];
                r0[2 * j] = r0[2 * j + 1] = v;
                r1[2 * j] = r1[2 * j + 1] = v;
            }
        }
    }
}

void orc_concat_channels(const float* a, const float* b, float* y, int64_t N, int64_t Ca, int64_t Cb, int64_t HW) {
    for (int64_t n = 0; n < N; ++n) {
        memcpy(y + n * (Ca + Cb) * HW, a + n * Ca * HW, (size_t)(Ca * HW) * sizeof(float));
        memcpy(y + (n * (Ca + Cb) + Ca) * HW, b + n * Cb * HW, (size_t)(Cb * HW) * sizeof(float));
    }
}

void orc_nchw_to_nlc(const float* x, float* y, int64_t N, int64_t C, int64_t HW) {
    for (int64_t nc = 0; nc < N * C; ++nc) {
        const int64_t n = nc / C, c = nc % C;
        const float* p = x + nc * HW;
        float* q = y + n * HW * C + c;
        for (int64_t i = 0; i < HW; ++i) q[i * C] = p[i];
    }
}

void orc_nlc_to_nchw(const float* x, float* y, int64_t N, int64_t C, int64_t HW) {
    for (int64_t nc = 0; nc < N * C; ++nc) {
        const int64_t n = nc / C, c = nc % C;
        if (g_plant == 7) { /* plant 7: input read as if it were already NCHW (no transpose) */
            memcpy(y + nc * HW, x + (n * C + c) * HW, (size_t)HW * sizeof(float));
            continue;
        }
        const float* p = x + n * HW * C + c;
        float* q = y + nc * HW;
        for (int64_t i = 0; i < HW; ++i) q[i] = p[i * C];
    }
}

void orc_patchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p) {
    const int64_t Ht = H / p, Wt = W / p;
    for (int64_t h = 0; h < Ht; ++h)
        for (int64_t w = 0; w < Wt; ++w) {
            float* tok = y + (h * Wt + w) * p * p * C;
            for (int64_t ph = 0; ph < p; ++ph)
                for (int64_t pw = 0; pw < p; ++pw)
                    for (int64_t c = 0; c < C; ++c) {
                        const int64_t f = (g_plant == 6) ? (pw * p + ph) : (ph * p + pw); /* plant 6: ph/pw swapped */
                        tok[f * C + c] = x[(c * H + h * p + ph) * W + w * p + pw];
                    }
        }
}

void orc_unpatchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p) {
    const int64_t Ht = H / p, Wt = W / p;
    for (int64_t h = 0; h < Ht; ++h)
        for (int64_t w = 0; w < Wt; ++w) {
            const float* tok = x + (h * Wt + w) * p * p * C;
            for (int64_t ph = 0; ph < p; ++ph)
                for (int64_t pw = 0; pw < p; ++pw)
                    for (int64_t c = 0; c < C; ++c) y[(c * H + h * p + ph) * W + w * p + pw] = tok[(ph * p + pw) * C + c];
        }
}

/* ------------------------------------------------------------------------ */
/* Compositions of the fused entry points                                    */
/* ------------------------------------------------------------------------ */
void orc_add_rms_norm(float* x, const float* r, float* y, int64_t rows, int64_t C, const float* gamma, float eps) {
    orc_add(x, r, rows * C);
    orc_rms_norm(x, y, rows, C, gamma, eps);
}

void orc_ln_modulate_gate(const float* x, float* res, const float* scale, const float* shift, const float* gate,
                          float* y_out, int64_t rows, int64_t C, float eps) {
    float* y = y_out ? y_out : (float*)malloc((size_t)(rows * C) * sizeof(float));
    float* s1 = (float*)malloc((size_t)C * sizeof(float));
    float* tg = (float*)malloc((size_t)C * sizeof(float));
    float* ones = (float*)malloc((size_t)(rows * C) * sizeof(float));
    for (int64_t i = 0; i < C; ++i) {
        s1[i] = scale[i];
        tg[i] = gate[i];
    }
    orc_layer_norm(x, y, rows, C, NULL, NULL, eps); /* zimage.cpp:223 form: no affine */
    orc_affine(s1, 1.0f, 1.0f, C);                  /* zimage.cpp:104-105, :221 */
    orc_tanh(tg, C);                                /* zimage.cpp:106-107 */
    orc_mul_rows(y, s1, rows, C);
    if (shift) {
        /* "+ shift" as add_rows_scaled_(y, ones, shift): y[r,i] += shift[i] * 1.0f */
        for (int64_t i = 0; i < rows * C; ++i) ones[i] = 1.0f;
        orc_add_rows_scaled(y, ones, shift, rows, C);
    }
    orc_add_rows_scaled(res, y, tg, rows, C);
    free(ones);
    free(tg);
    free(s1);
    if (!y_out) free(y);
}

// k_rownorm.hip - per-row reductions: rms_norm, layer_norm, the fused
// residual-add + rms_norm, the fused adaLN chain (layer_norm -> (1+scale) ->
// +shift -> res += tanh(gate) * y) and per-head rms_norm (QK-norm).
//
// Layout and mapping (gfx950, wave64):
//   * One wave owns one row at a time. A row of C floats is held in
//     registers as V float4 per lane (lane l holds float4 l, l+64, ...), so
//     HBM sees exactly one read of every input and one write of every output;
//     the statistics pass and the apply pass both run on registers.
//   * Reductions are wave-only (DPP + readlane, sdh_internal.hpp); no LDS and
//     no barrier, except the adaLN kernel (two waves per row, column vectors
//     staged in LDS once per 4 rows) and the norm + gated residual on rows
//     wider than 2048 floats (one 256-thread workgroup per row, measured
//     faster for that op's three row streams).
//   * The grid covers the rows exactly (4 rows per 256-thread workgroup, no
//     persistent loop): measured on MI355X, letting the dispatcher refill CUs
//     with fresh workgroups streams ~10 points of peak better than persistent
//     waves. Row data is loaded and stored non-temporally; per-column vectors
//     (gamma, beta, scale, shift) come from L2. Measured: with ordinary
//     (allocating) row loads the same kernels gain ~7 points when the
//     benchmark rotates few buffer sets and lose ~8 points when it rotates
//     many; non-temporal loads give the same bandwidth either way.
// Statistics: the reference accumulates in double (tensor.cpp:640-648,
// :672-674, :690-692). Here each lane accumulates its <= 4V values in fp32,
// the wave tree adds 64 partials in fp32, and the final mean / rstd are
// formed in double; the relative error of the sums stays below ~1e-6.
// Rows whose length is not a multiple of 4, unaligned rows or rows longer
// than 64 * 4 * 32 floats take the generic kernel (same arithmetic, strided
// scalar loops that re-read the row from cache).
#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

enum Mode { M_LN = 0, M_RMS = 1 };

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }
// The four floats summed in double, and their squares (each exact in double).
__device__ __forceinline__ double dsum4(const f4& v) {
    return ((double)v.x + (double)v.y) + ((double)v.z + (double)v.w);
}
__device__ __forceinline__ double dsq4(const f4& d) {
    return ((double)d.x * (double)d.x + (double)d.y * (double)d.y) +
           ((double)d.z * (double)d.z + (double)d.w * (double)d.w);
}
// rstd from a statistic summed in double: (float)(1 / sqrt(stat / C + eps)).
__device__ __forceinline__ float rstd_of_d(double stat, int64_t C, float eps) {
    return (float)(1.0 / sqrt(stat / (double)C + (double)eps));
}

using dev::rstd_of;

// y = layer_norm / rms_norm of each row of x (tensor.cpp:628-679).
template <int V, int MODE, bool HAS_G, bool HAS_B>
__global__ __launch_bounds__(kThreads) void k_rownorm(const float* __restrict__ x, float* __restrict__ y,
                                                     int64_t rows, int C, const float* __restrict__ gamma,
                                                     const float* __restrict__ beta, float eps) {
    const int lane = threadIdx.x & 63;
    const int n4 = C >> 2;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole wave: no barrier below
    const f4* xr = (const f4*)(x + row * C);
    f4* yr = (f4*)(y + row * C);
    f4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        v[j] = idx < n4 ? dev::ld_stream(xr + idx) : zero4();
    }
    float mean = 0.f, rstd;
    if constexpr (MODE == M_LN) {
        // both sums in double, as tensor.cpp:640-647 forms them: an fp32
        // sum moves the mean by ~1e-5 / C and rstd by ~1e-6 relative, which
        // outputs near zero (x near the mean, or cancelling beta) magnify
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < V; ++j) s += dsum4(v[j]);  // masked entries are zero
        mean = (float)(dev::wave_sum_d(s) / (double)C);
        double q = 0.0;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            if (lane + 64 * j < n4) q += dsq4(v[j] - mean);
        }
        rstd = rstd_of_d(dev::wave_sum_d(q), C, eps);
    } else {
        float q = 0.f;
#pragma unroll
        for (int j = 0; j < V; ++j) q += dev::sumsq4(v[j]);
        rstd = rstd_of(dev::wave_sum(q), C, eps);
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        if (idx < n4) {
            f4 o;
            if constexpr (MODE == M_LN) {
                // (x - mean) * rstd, then * gamma, then + beta, each rounded
                // on its own as tensor.cpp:650-652 does.
                o = (v[j] - mean) * rstd;
                if constexpr (HAS_G) {
                    const f4 g = ((const f4*)gamma)[idx];
                    o = f4{__fmul_rn(o.x, g.x), __fmul_rn(o.y, g.y), __fmul_rn(o.z, g.z), __fmul_rn(o.w, g.w)};
                }
                if constexpr (HAS_B) {
                    const f4 b = ((const f4*)beta)[idx];
                    o = f4{__fadd_rn(o.x, b.x), __fadd_rn(o.y, b.y), __fadd_rn(o.z, b.z), __fadd_rn(o.w, b.w)};
                }
            } else {
                o = v[j] * rstd;  // x * rstd * gamma (tensor.cpp:675)
                if constexpr (HAS_G) o = o * ((const f4*)gamma)[idx];
            }
            dev::st_stream(yr + idx, o);
        }
    }
}

// x += r; y = rms_norm(x) * gamma  (add_ then rms_norm, tensor.cpp:876, :673-675).
template <int V, bool HAS_G>
__global__ __launch_bounds__(kThreads) void k_add_rms(float* __restrict__ x, const float* __restrict__ r,
                                                     float* __restrict__ y, int64_t rows, int C,
                                                     const float* __restrict__ gamma, float eps) {
    const int lane = threadIdx.x & 63;
    const int n4 = C >> 2;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    f4* xr = (f4*)(x + row * C);
    const f4* rr = (const f4*)(r + row * C);
    f4* yr = (f4*)(y + row * C);
    // a load pair per vector and lane, added as it arrives: measured faster
    // (42.2 us at [4096,3840]) than issuing the whole row's loads first
    // (44.8 us), which needs 168 VGPRs and no longer fits every row on the GPU
    // at once
    f4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        v[j] = idx < n4 ? dev::ld_stream(xr + idx) + dev::ld_stream(rr + idx) : zero4();
    }
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        if (idx < n4) dev::st_stream(xr + idx, v[j]);
        q += dev::sumsq4(v[j]);
    }
    const float rstd = rstd_of(dev::wave_sum(q), C, eps);
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        if (idx < n4) {
            f4 o = v[j] * rstd;
            if constexpr (HAS_G) o = o * ((const f4*)gamma)[idx];
            dev::st_stream(yr + idx, o);
        }
    }
}

// Rows of 2048 < C <= 8192 floats can take one 256-thread workgroup per row,
// wave p lane l holding float4 l + 64 (p + 4 j). Measured on MI355X at
// [4096, 3840] against one wave per row: the norm + gated residual (two row
// reads, one write) gains 6-8 points of HBM peak; rms_norm (one read, one
// write) loses 5 and add + rms_norm (two reads, two writes) loses 2, so
// those keep one wave per row.
constexpr int kRowThreads = 256;

// Fused adaLN chain (see sdh_ln_modulate_gate). A 512-thread workgroup owns
// kModRows = 4 rows, two waves (128 threads, V float4 each) per row. It
// stages 1 + scale (affine_(scale, 1, 1)), shift and tanh(gate) for all C
// columns in LDS (the affine_ / tanh_ prologue of
// zimage.cpp:104-107, once per 4 rows), combines each row's two wave
// partials through LDS, and finishes from registers + LDS. Two waves per row
// halve the live registers per lane against one wave per row (168 -> ~90
// VGPRs), doubling the waves in flight; measured the fastest of the variants
// tried (1 wave/row with 8 rows per block, L2 gathers of the vectors, 2 or 8
// rows per block, 4 waves per row: 69.4 against 71 % of HBM peak).
constexpr int kModRows = 4;
constexpr int kModThreads = kModRows * 128;

template <int V, bool HAS_SHIFT, bool STORE_Y>
__global__ __launch_bounds__(kModThreads) void k_ln_mod_gate(const float* __restrict__ x, float* __restrict__ res,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ shift,
                                                            const float* __restrict__ gate, float* __restrict__ yout,
                                                            int64_t rows, int C, float eps) {
    extern __shared__ f4 lds[];  // [3][n4]: 1+scale | shift | tanh(gate)
    __shared__ double red[2 * kModRows * 2];
    const int n4 = C >> 2;
    f4* s1 = lds;
    f4* sh = lds + n4;
    f4* tg = lds + 2 * n4;
    const int sub = threadIdx.x >> 7, t = threadIdx.x & 127, w = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * kModRows + sub;
    const bool ok = row < rows;
    const f4* xr = (const f4*)(x + row * C);
    f4* rr = (f4*)(res + row * C);
    // Issue order: the column vectors (L2 hits) first, then x, then res.
    // Loads complete in order, so the staging below waits only for the
    // vectors while the row loads are in flight, and the mean only for x.
    constexpr int SV = (V + 3) / 4;  // staged float4 per thread: n4 <= 128 V
    f4 ssc[SV], ssh[SV], sgt[SV];
#pragma unroll
    for (int k = 0; k < SV; ++k) {
        const int i = threadIdx.x + kModThreads * k;
        if (i < n4) {
            ssc[k] = ((const f4*)scale)[i];
            if constexpr (HAS_SHIFT) ssh[k] = ((const f4*)shift)[i];
            sgt[k] = ((const f4*)gate)[i];
        }
    }
    f4 v[V], rv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = t + 128 * j;
        v[j] = (ok && idx < n4) ? dev::ld_stream(xr + idx) : zero4();
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = t + 128 * j;
        rv[j] = (ok && idx < n4) ? dev::ld_stream(rr + idx) : zero4();
    }
#pragma unroll
    for (int k = 0; k < SV; ++k) {
        const int i = threadIdx.x + kModThreads * k;
        if (i < n4) {
            s1[i] = ssc[k] * 1.0f + 1.0f;
            if constexpr (HAS_SHIFT) sh[i] = ssh[k];
            sgt[k] = f4{tanhf(sgt[k].x), tanhf(sgt[k].y), tanhf(sgt[k].z), tanhf(sgt[k].w)};
            tg[i] = sgt[k];
        }
    }
    // One pass of statistics: sum and sum of squares in double (every fp32
    // square is exact in double), so var = E[x^2] - mean^2 keeps the precision
    // of the reference's two-pass double form for any offset; one reduction
    // and one barrier instead of two.
    double s = 0.0, q = 0.0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const double a = v[j].x, b = v[j].y, c = v[j].z, e = v[j].w;
        s += (a + b) + (c + e);
        q += fma(a, a, fma(b, b, fma(c, c, e * e)));
    }
    s = dev::wave_sum_d(s);
    q = dev::wave_sum_d(q);
    if ((threadIdx.x & 63) == 0) {
        red[w] = s;
        red[2 * kModRows + w] = q;
    }
    __syncthreads();  // also publishes the staged vectors
    if (!ok) return;
    const double ms = (red[2 * sub] + red[2 * sub + 1]) / (double)C;
    const double var = fmax((red[2 * kModRows + 2 * sub] + red[2 * kModRows + 2 * sub + 1]) / (double)C - ms * ms, 0.0);
    const float mean = (float)ms;
    const float rstd = (float)(1.0 / sqrt(var + (double)eps));
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = t + 128 * j;
        if (idx < n4) {
            const f4 ln = (v[j] - mean) * rstd;  // layer_norm, no affine
            const f4 m = s1[idx];
            f4 yv = f4{__fmul_rn(ln.x, m.x), __fmul_rn(ln.y, m.y), __fmul_rn(ln.z, m.z), __fmul_rn(ln.w, m.w)};
            if constexpr (HAS_SHIFT) yv = yv + sh[idx];  // add_rows_scaled_(y, ones, shift)
            if constexpr (STORE_Y) dev::st_stream((f4*)(yout + row * C) + idx, yv);
            dev::st_stream(rr + idx, rv[j] + tg[idx] * yv);  // res += tanh(gate) * y
        }
    }
}

// In-place per-group RMS norm over groups of dim = L * 4 floats, L lanes per
// group (L = 4 .. 64), 64 / L groups per wave step (tensor.cpp:687-695).
template <int L, bool HAS_G>
__global__ __launch_bounds__(kThreads) void k_heads(float* __restrict__ x, int64_t groups, int dim,
                                                   const float* __restrict__ gamma, float eps) {
    constexpr int GPW = 64 / L;  // groups per wave
    const int lane = threadIdx.x & 63;
    const int sub = lane % L;
    const int64_t grp = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * GPW + lane / L;
    const bool ok = grp < groups;
    f4* p = (f4*)(x + grp * dim) + sub;
    const f4 v = ok ? *p : zero4();
    const float q = dev::group_sum<L>(dev::sumsq4(v));  // all 64 lanes take part
    const float rstd = dev::rstd_fast(q, 1.0f / (4 * L), eps);  // dim = 4 L
    f4 o = v * rstd;
    if constexpr (HAS_G) o = o * ((const f4*)gamma)[sub];
    if (ok) dev::st_stream(p, o);
}

// Generic fallback: one wave per row, strided scalar loops; handles any C
// and any alignment. MODE: LN or RMS. Also used for in-place QK-norm of odd
// group sizes (y == x).
template <int MODE>
__global__ __launch_bounds__(kThreads) void k_rownorm_generic(const float* x, float* y, int64_t rows, int64_t C,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows; row += stride) {
        const float* p = x + row * C;
        float* q = y + row * C;
        float mean = 0.f, rstd;
        if constexpr (MODE == M_LN) {
            double s = 0.0;
            for (int64_t i = lane; i < C; i += 64) s += (double)p[i];
            mean = (float)(dev::wave_sum_d(s) / (double)C);
            double ss = 0.0;
            for (int64_t i = lane; i < C; i += 64) {
                const float d = p[i] - mean;
                ss += (double)d * (double)d;
            }
            rstd = rstd_of_d(dev::wave_sum_d(ss), C, eps);
        } else {
            float ss = 0.f;
            for (int64_t i = lane; i < C; i += 64) ss += p[i] * p[i];
            rstd = rstd_of(dev::wave_sum(ss), C, eps);
        }
        for (int64_t i = lane; i < C; i += 64) {
            if constexpr (MODE == M_LN) {
                float o = (p[i] - mean) * rstd;
                if (gamma) o = __fmul_rn(o, gamma[i]);
                if (beta) o = __fadd_rn(o, beta[i]);
                q[i] = o;
            } else {
                q[i] = p[i] * rstd * (gamma ? gamma[i] : 1.0f);
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void k_add_rms_generic(float* x, const float* r, float* y, int64_t rows,
                                                             int64_t C, const float* __restrict__ gamma, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows; row += stride) {
        float* p = x + row * C;
        const float* rp = r + row * C;
        float* q = y + row * C;
        float ss = 0.f;
        for (int64_t i = lane; i < C; i += 64) {
            const float s = p[i] + rp[i];
            p[i] = s;
            ss += s * s;
        }
        const float rstd = rstd_of(dev::wave_sum(ss), C, eps);
        for (int64_t i = lane; i < C; i += 64) q[i] = p[i] * rstd * (gamma ? gamma[i] : 1.0f);
    }
}

__global__ __launch_bounds__(kThreads) void k_ln_mod_gate_generic(const float* x, float* res,
                                                                 const float* __restrict__ scale,
                                                                 const float* __restrict__ shift,
                                                                 const float* __restrict__ gate, float* yout,
                                                                 int64_t rows, int64_t C, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows; row += stride) {
        const float* p = x + row * C;
        float* rp = res + row * C;
        // statistics summed in double, as layer_norm's (tensor.cpp:640-647)
        double s = 0.0;
        for (int64_t i = lane; i < C; i += 64) s += (double)p[i];
        const float mean = (float)(dev::wave_sum_d(s) / (double)C);
        double ss = 0.0;
        for (int64_t i = lane; i < C; i += 64) {
            const float d = p[i] - mean;
            ss += (double)d * (double)d;
        }
        const float rstd = rstd_of_d(dev::wave_sum_d(ss), C, eps);
        for (int64_t i = lane; i < C; i += 64) {
            float yv = __fmul_rn((p[i] - mean) * rstd, scale[i] * 1.0f + 1.0f);
            if (shift) yv = yv + shift[i];
            if (yout) yout[row * C + i] = yv;
            rp[i] = rp[i] + tanhf(gate[i]) * yv;
        }
    }
}

// ---- the Z-Image block's fused row ops ---------------------------------------
// y16 = bf16(((x * rstd) * gamma) * scale): rms_norm(x, gamma), mul_rows_(.,
// scale) (zimage.cpp:115-116, :128-129) and the bf16 rounding gemm_nt_bf16
// applies to its A (backend_cuda.cu:183-188), with the same fp32 products in
// the same order, so the bits equal those of the three-op sequence. The bf16
// row is the A operand of the projections that follow.
// PAIR (rows of exactly 64 V float4, y 16-byte aligned): lanes 2i and 2i+1
// swap one bf16x4 (a DPP exchange), so every lane stores 16 contiguous bytes,
// the even lane two consecutive float4s' results of step j, the odd lane
// those of step j + 1; the loads and the sum keep the one-wave order, so
// rstd, and the output, are bit-equal to the unpaired form's.
template <int V, bool HAS_G, bool HAS_S, bool PAIR = false>
__global__ __launch_bounds__(kThreads) void k_rms_mod_bf16(const float* __restrict__ x, uint2* __restrict__ y,
                                                          int64_t rows, int C, const float* __restrict__ gamma,
                                                          const float* __restrict__ scale, float eps) {
    const int lane = threadIdx.x & 63;
    const int n4 = C >> 2;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const f4* xr = (const f4*)(x + row * C);
    uint2* yr = y + row * n4;
    f4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        v[j] = idx < n4 ? dev::ld_stream(xr + idx) : zero4();
    }
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) q += dev::sumsq4(v[j]);
    const float rstd = rstd_of(dev::wave_sum(q), C, eps);
    auto out = [&](int j) __attribute__((always_inline)) {
        const int idx = lane + 64 * j;
        f4 o = v[j] * rstd;
        if constexpr (HAS_G) o = o * ((const f4*)gamma)[idx];
        if constexpr (HAS_S) o = o * ((const f4*)scale)[idx];
        return dev::bf16x4(o);
    };
    if constexpr (PAIR) {
        const bool odd = lane & 1;
        // quad_perm(1, 0, 3, 2): each lane reads its pair partner
        auto swap = [](unsigned u) { return (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, false); };
#pragma unroll
        for (int j = 0; j + 1 < V; j += 2) {
            const uint2 b0 = out(j), b1 = out(j + 1);
            const uint2 send = odd ? b0 : b1;
            const uint2 r = {swap(send.x), swap(send.y)};
            const dev::u4v w = odd ? dev::u4v{r.x, r.y, b1.x, b1.y} : dev::u4v{b0.x, b0.y, r.x, r.y};
            const int pos = odd ? lane - 1 + 64 * (j + 1) : lane + 64 * j;  // in uint2 units, even
            __builtin_nontemporal_store(w, reinterpret_cast<dev::u4v*>(yr + pos));
        }
        if constexpr (V & 1) dev::st_stream(yr + lane + 64 * (V - 1), out(V - 1));
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j)
            if (lane + 64 * j < n4) dev::st_stream(yr + lane + 64 * j, out(j));
    }
}

// x += gate * (a * rstd * gamma): y = rms_norm(a, gamma) then add_rows_scaled_(x,
// y, gate), or add_(x, y) without a gate (zimage.cpp:124-127, :132-135), with
// the same fp32 expressions, so x equals the two-op sequence's.
template <int V, bool HAS_G, bool HAS_GATE>
__global__ __launch_bounds__(kThreads) void k_rms_gated_add(float* __restrict__ x, const float* __restrict__ a,
                                                           int64_t rows, int C, const float* __restrict__ gamma,
                                                           const float* __restrict__ gate, float eps) {
    const int lane = threadIdx.x & 63;
    const int n4 = C >> 2;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const f4* ar = (const f4*)(a + row * C);
    f4* xr = (f4*)(x + row * C);
    // both rows are loaded before the reduction, so the x stream is in
    // flight while the sum of squares is formed
    f4 v[V], xv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        v[j] = idx < n4 ? dev::ld_stream(ar + idx) : zero4();
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        xv[j] = idx < n4 ? dev::ld_stream(xr + idx) : zero4();
    }
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) q += dev::sumsq4(v[j]);
    const float rstd = rstd_of(dev::wave_sum(q), C, eps);
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        if (idx < n4) {
            // o is rounded on its own as rms_norm's output is: no contraction of
            // (a rstd) gamma into an FMA with x (the gate's FMA is explicit, as in
            // add_rows_scaled_)
#pragma clang fp contract(off)
            f4 o = v[j] * rstd;
            if constexpr (HAS_G) o = o * ((const f4*)gamma)[idx];
            const f4 xo = xv[j];
            f4 r;
            if constexpr (HAS_GATE) {
                const f4 g = ((const f4*)gate)[idx];
                r = f4{fmaf(g.x, o.x, xo.x), fmaf(g.y, o.y, xo.y), fmaf(g.z, o.z, xo.z), fmaf(g.w, o.w, xo.w)};
            } else {
                r = xo + o;
            }
            dev::st_stream(xr + idx, r);
        }
    }
}

// k_rms_gated_add with one 256-thread workgroup per row (2048 < C <= 8192).
// The sum of squares is formed in exactly the one-wave kernels' order (per
// lane l: float4 l, l + 64, l + 128, ... in sequence, then the wave tree),
// through LDS, so rstd has the bits rms_norm's has and x stays bit-equal to
// rms_norm then add_rows_scaled_.
template <int V, bool HAS_G, bool HAS_GATE>
__global__ __launch_bounds__(kRowThreads) void k_rms_gated_add_row(float* __restrict__ x, const float* __restrict__ a,
                                                                  int C, const float* __restrict__ gamma,
                                                                  const float* __restrict__ gate, float eps) {
    __shared__ float hs[4 * V][64];  // hs[k][l]: squared sum of float4 l + 64 k
    const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
    const int n4 = C >> 2;
    const int64_t row = blockIdx.x;
    const f4* ar = (const f4*)(a + row * C);
    f4* xr = (f4*)(x + row * C);
    f4 v[V], xv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * (p + 4 * j);
        v[j] = idx < n4 ? dev::ld_stream(ar + idx) : zero4();
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * (p + 4 * j);
        xv[j] = idx < n4 ? dev::ld_stream(xr + idx) : zero4();
    }
#pragma unroll
    for (int j = 0; j < V; ++j) hs[p + 4 * j][lane] = dev::sumsq4(v[j]);
    __syncthreads();
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < 4 * V; ++k) q += hs[k][lane];  // zero entries past the row add exactly 0
    const float rstd = rstd_of(dev::wave_sum(q), C, eps);
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * (p + 4 * j);
        if (idx < n4) {
#pragma clang fp contract(off)
            f4 o = v[j] * rstd;
            if constexpr (HAS_G) o = o * ((const f4*)gamma)[idx];
            const f4 xo = xv[j];
            f4 r;
            if constexpr (HAS_GATE) {
                const f4 g = ((const f4*)gate)[idx];
                r = f4{fmaf(g.x, o.x, xo.x), fmaf(g.y, o.y, xo.y), fmaf(g.z, o.z, xo.z), fmaf(g.w, o.w, xo.w)};
            } else {
                r = xo + o;
            }
            dev::st_stream(xr + idx, r);
        }
    }
}

// ---- residual add + RMSNorm + modulate: one sublayer's end and the next one's input ----
// x += gate * rms_norm(a, g1), then y16 = bf16(((x * rstd2) * g2) * scale) of
// the updated row: rms_norm_gated_add then rms_norm_modulate_bf16
// (zimage.cpp:124-129 and :132-135 -> :114-116), x read once instead of
// twice. Each half keeps its op's expressions and its sum of squares in the
// one-wave order (per lane l: float4 l, l + 64, ... in sequence, then the
// wave tree), so x and y16 are bit-equal to the two ops'. The vectors are
// optional (null: that product or the gate is left out, as in the two ops).

// x + gate * (a rstd gamma), k_rms_gated_add's expression
__device__ __forceinline__ f4 gated_add4(const f4& v, const f4& xo, float rstd, const float* g1, const float* gate,
                                         int idx) {
#pragma clang fp contract(off)
    f4 o = v * rstd;
    if (g1) o = o * ((const f4*)g1)[idx];
    if (!gate) return xo + o;
    const f4 g = ((const f4*)gate)[idx];
    return f4{fmaf(g.x, o.x, xo.x), fmaf(g.y, o.y, xo.y), fmaf(g.z, o.z, xo.z), fmaf(g.w, o.w, xo.w)};
}

// Stores y16 for V float4 of the updated row (r, zero past the row), lane's
// float4 at step j being lane + base(j); k_rms_mod_bf16's products. PAIR
// (n4 % 64 == 0, y 16-byte aligned): k_rms_mod_bf16's paired 16-byte stores.
template <int V, bool PAIR, class Base>
__device__ __forceinline__ void store_mod_bf16(uint2* yr, const f4 (&r)[V], float rstd, const float* g2,
                                               const float* scale, int lane, int n4, Base base) {
    auto out = [&](int j) __attribute__((always_inline)) {
        const int idx = lane + base(j);
        if (idx >= n4) return uint2{0u, 0u};
        f4 o = r[j] * rstd;
        if (g2) o = o * ((const f4*)g2)[idx];
        if (scale) o = o * ((const f4*)scale)[idx];
        return dev::bf16x4(o);
    };
    if constexpr (PAIR) {
        const bool odd = lane & 1;
        auto swap = [](unsigned u) { return (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, false); };
#pragma unroll
        for (int j = 0; j + 1 < V; j += 2) {
            const uint2 b0 = out(j), b1 = out(j + 1);
            const uint2 send = odd ? b0 : b1;
            const uint2 rr = {swap(send.x), swap(send.y)};
            const dev::u4v w = odd ? dev::u4v{rr.x, rr.y, b1.x, b1.y} : dev::u4v{b0.x, b0.y, rr.x, rr.y};
            const int pos = odd ? lane - 1 + base(j + 1) : lane + base(j);
            if (pos < n4) __builtin_nontemporal_store(w, reinterpret_cast<dev::u4v*>(yr + pos));
        }
        if constexpr (V & 1) {
            if (lane + base(V - 1) < n4) dev::st_stream(yr + lane + base(V - 1), out(V - 1));
        }
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j)
            if (lane + base(j) < n4) dev::st_stream(yr + lane + base(j), out(j));
    }
}

// one wave per row (rows of up to 64 V float4), 4 rows per workgroup
template <int V, bool PAIR>
__global__ __launch_bounds__(kThreads) void k_rms_gated_add_mod(float* __restrict__ x, const float* __restrict__ a,
                                                               uint2* __restrict__ y, int64_t rows, int C,
                                                               const float* __restrict__ g1,
                                                               const float* __restrict__ gate,
                                                               const float* __restrict__ g2,
                                                               const float* __restrict__ scale, float eps1,
                                                               float eps2) {
    const int lane = threadIdx.x & 63;
    const int n4 = C >> 2;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const f4* ar = (const f4*)(a + row * C);
    f4* xr = (f4*)(x + row * C);
    f4 v[V], xv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        v[j] = idx < n4 ? dev::ld_stream(ar + idx) : zero4();
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        xv[j] = idx < n4 ? dev::ld_stream(xr + idx) : zero4();
    }
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) q += dev::sumsq4(v[j]);
    const float rstd1 = rstd_of(dev::wave_sum(q), C, eps1);
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        if (idx < n4) {
            xv[j] = gated_add4(v[j], xv[j], rstd1, g1, gate, idx);
            dev::st_stream(xr + idx, xv[j]);
        }
    }
    float q2 = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) q2 += dev::sumsq4(xv[j]);
    const float rstd2 = rstd_of(dev::wave_sum(q2), C, eps2);
    store_mod_bf16<V, PAIR>(y + row * n4, xv, rstd2, g2, scale, lane, n4, [](int j) { return 64 * j; });
}

// one workgroup of W waves per row, wave p lane l holding float4 l + 64 (p +
// W j), j < V; both sums of squares in the one-wave order (float4 block k =
// p + W j in sequence, then the wave tree) through LDS. The column vectors
// are loaded ahead of the stores that precede their use: g1 and gate before
// the row, g2 and scale before the x stores. A wave's vector loads and
// stores are counted down in issue order, so a vector loaded after the x
// stores would have waited for every one of them to complete before the
// bf16 row could be formed. The vectors are never null here: the launcher
// passes a vector of ones for an absent one (an absent gate is the plain
// add), which leaves every product and sum bit-equal to leaving it out.
template <int W, int V, bool PAIR>
__global__ __launch_bounds__(64 * W) void k_rms_gated_add_mod_row(float* __restrict__ x, const float* __restrict__ a,
                                                                 uint2* __restrict__ y, int C,
                                                                 const float* __restrict__ g1,
                                                                 const float* __restrict__ gate,
                                                                 const float* __restrict__ g2,
                                                                 const float* __restrict__ scale, float eps1,
                                                                 float eps2) {
    __shared__ float hs[2][W * V][64];  // hs[h][k][l]: squared sum of float4 l + 64 k of a (h = 0), of x (h = 1)
    const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
    const int n4 = C >> 2;
    const int64_t row = blockIdx.x;
    const f4* ar = (const f4*)(a + row * C);
    f4* xr = (f4*)(x + row * C);
    auto pos = [&](int j) __attribute__((always_inline)) { return lane + 64 * (p + W * j); };
    // lanes past the row read a valid column vector (their values are never stored)
    auto col = [&](const float* vec, int j) __attribute__((always_inline)) {
        return ((const f4*)vec)[min(pos(j), n4 - 1)];
    };
    f4 c1[V], cg[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        c1[j] = col(g1, j);
        cg[j] = col(gate, j);
    }
    f4 v[V], xv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = pos(j) < n4 ? dev::ld_stream(ar + pos(j)) : zero4();
#pragma unroll
    for (int j = 0; j < V; ++j) xv[j] = pos(j) < n4 ? dev::ld_stream(xr + pos(j)) : zero4();
#pragma unroll
    for (int j = 0; j < V; ++j) hs[0][p + W * j][lane] = dev::sumsq4(v[j]);
    __syncthreads();
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < W * V; ++k) q += hs[0][k][lane];  // zero entries past the row add exactly 0
    const float rstd1 = rstd_of(dev::wave_sum(q), C, eps1);
#pragma unroll
    for (int j = 0; j < V; ++j) {
#pragma clang fp contract(off)
        f4 o = v[j] * rstd1;
        o = o * c1[j];
        const f4 g = cg[j], xo = xv[j];
        xv[j] = f4{fmaf(g.x, o.x, xo.x), fmaf(g.y, o.y, xo.y), fmaf(g.z, o.z, xo.z), fmaf(g.w, o.w, xo.w)};
    }
    // the second pair of vectors, into the registers the first pair and the a row leave
    f4 c2[V], cs[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        c2[j] = col(g2, j);
        cs[j] = col(scale, j);
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
        if (pos(j) < n4) {
            dev::st_stream(xr + pos(j), xv[j]);
            hs[1][p + W * j][lane] = dev::sumsq4(xv[j]);
        } else {
            hs[1][p + W * j][lane] = 0.f;
        }
    }
    __syncthreads();
    float q2 = 0.f;
#pragma unroll
    for (int k = 0; k < W * V; ++k) q2 += hs[1][k][lane];
    const float rstd2 = rstd_of(dev::wave_sum(q2), C, eps2);
    // y16 = bf16(((x * rstd2) * g2) * scale), k_rms_mod_bf16's products
    uint2 b[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
#pragma clang fp contract(off)
        f4 o = xv[j] * rstd2;
        o = o * c2[j];
        o = o * cs[j];
        b[j] = dev::bf16x4(o);
    }
    uint2* yr = y + row * n4;
    if constexpr (PAIR) {
        // adjacent lanes swap one bf16x4 so every lane stores 16 contiguous bytes
        const bool odd = lane & 1;
        auto swap = [](unsigned u) { return (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, false); };
#pragma unroll
        for (int j = 0; j + 1 < V; j += 2) {
            const uint2 b0 = b[j], b1 = b[j + 1];
            const uint2 send = odd ? b0 : b1;
            const uint2 rr = {swap(send.x), swap(send.y)};
            const dev::u4v w = odd ? dev::u4v{rr.x, rr.y, b1.x, b1.y} : dev::u4v{b0.x, b0.y, rr.x, rr.y};
            const int at = odd ? pos(j + 1) - 1 : pos(j);
            if (at < n4) __builtin_nontemporal_store(w, reinterpret_cast<dev::u4v*>(yr + at));
        }
        if constexpr (V & 1) {
            if (pos(V - 1) < n4) dev::st_stream(yr + pos(V - 1), b[V - 1]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j)
            if (pos(j) < n4) dev::st_stream(yr + pos(j), b[j]);
    }
}

// The same op over consecutive rows per workgroup, for rows of exactly
// 64 W V float4 (3840 = 64 x 15 x 1). The four column vectors are loaded once
// per workgroup and kept in registers: loaded once per row they are 61 KB of
// L2 reads per 45 KB row of HBM traffic, and measured they, not HBM, bound
// the one-row-per-workgroup kernel (its byte mix without them: 35 us at
// [4096, 3840]; with them: 44 us). Row i + 1 is loaded while row i is
// formed, ahead of row i's stores, through buffer loads over the row, so a
// workgroup's last prefetch covers an empty range (no memory access) and
// every load is issued unconditionally. Per row the arithmetic and both
// sums of squares are k_rms_gated_add_mod_row's, so the results are
// bit-equal to it and to the two ops.
template <int W, int V>
__device__ __forceinline__ void rows_load(f4 (&v)[V], const float* base, bool present) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, present ? 64 * W * V * 16 : 0, 0x00020000);
    const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < V; ++j)
        v[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (lane + 64 * p) * 16, 64 * W * 16 * j, 2));
}

// 1 / rms of a row from its per-block sums of squares h[k][lane] (block k =
// float4 lane + 64 k): wave 0 adds them per lane in block order, then the
// wave tree (the one-wave kernels' order), and broadcasts the result through
// *out; the other waves read one word instead of K per lane. Two barriers:
// the first publishes h, the second *out. The caller's next write of h comes
// after the second barrier, which every wave passes after wave 0's reads.
template <int K>
__device__ __forceinline__ float rows_rstd(const float (*h)[64], float* out, int C, float eps) {
    __syncthreads();
    if (threadIdx.x < 64) {
        float q = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) q += h[k][threadIdx.x];
        const float r = rstd_of(dev::wave_sum(q), C, eps);
        if (threadIdx.x == 0) *out = r;
    }
    __syncthreads();
    return *out;
}

template <int W, int V, bool PAIR>
__device__ __forceinline__ void rows_one(float* __restrict__ x, const float* __restrict__ a, uint2* __restrict__ y,
                                         int64_t rows, int64_t row, int C, f4 (&v)[V], f4 (&xc)[V], f4 (&an)[V],
                                         f4 (&xn)[V], int64_t next, const f4 (&c1)[V], const f4 (&cg)[V],
                                         const f4 (&c2)[V], const f4 (&cs)[V], float eps1, float eps2,
                                         float (*hs)[W * V][64], float* rs) {
    const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
    constexpr int n4 = 64 * W * V;
    auto pos = [&](int j) __attribute__((always_inline)) { return lane + 64 * (p + W * j); };
#pragma unroll
    for (int j = 0; j < V; ++j) hs[0][p + W * j][lane] = dev::sumsq4(v[j]);
    const float rstd1 = rows_rstd<W * V>(hs[0], rs, C, eps1);
#pragma unroll
    for (int j = 0; j < V; ++j) {
#pragma clang fp contract(off)
        f4 o = v[j] * rstd1;
        o = o * c1[j];
        const f4 g = cg[j], xo = xc[j];
        xc[j] = f4{fmaf(g.x, o.x, xo.x), fmaf(g.y, o.y, xo.y), fmaf(g.z, o.z, xo.z), fmaf(g.w, o.w, xo.w)};
    }
    // row `next`, ahead of this row's stores (an empty range past the workgroup's last row)
    const bool more = next < rows;
    rows_load<W, V>(an, a + (more ? next : row) * (int64_t)C, more);
    rows_load<W, V>(xn, x + (more ? next : row) * (int64_t)C, more);
    f4* xr = (f4*)(x + row * (int64_t)C);
#pragma unroll
    for (int j = 0; j < V; ++j) {
        dev::st_stream(xr + pos(j), xc[j]);
        hs[1][p + W * j][lane] = dev::sumsq4(xc[j]);
    }
    const float rstd2 = rows_rstd<W * V>(hs[1], rs + 1, C, eps2);
    uint2 b[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
#pragma clang fp contract(off)
        f4 o = xc[j] * rstd2;
        o = o * c2[j];
        o = o * cs[j];
        b[j] = dev::bf16x4(o);
    }
    uint2* yr = y + row * (int64_t)n4;
    if constexpr (PAIR) {
        const bool odd = lane & 1;
        auto swap = [](unsigned u) { return (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, false); };
#pragma unroll
        for (int j = 0; j + 1 < V; j += 2) {
            const uint2 b0 = b[j], b1 = b[j + 1];
            const uint2 send = odd ? b0 : b1;
            const uint2 rr = {swap(send.x), swap(send.y)};
            const dev::u4v w = odd ? dev::u4v{rr.x, rr.y, b1.x, b1.y} : dev::u4v{b0.x, b0.y, rr.x, rr.y};
            __builtin_nontemporal_store(w, reinterpret_cast<dev::u4v*>(yr + (odd ? pos(j + 1) - 1 : pos(j))));
        }
        if constexpr (V & 1) dev::st_stream(yr + pos(V - 1), b[V - 1]);
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j) dev::st_stream(yr + pos(j), b[j]);
    }
}

// Workgroup b of G takes rows [b rows / G, (b + 1) rows / G): G at most one
// round of resident workgroups, so every workgroup starts at once and each
// runs rows / G rows, give or take one.
template <int W, int V, bool PAIR>
__global__ __launch_bounds__(64 * W) void k_rms_gated_add_mod_rows(float* __restrict__ x, const float* __restrict__ a,
                                                                  uint2* __restrict__ y, int64_t rows, int C,
                                                                  const float* __restrict__ g1,
                                                                  const float* __restrict__ gate,
                                                                  const float* __restrict__ g2,
                                                                  const float* __restrict__ scale, float eps1,
                                                                  float eps2) {
    __shared__ float hs[2][W * V][64];
    __shared__ float rs[2];
    const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * rows / gridDim.x;
    const int64_t end = (int64_t)(blockIdx.x + 1) * rows / gridDim.x;  // this workgroup's rows [r0, end)
    f4 c1[V], cg[V], c2[V], cs[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int i = lane + 64 * (p + W * j);
        c1[j] = ((const f4*)g1)[i];
        cg[j] = ((const f4*)gate)[i];
        c2[j] = ((const f4*)g2)[i];
        cs[j] = ((const f4*)scale)[i];
    }
    f4 v[V], xa[V], xb[V];
    rows_load<W, V>(v, a + r0 * (int64_t)C, true);
    rows_load<W, V>(xa, x + r0 * (int64_t)C, true);
    for (int64_t row = r0; row < end; row += 2) {
        rows_one<W, V, PAIR>(x, a, y, end, row, C, v, xa, v, xb, row + 1, c1, cg, c2, cs, eps1, eps2, hs, rs);
        if (row + 1 >= end) break;
        rows_one<W, V, PAIR>(x, a, y, end, row + 1, C, v, xb, v, xa, row + 2, c1, cg, c2, cs, eps1, eps2, hs, rs);
    }
}

// Workgroups of k_rms_gated_add_mod_rows<15, 1, pair> the GPU holds at once
// (resident per CU x CUs; 2 x 256 on MI355X); cached.
int64_t rows15_slots(bool pair) {
    static int64_t cache[2] = {0, 0};
    int64_t& c = cache[pair];
    if (!c) {
        int nb = 0;
        const void* k = pair ? reinterpret_cast<const void*>(k_rms_gated_add_mod_rows<15, 1, true>)
                             : reinterpret_cast<const void*>(k_rms_gated_add_mod_rows<15, 1, false>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, 960, 0) != hipSuccess || nb < 1) nb = 1;
        c = (int64_t)nb * num_cus();
    }
    return c;
}

// the row-per-workgroup kernels' float4 per lane for a row of n4 float4, or 0
int pick_row_v(int64_t n4) {
    if (n4 <= 512) return 0;  // narrower rows: one wave per row
    if (n4 <= 1024) return 4;
    if (n4 <= 2048) return 8;
    return 0;
}

// any C / alignment: one wave per row, strided loops over the row
template <bool GATED>
__global__ __launch_bounds__(kThreads) void k_rms_fused_generic(const float* __restrict__ src, float* __restrict__ x,
                                                               unsigned short* __restrict__ y16, int64_t rows,
                                                               int64_t C, const float* __restrict__ gamma,
                                                               const float* __restrict__ vec, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows; row += stride) {
        const float* p = src + row * C;
        float ss = 0.f;
        for (int64_t i = lane; i < C; i += 64) ss += p[i] * p[i];
        const float rstd = rstd_of(dev::wave_sum(ss), C, eps);
        for (int64_t i = lane; i < C; i += 64) {
#pragma clang fp contract(off)
            float o = p[i] * rstd * (gamma ? gamma[i] : 1.0f);
            if constexpr (GATED) {
                float* xp = x + row * C + i;
                *xp = vec ? fmaf(vec[i], o, *xp) : *xp + o;
            } else {
                if (vec) o = o * vec[i];
                y16[row * C + i] = dev::bf16_rne(o);
            }
        }
    }
}

// ---- dispatch helpers ------------------------------------------------------
constexpr int kMaxV = 32;

// Smallest supported V with 64 * V >= n4, or 0 if n4 is too large.
int pick_v(int64_t n4) {
    static const int vs[] = {1, 2, 4, 8, 12, 15, 16, 24, 32};
    for (int v : vs)
        if (64 * (int64_t)v >= n4) return v;
    return 0;
}

unsigned row_grid(int64_t rows, int waves_per_cu) {
    const int64_t want = (rows + kWaves - 1) / kWaves;
    const int64_t cap = (int64_t)num_cus() * waves_per_cu / kWaves;
    return (unsigned)std::max<int64_t>(1, std::min(want, std::max<int64_t>(cap, 1)));
}

// One wave per row (or per unit), 4 per workgroup, covering all of them.
unsigned exact_grid(int64_t units) {
    const int64_t b = (units + kWaves - 1) / kWaves;
    need(b * kThreads <= kMaxGridItems, "backend_hip", "too many rows for one launch");
    return (unsigned)std::max<int64_t>(1, b);
}

// Rows one launch of the one-wave-per-row kernels covers; the entry points
// split larger tensors into launches of at most this many rows.
int64_t rows_per_launch() { return units_per_launch(64); }

// Calls f(std::integral_constant<int, V>) for the runtime V.
template <class F>
void with_v(int v, F&& f) {
    switch (v) {
        case 1: f(std::integral_constant<int, 1>()); break;
        case 2: f(std::integral_constant<int, 2>()); break;
        case 4: f(std::integral_constant<int, 4>()); break;
        case 8: f(std::integral_constant<int, 8>()); break;
        case 12: f(std::integral_constant<int, 12>()); break;
        case 15: f(std::integral_constant<int, 15>()); break;
        case 16: f(std::integral_constant<int, 16>()); break;
        case 24: f(std::integral_constant<int, 24>()); break;
        case 32: f(std::integral_constant<int, 32>()); break;
        default: fail(SDH_ERR_INVALID, "internal: unsupported row width");
    }
}

bool vec_ok(int64_t C, std::initializer_list<const void*> ptrs) {
    if (C % 4 != 0 || pick_v(C / 4) == 0 || C > (int64_t)64 * 4 * kMaxV) return false;
    for (const void* p : ptrs)
        if (p && !aligned16(p)) return false;
    return true;
}

void run_rownorm(const char* op, int mode, const float* x, float* y, int64_t rows, int64_t C, const float* gamma,
                 const float* beta, float eps) {
    need(rows >= 0 && C >= 0, op, "negative size");
    if (rows == 0 || C == 0) return;
    ensure_init();
    const size_t bytes = (size_t)(rows * C) * 4;
    check_range(x, bytes, op, "x");
    check_range(y, bytes, op, "y");
    if (gamma) check_range(gamma, (size_t)C * 4, op, "gamma");
    if (beta) check_range(beta, (size_t)C * 4, op, "beta");
    if (rows > rows_per_launch()) {
        in_pieces(rows, rows_per_launch(), [&](int64_t r0, int64_t nr) {
            run_rownorm(op, mode, x + r0 * C, y + r0 * C, nr, C, gamma, beta, eps);
        });
        return;
    }
    if (vec_ok(C, {x, y, gamma, beta})) {
        const int v = pick_v(C / 4);
        const unsigned grid = exact_grid(rows);
        with_v(v, [&](auto vc) {
            constexpr int V = decltype(vc)::value;
            if (mode == M_RMS) {
                if (gamma)
                    k_rownorm<V, M_RMS, true, false><<<grid, kThreads, 0, stream()>>>(x, y, rows, (int)C, gamma, beta, eps);
                else
                    k_rownorm<V, M_RMS, false, false><<<grid, kThreads, 0, stream()>>>(x, y, rows, (int)C, gamma, beta, eps);
            } else {
                if (gamma && beta)
                    k_rownorm<V, M_LN, true, true><<<grid, kThreads, 0, stream()>>>(x, y, rows, (int)C, gamma, beta, eps);
                else if (gamma)
                    k_rownorm<V, M_LN, true, false><<<grid, kThreads, 0, stream()>>>(x, y, rows, (int)C, gamma, beta, eps);
                else if (beta)
                    k_rownorm<V, M_LN, false, true><<<grid, kThreads, 0, stream()>>>(x, y, rows, (int)C, gamma, beta, eps);
                else
                    k_rownorm<V, M_LN, false, false><<<grid, kThreads, 0, stream()>>>(x, y, rows, (int)C, gamma, beta, eps);
            }
        });
    } else {
        const unsigned grid = row_grid(rows, 32);
        if (mode == M_RMS)
            k_rownorm_generic<M_RMS><<<grid, kThreads, 0, stream()>>>(x, y, rows, C, gamma, beta, eps);
        else
            k_rownorm_generic<M_LN><<<grid, kThreads, 0, stream()>>>(x, y, rows, C, gamma, beta, eps);
    }
    launched(op);
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + nb && y < x + na;
}

void run_rms_mod_bf16(const float* x, uint16_t* y, int64_t rows, int64_t C, const float* gamma, const float* scale,
                      float eps) {
    const char* op = "sdh_rms_norm_modulate_bf16";
    need(rows >= 0 && C >= 0, op, "negative size");
    if (rows == 0 || C == 0) return;
    ensure_init();
    check_range(x, (size_t)(rows * C) * 4, op, "x");
    check_range(y, (size_t)(rows * C) * 2, op, "y");
    if (gamma) check_range(gamma, (size_t)C * 4, op, "gamma");
    if (scale) check_range(scale, (size_t)C * 4, op, "scale");
    need(!overlaps(x, (size_t)(rows * C) * 4, y, (size_t)(rows * C) * 2), op, "y overlaps x");
    if (rows > rows_per_launch()) {
        in_pieces(rows, rows_per_launch(), [&](int64_t r0, int64_t nr) {
            run_rms_mod_bf16(x + r0 * C, y + r0 * C, nr, C, gamma, scale, eps);
        });
        return;
    }
    if (vec_ok(C, {x, gamma, scale}) && ((uintptr_t)y & 7) == 0) {
        const unsigned grid = exact_grid(rows);
        with_v(pick_v(C / 4), [&](auto vc) {
            constexpr int V = decltype(vc)::value;
            uint2* yy = (uint2*)y;
            if (gamma && scale && C == 256 * V && ((uintptr_t)y & 15) == 0)
                k_rms_mod_bf16<V, true, true, true><<<grid, kThreads, 0, stream()>>>(x, yy, rows, (int)C, gamma, scale,
                                                                                   eps);
            else if (gamma && scale)
                k_rms_mod_bf16<V, true, true><<<grid, kThreads, 0, stream()>>>(x, yy, rows, (int)C, gamma, scale, eps);
            else if (gamma)
                k_rms_mod_bf16<V, true, false><<<grid, kThreads, 0, stream()>>>(x, yy, rows, (int)C, gamma, scale, eps);
            else if (scale)
                k_rms_mod_bf16<V, false, true><<<grid, kThreads, 0, stream()>>>(x, yy, rows, (int)C, gamma, scale, eps);
            else
                k_rms_mod_bf16<V, false, false><<<grid, kThreads, 0, stream()>>>(x, yy, rows, (int)C, gamma, scale, eps);
        });
    } else {
        k_rms_fused_generic<false><<<row_grid(rows, 32), kThreads, 0, stream()>>>(x, nullptr, (unsigned short*)y, rows,
                                                                                   C, gamma, scale, eps);
    }
    launched(op);
}

void run_rms_gated_add(float* x, const float* a, int64_t rows, int64_t C, const float* gamma, const float* gate,
                       float eps) {
    const char* op = "sdh_rms_norm_gated_add";
    need(rows >= 0 && C >= 0, op, "negative size");
    if (rows == 0 || C == 0) return;
    ensure_init();
    const size_t bytes = (size_t)(rows * C) * 4;
    check_range(x, bytes, op, "x");
    check_range(a, bytes, op, "a");
    if (gamma) check_range(gamma, (size_t)C * 4, op, "gamma");
    if (gate) check_range(gate, (size_t)C * 4, op, "gate");
    need(!overlaps(x, bytes, a, bytes), op, "x overlaps a");
    if (rows > rows_per_launch()) {
        in_pieces(rows, rows_per_launch(), [&](int64_t r0, int64_t nr) {
            run_rms_gated_add(x + r0 * C, a + r0 * C, nr, C, gamma, gate, eps);
        });
        return;
    }
    const int rv = pick_row_v(C / 4);
    if (rv && vec_ok(C, {x, a, gamma, gate})) {
        // one workgroup per row
        in_pieces(rows, units_per_launch(kRowThreads), [&](int64_t r0, int64_t nr) {
            float* xp = x + r0 * C;
            const float* ap = a + r0 * C;
            auto go = [&](auto vc) {
                constexpr int V = decltype(vc)::value;
                const unsigned g = (unsigned)nr;
                if (gamma && gate)
                    k_rms_gated_add_row<V, true, true><<<g, kRowThreads, 0, stream()>>>(xp, ap, (int)C, gamma, gate, eps);
                else if (gamma)
                    k_rms_gated_add_row<V, true, false><<<g, kRowThreads, 0, stream()>>>(xp, ap, (int)C, gamma, gate, eps);
                else if (gate)
                    k_rms_gated_add_row<V, false, true><<<g, kRowThreads, 0, stream()>>>(xp, ap, (int)C, gamma, gate, eps);
                else
                    k_rms_gated_add_row<V, false, false><<<g, kRowThreads, 0, stream()>>>(xp, ap, (int)C, gamma, gate, eps);
            };
            if (rv == 4) go(std::integral_constant<int, 4>());
            else go(std::integral_constant<int, 8>());
        });
    } else if (vec_ok(C, {x, a, gamma, gate})) {
        const unsigned grid = exact_grid(rows);
        with_v(pick_v(C / 4), [&](auto vc) {
            constexpr int V = decltype(vc)::value;
            if (gamma && gate)
                k_rms_gated_add<V, true, true><<<grid, kThreads, 0, stream()>>>(x, a, rows, (int)C, gamma, gate, eps);
            else if (gamma)
                k_rms_gated_add<V, true, false><<<grid, kThreads, 0, stream()>>>(x, a, rows, (int)C, gamma, gate, eps);
            else if (gate)
                k_rms_gated_add<V, false, true><<<grid, kThreads, 0, stream()>>>(x, a, rows, (int)C, gamma, gate, eps);
            else
                k_rms_gated_add<V, false, false><<<grid, kThreads, 0, stream()>>>(x, a, rows, (int)C, gamma, gate, eps);
        });
    } else {
        k_rms_fused_generic<true><<<row_grid(rows, 32), kThreads, 0, stream()>>>(a, x, nullptr, rows, C, gamma, gate,
                                                                                  eps);
    }
    launched(op);
}

void run_rms_gated_add_mod(float* x, const float* a, uint16_t* y, int64_t rows, int64_t C, const float* g1,
                           const float* gate, const float* g2, const float* scale, float eps1, float eps2) {
    const char* op = "sdh_rms_norm_gated_add_modulate_bf16";
    need(rows >= 0 && C >= 0, op, "negative size");
    if (rows == 0 || C == 0) return;
    ensure_init();
    const size_t bytes = (size_t)(rows * C) * 4, ybytes = (size_t)(rows * C) * 2;
    check_range(x, bytes, op, "x");
    check_range(a, bytes, op, "a");
    check_range(y, ybytes, op, "y");
    for (const float* vec : {g1, gate, g2, scale})
        if (vec) check_range(vec, (size_t)C * 4, op, "a column vector");
    need(!overlaps(x, bytes, a, bytes), op, "x overlaps a");
    need(!overlaps(y, ybytes, x, bytes) && !overlaps(y, ybytes, a, bytes), op, "y overlaps x or a");
    const int64_t n4 = C / 4;
    const bool vec = vec_ok(C, {x, a, g1, gate, g2, scale}) && ((uintptr_t)y & 7) == 0;
    if (!vec) {
        // the two ops, each on its own general kernel
        run_rms_gated_add(x, a, rows, C, g1, gate, eps1);
        run_rms_mod_bf16(x, y, rows, C, g2, scale, eps2);
        return;
    }
    const bool pair = n4 % 64 == 0 && ((uintptr_t)y & 15) == 0;
    uint2* yy = (uint2*)y;
    const int rv = pick_row_v(n4);
    if (rv) {
        // absent column vectors become a vector of ones (bit-equal, see the kernel)
        const float* one = ones_vector(C);
        const float *v1 = g1 ? g1 : one, *vg = gate ? gate : one, *v2 = g2 ? g2 : one, *vs = scale ? scale : one;
        // rows of exactly 960 float4 (C = 3840, the Z-Image width) take the
        // multi-row kernel: 15 waves, one float4 per lane, 8 rows per workgroup
        const bool rows15 = n4 == 64 * 15;
        in_pieces(rows, units_per_launch(rows15 ? 960 / 8 : kRowThreads), [&](int64_t r0, int64_t nr) {
            const int64_t o = r0 * C;
            auto go = [&](auto wc, auto vc, auto pc) {
                constexpr int W = decltype(wc)::value, V = decltype(vc)::value;
                constexpr bool P = decltype(pc)::value;
                k_rms_gated_add_mod_row<W, V, P><<<(unsigned)nr, 64 * W, 0, stream()>>>(
                    x + o, a + o, yy + r0 * n4, (int)C, v1, vg, v2, vs, eps1, eps2);
            };
            using I4 = std::integral_constant<int, 4>;
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (rows15) {
                // measured at [4096, 3840]: 15 waves x 1 float4 over 8 rows
                // per workgroup (512 workgroups: two per CU, one round)
                // 39.3 us; 5 x 3 over 8 rows 45 us; 15 x 1 over 4 rows (two
                // rounds) 42 us, over 16 rows (one workgroup per CU) 43.6 us;
                // two rows ahead 41.9 us. So: one round of resident
                // workgroups, the rows shared out evenly.
                const unsigned g = (unsigned)std::min<int64_t>(nr, rows15_slots(pair));
                if (pair)
                    k_rms_gated_add_mod_rows<15, 1, true><<<g, 960, 0, stream()>>>(
                        x + o, a + o, yy + r0 * n4, nr, (int)C, v1, vg, v2, vs, eps1, eps2);
                else
                    k_rms_gated_add_mod_rows<15, 1, false><<<g, 960, 0, stream()>>>(
                        x + o, a + o, yy + r0 * n4, nr, (int)C, v1, vg, v2, vs, eps1, eps2);
            }
            else if (rv == 4) pair ? go(I4(), I4(), T_()) : go(I4(), I4(), F_());
            else pair ? go(I4(), std::integral_constant<int, 8>(), T_()) : go(I4(), std::integral_constant<int, 8>(), F_());
        });
    } else {
        in_pieces(rows, rows_per_launch(), [&](int64_t r0, int64_t nr) {
            const int64_t o = r0 * C;
            with_v(pick_v(n4), [&](auto vc) {
                constexpr int V = decltype(vc)::value;
                if (pair)
                    k_rms_gated_add_mod<V, true><<<exact_grid(nr), kThreads, 0, stream()>>>(
                        x + o, a + o, yy + r0 * n4, nr, (int)C, g1, gate, g2, scale, eps1, eps2);
                else
                    k_rms_gated_add_mod<V, false><<<exact_grid(nr), kThreads, 0, stream()>>>(
                        x + o, a + o, yy + r0 * n4, nr, (int)C, g1, gate, g2, scale, eps1, eps2);
            });
        });
    }
    launched(op);
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_rms_norm_modulate_bf16(const float* x, uint16_t* y, int64_t rows, int64_t C, const float* gamma,
                               const float* scale, float eps) {
    return guarded([&] { run_rms_mod_bf16(x, y, rows, C, gamma, scale, eps); });
}

int sdh_rms_norm_gated_add(float* x, const float* a, int64_t rows, int64_t C, const float* gamma, const float* gate,
                           float eps) {
    return guarded([&] { run_rms_gated_add(x, a, rows, C, gamma, gate, eps); });
}

int sdh_rms_norm_gated_add_modulate_bf16(float* x, const float* a, uint16_t* y, int64_t rows, int64_t C,
                                         const float* gamma_out, const float* gate, const float* gamma_in,
                                         const float* scale, float eps_out, float eps_in) {
    return guarded([&] { run_rms_gated_add_mod(x, a, y, rows, C, gamma_out, gate, gamma_in, scale, eps_out, eps_in); });
}

int sdh_rms_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, float eps) {
    return guarded([&] { run_rownorm("sdh_rms_norm", M_RMS, x, y, rows, C, gamma, nullptr, eps); });
}

int sdh_layer_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, const float* beta,
                   float eps) {
    return guarded([&] { run_rownorm("sdh_layer_norm", M_LN, x, y, rows, C, gamma, beta, eps); });
}

int sdh_add_rms_norm(float* x, const float* r, float* y, int64_t rows, int64_t C, const float* gamma, float eps) {
    return guarded([&] {
        const char* op = "sdh_add_rms_norm";
        need(rows >= 0 && C >= 0, op, "negative size");
        if (rows == 0 || C == 0) return;
        ensure_init();
        const size_t bytes = (size_t)(rows * C) * 4;
        check_range(x, bytes, op, "x");
        check_range(r, bytes, op, "r");
        check_range(y, bytes, op, "y");
        if (gamma) check_range(gamma, (size_t)C * 4, op, "gamma");
        if (vec_ok(C, {x, r, y, gamma})) {
            in_pieces(rows, rows_per_launch(), [&](int64_t r0, int64_t nr) {
                const unsigned grid = exact_grid(nr);
                const int64_t o = r0 * C;
                with_v(pick_v(C / 4), [&](auto vc) {
                    constexpr int V = decltype(vc)::value;
                    if (gamma)
                        k_add_rms<V, true><<<grid, kThreads, 0, stream()>>>(x + o, r + o, y + o, nr, (int)C, gamma, eps);
                    else
                        k_add_rms<V, false><<<grid, kThreads, 0, stream()>>>(x + o, r + o, y + o, nr, (int)C, gamma, eps);
                });
            });
        } else {
            k_add_rms_generic<<<row_grid(rows, 32), kThreads, 0, stream()>>>(x, r, y, rows, C, gamma, eps);
        }
        launched(op);
    });
}

int sdh_ln_modulate_gate(const float* x, float* res, const float* scale, const float* shift, const float* gate,
                         float* y_out, int64_t rows, int64_t C, float eps) {
    return guarded([&] {
        const char* op = "sdh_ln_modulate_gate";
        need(rows >= 0 && C >= 0, op, "negative size");
        if (rows == 0 || C == 0) return;
        ensure_init();
        const size_t bytes = (size_t)(rows * C) * 4;
        check_range(x, bytes, op, "x");
        check_range(res, bytes, op, "res");
        check_range(scale, (size_t)C * 4, op, "scale");
        check_range(gate, (size_t)C * 4, op, "gate");
        if (shift) check_range(shift, (size_t)C * 4, op, "shift");
        if (y_out) check_range(y_out, bytes, op, "y_out");
        const size_t lds = (size_t)3 * C * 4;
        const int64_t n4 = C / 4;
        const int v = n4 <= 128 ? 1 : n4 <= 256 ? 2 : n4 <= 512 ? 4 : n4 <= 1024 ? 8 : n4 <= 1536 ? 12 : n4 <= 2048 ? 16 : 0;
        if (vec_ok(C, {x, res, scale, shift, gate, y_out}) && lds <= 64 * 1024 && v) {
            // two waves (128 work-items) per row
            in_pieces(rows, units_per_launch(128), [&](int64_t r0, int64_t nr) {
                const unsigned grid = blocks_for(nr, kModRows);
                const int64_t o = r0 * C;
                const float* xp = x + o;
                float* rp = res + o;
                float* yp = y_out ? y_out + o : nullptr;
                auto go = [&](auto vc) {
                    constexpr int V = decltype(vc)::value;
                    if (shift && y_out)
                        k_ln_mod_gate<V, true, true><<<grid, kModThreads, lds, stream()>>>(xp, rp, scale, shift, gate, yp, nr, (int)C, eps);
                    else if (shift)
                        k_ln_mod_gate<V, true, false><<<grid, kModThreads, lds, stream()>>>(xp, rp, scale, shift, gate, yp, nr, (int)C, eps);
                    else if (y_out)
                        k_ln_mod_gate<V, false, true><<<grid, kModThreads, lds, stream()>>>(xp, rp, scale, shift, gate, yp, nr, (int)C, eps);
                    else
                        k_ln_mod_gate<V, false, false><<<grid, kModThreads, lds, stream()>>>(xp, rp, scale, shift, gate, yp, nr, (int)C, eps);
                };
                switch (v) {
                    case 1: go(std::integral_constant<int, 1>()); break;
                    case 2: go(std::integral_constant<int, 2>()); break;
                    case 4: go(std::integral_constant<int, 4>()); break;
                    case 8: go(std::integral_constant<int, 8>()); break;
                    case 12: go(std::integral_constant<int, 12>()); break;
                    default: go(std::integral_constant<int, 16>()); break;
                }
            });
        } else {
            k_ln_mod_gate_generic<<<row_grid(rows, 32), kThreads, 0, stream()>>>(x, res, scale, shift, gate, y_out,
                                                                                rows, C, eps);
        }
        launched(op);
    });
}

int sdh_rms_norm_heads(float* x, int64_t groups, int64_t dim, const float* gamma, float eps) {
    return guarded([&] {
        const char* op = "sdh_rms_norm_heads";
        need(groups >= 0 && dim >= 0, op, "negative size");
        if (groups == 0 || dim == 0) return;
        ensure_init();
        check_range(x, (size_t)(groups * dim) * 4, op, "x");
        if (gamma) check_range(gamma, (size_t)dim * 4, op, "gamma");
        const int64_t L = dim / 4;
        const bool vec = dim % 4 == 0 && (L == 4 || L == 8 || L == 16 || L == 32 || L == 64) && aligned16(x) &&
                         (!gamma || aligned16(gamma));
        if (vec) {
            // L work-items per group; pieces of 2^31 / L groups are whole waves
            in_pieces(groups, units_per_launch(L), [&](int64_t g0, int64_t ng) {
                const unsigned grid = exact_grid((ng + (64 / L) - 1) / (64 / L));
                float* xp = x + g0 * dim;
                auto go = [&](auto lc) {
                    constexpr int LL = decltype(lc)::value;
                    if (gamma)
                        k_heads<LL, true><<<grid, kThreads, 0, stream()>>>(xp, ng, (int)dim, gamma, eps);
                    else
                        k_heads<LL, false><<<grid, kThreads, 0, stream()>>>(xp, ng, (int)dim, gamma, eps);
                };
                switch (L) {
                    case 4: go(std::integral_constant<int, 4>()); break;
                    case 8: go(std::integral_constant<int, 8>()); break;
                    case 16: go(std::integral_constant<int, 16>()); break;
                    case 32: go(std::integral_constant<int, 32>()); break;
                    default: go(std::integral_constant<int, 64>()); break;
                }
            });
        } else {
            k_rownorm_generic<M_RMS><<<row_grid(groups, 32), kThreads, 0, stream()>>>(x, x, groups, dim, gamma,
                                                                                     nullptr, eps);
        }
        launched(op);
    });
}

}  // extern "C"

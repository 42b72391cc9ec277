// k_elementwise.hip - streaming elementwise ops: swiglu, silu, tanh, gelu,
// quick_gelu, add, scale, affine, geglu, the device zero fill and the seeded
// normal generator.
//
// Roofline: HBM-bound (well under 1 flop per byte). Each thread moves one
// 128-bit vector per operand and the grid covers the tensor exactly (no
// persistent loop): on MI355X many small workgroups with non-temporal loads
// and stores stream best. Measured (swiglu [4096,10240], 503 MB; a plain
// copy of 336 MB): one-wave workgroups 75.2-75.6 us (83.2-83.6 % of 8 TB/s),
// copy 83.7-83.9 %; 128 threads alike for swiglu, 81.7 % for the copy; 256
// threads 78.9 us (79.7 %), copy 81.8 %; two or four vectors per thread
// 76-79 %; ordinary (allocating) loads or stores 72-76 %. Arithmetic
// follows the reference's expression order (tensor.cpp:745, :847, :852,
// :859, :866, :876, :881, :886, :830) with ROCm's device libm (expf, tanhf,
// erff).
#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 64;  // one wave per workgroup (see above)
constexpr int kUnroll = 1;
constexpr int64_t kPerBlock = (int64_t)kThreads * kUnroll;  // float4 per block

enum UnaryKind { U_SILU, U_TANH, U_GELU, U_QGELU, U_SCALE, U_AFFINE };

template <int K>
__device__ __forceinline__ float unary(float v, float a, float b) {
    if constexpr (K == U_SILU) return dev::silu(v);
    if constexpr (K == U_TANH) return tanhf(v);
    if constexpr (K == U_GELU) return dev::gelu_erf(v);
    if constexpr (K == U_QGELU) return dev::quick_gelu(v);
    if constexpr (K == U_SCALE) return v * a;
    if constexpr (K == U_AFFINE) return v * a + b;
    return v;
}

template <int K>
__device__ __forceinline__ f4 unary4(f4 v, float a, float b) {
    return f4{unary<K>(v.x, a, b), unary<K>(v.y, a, b), unary<K>(v.z, a, b), unary<K>(v.w, a, b)};
}

// In-place unary map over n4 float4 plus a scalar tail of `tail` floats.
template <int K>
__global__ __launch_bounds__(kThreads) void k_unary(f4* __restrict__ x, int64_t n4, float* __restrict__ tail_ptr,
                                                   int tail, float a, float b) {
    const int64_t base = (int64_t)blockIdx.x * kPerBlock + threadIdx.x;
    f4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t i = base + (int64_t)u * kThreads;
        if (i < n4) v[u] = dev::ld_stream(x + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t i = base + (int64_t)u * kThreads;
        if (i < n4) dev::st_stream(x + i, unary4<K>(v[u], a, b));
    }
    if (blockIdx.x == 0 && (int)threadIdx.x < tail) tail_ptr[threadIdx.x] = unary<K>(tail_ptr[threadIdx.x], a, b);
}

// The adaLN modulation rows of a block, in place: rows 2p (scales) become
// 1 + x, rows 2p + 1 (gates) tanh(x), with the expressions of affine_ and
// tanh_ (one launch for the four ops of zimage.cpp:104-107).
__global__ __launch_bounds__(kThreads) void k_modulation_rows(float* __restrict__ x, int64_t n, int64_t dim) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
        const float v = x[i];
        x[i] = ((i / dim) & 1) ? unary<U_TANH>(v, 0.f, 0.f) : unary<U_AFFINE>(v, 1.0f, 1.0f);
    }
}

template <int K>
__global__ __launch_bounds__(kThreads) void k_unary_scalar(float* __restrict__ x, int64_t n, float a, float b) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        x[i] = unary<K>(x[i], a, b);
}

// y = g / (1 + exp(-g)) * u  (tensor.cpp:745)
__device__ __forceinline__ float swiglu1(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__global__ __launch_bounds__(kThreads) void k_swiglu(const f4* __restrict__ g, const f4* __restrict__ u,
                                                    f4* __restrict__ y, int64_t n4, const float* __restrict__ gt,
                                                    const float* __restrict__ ut, float* __restrict__ yt, int tail) {
    const int64_t base = (int64_t)blockIdx.x * kPerBlock + threadIdx.x;
    f4 gv[kUnroll], uv[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t i = base + (int64_t)k * kThreads;
        if (i < n4) {
            gv[k] = dev::ld_stream(g + i);
            uv[k] = dev::ld_stream(u + i);
        }
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t i = base + (int64_t)k * kThreads;
        if (i < n4) {
            const f4 a = gv[k], b = uv[k];
            dev::st_stream(y + i, f4{swiglu1(a.x, b.x), swiglu1(a.y, b.y), swiglu1(a.z, b.z), swiglu1(a.w, b.w)});
        }
    }
    if (blockIdx.x == 0 && (int)threadIdx.x < tail) yt[threadIdx.x] = swiglu1(gt[threadIdx.x], ut[threadIdx.x]);
}

__global__ __launch_bounds__(kThreads) void k_swiglu_scalar(const float* __restrict__ g, const float* __restrict__ u,
                                                           float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        y[i] = swiglu1(g[i], u[i]);
}

// y16 = bf16(swiglu(g, u)): swiglu, then the rounding gemm_nt_bf16 applies to
// its A (the input of the FFN's w2, zimage.cpp:130), bit for bit.
__global__ __launch_bounds__(kThreads) void k_swiglu_bf16(const f4* __restrict__ g, const f4* __restrict__ u,
                                                         uint2* __restrict__ y, int64_t n4,
                                                         const float* __restrict__ gt, const float* __restrict__ ut,
                                                         unsigned short* __restrict__ yt, int tail) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n4) {
        const f4 a = dev::ld_stream(g + i), b = dev::ld_stream(u + i);
        y[i] = dev::bf16x4(f4{swiglu1(a.x, b.x), swiglu1(a.y, b.y), swiglu1(a.z, b.z), swiglu1(a.w, b.w)});
    }
    if (blockIdx.x == 0 && (int)threadIdx.x < tail) yt[threadIdx.x] = dev::bf16_rne(swiglu1(gt[threadIdx.x], ut[threadIdx.x]));
}

__global__ __launch_bounds__(kThreads) void k_swiglu_bf16_scalar(const float* __restrict__ g,
                                                                const float* __restrict__ u,
                                                                unsigned short* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        y[i] = dev::bf16_rne(swiglu1(g[i], u[i]));
}

// a += b  (tensor.cpp:876)
__global__ __launch_bounds__(kThreads) void k_add(f4* __restrict__ a, const f4* __restrict__ b, int64_t n4,
                                                 float* __restrict__ at, const float* __restrict__ bt, int tail) {
    const int64_t base = (int64_t)blockIdx.x * kPerBlock + threadIdx.x;
    f4 av[kUnroll], bv[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t i = base + (int64_t)k * kThreads;
        if (i < n4) {
            av[k] = dev::ld_stream(a + i);
            bv[k] = dev::ld_stream(b + i);
        }
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t i = base + (int64_t)k * kThreads;
        if (i < n4) dev::st_stream(a + i, av[k] + bv[k]);
    }
    if (blockIdx.x == 0 && (int)threadIdx.x < tail) at[threadIdx.x] += bt[threadIdx.x];
}

__global__ __launch_bounds__(kThreads) void k_add_scalar(float* __restrict__ a, const float* __restrict__ b,
                                                        int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        a[i] += b[i];
}

// y[r, i] = a * 0.5 * g * (1 + erf(g / sqrt 2)), a = x[r, i], g = x[r, D + i]
// (tensor.cpp:828-831). One thread per output element; rows of any D.
__global__ __launch_bounds__(kThreads) void k_geglu(const float* __restrict__ x, float* __restrict__ y, int64_t rows,
                                                   int64_t D) {
    const int64_t n = rows * D;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * kThreads) {
        const int64_t r = idx / D, i = idx - r * D;
        const float a = x[r * 2 * D + i];
        const float gg = x[r * 2 * D + D + i];
        y[idx] = a * 0.5f * gg * (1.0f + erff(gg * 0.70710678118654752f));
    }
}

// Vectorised GEGLU for D % 4 == 0: one float4 of the output per thread.
__global__ __launch_bounds__(kThreads) void k_geglu_vec(const f4* __restrict__ x, f4* __restrict__ y, int64_t n4,
                                                       int64_t D4) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n4) return;
    const int64_t r = i / D4, c = i - r * D4;
    const f4 a = dev::ld_stream(x + r * 2 * D4 + c);
    const f4 g = dev::ld_stream(x + r * 2 * D4 + D4 + c);
    auto one = [](float av, float gg) { return av * 0.5f * gg * (1.0f + erff(gg * 0.70710678118654752f)); };
    dev::st_stream(y + i, f4{one(a.x, g.x), one(a.y, g.y), one(a.z, g.z), one(a.w, g.w)});
}

// Zero fill (used instead of hipMemsetAsync so the library queues no memset
// nodes into a stream a caller might capture into a graph).
__global__ __launch_bounds__(kThreads) void k_zero(f4* __restrict__ p, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += (int64_t)gridDim.x * kThreads)
        p[i] = f4{0.f, 0.f, 0.f, 0.f};
}
__global__ __launch_bounds__(kThreads) void k_zero_bytes(unsigned char* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        p[i] = 0;
}

// Seeded N(mean, std): counter-based splitmix64 -> Box-Muller in double.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(kThreads) void k_fill_normal(float* __restrict__ out, int64_t n, uint64_t seed,
                                                         double mean, double stdv) {
    const uint64_t golden = 0x9E3779B97F4A7C15ULL;
    const uint64_t key = mix64(seed + golden);
    const int64_t pairs = (n + 1) / 2;
    for (int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x; j < pairs; j += (int64_t)gridDim.x * kThreads) {
        const uint64_t h1 = mix64(key + (uint64_t)(2 * j + 1) * golden);
        const uint64_t h2 = mix64(key + (uint64_t)(2 * j + 2) * golden);
        const double u1 = (double)((h1 >> 11) + 1) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        const double th = 6.283185307179586476925286766559 * u2;
        out[2 * j] = (float)(mean + stdv * (r * cos(th)));
        if (2 * j + 1 < n) out[2 * j + 1] = (float)(mean + stdv * (r * sin(th)));
    }
}

// The float4 kernels above map one work-item to one float4 (kUnroll = 1):
// calls launch(first, count, last) over [0, n4) in pieces a dispatch can
// cover; the scalar tail goes with the last piece (n4 = 0: one empty piece
// that only does the tail).
template <class F>
void vec_pieces(int64_t n4, F&& launch) {
    static_assert(kUnroll == 1, "pieces are sized for one float4 per work-item");
    const int64_t units = std::max<int64_t>(n4, 1);
    in_pieces(units, launch_items(), [&](int64_t f, int64_t c) { launch(f, std::min(c, n4 - f), f + c == units); });
}

// Grid for grid-stride scalar kernels: enough blocks to fill the chip.
unsigned stride_grid(int64_t n) {
    const int64_t want = (n + kThreads - 1) / kThreads;
    const int64_t cap = (int64_t)num_cus() * 128;  // 8192 work-items per CU
    return (unsigned)std::max<int64_t>(1, std::min(want, cap));
}

template <int K>
void run_unary(const char* op, float* x, int64_t n, float a, float b) {
    need(n >= 0, op, "negative element count");
    if (n == 0) return;
    ensure_init();
    check_range(x, (size_t)n * 4, op, "x");
    if (aligned16(x)) {
        const int64_t n4 = n / 4;
        const int tail = (int)(n - n4 * 4);
        vec_pieces(n4, [&](int64_t f, int64_t c, bool last) {
            k_unary<K><<<blocks_for(std::max<int64_t>(c, 1), kPerBlock), kThreads, 0, stream()>>>(
                (f4*)x + f, c, x + n4 * 4, last ? tail : 0, a, b);
        });
    } else {
        k_unary_scalar<K><<<stride_grid(n), kThreads, 0, stream()>>>(x, n, a, b);
    }
    launched(op);
}

}  // namespace

void launch_swiglu(const float* gate, const float* up, float* y, int64_t n) {
    if (aligned16(gate) && aligned16(up) && aligned16(y)) {
        const int64_t n4 = n / 4;
        const int tail = (int)(n - n4 * 4);
        vec_pieces(n4, [&](int64_t f, int64_t c, bool last) {
            k_swiglu<<<blocks_for(std::max<int64_t>(c, 1), kPerBlock), kThreads, 0, stream()>>>(
                (const f4*)gate + f, (const f4*)up + f, (f4*)y + f, c, gate + n4 * 4, up + n4 * 4, y + n4 * 4,
                last ? tail : 0);
        });
    } else {
        k_swiglu_scalar<<<stride_grid(n), kThreads, 0, stream()>>>(gate, up, y, n);
    }
}

void zero_device(void* p, size_t bytes) {
    if (bytes == 0) return;
    const int64_t n4 = aligned16(p) ? (int64_t)(bytes / 16) : 0;
    const int64_t rest = (int64_t)bytes - n4 * 16;
    if (n4) k_zero<<<stride_grid(n4), kThreads, 0, stream()>>>((f4*)p, n4);
    if (rest) k_zero_bytes<<<stride_grid(rest), kThreads, 0, stream()>>>((unsigned char*)p + n4 * 16, rest);
    launched("zero");
}

}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_swiglu_bf16(const float* gate, const float* up, uint16_t* y, int64_t n) {
    return guarded([&] {
        const char* op = "sdh_swiglu_bf16";
        need(n >= 0, op, "negative element count");
        if (n == 0) return;
        ensure_init();
        check_range(gate, (size_t)n * 4, op, "gate");
        check_range(up, (size_t)n * 4, op, "up");
        check_range(y, (size_t)n * 2, op, "y");
        if (aligned16(gate) && aligned16(up) && ((uintptr_t)y & 7) == 0) {
            const int64_t n4 = n / 4;
            const int tail = (int)(n - n4 * 4);
            vec_pieces(n4, [&](int64_t f, int64_t c, bool last) {
                k_swiglu_bf16<<<blocks_for(std::max<int64_t>(c, 1), kThreads), kThreads, 0, stream()>>>(
                    (const f4*)gate + f, (const f4*)up + f, (uint2*)y + f, c, gate + n4 * 4, up + n4 * 4,
                    (unsigned short*)y + n4 * 4, last ? tail : 0);
            });
        } else {
            k_swiglu_bf16_scalar<<<stride_grid(n), kThreads, 0, stream()>>>(gate, up, (unsigned short*)y, n);
        }
        launched(op);
    });
}

int sdh_swiglu(const float* gate, const float* up, float* y, int64_t n) {
    return guarded([&] {
        const char* op = "sdh_swiglu";
        need(n >= 0, op, "negative element count");
        if (n == 0) return;
        ensure_init();
        check_range(gate, (size_t)n * 4, op, "gate");
        check_range(up, (size_t)n * 4, op, "up");
        check_range(y, (size_t)n * 4, op, "y");
        launch_swiglu(gate, up, y, n);
        launched(op);
    });
}

int sdh_geglu(const float* x, float* y, int64_t rows, int64_t D) {
    return guarded([&] {
        const char* op = "sdh_geglu";
        need(rows >= 0 && D >= 0, op, "negative size");
        if (rows == 0 || D == 0) return;
        ensure_init();
        check_range(x, (size_t)(rows * 2 * D) * 4, op, "x");
        check_range(y, (size_t)(rows * D) * 4, op, "y");
        if (D % 4 == 0 && D / 4 <= kMaxGridItems && aligned16(x) && aligned16(y)) {
            const int64_t D4 = D / 4;
            in_pieces(rows, units_per_launch(D4), [&](int64_t r0, int64_t nr) {
                k_geglu_vec<<<blocks_for(nr * D4, kThreads), kThreads, 0, stream()>>>(
                    (const f4*)x + r0 * 2 * D4, (f4*)y + r0 * D4, nr * D4, D4);
            });
        } else {
            k_geglu<<<stride_grid(rows * D), kThreads, 0, stream()>>>(x, y, rows, D);
        }
        launched(op);
    });
}

int sdh_silu(float* x, int64_t n) { return guarded([&] { run_unary<U_SILU>("sdh_silu", x, n, 0.f, 0.f); }); }
int sdh_tanh(float* x, int64_t n) { return guarded([&] { run_unary<U_TANH>("sdh_tanh", x, n, 0.f, 0.f); }); }
int sdh_gelu(float* x, int64_t n) { return guarded([&] { run_unary<U_GELU>("sdh_gelu", x, n, 0.f, 0.f); }); }
int sdh_quick_gelu(float* x, int64_t n) {
    return guarded([&] { run_unary<U_QGELU>("sdh_quick_gelu", x, n, 0.f, 0.f); });
}
int sdh_scale(float* x, float s, int64_t n) { return guarded([&] { run_unary<U_SCALE>("sdh_scale", x, n, s, 0.f); }); }
int sdh_affine(float* x, float a, float b, int64_t n) {
    return guarded([&] { run_unary<U_AFFINE>("sdh_affine", x, n, a, b); });
}

int sdh_modulation_rows(float* x, int64_t pairs, int64_t dim) {
    return guarded([&] {
        const char* op = "sdh_modulation_rows";
        need(pairs >= 0 && dim >= 0, op, "negative size");
        need(dim == 0 || pairs <= (INT64_MAX / 8) / dim, op, "size overflows");
        const int64_t n = 2 * pairs * dim;
        if (n == 0) return;
        ensure_init();
        check_range(x, (size_t)n * 4, op, "x");
        k_modulation_rows<<<stride_grid(n), kThreads, 0, stream()>>>(x, n, dim);
        launched(op);
    });
}

int sdh_add(float* a, const float* b, int64_t n) {
    return guarded([&] {
        const char* op = "sdh_add";
        need(n >= 0, op, "negative element count");
        if (n == 0) return;
        ensure_init();
        check_range(a, (size_t)n * 4, op, "a");
        check_range(b, (size_t)n * 4, op, "b");
        if (aligned16(a) && aligned16(b)) {
            const int64_t n4 = n / 4;
            const int tail = (int)(n - n4 * 4);
            vec_pieces(n4, [&](int64_t f, int64_t c, bool last) {
                k_add<<<blocks_for(std::max<int64_t>(c, 1), kPerBlock), kThreads, 0, stream()>>>(
                    (f4*)a + f, (const f4*)b + f, c, a + n4 * 4, b + n4 * 4, last ? tail : 0);
            });
        } else {
            k_add_scalar<<<stride_grid(n), kThreads, 0, stream()>>>(a, b, n);
        }
        launched(op);
    });
}

int sdh_zero(void* dst, size_t bytes) {
    return guarded([&] {
        if (bytes == 0) return;
        ensure_init();
        check_range(dst, bytes, "sdh_zero", "dst");
        zero_device(dst, bytes);
    });
}

int sdh_fill_normal(float* x, int64_t n, uint64_t seed, float mean, float stdv) {
    return guarded([&] {
        const char* op = "sdh_fill_normal";
        need(n >= 0, op, "negative element count");
        if (n == 0) return;
        ensure_init();
        check_range(x, (size_t)n * 4, op, "x");
        k_fill_normal<<<stride_grid((n + 1) / 2), kThreads, 0, stream()>>>(x, n, seed, (double)mean, (double)stdv);
        launched(op);
    });
}

}  // extern "C"

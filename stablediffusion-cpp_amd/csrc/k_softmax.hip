// k_softmax.hip - in-place row softmax with pre-scale and optional causal
// mask (tensor.cpp:752-769; the `period` form of backend_cuda.cu:351-367).
//
// One wave owns one row: the row is loaded once into registers (V float4 per
// lane), the max and the exp-sum are wave reductions, and the normalised row
// is stored once, so HBM sees one read and one write per element (the
// reference's GPU kernel makes three reads and two writes). Waves are
// persistent over rows. Per element: t = x * scale; m = max t;
// e = expf(t - m); out = e * (1 / sum e), the reference's order.
#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <int V, bool CAUSAL>
__global__ __launch_bounds__(kThreads) void k_softmax(float* __restrict__ x, int64_t rows, int cols, float scale,
                                                     int64_t period) {
    const int lane = threadIdx.x & 63;
    const int n4 = cols >> 2;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows; row += stride) {
        f4* p = (f4*)(x + row * cols);
        int valid = cols;
        if constexpr (CAUSAL) {
            const int64_t rr = row % period;
            valid = rr + 1 < cols ? (int)(rr + 1) : cols;
        }
        f4 v[V];
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int idx = lane + 64 * j;
            if (idx < n4) {
                v[j] = dev::ld_stream(p + idx) * scale;
                if constexpr (CAUSAL) {
                    const int c0 = idx * 4;
                    if (c0 + 0 >= valid) v[j].x = -INFINITY;
                    if (c0 + 1 >= valid) v[j].y = -INFINITY;
                    if (c0 + 2 >= valid) v[j].z = -INFINITY;
                    if (c0 + 3 >= valid) v[j].w = -INFINITY;
                }
                m = fmaxf(m, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
            } else {
                v[j] = f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            }
        }
        m = dev::wave_max(m);
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            // masked entries are -inf: expf(-inf) = 0, the exact zero the
            // causal tail must hold
            v[j] = f4{expf(v[j].x - m), expf(v[j].y - m), expf(v[j].z - m), expf(v[j].w - m)};
            s += dev::hsum(v[j]);
        }
        const float inv = 1.0f / dev::wave_sum(s);
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int idx = lane + 64 * j;
            if (idx < n4) dev::st_stream(p + idx, v[j] * inv);
        }
    }
}

// Generic: any cols / alignment; three strided passes over the row (the row
// stays in L1/L2 between them).
__global__ __launch_bounds__(kThreads) void k_softmax_generic(float* __restrict__ x, int64_t rows, int64_t cols,
                                                             float scale, int causal, int64_t period) {
    const int lane = threadIdx.x & 63;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows; row += stride) {
        float* p = x + row * cols;
        const int64_t rr = row % period;
        const int64_t valid = causal ? (rr + 1 < cols ? rr + 1 : cols) : cols;
        float m = -INFINITY;
        for (int64_t j = lane; j < valid; j += 64) m = fmaxf(m, p[j] * scale);
        m = dev::wave_max(m);
        float s = 0.f;
        for (int64_t j = lane; j < valid; j += 64) {
            const float e = expf(p[j] * scale - m);
            p[j] = e;
            s += e;
        }
        const float inv = 1.0f / dev::wave_sum(s);
        for (int64_t j = lane; j < valid; j += 64) p[j] *= inv;
        for (int64_t j = valid + lane; j < cols; j += 64) p[j] = 0.0f;
    }
}

int pick_v(int64_t n4) {
    static const int vs[] = {1, 2, 4, 8, 12, 16, 17, 24, 32};
    for (int v : vs)
        if (64 * (int64_t)v >= n4) return v;
    return 0;
}

template <class F>
void with_v(int v, F&& f) {
    switch (v) {
        case 1: f(std::integral_constant<int, 1>()); break;
        case 2: f(std::integral_constant<int, 2>()); break;
        case 4: f(std::integral_constant<int, 4>()); break;
        case 8: f(std::integral_constant<int, 8>()); break;
        case 12: f(std::integral_constant<int, 12>()); break;
        case 16: f(std::integral_constant<int, 16>()); break;
        case 17: f(std::integral_constant<int, 17>()); break;
        case 24: f(std::integral_constant<int, 24>()); break;
        case 32: f(std::integral_constant<int, 32>()); break;
        default: fail(SDH_ERR_INVALID, "internal: unsupported softmax width");
    }
}

unsigned row_grid(int64_t rows, int waves_per_cu) {
    const int64_t want = (rows + kWaves - 1) / kWaves;
    const int64_t cap = (int64_t)num_cus() * waves_per_cu / kWaves;
    return (unsigned)std::max<int64_t>(1, std::min(want, std::max<int64_t>(cap, 1)));
}

void run_softmax(float* x, int64_t rows, int64_t cols, float scale, int causal, int64_t period) {
    const char* op = "sdh_softmax_rows";
    need(rows >= 0 && cols >= 0, op, "negative size");
    need(period > 0, op, "period must be positive");
    if (rows == 0 || cols == 0) return;
    ensure_init();
    check_range(x, (size_t)(rows * cols) * 4, op, "x");
    const int v = (cols % 4 == 0 && aligned16(x)) ? pick_v(cols / 4) : 0;
    if (v) {
        const unsigned grid = row_grid(rows, 16);
        with_v(v, [&](auto vc) {
            constexpr int V = decltype(vc)::value;
            if (causal)
                k_softmax<V, true><<<grid, kThreads, 0, stream()>>>(x, rows, (int)cols, scale, period);
            else
                k_softmax<V, false><<<grid, kThreads, 0, stream()>>>(x, rows, (int)cols, scale, period);
        });
    } else {
        k_softmax_generic<<<row_grid(rows, 32), kThreads, 0, stream()>>>(x, rows, cols, scale, causal, period);
    }
    launched(op);
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_softmax_rows(float* x, int64_t rows, int64_t cols, float scale, int causal) {
    return guarded([&] { run_softmax(x, rows, cols, scale, causal, rows > 0 ? rows : 1); });
}

int sdh_softmax_rows_batched(float* x, int64_t rows, int64_t cols, float scale, int causal, int64_t period) {
    return guarded([&] { run_softmax(x, rows, cols, scale, causal, period); });
}

}  // extern "C"

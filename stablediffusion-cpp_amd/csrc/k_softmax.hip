// k_softmax.hip - in-place row softmax with pre-scale and optional causal
// mask (tensor.cpp:752-769; the `period` form of backend_cuda.cu:351-367).
//
// Each row is loaded once into registers, the max and the exp-sum are
// reductions over the row's threads, and the normalised row is stored once,
// so HBM sees one read and one write per element (the reference's GPU kernel
// makes three reads and two writes). Two layouts, both with a grid that
// covers the rows exactly (no persistent loop):
//   * rows of <= 1024 floats: one wave per row, 4 rows per workgroup, wave
//     reductions only;
//   * longer rows (<= 16384 floats): one workgroup per row, TPB threads with
//     V float4 each, wave reductions combined through LDS. For the 4096-wide
//     attention rows this is 512 threads x 2 float4, measured ~10 points of
//     HBM peak faster on MI355X than a persistent wave-per-row loop.
// Loads and stores are non-temporal. Per element: t = x * scale; m = max t;
// e = expf(t - m); out = e * (1 / sum e), the reference's order.
#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ f4 neg_inf4() { return f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY}; }

// Loads float4 `idx` of a row scaled, with columns >= valid set to -inf.
template <bool CAUSAL>
__device__ __forceinline__ f4 load_scaled(const f4* p, int idx, int n4, int valid, float scale) {
    if (idx >= n4) return neg_inf4();
    f4 v = dev::ld_stream(p + idx) * scale;
    if constexpr (CAUSAL) {
        const int c0 = idx * 4;
        if (c0 + 0 >= valid) v.x = -INFINITY;
        if (c0 + 1 >= valid) v.y = -INFINITY;
        if (c0 + 2 >= valid) v.z = -INFINITY;
        if (c0 + 3 >= valid) v.w = -INFINITY;
    }
    return v;
}

__device__ __forceinline__ float max4(f4 v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }
// masked entries are -inf: expf(-inf) = 0, the exact zero the causal tail must hold
__device__ __forceinline__ f4 exp4(f4 v, float m) { return f4{expf(v.x - m), expf(v.y - m), expf(v.z - m), expf(v.w - m)}; }

__device__ __forceinline__ int valid_cols(int64_t row, int64_t period, int cols, bool causal) {
    if (!causal) return cols;
    const int64_t rr = row % period;
    return rr + 1 < cols ? (int)(rr + 1) : cols;
}

// One wave per row (n4 <= 64 * V).
template <int V, bool CAUSAL>
__global__ __launch_bounds__(kThreads) void k_softmax_wave(float* __restrict__ x, int64_t rows, int cols, float scale,
                                                          int64_t period, int64_t row0) {
    const int lane = threadIdx.x & 63;
    const int n4 = cols >> 2;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    f4* p = (f4*)(x + row * cols);
    const int valid = valid_cols(row0 + row, period, cols, CAUSAL);
    f4 v[V];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        v[j] = load_scaled<CAUSAL>(p, lane + 64 * j, n4, valid, scale);
        m = fmaxf(m, max4(v[j]));
    }
    m = dev::wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        v[j] = exp4(v[j], m);
        s += dev::hsum(v[j]);
    }
    const float inv = 1.0f / dev::wave_sum(s);
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = lane + 64 * j;
        if (idx < n4) dev::st_stream(p + idx, v[j] * inv);
    }
}

// One workgroup of TPB threads per row (n4 <= TPB * V).
template <int TPB, int V, bool CAUSAL>
__global__ __launch_bounds__(TPB) void k_softmax_block(float* __restrict__ x, int cols, float scale, int64_t period, int64_t row0) {
    constexpr int W = TPB / 64;
    __shared__ float sh[2 * W];
    const int w = threadIdx.x >> 6;
    const int n4 = cols >> 2;
    const int64_t row = blockIdx.x;
    f4* p = (f4*)(x + row * cols);
    const int valid = valid_cols(row0 + row, period, cols, CAUSAL);
    f4 v[V];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        v[j] = load_scaled<CAUSAL>(p, threadIdx.x + TPB * j, n4, valid, scale);
        m = fmaxf(m, max4(v[j]));
    }
    m = dev::wave_max(m);
    if ((threadIdx.x & 63) == 0) sh[w] = m;
    __syncthreads();
    m = sh[0];
#pragma unroll
    for (int k = 1; k < W; ++k) m = fmaxf(m, sh[k]);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        v[j] = exp4(v[j], m);
        s += dev::hsum(v[j]);
    }
    s = dev::wave_sum(s);
    if ((threadIdx.x & 63) == 0) sh[W + w] = s;
    __syncthreads();
    s = sh[W];
#pragma unroll
    for (int k = 1; k < W; ++k) s += sh[W + k];
    const float inv = 1.0f / s;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = threadIdx.x + TPB * j;
        if (idx < n4) dev::st_stream(p + idx, v[j] * inv);
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

// The vector kernels' grids cover their rows exactly, so rows beyond what one
// dispatch covers go in several launches; row0 keeps the causal phase.
template <bool CAUSAL>
bool launch_vec(float* x, int64_t rows, int cols, float scale, int64_t period) {
    const int n4 = cols / 4;
    hipStream_t st = stream();
    if (n4 <= 256) {
        in_pieces(rows, units_per_launch(64), [&](int64_t r0, int64_t nr) {
            const unsigned g = blocks_for(nr, kWaves);
            float* xp = x + r0 * cols;
            if (n4 <= 64) k_softmax_wave<1, CAUSAL><<<g, kThreads, 0, st>>>(xp, nr, cols, scale, period, r0);
            else if (n4 <= 128) k_softmax_wave<2, CAUSAL><<<g, kThreads, 0, st>>>(xp, nr, cols, scale, period, r0);
            else if (n4 <= 192) k_softmax_wave<3, CAUSAL><<<g, kThreads, 0, st>>>(xp, nr, cols, scale, period, r0);
            else k_softmax_wave<4, CAUSAL><<<g, kThreads, 0, st>>>(xp, nr, cols, scale, period, r0);
        });
        return true;
    }
    const int tpb = n4 <= 512 ? 256 : n4 <= 1024 ? 512 : 1024;
    if (n4 > 4096) return false;
    in_pieces(rows, units_per_launch(tpb), [&](int64_t r0, int64_t nr) {
        const unsigned g = (unsigned)nr;
        float* xp = x + r0 * cols;
        if (n4 <= 512) k_softmax_block<256, 2, CAUSAL><<<g, 256, 0, st>>>(xp, cols, scale, period, r0);
        else if (n4 <= 1024) k_softmax_block<512, 2, CAUSAL><<<g, 512, 0, st>>>(xp, cols, scale, period, r0);
        else if (n4 <= 2048) k_softmax_block<1024, 2, CAUSAL><<<g, 1024, 0, st>>>(xp, cols, scale, period, r0);
        else k_softmax_block<1024, 4, CAUSAL><<<g, 1024, 0, st>>>(xp, cols, scale, period, r0);
    });
    return true;
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
    bool done = false;
    if (cols % 4 == 0 && aligned16(x) && cols <= 0x7fffffff)
        done = causal ? launch_vec<true>(x, rows, (int)cols, scale, period)
                      : launch_vec<false>(x, rows, (int)cols, scale, period);
    if (!done)
        k_softmax_generic<<<row_grid(rows, 32), kThreads, 0, stream()>>>(x, rows, cols, scale, causal, period);
    launched(op);
}

}  // namespace

void softmax_rows_device(const char* op, float* x, int64_t rows, int64_t cols, float scale, bool causal) {
    (void)op;
    run_softmax(x, rows, cols, scale, causal ? 1 : 0, rows > 0 ? rows : 1);
}

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

// k_broadcast.hip - row-vector and per-channel broadcasts, in place:
//   mul_rows         x[r, :] *= v            (tensor.cpp:889-901)
//   add_rows_scaled  x[r, :] += g * y[r, :]  (tensor.cpp:903-917)
//   add_rows         x[r, :] += v            (linear's bias epilogue,
//                                             backend_cuda.cu:239-241)
//   add_channel_bias x[n, c, :] += b[n, c]   (tensor.cpp:919-929)
// HBM-bound. When the row length is a multiple of 4 and the pointers are
// 16-byte aligned, each thread handles one 128-bit vector, the grid covers
// the tensor exactly, and the broadcast operand (a [dim] vector, resident in
// L2) is indexed with a 32-bit column computed once per vector instead of a
// 64-bit i % dim per element (backend_cuda.cu:394-402).
#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;
// k_rows_vec streams one float4 per thread in one-wave workgroups (many
// small workgroups stream best on MI355X), non-temporal loads and stores.
// Measured at [4096, 3840] over 504 MB of rotated inputs: mul_rows 23.1 ->
// 21.0 us, add_rows_scaled 33.1 -> 29.8 us (from 256-thread workgroups with
// ordinary loads).
constexpr int kVecThreads = 64;

enum BKind { B_MUL, B_ADD_SCALED, B_ADD };

template <int K>
__global__ __launch_bounds__(kVecThreads) void k_rows_vec(f4* __restrict__ x, const f4* __restrict__ y,
                                                         const f4* __restrict__ v, int64_t n4, unsigned dim4) {
    const int64_t i = (int64_t)blockIdx.x * kVecThreads + threadIdx.x;
    if (i >= n4) return;
    const unsigned c = (unsigned)i % dim4;  // n4 <= kMaxGridItems per launch
    const f4 vv = v[c];
    const f4 xv = dev::ld_stream(x + i);
    f4 o;
    if constexpr (K == B_MUL) o = xv * vv;
    if constexpr (K == B_ADD_SCALED) o = xv + vv * dev::ld_stream(y + i);
    if constexpr (K == B_ADD) o = xv + vv;
    dev::st_stream(x + i, o);
}

template <int K>
__global__ __launch_bounds__(kThreads) void k_rows_scalar(float* __restrict__ x, const float* __restrict__ y,
                                                         const float* __restrict__ v, int64_t rows, int64_t dim) {
    const int64_t n = rows * dim;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
        const float vv = v[i % dim];
        if constexpr (K == B_MUL) x[i] *= vv;
        if constexpr (K == B_ADD_SCALED) x[i] += vv * y[i];
        if constexpr (K == B_ADD) x[i] += vv;
    }
}

// x[n, c, :] += b[n, c]: blockIdx.y = n*C + c, blockIdx.x sweeps the plane.
__global__ __launch_bounds__(kThreads) void k_channel_bias_vec(f4* __restrict__ x, const float* __restrict__ b,
                                                              int64_t hw4) {
    const int64_t nc = blockIdx.y;
    const float add = b[nc];
    f4* p = x + nc * hw4;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < hw4; i += (int64_t)gridDim.x * kThreads)
        dev::st_stream(p + i, dev::ld_stream(p + i) + add);
}

__global__ __launch_bounds__(kThreads) void k_channel_bias_scalar(float* __restrict__ x, const float* __restrict__ b,
                                                                 int64_t n, int64_t HW) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        x[i] += b[i / HW];
}

unsigned stride_grid(int64_t n) {
    const int64_t want = (n + kThreads - 1) / kThreads;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)num_cus() * 32));
}

template <int K>
void run_rows(const char* op, float* x, const float* y, const float* v, int64_t rows, int64_t dim) {
    need(rows >= 0 && dim >= 0, op, "negative size");
    if (rows == 0 || dim == 0) return;
    ensure_init();
    check_range(x, (size_t)(rows * dim) * 4, op, "x");
    if (K == B_ADD_SCALED) check_range(y, (size_t)(rows * dim) * 4, op, "y");
    check_range(v, (size_t)dim * 4, op, K == B_ADD_SCALED ? "g" : "v");
    const bool vec = dim % 4 == 0 && dim / 4 <= kMaxGridItems && aligned16(x) && aligned16(v) &&
                     (K != B_ADD_SCALED || aligned16(y));
    if (vec) {
        // whole rows per launch, so the column of element i is i % dim4 in every launch
        const int64_t dim4 = dim / 4;
        in_pieces(rows, units_per_launch(dim4), [&](int64_t r0, int64_t nr) {
            k_rows_vec<K><<<blocks_for(nr * dim4, kVecThreads), kVecThreads, 0, stream()>>>(
                (f4*)x + r0 * dim4, K == B_ADD_SCALED ? (const f4*)y + r0 * dim4 : nullptr, (const f4*)v, nr * dim4,
                (unsigned)dim4);
        });
    } else {
        k_rows_scalar<K><<<stride_grid(rows * dim), kThreads, 0, stream()>>>(x, y, v, rows, dim);
    }
    launched(op);
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_mul_rows(float* x, const float* v, int64_t rows, int64_t dim) {
    return guarded([&] { run_rows<B_MUL>("sdh_mul_rows", x, nullptr, v, rows, dim); });
}

int sdh_add_rows_scaled(float* x, const float* y, const float* g, int64_t rows, int64_t dim) {
    return guarded([&] { run_rows<B_ADD_SCALED>("sdh_add_rows_scaled", x, y, g, rows, dim); });
}

int sdh_add_rows(float* x, const float* v, int64_t rows, int64_t dim) {
    return guarded([&] { run_rows<B_ADD>("sdh_add_rows", x, nullptr, v, rows, dim); });
}

int sdh_add_channel_bias(float* x, const float* b, int64_t N, int64_t C, int64_t HW) {
    return guarded([&] {
        const char* op = "sdh_add_channel_bias";
        need(N >= 0 && C >= 0 && HW >= 0, op, "negative size");
        if (N == 0 || C == 0 || HW == 0) return;
        ensure_init();
        check_range(x, (size_t)(N * C * HW) * 4, op, "x");
        check_range(b, (size_t)(N * C) * 4, op, "b");
        if (HW % 4 == 0 && aligned16(x) && N * C <= 65535) {
            const int64_t hw4 = HW / 4;
            const int64_t want = (hw4 + kThreads - 1) / kThreads;
            const int64_t per_plane = std::max<int64_t>(1, (int64_t)num_cus() * 8 / (N * C));
            const unsigned gx = (unsigned)std::max<int64_t>(1, std::min(want, per_plane));
            k_channel_bias_vec<<<dim3(gx, (unsigned)(N * C)), kThreads, 0, stream()>>>((f4*)x, b, hw4);
        } else {
            k_channel_bias_scalar<<<stride_grid(N * C * HW), kThreads, 0, stream()>>>(x, b, N * C * HW, HW);
        }
        launched(op);
    });
}

}  // extern "C"

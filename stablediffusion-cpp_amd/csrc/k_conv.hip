// k_conv.hip - conv2d (backend_cuda.h:45-47; tensor.cpp:520-560) as gather +
// library GEMM, so that backend_hip covers every function of the reference's
// backend interface and tensor.cpp's device branches run unchanged on it.
//
// Not a tuned path (convolutions are outside this backend's elementwise /
// reduction scope): per sample, pixels are taken in chunks of at most 2^25
// gathered floats; k_gather_patches writes cols[p, (ci, ky, kx)] (the patch
// that output pixel p sees, zero over the padding; (ci, ky, kx) is the
// [Cout, Cin, kh, kw] weight's own order, so the weight is already a
// [Cout, K] matrix); then out[Cout, pixels] = W cols^T through
// sdh_gemm_nt_f32 (hipBLASLt with fp32 operands), written straight into the
// NCHW output (ldc = Ho * Wo); the bias is added per output channel after
// the last chunk (sdh_add_channel_bias).
#include <algorithm>

#include "sdh_backend.h"
#include "sdh_internal.hpp"

namespace sdh {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kChunkFloats = int64_t(1) << 25;  // gathered floats per chunk (128 MB)

// cols[p, k] for p in [0, P), k in [0, K): K fastest, so the stores of a wave
// are contiguous; 32-bit index math (P * K <= 2^25).
__global__ __launch_bounds__(kThreads) void k_gather_patches(const float* __restrict__ x, float* __restrict__ cols,
                                                            int H, int W, int kh, int kw, int Wo, int stride, int pad,
                                                            int p0, int P, int K) {
    const unsigned i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= (unsigned)P * (unsigned)K) return;
    const unsigned p = i / (unsigned)K, k = i - p * (unsigned)K;
    const unsigned khw = (unsigned)(kh * kw);
    const unsigned ci = k / khw, r = k - ci * khw;
    const int ky = (int)(r / (unsigned)kw), kx = (int)(r - (unsigned)ky * (unsigned)kw);
    const int op = p0 + (int)p, oy = op / Wo, ox = op - oy * Wo;
    const int iy = oy * stride - pad + ky, ix = ox * stride - pad + kx;
    cols[i] = (iy >= 0 && iy < H && ix >= 0 && ix < W) ? x[((int64_t)ci * H + iy) * W + ix] : 0.0f;
}

void check_status(int st) {
    if (st != SDH_OK) fail(st, sdh_last_error());
}

void run_conv2d(const float* x, int64_t N, int64_t Cin, int64_t H, int64_t W, const float* w, int64_t Cout,
                int64_t kh, int64_t kw, const float* bias, int stride, int pad, float* out, int64_t Ho, int64_t Wo) {
    const char* op = "sdh_conv2d";
    need(N >= 0 && Cin > 0 && H >= 0 && W >= 0 && Cout >= 0 && kh > 0 && kw > 0, op, "bad size");
    need(stride > 0 && pad >= 0, op, "stride must be positive and pad non-negative");
    need(Ho == (H + 2 * pad - kh) / stride + 1 && Wo == (W + 2 * pad - kw) / stride + 1 && Ho > 0 && Wo > 0, op,
         "output size does not match (H + 2 pad - kh) / stride + 1");  // tensor.cpp:533
    if (N == 0 || Cout == 0) return;
    ensure_init();
    const int64_t K = Cin * kh * kw, HW = Ho * Wo;
    need(K <= kChunkFloats && H * W < (int64_t(1) << 31) && HW < (int64_t(1) << 31), op, "convolution too large");
    check_range(x, (size_t)(N * Cin * H * W) * 4, op, "x");
    check_range(w, (size_t)(Cout * K) * 4, op, "w");
    check_range(out, (size_t)(N * Cout * HW) * 4, op, "out");
    if (bias) check_range(bias, (size_t)Cout * 4, op, "bias");
    const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(HW, kChunkFloats / K));
    float* cols = (float*)scratch((size_t)(chunk * K) * 4);
    for (int64_t n = 0; n < N; ++n) {
        const float* xn = x + n * Cin * H * W;
        float* on = out + n * Cout * HW;
        for (int64_t p0 = 0; p0 < HW; p0 += chunk) {
            const int64_t P = std::min(chunk, HW - p0);
            k_gather_patches<<<blocks_for(P * K, kThreads), kThreads, 0, stream()>>>(
                xn, cols, (int)H, (int)W, (int)kh, (int)kw, (int)Wo, stride, pad, (int)p0, (int)P, (int)K);
            launched(op);
            // out[co, p0 + p] = sum_k w[co, k] cols[p, k]  (ldc = HW)
            check_status(sdh_gemm_nt_f32(Cout, P, K, w, K, cols, K, on + p0, HW, nullptr, 0));
        }
        if (bias) check_status(sdh_add_channel_bias(on, bias, 1, Cout, HW));
    }
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_conv2d(const float* x, int64_t N, int64_t Cin, int64_t H, int64_t W, const float* w, int64_t Cout, int64_t kh,
               int64_t kw, const float* bias, int stride, int pad, float* out, int64_t Ho, int64_t Wo) {
    return guarded([&] { run_conv2d(x, N, Cin, H, W, w, Cout, kh, kw, bias, stride, pad, out, Ho, Wo); });
}

}  // extern "C"

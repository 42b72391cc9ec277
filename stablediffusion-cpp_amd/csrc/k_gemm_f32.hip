// k_gemm_f32.hip - the linear layer with fp32 weights: C[M,N] = A[M,K] * B[N,K]^T
// (+ C) (+ bias[N]) in fp32 (backend_cuda.h:38-40, gemm_nt_f32; the reference's
// device path is an fp32 SGEMM, backend_cuda.cu:453-464, its CPU path fp32
// micro-kernels, tensor.cpp:354-406). Z-Image keeps every weight under 2^20
// elements in fp32 (safetensors.cpp:110-116 with keep_bf16, pipeline.cpp:113):
// the patch and caption embedders' small relatives, the timestep MLP, the
// final layer's modulation and projection. Those layers are small (at most
// about 1 GFLOP at 1024x1024), so this is a plain register-blocked fp32 FMA
// kernel on the vector ALUs, exact in fp32 like both reference paths:
// 64 x 64 output tile per 256-thread workgroup, 4 x 4 per thread, K in steps
// of 16 through LDS (A and B tiles stored k-major, so a thread's four rows or
// columns are one float4 read).
//
// Also sdh_to_bf16: float32 -> bf16 bits on the device with the reference's
// rounding (nearest even; inf and NaN keep their top bits; tensor.cpp:114-121).
#include <algorithm>

#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;
constexpr int kT = 64, kKS = 16, kThreads = 256;

// VEC: K % 4 == 0, lda % 4 == 0, ldb % 4 == 0 and 16-B aligned A and B.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_gemm_f32(const float* __restrict__ A, int64_t lda,
                                                       const float* __restrict__ B, int64_t ldb, float* __restrict__ C,
                                                       int64_t ldc, const float* __restrict__ bias, int64_t M,
                                                       int64_t N, int64_t K, int accumulate) {
    __shared__ float sA[kKS][kT + 4];
    __shared__ float sB[kKS][kT + 4];
    const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
    const int64_t m0 = (int64_t)blockIdx.y * kT, n0 = (int64_t)blockIdx.x * kT;
    // loader mapping: thread t loads row (t >> 2) of the tile, k quad (t & 3)
    const int lr = t >> 2, lk = (t & 3) * 4;
    const int64_t am = m0 + lr, bn = n0 + lr;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int64_t k0 = 0; k0 < K; k0 += kKS) {
        f4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
        if constexpr (VEC) {
            if (am < M && k0 + lk < K) a = *(const f4*)(A + am * lda + k0 + lk);
            if (bn < N && k0 + lk < K) b = *(const f4*)(B + bn * ldb + k0 + lk);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t k = k0 + lk + e;
                if (am < M && k < K) a[e] = A[am * lda + k];
                if (bn < N && k < K) b[e] = B[bn * ldb + k];
            }
        }
        __syncthreads();  // every thread is done with the previous tiles
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sA[lk + e][lr] = a[e];
            sB[lk + e][lr] = b[e];
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kKS; ++kk) {
            const f4 av = *(const f4*)&sA[kk][ty * 4];
            const f4 bv = *(const f4*)&sB[kk][tx * 4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tx * 4 + j;
            if (n >= N) continue;
            float* cp = C + m * ldc + n;
            float v = acc[i][j];
            if (bias) v += bias[n];
            if (accumulate) v += *cp;
            *cp = v;
        }
    }
}

// Nearest-even float -> bf16 bits; inf and NaN keep their top 16 bits.
__device__ __forceinline__ unsigned short to_bf16_bits(float f) {
    const unsigned b = __float_as_uint(f);
    if ((b & 0x7F800000u) == 0x7F800000u) return (unsigned short)(b >> 16);
    return (unsigned short)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

__global__ __launch_bounds__(256) void k_to_bf16(const float* __restrict__ x, unsigned short* __restrict__ y,
                                                 int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) y[i] = to_bf16_bits(x[i]);
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

void run_gemm_f32(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                  int64_t ldc, const float* bias, bool accumulate) {
    const char* op = "sdh_gemm_nt_f32";
    need(M >= 0 && N >= 0 && K >= 0, op, "negative size");
    need(lda >= K && ldb >= K && ldc >= N, op, "leading dimension smaller than the row");
    if (M == 0 || N == 0) return;
    ensure_init();
    if (K > 0) {
        check_range(A, (size_t)((M - 1) * lda + K) * 4, op, "A");
        check_range(B, (size_t)((N - 1) * ldb + K) * 4, op, "B");
    }
    check_range(C, (size_t)((M - 1) * ldc + N) * 4, op, "C");
    if (bias) check_range(bias, (size_t)N * 4, op, "bias");
    // the library GEMM for aligned operands (fp32 products, fp32 accumulation)
    if (K > 0 && lda % 4 == 0 && ldb % 4 == 0 && ldc % 4 == 0 && aligned(A, 16) && aligned(B, 16) && aligned(C, 16) &&
        (!bias || aligned(bias, 16)) && blaslt_gemm(true, M, N, K, A, lda, B, ldb, C, ldc, bias, accumulate)) {
        launched(op);
        return;
    }
    const int64_t gx = (N + kT - 1) / kT, gy = (M + kT - 1) / kT;
    need(gy <= 65535 && gx * kThreads <= kMaxGridItems, op, "matrix too large for one launch");
    const bool vec = K % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0 && aligned(A, 16) && aligned(B, 16);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    if (vec)
        k_gemm_f32<true><<<grid, kThreads, 0, stream()>>>(A, lda, B, ldb, C, ldc, bias, M, N, K, accumulate ? 1 : 0);
    else
        k_gemm_f32<false><<<grid, kThreads, 0, stream()>>>(A, lda, B, ldb, C, ldc, bias, M, N, K, accumulate ? 1 : 0);
    launched(op);
}

}  // namespace

void to_bf16_device(const char* op, const float* x, uint16_t* y, int64_t n) {
    (void)op;
    if (n <= 0) return;
    const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, (int64_t)num_cus() * 32);
    k_to_bf16<<<grid, 256, 0, stream()>>>(x, y, n);
}

}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_gemm_nt_f32(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B, int64_t ldb,
                    float* C, int64_t ldc, const float* bias, int accumulate) {
    return guarded([&] { run_gemm_f32(M, N, K, A, lda, B, ldb, C, ldc, bias, accumulate != 0); });
}

int sdh_to_bf16(const float* x, uint16_t* y, int64_t n) {
    return guarded([&] {
        const char* op = "sdh_to_bf16";
        need(n >= 0, op, "negative size");
        if (n == 0) return;
        ensure_init();
        check_range(x, (size_t)n * 4, op, "x");
        check_range(y, (size_t)n * 2, op, "y");
        const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, (int64_t)num_cus() * 32);
        k_to_bf16<<<grid, 256, 0, stream()>>>(x, y, n);
        launched(op);
    });
}

}  // extern "C"

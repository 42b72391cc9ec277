// k_gemm.hip - the linear layer's GEMM on the MFMA units, with fused
// epilogues: C[M,N] = A[M,K] * B[N,K]^T (+ C) (+ bias[N]) with fp32 A and bf16
// weights B (backend_cuda.h:38-43, gemm_nt_bf16), and the Z-Image FFN front
// half y = swiglu(A W1^T, A W3^T) (zimage.cpp:130) in one GEMM.
//
// Dispatch: A is rounded to bf16 by k_pack_bf16; the product then runs on
// hipBLASLt (bf16 x bf16 -> fp32 with the bias epilogue, the library GEMM,
// measured 1.35-1.83 PFLOP/s at the Z-Image shapes against 0.88 for the
// kernels below) whenever the operands are 16-B aligned with aligned leading
// dimensions; for SwiGLU as two GEMMs into scratch and the elementwise
// kernel. The hand-written MFMA kernels below cover the other shapes.
//
// Numerics are the reference GPU path's (backend_cuda.cu:236-238, :466-479):
// A is rounded to bf16 (nearest even; inf/NaN truncated) once per call into
// library scratch, products of bf16 pairs are exact in fp32, and they are
// accumulated in fp32 by the MFMA units. Only the accumulation order differs
// from cuBLAS.
//
// Main kernel (K % 64 == 0): 256 x 128 output tile per 512-thread workgroup
// (eight waves of 64 x 64, each 2 x 2 tiles of v_mfma_f32_32x32x16_bf16:
// lane l holds A row l%32 and B row l%32, k (l/32)*8..+7; result column l%32,
// rows (i/4)*8 + (l/32)*4 + i%4), K in steps of 64.
//   * Operands go from global memory straight into LDS
//     (global_load_lds_dwordx4: lane i of a wave's load lands at base + 16 i),
//     two stages; the next stage's loads are in flight while the current one
//     multiplies, one barrier per step.
//   * LDS rows are 128 B (64 bf16) with no padding; 16-B chunk c of row r
//     sits at position c ^ ((r >> 1) & 7). gfx950's LDS serves 16 lanes of a
//     128-bit read from one 256-byte window (two rows), and the fragment
//     reads of 16 consecutive rows then hit 16 distinct chunks: no bank
//     conflicts (SQ_LDS_BANK_CONFLICT = 0; the (r & 7) form measured 50 % of
//     LDS cycles in conflicts). The global side picks for each lane the chunk
//     that belongs at its LDS slot.
//   * Fragments are double-buffered in registers across the four 16-k slices
//     and the compiler's MFMA/LDS interleaving (iglp_opt 0) is requested.
// Measured on MI355X at [4096 x 3840] x [3840 x 3840]^T: 35 % of the dense
// bf16 peak, against 26 % for register staging with padded LDS rows (the
// kernel kept for K % 64 != 0) and 84 % for MFMAs fed from registers only.
// For the SwiGLU epilogue the B tile holds 64 rows of W1 and the same 64 rows
// of W3, and each wave's two column sub-tiles are a W1 and a W3 sub-tile of
// the same output columns, so g and u of an output element sit in one lane.
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "sdh_internal.hpp"

namespace sdh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // 8 bf16
typedef unsigned short u16;
using dev::f4;

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kRow = kBK + 8;  // LDS row length in bf16 (144 B)
constexpr int kGT = 256;

enum Epi { E_LINEAR = 0, E_SWIGLU = 1 };

// Nearest-even float -> bf16 bits; inf and NaN keep their top 16 bits.
__device__ __forceinline__ unsigned bf16_bits(float f) {
    const unsigned b = __float_as_uint(f);
    if ((b & 0x7F800000u) == 0x7F800000u) return b >> 16;
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// A fp32 [M, lda] -> P bf16 [M, K] (dense rows). One thread per 8 elements;
// grid.y walks rows (K % 8 == 0, lda % 4 == 0, A 16-byte aligned).
// Rows r0 .. r0 + rows of A rounded to bf16 into the dense P: one thread per
// 8 columns (two float4 in, one 16-B vector out), flat over the rows in
// one-wave workgroups (many small workgroups stream best on MI355X);
// rows * (K / 8) < 2^31 per launch.
constexpr int kPackThreads = 64;
__global__ __launch_bounds__(kPackThreads) void k_pack_bf16(const float* __restrict__ A, int64_t lda,
                                                           u32x4* __restrict__ P, unsigned n8, unsigned kg) {
    const unsigned i = blockIdx.x * kPackThreads + threadIdx.x;
    if (i >= n8) return;
    const unsigned m = i / kg, g = i - m * kg;
    const f4* p = (const f4*)(A + (int64_t)m * lda) + 2 * g;
    const f4 a = dev::ld_stream(p), b = dev::ld_stream(p + 1);
    u32x4 o;
    o.x = bf16_bits(a.x) | (bf16_bits(a.y) << 16);
    o.y = bf16_bits(a.z) | (bf16_bits(a.w) << 16);
    o.z = bf16_bits(b.x) | (bf16_bits(b.y) << 16);
    o.w = bf16_bits(b.z) | (bf16_bits(b.w) << 16);
    P[i] = o;  // re-read by the GEMM right after: ordinary store
}

// P bf16 [M, K] dense; B0 (and B1 for SwiGLU) bf16 [N, ldb]. EPI E_LINEAR:
// the block covers output columns n0 .. n0+127 of B0. E_SWIGLU: n0 .. n0+63,
// B tile rows 0..63 from B0 (W1), 64..127 from B1 (W3).
template <int EPI>
__global__ __launch_bounds__(kGT, 2) void k_gemm_bf16(const u16* __restrict__ P, const u16* __restrict__ B0,
                                                     const u16* __restrict__ B1, int64_t ldb, float* __restrict__ C,
                                                     int64_t ldc, const float* __restrict__ bias, int M, int N, int K,
                                                     int accumulate) {
    __shared__ __attribute__((aligned(16))) u16 sA[2][kBM * kRow];
    __shared__ __attribute__((aligned(16))) u16 sB[2][kBN * kRow];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wm = w >> 1, wn = w & 1;
    const int m0 = blockIdx.y * kBM;
    const int n0 = blockIdx.x * (EPI == E_SWIGLU ? kBN / 2 : kBN);
    const int c8 = (t & 7) * 8, r0 = t >> 3;  // global/LDS staging: 16 B chunk c8 of rows r0 + 32 j
    const u32x4 zero = {0u, 0u, 0u, 0u};
    u32x4 ra[4], rb[4];

    auto gload = [&](int k0) {
        const int kk = k0 + c8;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = r0 + 32 * j;
            const int am = m0 + r;
            ra[j] = (am < M && kk < K) ? *(const u32x4*)(P + (int64_t)am * K + kk) : zero;
            const u16* bp = B0;
            int bn = n0 + r;
            if constexpr (EPI == E_SWIGLU) {
                bp = r < 64 ? B0 : B1;
                bn = n0 + (r & 63);
            }
            rb[j] = (bn < N && kk < K) ? *(const u32x4*)(bp + (int64_t)bn * ldb + kk) : zero;
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            *(u32x4*)(&sA[buf][(r0 + 32 * j) * kRow + c8]) = ra[j];
            *(u32x4*)(&sB[buf][(r0 + 32 * j) * kRow + c8]) = rb[j];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.f;

    // B rows of this wave's two column sub-tiles
    const int nb0 = EPI == E_SWIGLU ? wn * 32 : wn * 64;
    const int nb1 = EPI == E_SWIGLU ? 64 + wn * 32 : wn * 64 + 32;
    const int fr = lane & 31, fk = (lane >> 5) * 8;

    const int nk = (K + kBK - 1) / kBK;
    gload(0);
    swrite(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const int col = ks * 16 + fk;
            bf16x8 af[2], bfr[2];
#pragma unroll
            for (int ms = 0; ms < 2; ++ms) af[ms] = *(const bf16x8*)(&sA[buf][(wm * 64 + ms * 32 + fr) * kRow + col]);
            bfr[0] = *(const bf16x8*)(&sB[buf][(nb0 + fr) * kRow + col]);
            bfr[1] = *(const bf16x8*)(&sB[buf][(nb1 + fr) * kRow + col]);
#pragma unroll
            for (int ms = 0; ms < 2; ++ms)
#pragma unroll
                for (int ns = 0; ns < 2; ++ns)
                    acc[ms][ns] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ms], bfr[ns], acc[ms][ns], 0, 0, 0);
        }
        if (kt + 1 < nk) swrite(buf ^ 1);
        __syncthreads();
    }

    // epilogue
#pragma unroll
    for (int ms = 0; ms < 2; ++ms) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = m0 + wm * 64 + ms * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            if (m >= M) continue;
            if constexpr (EPI == E_SWIGLU) {
                const int n = n0 + wn * 32 + fr;
                if (n < N) {
                    const float g = acc[ms][0][i], u = acc[ms][1][i];
                    C[(int64_t)m * ldc + n] = g / (1.0f + expf(-g)) * u;  // tensor.cpp:745 order
                }
            } else {
#pragma unroll
                for (int ns = 0; ns < 2; ++ns) {
                    const int n = n0 + wn * 64 + ns * 32 + fr;
                    if (n < N) {
                        float v = acc[ms][ns][i];
                        float* cp = C + (int64_t)m * ldc + n;
                        if (accumulate) v = *cp + v;
                        if (bias) v += bias[n];
                        *cp = v;
                    }
                }
            }
        }
    }
}


// K % 64 == 0: direct-to-LDS loads, swizzled rows, 2 stages (see above).
constexpr int kDM = 256, kDN = 128, kDWaves = 8, kDT = 64 * kDWaves;
constexpr int kDIA = kDM / 8 / kDWaves, kDIB = kDN / 8 / kDWaves;  // load instructions per wave per stage

template <int EPI>
__global__ __launch_bounds__(kDT, 1) void k_gemm_dl(const u16* __restrict__ P, const u16* __restrict__ B0,
                                                   const u16* __restrict__ B1, int64_t ldb, float* __restrict__ C,
                                                   int64_t ldc, const float* __restrict__ bias, int M, int N, int K,
                                                   int accumulate) {
    __shared__ __attribute__((aligned(1024))) u16 sA0[kDM * 64];
    __shared__ __attribute__((aligned(1024))) u16 sA1[kDM * 64];
    __shared__ __attribute__((aligned(1024))) u16 sB0[kDN * 64];
    __shared__ __attribute__((aligned(1024))) u16 sB1[kDN * 64];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wm = w >> 1, wn = w & 1;  // 4 x 2 waves of 64 x 64
    const int m0 = blockIdx.y * kDM;
    const int n0 = blockIdx.x * (EPI == E_SWIGLU ? kDN / 2 : kDN);
    const int lrow = lane >> 3;
    // global sources of this lane in each of the wave's load instructions;
    // rows past the matrix read its last row (their results are not stored)
    const u16* ga[kDIA];
    const u16* gb[kDIB];
#pragma unroll
    for (int j = 0; j < kDIA; ++j) {
        const int r = (w * kDIA + j) * 8 + lrow;
        ga[j] = P + (int64_t)min(m0 + r, M - 1) * K + ((lane & 7) ^ ((r >> 1) & 7)) * 8;
    }
#pragma unroll
    for (int j = 0; j < kDIB; ++j) {
        const int r = (w * kDIB + j) * 8 + lrow;
        const u16* bp = B0;
        int bn = n0 + r;
        if constexpr (EPI == E_SWIGLU) {
            bp = r < kDN / 2 ? B0 : B1;
            bn = n0 + (r & (kDN / 2 - 1));
        }
        gb[j] = bp + (int64_t)min(bn, N - 1) * ldb + ((lane & 7) ^ ((r >> 1) & 7)) * 8;
    }
    auto issue = [&](int k0, u16* dA, u16* dB) {
#pragma unroll
        for (int j = 0; j < kDIA; ++j)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(ga[j] + k0),
                                             (__attribute__((address_space(3))) void*)(dA + (w * kDIA + j) * 512), 16, 0,
                                             0);
#pragma unroll
        for (int j = 0; j < kDIB; ++j)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(gb[j] + k0),
                                             (__attribute__((address_space(3))) void*)(dB + (w * kDIB + j) * 512), 16, 0,
                                             0);
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.f;
    // B rows of this wave's two column sub-tiles
    const int nb0 = EPI == E_SWIGLU ? wn * 32 : wn * 64;
    const int nb1 = EPI == E_SWIGLU ? kDN / 2 + wn * 32 : wn * 64 + 32;
    const int fr = lane & 31, fh = lane >> 5;
    auto frag = [&](const u16* tA, const u16* tB, int ks, bf16x8* af, bf16x8* bfr) {
        const int c = ks * 2 + fh;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            const int r = wm * 64 + a * 32 + fr;
            af[a] = *(const bf16x8*)(tA + r * 64 + ((c ^ ((r >> 1) & 7)) << 3));
        }
        const int r0 = nb0 + fr, r1 = nb1 + fr;
        bfr[0] = *(const bf16x8*)(tB + r0 * 64 + ((c ^ ((r0 >> 1) & 7)) << 3));
        bfr[1] = *(const bf16x8*)(tB + r1 * 64 + ((c ^ ((r1 >> 1) & 7)) << 3));
    };
    auto mma = [&](const bf16x8* af, const bf16x8* bfr) {
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfr[b], acc[a][b], 0, 0, 0);
    };
    auto compute = [&](const u16* tA, const u16* tB) {
        bf16x8 af0[2], bf0[2], af1[2], bf1[2];
        frag(tA, tB, 0, af0, bf0);
        frag(tA, tB, 1, af1, bf1);
        mma(af0, bf0);
        frag(tA, tB, 2, af0, bf0);
        mma(af1, bf1);
        frag(tA, tB, 3, af1, bf1);
        mma(af0, bf0);
        mma(af1, bf1);
        __builtin_amdgcn_iglp_opt(0);
    };
    const int nk = K / 64;
    issue(0, sA0, sB0);
    for (int kt = 0; kt < nk; kt += 2) {
        // stage kt has landed in buffer 0 and every wave is done with buffer 1
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + 1 < nk) issue((kt + 1) * 64, sA1, sB1);
        compute(sA0, sB0);
        if (kt + 1 >= nk) break;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + 2 < nk) issue((kt + 2) * 64, sA0, sB0);
        compute(sA1, sB1);
    }

#pragma unroll
    for (int ms = 0; ms < 2; ++ms) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = m0 + wm * 64 + ms * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            if (m >= M) continue;
            if constexpr (EPI == E_SWIGLU) {
                const int n = n0 + wn * 32 + fr;
                if (n < N) {
                    const float g = acc[ms][0][i], u = acc[ms][1][i];
                    C[(int64_t)m * ldc + n] = g / (1.0f + expf(-g)) * u;  // tensor.cpp:745 order
                }
            } else {
#pragma unroll
                for (int ns = 0; ns < 2; ++ns) {
                    const int n = n0 + wn * 64 + ns * 32 + fr;
                    if (n < N) {
                        float v = acc[ms][ns][i];
                        float* cp = C + (int64_t)m * ldc + n;
                        if (accumulate) v = *cp + v;
                        if (bias) v += bias[n];
                        *cp = v;
                    }
                }
            }
        }
    }
}

// Any alignment and K: one thread per output element, bf16-rounded A times
// bf16 B accumulated in fp32 in k order.
template <int EPI>
__global__ __launch_bounds__(kGT) void k_gemm_scalar(const float* __restrict__ A, int64_t lda,
                                                    const u16* __restrict__ B0, const u16* __restrict__ B1,
                                                    int64_t ldb, float* __restrict__ C, int64_t ldc,
                                                    const float* __restrict__ bias, int64_t M, int64_t N, int64_t K,
                                                    int accumulate) {
    for (int64_t idx = (int64_t)blockIdx.x * kGT + threadIdx.x; idx < M * N; idx += (int64_t)gridDim.x * kGT) {
        const int64_t m = idx / N, n = idx - m * N;
        const float* a = A + m * lda;
        const u16* b0 = B0 + n * ldb;
        float s0 = 0.f, s1 = 0.f;
        for (int64_t k = 0; k < K; ++k) {
            const float av = __uint_as_float(bf16_bits(a[k]) << 16);
            s0 += av * __uint_as_float((unsigned)b0[k] << 16);
            if constexpr (EPI == E_SWIGLU) s1 += av * __uint_as_float((unsigned)B1[n * ldb + k] << 16);
        }
        float* cp = C + m * ldc + n;
        if constexpr (EPI == E_SWIGLU) {
            *cp = s0 / (1.0f + expf(-s0)) * s1;
        } else {
            float v = s0;
            if (accumulate) v = *cp + v;
            if (bias) v += bias[n];
            *cp = v;
        }
    }
}

bool aligned(const void* p, unsigned a) { return ((uintptr_t)p & (a - 1)) == 0; }

// ---------------------------------------------------------------------------
// The plain GEMM on hipBLASLt: D[M,N] = P[M,K] (bf16, packed, ld K) x B[N,K]^T
// (bf16, ld ldb) (+ bias[N]) (+ D), fp32 accumulation and output. In
// hipBLASLt's column-major terms D^T (N x M, ld ldc) = op_T(B as K x N, ld ldb)
// x (P as K x M, ld K). One plan (descriptors + the heuristic's first
// algorithm) per shape, created on first use and kept for the process.
// ---------------------------------------------------------------------------
constexpr size_t kBlasWorkspace = (size_t)64 << 20;

struct BlasPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};
struct Blas {
    std::mutex mu;
    hipblasLtHandle_t h = nullptr;
    bool tried = false;
    std::map<std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int, int>, BlasPlan> plans;
};
Blas& blas() {
    static Blas b;
    return b;
}

void blas_check(hipblasStatus_t st, const char* what) {
    if (st != HIPBLAS_STATUS_SUCCESS) fail(SDH_ERR_HIP, std::string(what) + ": hipBLASLt status " + std::to_string((int)st));
}

}  // namespace

// C[M,N] = P[M,K] B[N,K]^T (+ bias) (+ C) on hipBLASLt with fp32 accumulation,
// P and B bf16 (f32 = false) or fp32 (f32 = true; fp32 products). Returns
// false when hipBLASLt has no algorithm for the shape (the caller then runs
// its own kernels); throws on a failed launch.
bool blaslt_gemm(bool f32, int64_t M, int64_t N, int64_t K, const void* P, int64_t ldp, const void* B, int64_t ldb,
                 float* C, int64_t ldc, const float* bias, bool accumulate) {
    Blas& b = blas();
    std::lock_guard<std::mutex> lk(b.mu);
    if (!b.h) {
        if (b.tried) return false;
        b.tried = true;
        if (hipblasLtCreate(&b.h) != HIPBLAS_STATUS_SUCCESS) {
            b.h = nullptr;
            return false;
        }
    }
    const auto key = std::make_tuple(M, N, K, ldp, ldb, ldc, bias ? 1 : 0, f32 ? 1 : 0);
    const hipDataType ab = f32 ? HIP_R_32F : HIP_R_16BF;
    auto it = b.plans.find(key);
    if (it == b.plans.end()) {
        BlasPlan p;
        blas_check(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "hipblasLtMatmulDescCreate");
        const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
        blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta), "transA");
        blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb), "transB");
        const hipblasLtEpilogue_t epi = bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT;
        blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof epi), "epilogue");
        if (bias) {
            const hipDataType bt = HIP_R_32F;
            blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof bt),
                       "bias type");
        }
        blas_check(hipblasLtMatrixLayoutCreate(&p.la, ab, (uint64_t)K, (uint64_t)N, ldb), "layout B");
        blas_check(hipblasLtMatrixLayoutCreate(&p.lb, ab, (uint64_t)K, (uint64_t)M, ldp), "layout A");
        blas_check(hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, (uint64_t)N, (uint64_t)M, ldc), "layout C");
        hipblasLtMatmulPreference_t pref;
        blas_check(hipblasLtMatmulPreferenceCreate(&pref), "preference");
        const size_t wsb = kBlasWorkspace;
        blas_check(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof wsb),
                   "workspace size");
        hipblasLtMatmulHeuristicResult_t res[1];
        int n = 0;
        if (hipblasLtMatmulAlgoGetHeuristic(b.h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, res, &n) ==
                HIPBLAS_STATUS_SUCCESS &&
            n > 0) {
            p.algo = res[0].algo;
            p.ok = true;
        }
        hipblasLtMatmulPreferenceDestroy(pref);
        it = b.plans.emplace(key, p).first;
    }
    BlasPlan& p = it->second;
    if (!p.ok) return false;
    if (bias)
        blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof bias),
                   "bias pointer");
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    void* ws = workspace(kBlasWorkspace);
    blas_check(hipblasLtMatmul(b.h, p.desc, &alpha, B, p.la, P, p.lb, &beta, C, p.lc, C, p.lc, &p.algo, ws,
                               kBlasWorkspace, stream()),
               "hipblasLtMatmul");
    return true;
}

namespace {

template <int EPI>
void run_gemm(const char* op, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const u16* B0,
              const u16* B1, int64_t ldb, float* C, int64_t ldc, const float* bias, bool accumulate) {
    need(M >= 0 && N >= 0 && K >= 0, op, "negative size");
    need(lda >= K && ldb >= K && ldc >= N, op, "leading dimension smaller than the row");
    if (M == 0 || N == 0) return;
    ensure_init();
    if (K > 0) {
        check_range(A, (size_t)((M - 1) * lda + K) * 4, op, "A");
        check_range(B0, (size_t)((N - 1) * ldb + K) * 2, op, EPI == E_SWIGLU ? "w1" : "B");
        if (EPI == E_SWIGLU) check_range(B1, (size_t)((N - 1) * ldb + K) * 2, op, "w3");
    }
    check_range(C, (size_t)((M - 1) * ldc + N) * 4, op, EPI == E_SWIGLU ? "y" : "C");
    if (bias) check_range(bias, (size_t)N * 4, op, "bias");
    const bool fast = K > 0 && K % 8 == 0 && lda % 4 == 0 && ldb % 8 == 0 && aligned(A, 16) && aligned(B0, 16) &&
                      (EPI != E_SWIGLU || aligned(B1, 16)) && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31);
    if (fast) {
        // hipBLASLt takes the plain GEMM when the operands are 16-B aligned with
        // aligned leading dimensions; SwiGLU then runs as two GEMMs into scratch
        // and the elementwise kernel (faster than the fused kernel below, which
        // stays for the shapes hipBLASLt has no algorithm for)
        const bool lt = ldb % 8 == 0 && ldc % 4 == 0 && aligned(C, 16) && (!bias || aligned(bias, 16));
        const bool swi_lt = EPI == E_SWIGLU && lt && ldc == N;
        const size_t pbytes = ((size_t)(M * K) * 2 + 255) / 256 * 256, gbytes = (size_t)(M * N) * 4;
        char* base = (char*)scratch(pbytes + (swi_lt ? 2 * gbytes : 0));
        u16* P = (u16*)base;
        const int64_t kg = K / 8;
        in_pieces(M, std::max<int64_t>(1, ((int64_t)1 << 31) / kg - 1), [&](int64_t m0, int64_t nm) {
            const unsigned n8 = (unsigned)(nm * kg);
            k_pack_bf16<<<blocks_for(n8, kPackThreads), kPackThreads, 0, stream()>>>(
                A + m0 * lda, lda, (u32x4*)P + m0 * kg, n8, (unsigned)kg);
        });
        launched(op);
        if constexpr (EPI == E_LINEAR) {
            if (lt && blaslt_gemm(false, M, N, K, P, K, B0, ldb, C, ldc, bias, accumulate)) {
                launched(op);
                return;
            }
        } else {
            float* G = (float*)(base + pbytes);
            float* U = G + M * N;
            if (swi_lt && blaslt_gemm(false, M, N, K, P, K, B0, ldb, G, N, nullptr, false)) {
                blaslt_gemm(false, M, N, K, P, K, B1, ldb, U, N, nullptr, false);
                launch_swiglu(G, U, C, M * N);  // tensor.cpp:745 order, as the fused epilogue
                launched(op);
                return;
            }
        }
        if (K % 64 == 0) {
            const int bn = EPI == E_SWIGLU ? kDN / 2 : kDN;
            const int64_t gx = (N + bn - 1) / bn, gym = (M + kDM - 1) / kDM;
            need(gym <= 65535 && gx * kDT <= kMaxGridItems, op, "matrix too large for one launch");
            k_gemm_dl<EPI><<<dim3((unsigned)gx, (unsigned)gym), kDT, 0, stream()>>>(
                P, B0, B1, ldb, C, ldc, bias, (int)M, (int)N, (int)K, accumulate ? 1 : 0);
        } else {
            const int bn = EPI == E_SWIGLU ? kBN / 2 : kBN;
            const int64_t gx = (N + bn - 1) / bn, gym = (M + kBM - 1) / kBM;
            need(gym <= 65535 && gx * kGT <= kMaxGridItems, op, "matrix too large for one launch");
            k_gemm_bf16<EPI><<<dim3((unsigned)gx, (unsigned)gym), kGT, 0, stream()>>>(
                P, B0, B1, ldb, C, ldc, bias, (int)M, (int)N, (int)K, accumulate ? 1 : 0);
        }
    } else {
        const int64_t want = (M * N + kGT - 1) / kGT;
        const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)num_cus() * 16));
        k_gemm_scalar<EPI><<<grid, kGT, 0, stream()>>>(A, lda, B0, B1, ldb, C, ldc, bias, M, N, K, accumulate ? 1 : 0);
    }
    launched(op);
}

// C[M,N] = A[M,K] x B[N,K]^T (+ bias) (+ C) with A already bf16 (ld lda).
void run_gemm_packed(int64_t M, int64_t N, int64_t K, const u16* A, int64_t lda, const u16* B, int64_t ldb, float* C,
                     int64_t ldc, const float* bias, bool accumulate) {
    const char* op = "sdh_gemm_nt_bf16_packed";
    need(M >= 0 && N >= 0 && K >= 0, op, "negative size");
    need(lda >= K && ldb >= K && ldc >= N, op, "leading dimension smaller than the row");
    if (M == 0 || N == 0) return;
    ensure_init();
    if (K > 0) {
        check_range(A, (size_t)((M - 1) * lda + K) * 2, op, "A");
        check_range(B, (size_t)((N - 1) * ldb + K) * 2, op, "B");
    }
    check_range(C, (size_t)((M - 1) * ldc + N) * 4, op, "C");
    if (bias) check_range(bias, (size_t)N * 4, op, "bias");
    const bool lt = K > 0 && lda % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0 && aligned(A, 16) && aligned(B, 16) &&
                    aligned(C, 16) && (!bias || aligned(bias, 16));
    if (lt && blaslt_gemm(false, M, N, K, A, lda, B, ldb, C, ldc, bias, accumulate)) {
        launched(op);
        return;
    }
    // the MFMA kernels read A with ld K: rows of a wider A are copied together first
    need(K > 0 && K % 8 == 0 && ldb % 8 == 0 && aligned(B, 16) && M < (1LL << 31) && N < (1LL << 31), op,
         "unsupported shape or alignment (K and ldb multiples of 8, 16-byte aligned operands)");
    const u16* P = A;
    if (lda != K || !aligned(A, 16)) {
        u16* Q = (u16*)scratch((size_t)(M * K) * 2);
        hip_check(hipMemcpy2DAsync(Q, (size_t)K * 2, A, (size_t)lda * 2, (size_t)K * 2, (size_t)M,
                                   hipMemcpyDeviceToDevice, stream()),
                  "hipMemcpy2DAsync");
        P = Q;
    }
    if (K % 64 == 0) {
        const int64_t gx = (N + kDN - 1) / kDN, gym = (M + kDM - 1) / kDM;
        need(gym <= 65535 && gx * kDT <= kMaxGridItems, op, "matrix too large for one launch");
        k_gemm_dl<E_LINEAR><<<dim3((unsigned)gx, (unsigned)gym), kDT, 0, stream()>>>(
            P, B, nullptr, ldb, C, ldc, bias, (int)M, (int)N, (int)K, accumulate ? 1 : 0);
    } else {
        const int64_t gx = (N + kBN - 1) / kBN, gym = (M + kBM - 1) / kBM;
        need(gym <= 65535 && gx * kGT <= kMaxGridItems, op, "matrix too large for one launch");
        k_gemm_bf16<E_LINEAR><<<dim3((unsigned)gx, (unsigned)gym), kGT, 0, stream()>>>(
            P, B, nullptr, ldb, C, ldc, bias, (int)M, (int)N, (int)K, accumulate ? 1 : 0);
    }
    launched(op);
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_gemm_nt_bf16_packed(int64_t M, int64_t N, int64_t K, const uint16_t* A, int64_t lda, const uint16_t* B,
                            int64_t ldb, float* C, int64_t ldc, const float* bias, int accumulate) {
    return guarded([&] { run_gemm_packed(M, N, K, A, lda, B, ldb, C, ldc, bias, accumulate != 0); });
}

int sdh_gemm_nt_bf16(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const uint16_t* B, int64_t ldb,
                     float* C, int64_t ldc, const float* bias, int accumulate) {
    return guarded([&] {
        run_gemm<E_LINEAR>("sdh_gemm_nt_bf16", M, N, K, A, lda, B, nullptr, ldb, C, ldc, bias, accumulate != 0);
    });
}

int sdh_linear_swiglu(const float* x, const uint16_t* w1, const uint16_t* w3, float* y, int64_t rows, int64_t in,
                      int64_t hidden) {
    return guarded([&] {
        need(w1 != nullptr && w3 != nullptr, "sdh_linear_swiglu", "w1 and w3 are required");
        run_gemm<E_SWIGLU>("sdh_linear_swiglu", rows, hidden, in, x, in, w1, w3, in, y, hidden, nullptr, false);
    });
}

}  // extern "C"

// k_layout.hip - the tensor library's layout ops (tensor.cpp:931-1099): nearest
// 2x upsampling, channel concatenation, NCHW <-> NLC, and the Z-Image
// patchify / unpatchify. Pure data movement: every output element is a copy
// of one input element, so results are bit-exact by construction, and every
// kernel is bound by HBM at (bytes read + bytes written) per element.
//
//   upsample_nearest2x  [NC, H, W] -> [NC, 2H, 2W]. One thread per input
//       float2 (2 consecutive columns): it writes the 4 output floats of its
//       columns into both output rows as two 128-bit stores. The flattened
//       input row (nc * H + i) maps to output rows 2 (nc * H + i) and +1, so
//       no division splits n, c and i.
//   concat_channels     y[n] = a[n] ++ b[n] (Ca * HW, then Cb * HW floats).
//       grid.y = n; each thread copies one float4, from a or b by one compare.
//   nchw_to_nlc / nlc_to_nchw  a batched 2-D transpose [B, R, K] -> [B, K, R]
//       (R = C, K = HW for NCHW -> NLC; R = HW, K = C back). 64 x 64 tiles
//       staged in LDS with a padded row (65 floats), so the column reads of
//       the store phase fall in distinct banks; both global sides move
//       128-bit vectors along their contiguous axis.
//   patchify / unpatchify  [C, H, W] <-> [(H/p)(W/p), p*p*C], features in
//       (ph, pw, c) order (tensor.cpp:931-966). One thread per output element
//       (coalesced stores, gathered loads that hit L2): the Z-Image latent is
//       1 MB, so these launches are latency-bound, not bandwidth-bound.
//
// Unaligned pointers, or sizes the vector kernels cannot tile (odd widths
// for upsample, channel planes or rows that are not whole float4), take
// scalar kernels with the reference's index arithmetic
// (backend_cuda.cu:405-446).
#include <algorithm>

#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;
// The streaming kernels (upsample, concat) run one wave per workgroup: on
// MI355X many one-wave workgroups stream faster than 256-thread ones
// (measured: upsample [1,512,256,256] 108-110 against 111-113 us, concat
// [2,960,64,64] 11.4 against 11.9 us).
constexpr int kStreamThreads = 64;

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + nb && y < x + na;
}

unsigned stride_grid(int64_t n) {
    const int64_t want = (n + kThreads - 1) / kThreads;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)num_cus() * 32));
}

// ---- upsample ------------------------------------------------------------------
// One thread per input float2 (columns 2q, 2q+1 of input row `row`), which
// becomes output float4 q of output rows 2 row and 2 row + 1. Every store
// instruction thus writes whole lines across the wave; a float4-per-thread
// mapping that stores two interleaved float4 per row measured 2.7x slower on
// MI355X (non-temporal stores that cover half of each line).
typedef float f2 __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(kStreamThreads) void k_upsample2x_vec(const f2* __restrict__ x, f4* __restrict__ y,
                                                                  unsigned n2, unsigned w2) {
    const unsigned g = blockIdx.x * kStreamThreads + threadIdx.x;
    if (g >= n2) return;
    const unsigned row = g / w2, q = g - row * w2;
    const f2 v = __builtin_nontemporal_load(x + g);
    const f4 o = f4{v.x, v.x, v.y, v.y};
    f4* r0 = y + (size_t)row * (2u * w2) + q;  // output rows are w2 float4 wide
    dev::st_stream(r0, o);
    dev::st_stream(r0 + w2, o);
}

__global__ __launch_bounds__(kThreads) void k_upsample2x_scalar(const float* __restrict__ x, float* __restrict__ y,
                                                               int64_t total, int64_t H, int64_t W) {
    const int64_t H2 = 2 * H, W2 = 2 * W;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t nc = idx / (H2 * W2), r = idx - nc * (H2 * W2), i = r / W2, j = r - i * W2;
        y[idx] = x[(nc * H + i / 2) * W + j / 2];
    }
}

// ---- concat ----------------------------------------------------------------------
__global__ __launch_bounds__(kStreamThreads) void k_concat_vec(const f4* __restrict__ a, const f4* __restrict__ b,
                                                              f4* __restrict__ y, unsigned na4, unsigned nb4) {
    const unsigned i = blockIdx.x * kStreamThreads + threadIdx.x;
    const unsigned n = blockIdx.y, nt = na4 + nb4;
    if (i >= nt) return;
    const f4 v = i < na4 ? dev::ld_stream(a + (size_t)n * na4 + i) : dev::ld_stream(b + (size_t)n * nb4 + (i - na4));
    dev::st_stream(y + (size_t)n * nt + i, v);
}

__global__ __launch_bounds__(kThreads) void k_concat_scalar(const float* __restrict__ a, const float* __restrict__ b,
                                                           float* __restrict__ y, int64_t N, int64_t Ca, int64_t Cb,
                                                           int64_t HW) {
    const int64_t C = Ca + Cb, total = N * C * HW;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t n = idx / (C * HW), c = (idx / HW) % C, i = idx % HW;
        y[idx] = c < Ca ? a[(n * Ca + c) * HW + i] : b[(n * Cb + (c - Ca)) * HW + i];
    }
}

// ---- transpose [B, R, K] -> [B, K, R] ----------------------------------------------
constexpr int kTile = 64;
constexpr int kPad = kTile + 1;

__global__ __launch_bounds__(kThreads) void k_transpose_vec(const float* __restrict__ x, float* __restrict__ y,
                                                           int R, int K) {
    __shared__ float tile[kTile * kPad];
    const int k0 = blockIdx.x * kTile, r0 = blockIdx.y * kTile;
    const size_t base = (size_t)blockIdx.z * (size_t)R * (size_t)K;
    const int c4 = threadIdx.x & 15, rr = threadIdx.x >> 4;
    // load: rows r0 + rr + 16 it, columns k0 + 4 c4 .. +3 (K % 4 == 0, so a
    // float4 that starts inside the row ends inside it)
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int r = r0 + rr + 16 * it, k = k0 + 4 * c4;
        if (r < R && k < K) {
            const f4 v = dev::ld_stream((const f4*)(x + base + (size_t)r * K + k));
            float* t = tile + (rr + 16 * it) * kPad + 4 * c4;
            t[0] = v.x;
            t[1] = v.y;
            t[2] = v.z;
            t[3] = v.w;
        }
    }
    __syncthreads();
    // store: output rows k0 + rr + 16 it, columns r0 + 4 c4 .. +3 (R % 4 == 0)
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int k = k0 + rr + 16 * it, r = r0 + 4 * c4;
        if (k < K && r < R) {
            const int kk = rr + 16 * it;
            const f4 v = f4{tile[(4 * c4) * kPad + kk], tile[(4 * c4 + 1) * kPad + kk], tile[(4 * c4 + 2) * kPad + kk],
                            tile[(4 * c4 + 3) * kPad + kk]};
            dev::st_stream((f4*)(y + base + (size_t)k * R + r), v);
        }
    }
}

__global__ __launch_bounds__(kThreads) void k_transpose_scalar(const float* __restrict__ x, float* __restrict__ y,
                                                              int64_t B, int64_t R, int64_t K) {
    const int64_t total = B * R * K;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {  // idx indexes the output [B, K, R]
        const int64_t b = idx / (K * R), k = (idx / R) % K, r = idx % R;
        y[idx] = x[(b * R + r) * K + k];
    }
}

// ---- patchify / unpatchify ------------------------------------------------------------
// I: index type (uint32 when the tensor allows, else int64).
template <class I>
__global__ __launch_bounds__(kThreads) void k_patchify(const float* __restrict__ x, float* __restrict__ y, I C, I H,
                                                      I W, I p, I total) {
    const I Wt = W / p, F = p * p * C;
    for (I idx = (I)blockIdx.x * kThreads + threadIdx.x; idx < total; idx += (I)gridDim.x * kThreads) {
        const I t = idx / F, f = idx - t * F, h = t / Wt, w = t - h * Wt;
        const I c = f % C, pw = (f / C) % p, ph = f / (C * p);
        y[idx] = x[(c * H + h * p + ph) * W + w * p + pw];
    }
}

template <class I>
__global__ __launch_bounds__(kThreads) void k_unpatchify(const float* __restrict__ x, float* __restrict__ y, I C,
                                                        I H, I W, I p, I total) {
    const I Wt = W / p, F = p * p * C;
    for (I idx = (I)blockIdx.x * kThreads + threadIdx.x; idx < total; idx += (I)gridDim.x * kThreads) {
        const I c = idx / (H * W), hw = idx - c * (H * W), hh = hw / W, ww = hw - hh * W;
        const I h = hh / p, ph = hh - h * p, w = ww / p, pw = ww - w * p;
        y[idx] = x[(h * Wt + w) * F + (ph * p + pw) * C + c];
    }
}

// ---- launchers ---------------------------------------------------------------------------
void run_transpose(const char* op, const float* x, float* y, int64_t B, int64_t R, int64_t K) {
    need(B >= 0 && R >= 0 && K >= 0, op, "negative size");
    if (B == 0 || R == 0 || K == 0) return;
    ensure_init();
    const size_t bytes = (size_t)(B * R * K) * 4;
    check_range(x, bytes, op, "x");
    check_range(y, bytes, op, "y");
    need(!overlaps(x, bytes, y, bytes), op, "output overlaps input");
    const bool vec = R % 4 == 0 && K % 4 == 0 && aligned16(x) && aligned16(y) && R < (1LL << 31) &&
                     K < (1LL << 31) && B <= 65535 && (R + kTile - 1) / kTile <= 65535 &&
                     (K + kTile - 1) / kTile * kThreads <= kMaxGridItems;
    if (vec) {
        const dim3 grid((unsigned)((K + kTile - 1) / kTile), (unsigned)((R + kTile - 1) / kTile), (unsigned)B);
        k_transpose_vec<<<grid, kThreads, 0, stream()>>>(x, y, (int)R, (int)K);
    } else {
        k_transpose_scalar<<<stride_grid(B * R * K), kThreads, 0, stream()>>>(x, y, B, R, K);
    }
    launched(op);
}

void run_patch(const char* op, bool forward, const float* x, float* y, int64_t C, int64_t H, int64_t W, int p) {
    need(C >= 0 && H >= 0 && W >= 0, op, "negative size");
    need(p > 0, op, "patch size must be positive");
    need(H % p == 0 && W % p == 0, op, "H and W must be multiples of the patch size");
    if (C == 0 || H == 0 || W == 0) return;
    ensure_init();
    const int64_t total = C * H * W;
    const size_t bytes = (size_t)total * 4;
    check_range(x, bytes, op, "x");
    check_range(y, bytes, op, "y");
    need(!overlaps(x, bytes, y, bytes), op, "output overlaps input");
    const unsigned grid = stride_grid(total);
    if (total < (1LL << 31)) {
        using U = unsigned;
        if (forward)
            k_patchify<U><<<grid, kThreads, 0, stream()>>>(x, y, (U)C, (U)H, (U)W, (U)p, (U)total);
        else
            k_unpatchify<U><<<grid, kThreads, 0, stream()>>>(x, y, (U)C, (U)H, (U)W, (U)p, (U)total);
    } else {
        if (forward)
            k_patchify<int64_t><<<grid, kThreads, 0, stream()>>>(x, y, C, H, W, (int64_t)p, total);
        else
            k_unpatchify<int64_t><<<grid, kThreads, 0, stream()>>>(x, y, C, H, W, (int64_t)p, total);
    }
    launched(op);
}

}  // namespace

void transpose_device(const char* op, const float* x, float* y, int64_t B, int64_t R, int64_t K) {
    run_transpose(op, x, y, B, R, K);
}

}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_upsample_nearest2x(const float* x, float* y, int64_t NC, int64_t H, int64_t W) {
    return guarded([&] {
        const char* op = "sdh_upsample_nearest2x";
        need(NC >= 0 && H >= 0 && W >= 0, op, "negative size");
        if (NC == 0 || H == 0 || W == 0) return;
        ensure_init();
        const size_t in = (size_t)(NC * H * W) * 4;
        check_range(x, in, op, "x");
        check_range(y, 4 * in, op, "y");
        need(!overlaps(x, in, y, 4 * in), op, "output overlaps input");
        const int64_t n2 = NC * H * W / 2;
        if (W % 2 == 0 && ((uintptr_t)x & 7u) == 0 && aligned16(y) && n2 < (1LL << 31)) {
            k_upsample2x_vec<<<blocks_for(n2, kStreamThreads), kStreamThreads, 0, stream()>>>(
                (const f2*)x, (f4*)y, (unsigned)n2, (unsigned)(W / 2));
        } else {
            k_upsample2x_scalar<<<stride_grid(4 * NC * H * W), kThreads, 0, stream()>>>(x, y, 4 * NC * H * W, H, W);
        }
        launched(op);
    });
}

int sdh_concat_channels(const float* a, const float* b, float* y, int64_t N, int64_t Ca, int64_t Cb, int64_t HW) {
    return guarded([&] {
        const char* op = "sdh_concat_channels";
        need(N >= 0 && Ca >= 0 && Cb >= 0 && HW >= 0, op, "negative size");
        if (N == 0 || Ca + Cb == 0 || HW == 0) return;
        ensure_init();
        const size_t na = (size_t)(N * Ca * HW) * 4, nb = (size_t)(N * Cb * HW) * 4, ny = na + nb;
        if (na) check_range(a, na, op, "a");
        if (nb) check_range(b, nb, op, "b");
        check_range(y, ny, op, "y");
        need(!(na && overlaps(a, na, y, ny)) && !(nb && overlaps(b, nb, y, ny)), op, "output overlaps an input");
        const int64_t na4 = Ca * HW / 4, nb4 = Cb * HW / 4;
        const bool vec = (Ca * HW) % 4 == 0 && (Cb * HW) % 4 == 0 && (na == 0 || aligned16(a)) &&
                         (nb == 0 || aligned16(b)) && aligned16(y) && na4 + nb4 <= kMaxGridItems && N <= 65535;
        if (vec) {
            const dim3 grid(blocks_for(na4 + nb4, kStreamThreads), (unsigned)N);
            k_concat_vec<<<grid, kStreamThreads, 0, stream()>>>((const f4*)a, (const f4*)b, (f4*)y, (unsigned)na4,
                                                          (unsigned)nb4);
        } else {
            k_concat_scalar<<<stride_grid(N * (Ca + Cb) * HW), kThreads, 0, stream()>>>(a, b, y, N, Ca, Cb, HW);
        }
        launched(op);
    });
}

int sdh_nchw_to_nlc(const float* x, float* y, int64_t N, int64_t C, int64_t HW) {
    return guarded([&] { run_transpose("sdh_nchw_to_nlc", x, y, N, C, HW); });
}

int sdh_nlc_to_nchw(const float* x, float* y, int64_t N, int64_t C, int64_t HW) {
    return guarded([&] { run_transpose("sdh_nlc_to_nchw", x, y, N, HW, C); });
}

int sdh_patchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p) {
    return guarded([&] { run_patch("sdh_patchify", true, x, y, C, H, W, p); });
}

int sdh_unpatchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p) {
    return guarded([&] { run_patch("sdh_unpatchify", false, x, y, C, H, W, p); });
}

}  // extern "C"

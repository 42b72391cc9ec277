// k_groupnorm.hip - GroupNorm and the fused GroupNorm + SiLU
// (tensor.cpp:592-625 then :843-849).
//
// A "segment" is one (sample, group): cg * HW contiguous floats, channels
// g*cg .. g*cg+cg-1 of sample n. Statistics follow the reference's two-pass
// definition (mean, then the sum of squared deviations M2 around it); the
// apply step uses the reference's folded form y = x * a + (beta - mean * a),
// a = rstd * gamma[c], then SiLU as x / (1 + exp(-x)).
//
// Two schedules:
//   * single: one workgroup (256 or 1024 threads) per segment when the
//     segment fits in its registers (<= 65536 floats). One HBM read, one
//     write. Used by the SD 1.5 shapes.
//   * split: the segment is cut into chunks of kChunk floats.
//       pass A (k_gn_partial): one workgroup per chunk computes the chunk's
//         sum and its M2 around the chunk mean from registers and stores the
//         pair. No atomics: cross-workgroup publication through device-scope
//         release/acquire would write back and invalidate the per-XCD L2s
//         from every workgroup; the kernel boundary publishes instead.
//       finalize (k_gn_finalize): one wave per segment merges the
//         segment's chunk pairs in double in a fixed order (M2 = sum M2_i +
//         n_i (mean_i - mean)^2, the exact pairwise identity) into
//         (mean, rstd). Segments of at most 64 chunks skip this launch: each
//         pass-B wave merges the pairs itself, loading them before its x
//         loads so the merge overlaps them (4a: 16.6 -> 14.7 us).
//       pass B (k_gn_apply): one workgroup per chunk, with the same
//         workgroup -> chunk mapping as pass A, so each chunk is re-read on
//         the XCD whose L2 read it in pass A (tensors up to the 32 MB of
//         total L2 are mostly re-read from cache); it applies the affine (and
//         SiLU).
//     Measured on MI355X the Infinity Cache does not keep streamed reads
//     (re-reading 64-512 MB is no faster than the first read), so for
//     tensors much larger than L2 this schedule moves three streams (x, x,
//     y) against the two of the algorithmic minimum.
#include <algorithm>
#include <cstdlib>

#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;
constexpr int kChunkV = 8;                               // float4 per thread per chunk
constexpr int64_t kChunk = (int64_t)kThreads * 4 * kChunkV;  // floats per chunk (8192)
constexpr int64_t kGnBlockMB = 0;

// SiLU on the hardware exp2 and reciprocal: x * rcp(1 + 2^(-x log2 e)). Its
// error against the correctly rounded x / (1 + expf(-x)) is a few ulp (the
// exp argument's rounding contributes |x| 2^-24 relatively, v_exp_f32 and
// v_rcp_f32 1 ulp each), far inside the 1e-4 relative bound of this op.
__device__ __forceinline__ float silu1(float v) { return dev::silu_fast(v); }

template <bool SILU>
__device__ __forceinline__ f4 apply4(f4 v, float a, float b) {
    f4 o = v * a + b;
    if constexpr (SILU) o = f4{silu1(o.x), silu1(o.y), silu1(o.z), silu1(o.w)};
    return o;
}

// ---- single-workgroup schedule ---------------------------------------------
template <int TPB>
__device__ __forceinline__ float block_sum(float v, float* sh) {
    constexpr int W = TPB / 64;
    v = dev::wave_sum(v);
    __syncthreads();  // sh may still be read by the previous reduction
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = sh[0];
#pragma unroll
    for (int k = 1; k < W; ++k) t += sh[k];
    return t;
}

template <int TPB, int V, bool SILU>
__global__ __launch_bounds__(TPB) void k_gn_single(const float* __restrict__ x, float* __restrict__ y, int C, int HW,
                                                  int groups, const float* __restrict__ gamma,
                                                  const float* __restrict__ beta, float eps) {
    __shared__ float sh[TPB / 64];
    const int64_t seg = blockIdx.x;
    const int n = (int)(seg / groups), g = (int)(seg % groups);
    const int cg = C / groups;
    const int L = cg * HW, n4 = L >> 2;
    const f4* p = (const f4*)(x + ((int64_t)n * C + (int64_t)g * cg) * HW);
    f4* q = (f4*)(y + ((int64_t)n * C + (int64_t)g * cg) * HW);
    f4 v[V];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = threadIdx.x + TPB * j;
        v[j] = idx < n4 ? dev::ld_stream(p + idx) : f4{0.f, 0.f, 0.f, 0.f};
        s += dev::hsum(v[j]);
    }
    const double mean = (double)block_sum<TPB>(s, sh) / (double)L;
    const float meanf = (float)mean;
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = threadIdx.x + TPB * j;
        if (idx < n4) {
            const f4 d = v[j] - meanf;
            m2 += dev::hsum(d * d);
        }
    }
    const double var = (double)block_sum<TPB>(m2, sh);
    const float rstd = (float)(1.0 / sqrt(var / (double)L + (double)eps));
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = threadIdx.x + TPB * j;
        if (idx < n4) {
            const int ch = g * cg + (idx * 4) / HW;
            const float a = rstd * gamma[ch];
            const float b = beta[ch] - meanf * a;
            dev::st_stream(q + idx, apply4<SILU>(v[j], a, b));
        }
    }
}

// ---- split schedule -----------------------------------------------------------
// Pass A. grid = (chunks per segment, segments). Ordinary loads: measured
// faster here than non-temporal ones (4a 17 vs 21 us), although the traffic
// counters show pass B's re-read is not served from L2.
__global__ __launch_bounds__(kThreads) void k_gn_partial(const float* __restrict__ x, int64_t L, int64_t nchunks,
                                                        float2* __restrict__ part) {
    __shared__ float sh[kThreads / 64];
    const int64_t seg = blockIdx.y, chunk = blockIdx.x;
    const int64_t off = chunk * kChunk;
    const int64_t cnt = L - off < kChunk ? L - off : kChunk;
    const f4* p = (const f4*)(x + seg * L + off);
    const int n4 = (int)(cnt >> 2);
    f4 v[kChunkV];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kChunkV; ++j) {
        const int idx = threadIdx.x + kThreads * j;
        v[j] = idx < n4 ? p[idx] : f4{0.f, 0.f, 0.f, 0.f};
        s += dev::hsum(v[j]);
    }
    const float sum = block_sum<kThreads>(s, sh);
    const float mc = sum / (float)cnt;
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < kChunkV; ++j) {
        const int idx = threadIdx.x + kThreads * j;
        if (idx < n4) {
            const f4 d = v[j] - mc;
            m2 += dev::hsum(d * d);
        }
    }
    const float M2 = block_sum<kThreads>(m2, sh);
    if (threadIdx.x == 0) part[seg * nchunks + chunk] = make_float2(sum, M2);
}

__device__ __forceinline__ double wave_dsum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Merge of one segment's chunk pairs in double, in chunk order (fixed
// butterfly): M2 = sum_i M2_i + n_i (mean_i - mean)^2. One wave per segment,
// no LDS and no barrier. grid = segments, 64 threads.
__global__ __launch_bounds__(64) void k_gn_finalize(const float2* __restrict__ part, int64_t L, int64_t nchunks,
                                                   float2* __restrict__ stats, float eps) {
    const int64_t seg = blockIdx.x;
    const float2* pp = part + seg * nchunks;
    double tot = 0.0;
    for (int64_t i = threadIdx.x; i < nchunks; i += 64) tot += (double)pp[i].x;
    const double mean = wave_dsum(tot) / (double)L;
    double m2t = 0.0;
    for (int64_t i = threadIdx.x; i < nchunks; i += 64) {
        const float2 pr = pp[i];
        const double ni = (double)(L - i * kChunk < kChunk ? L - i * kChunk : kChunk);
        const double dm = (double)pr.x / ni - mean;
        m2t += (double)pr.y + ni * dm * dm;
    }
    const double m2 = wave_dsum(m2t);
    if (threadIdx.x == 0) stats[seg] = make_float2((float)mean, (float)(1.0 / sqrt(m2 / (double)L + (double)eps)));
}

// Pass B. grid = (chunks per segment, segments), same mapping as pass A.
// UNIFORM: HW % kChunk == 0, so every chunk is full and lies inside one
// channel (channel = chunk / (HW / kChunk)): no masks, one set of affine
// coefficients per workgroup. Otherwise each vector finds its channel with
// 32-bit arithmetic (a vector never straddles channels since HW % 4 == 0;
// segments are < 2^31 floats on this path). Index math stays 32-bit: a
// 64-bit division here expands into a software routine that doubled the
// kernel's VGPR count and cost a third of its bandwidth.
// MERGE (segments of at most 64 chunks): no finalize launch; every wave
// merges its segment's chunk pairs itself with k_gn_finalize's arithmetic
// (one pair per lane) and takes lane 0's result, the value the finalize
// kernel would store. The pair loads are issued before the x loads: loads
// complete in order, so the merge runs while the x loads are in flight
// instead of after them.
template <bool SILU, bool UNIFORM, bool MERGE>
__global__ __launch_bounds__(kThreads) void k_gn_apply(const float* __restrict__ x, float* __restrict__ y, int64_t L,
                                                      int HW, int chunks_per_ch, int cg, int groups, int seg0,
                                                      const float2* __restrict__ stats,
                                                      const float2* __restrict__ part, int nchunks, float eps,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ beta) {
    const int seg = blockIdx.y, chunk = blockIdx.x;
    const int off = chunk * (int)kChunk;
    const f4* p = (const f4*)(x + (int64_t)seg * L + off);
    f4* q = (f4*)(y + (int64_t)seg * L + off);
    const int lane = threadIdx.x & 63;
    float2 st = make_float2(0.f, 0.f);
    if constexpr (MERGE) st = lane < nchunks ? part[(int64_t)seg * nchunks + lane] : make_float2(0.f, 0.f);
    else st = stats[seg];
    const int cnt = UNIFORM ? (int)kChunk : (int)(L - off < kChunk ? L - off : kChunk);
    const int n4 = cnt >> 2;
    f4 v[kChunkV];
#pragma unroll
    for (int j = 0; j < kChunkV; ++j) {
        const int idx = threadIdx.x + kThreads * j;
        if (UNIFORM || idx < n4) v[j] = dev::ld_stream(p + idx);
    }
    float meanf, rstd;
    if constexpr (MERGE) {
        const double tot = lane < nchunks ? (double)st.x : 0.0;
        const double mean = wave_dsum(tot) / (double)L;
        double m2t = 0.0;
        if (lane < nchunks) {
            const int64_t o = (int64_t)lane * kChunk;
            const double ni = (double)(L - o < kChunk ? L - o : kChunk);
            const double dm = (double)st.x / ni - mean;
            m2t = (double)st.y + ni * dm * dm;
        }
        const double m2 = wave_dsum(m2t);
        meanf = dev::readlane((float)mean, 0);
        rstd = dev::readlane((float)(1.0 / sqrt(m2 / (double)L + (double)eps)), 0);
    } else {
        meanf = st.x;
        rstd = st.y;
    }
    const int gc = ((seg0 + seg) % groups) * cg;
    if constexpr (UNIFORM) {
        const int ch = gc + chunk / chunks_per_ch;
        const float a = rstd * gamma[ch];
        const float b = beta[ch] - meanf * a;
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) dev::st_stream(q + threadIdx.x + kThreads * j, apply4<SILU>(v[j], a, b));
    } else {
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) {
            const int idx = threadIdx.x + kThreads * j;
            if (idx < n4) {
                const int ch = gc + (int)((unsigned)(off + idx * 4) / (unsigned)HW);
                const float a = rstd * gamma[ch];
                const float b = beta[ch] - meanf * a;
                dev::st_stream(q + idx, apply4<SILU>(v[j], a, b));
            }
        }
    }
}

// ---- generic (any HW / alignment): one workgroup per segment, three strided
// passes; statistics in double per thread, like the reference's loops.
template <bool SILU>
__global__ __launch_bounds__(kThreads) void k_gn_generic(const float* x, float* y, int64_t C, int64_t HW, int groups,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, float eps) {
    __shared__ double dsh[kThreads];
    const int64_t seg = blockIdx.x;
    const int64_t n = seg / groups, g = seg % groups, cg = C / groups, L = cg * HW;
    const float* p = x + (n * C + g * cg) * HW;
    float* q = y + (n * C + g * cg) * HW;
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < L; i += kThreads) s += p[i];
    dsh[threadIdx.x] = s;
    __syncthreads();
    for (int w = kThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) dsh[threadIdx.x] += dsh[threadIdx.x + w];
        __syncthreads();
    }
    const double mean = dsh[0] / (double)L;
    __syncthreads();
    double m2 = 0.0;
    for (int64_t i = threadIdx.x; i < L; i += kThreads) {
        const double d = p[i] - mean;
        m2 += d * d;
    }
    dsh[threadIdx.x] = m2;
    __syncthreads();
    for (int w = kThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) dsh[threadIdx.x] += dsh[threadIdx.x + w];
        __syncthreads();
    }
    const float rstd = (float)(1.0 / sqrt(dsh[0] / (double)L + (double)eps));
    const float meanf = (float)mean;
    for (int64_t i = threadIdx.x; i < L; i += kThreads) {
        const int64_t ch = g * cg + i / HW;
        const float a = rstd * gamma[ch];
        const float b = beta[ch] - meanf * a;
        float o = p[i] * a + b;
        if (SILU) o = silu1(o);
        q[i] = o;
    }
}

// Bytes of input per block of the split schedule (SDH_GN_BLOCK_MB; 0 = the
// whole tensor in one block, the default). Blocks exist for the grid's
// 65535-segment limit; smaller blocks, so that the apply pass would re-read
// a block from cache, measured slower on MI355X at every size from 8 to 128
// MB (4b: 249 us whole, 258-431 us blocked), so the knob serves tests of the
// multi-block path at small sizes.
int64_t gn_block_bytes() {
    static const int64_t v = [] {
        const char* e = std::getenv("SDH_GN_BLOCK_MB");
        if (!e || !*e) return (int64_t)kGnBlockMB << 20;
        char* end = nullptr;
        const long long mb = std::strtoll(e, &end, 10);
        return (end && *end == 0 && mb >= 0) ? (int64_t)mb << 20 : (int64_t)kGnBlockMB << 20;
    }();
    return v;
}

void run_gn(const char* op, bool silu, const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups,
            const float* gamma, const float* beta, float eps) {
    need(N >= 0 && C >= 0 && HW >= 0, op, "negative size");
    need(groups > 0, op, "groups must be positive");
    need(C % groups == 0, op, "channels not divisible by groups");
    if (N == 0 || C == 0 || HW == 0) return;
    ensure_init();
    const size_t bytes = (size_t)(N * C * HW) * 4;
    check_range(x, bytes, op, "x");
    check_range(y, bytes, op, "y");
    check_range(gamma, (size_t)C * 4, op, "gamma");
    check_range(beta, (size_t)C * 4, op, "beta");
    // the single-pass and generic kernels run one workgroup (up to 1024
    // work-items) per (sample, group) segment: samples beyond what one
    // dispatch covers go in several launches
    need((int64_t)groups * 1024 <= kMaxGridItems, op, "too many groups for one launch");
    const int64_t samples_per_launch = units_per_launch((int64_t)groups * 1024);
    if (N > samples_per_launch) {
        in_pieces(N, samples_per_launch, [&](int64_t n0, int64_t nn) {
            run_gn(op, silu, x + n0 * C * HW, y + n0 * C * HW, nn, C, HW, groups, gamma, beta, eps);
        });
        return;
    }
    const int64_t cg = C / groups, L = cg * HW, nseg = N * groups;
    const bool vec = HW % 4 == 0 && aligned16(x) && aligned16(y) && L < (1LL << 31);
    if (vec && L <= (int64_t)1024 * 4 * 16 && nseg <= 0x7fffffffLL) {
        const int64_t n4 = L / 4;
        auto go = [&](auto tc, auto vc) {
            constexpr int TPB = decltype(tc)::value, V = decltype(vc)::value;
            if (silu)
                k_gn_single<TPB, V, true><<<(unsigned)nseg, TPB, 0, stream()>>>(x, y, (int)C, (int)HW, groups, gamma,
                                                                               beta, eps);
            else
                k_gn_single<TPB, V, false><<<(unsigned)nseg, TPB, 0, stream()>>>(x, y, (int)C, (int)HW, groups, gamma,
                                                                                beta, eps);
        };
        using I = std::integral_constant<int, 256>;
        using K = std::integral_constant<int, 1024>;
        if (n4 <= 256) go(I(), std::integral_constant<int, 1>());
        else if (n4 <= 512) go(I(), std::integral_constant<int, 2>());
        else if (n4 <= 1024) go(I(), std::integral_constant<int, 4>());
        else if (n4 <= 2048) go(I(), std::integral_constant<int, 8>());
        else if (n4 <= 4096) go(K(), std::integral_constant<int, 4>());
        else if (n4 <= 8192) go(K(), std::integral_constant<int, 8>());
        else if (n4 <= 12288) go(K(), std::integral_constant<int, 12>());
        else go(K(), std::integral_constant<int, 16>());
    } else if (vec) {
        const int64_t nchunks = (L + kChunk - 1) / kChunk;
        // segments per block: the apply pass re-reads a block right after
        // the partial pass read it, while it is still cached
        int64_t sb = nseg;
        const int64_t budget = gn_block_bytes();
        if (budget > 0) sb = std::max<int64_t>(1, std::min<int64_t>(nseg, budget / (L * 4)));
        sb = std::min<int64_t>(sb, 65535);
        const size_t part_bytes = ((size_t)(sb * nchunks) * sizeof(float2) + 255) / 256 * 256;
        char* scr = (char*)scratch(part_bytes + (size_t)sb * sizeof(float2));
        float2* part = (float2*)scr;
        float2* stats = (float2*)(scr + part_bytes);
        const bool uniform = HW % kChunk == 0;
        const int cpc = uniform ? (int)(HW / kChunk) : 1;
        for (int64_t s0 = 0; s0 < nseg; s0 += sb) {
            const int64_t k = std::min<int64_t>(sb, nseg - s0);
            const float* xb = x + s0 * L;
            float* yb = y + s0 * L;
            const dim3 grid((unsigned)nchunks, (unsigned)k);
            k_gn_partial<<<grid, kThreads, 0, stream()>>>(xb, L, nchunks, part);
            launched(op);
            const bool merge = nchunks <= 64;  // one chunk pair per lane: merged inside pass B
            if (!merge) {
                k_gn_finalize<<<(unsigned)k, 64, 0, stream()>>>(part, L, nchunks, stats, eps);
                launched(op);
            }
            const int seg0 = (int)(s0 % groups);
            auto apply = [&](auto sc, auto uc) {
                constexpr bool S = decltype(sc)::value, U = decltype(uc)::value;
                if (merge)
                    k_gn_apply<S, U, true><<<grid, kThreads, 0, stream()>>>(xb, yb, L, (int)HW, cpc, (int)cg, groups,
                                                                            seg0, stats, part, (int)nchunks, eps,
                                                                            gamma, beta);
                else
                    k_gn_apply<S, U, false><<<grid, kThreads, 0, stream()>>>(xb, yb, L, (int)HW, cpc, (int)cg, groups,
                                                                             seg0, stats, part, (int)nchunks, eps,
                                                                             gamma, beta);
            };
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (silu) uniform ? apply(T_(), T_()) : apply(T_(), F_());
            else uniform ? apply(F_(), T_()) : apply(F_(), F_());
            if (s0 + sb < nseg) launched(op);
        }
    } else {
        need(nseg <= 0x7fffffffLL, op, "too many groups");
        if (silu)
            k_gn_generic<true><<<(unsigned)nseg, kThreads, 0, stream()>>>(x, y, C, HW, groups, gamma, beta, eps);
        else
            k_gn_generic<false><<<(unsigned)nseg, kThreads, 0, stream()>>>(x, y, C, HW, groups, gamma, beta, eps);
    }
    launched(op);
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_group_norm(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                   const float* beta, float eps) {
    return guarded([&] { run_gn("sdh_group_norm", false, x, y, N, C, HW, groups, gamma, beta, eps); });
}

int sdh_group_norm_silu(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                        const float* beta, float eps) {
    return guarded([&] { run_gn("sdh_group_norm_silu", true, x, y, N, C, HW, groups, gamma, beta, eps); });
}

}  // extern "C"

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
//   * single: one workgroup per segment when the segment fits in the
//     workgroup's registers (<= 256 threads x 16 float4). One HBM read, one
//     write. Used by the SD 1.5 mid-block shapes.
//   * split: the segment is cut into chunks of kChunk floats.
//       pass A (k_gn_partial): one workgroup per chunk computes the chunk's
//         sum and its M2 around the chunk mean from registers and stores the
//         pair; it then bumps the segment's arrival counter, and the last
//         arriving workgroup merges all chunk pairs in double
//         (M2 = sum M2_i + n_i (mean_i - mean)^2, the exact pairwise identity),
//         writes (mean, rstd) and re-arms the counter to zero. No workgroup
//         ever waits for another.
//       pass B (k_gn_apply): one workgroup per chunk applies the affine (and
//         SiLU), walking the chunks in the reverse of pass A's order so that
//         its first reads find the most recently read data still in the
//         last-level (Infinity) cache.
#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;
constexpr int kChunkV = 8;                               // float4 per thread per chunk
constexpr int64_t kChunk = (int64_t)kThreads * 4 * kChunkV;  // floats per chunk (8192)

struct SegStat {
    double mean;
    float rstd;
    float pad;
};

// Block-wide sum of 4 waves: wave DPP reduction, then 4 partials via LDS.
__device__ __forceinline__ float block_sum4(float v, float* sh) {
    v = dev::wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();  // sh may still be read from a previous call
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

__device__ __forceinline__ float silu1(float v) { return v / (1.0f + expf(-v)); }

template <bool SILU>
__device__ __forceinline__ f4 apply4(f4 v, float a, float b) {
    f4 o = v * a + b;
    if constexpr (SILU) o = f4{silu1(o.x), silu1(o.y), silu1(o.z), silu1(o.w)};
    return o;
}

// ---- single-workgroup schedule ---------------------------------------------
template <int V, bool SILU>
__global__ __launch_bounds__(kThreads) void k_gn_single(const float* __restrict__ x, float* __restrict__ y, int C,
                                                       int HW, int groups, const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, float eps) {
    __shared__ float sh[4];
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
        const int idx = threadIdx.x + kThreads * j;
        v[j] = idx < n4 ? dev::ld_stream(p + idx) : f4{0.f, 0.f, 0.f, 0.f};
        s += dev::hsum(v[j]);
    }
    const double mean = (double)block_sum4(s, sh) / (double)L;
    const float meanf = (float)mean;
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = threadIdx.x + kThreads * j;
        if (idx < n4) {
            const f4 d = v[j] - meanf;
            m2 += dev::hsum(d * d);
        }
    }
    const double var = (double)block_sum4(m2, sh);
    const float rstd = (float)(1.0 / sqrt(var / (double)L + (double)eps));
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = threadIdx.x + kThreads * j;
        if (idx < n4) {
            const int ch = g * cg + (idx * 4) / HW;
            const float a = rstd * gamma[ch];
            const float b = beta[ch] - meanf * a;
            dev::st_stream(q + idx, apply4<SILU>(v[j], a, b));
        }
    }
}

// ---- split schedule -----------------------------------------------------------
// grid = (chunks per segment, segments)
__global__ __launch_bounds__(kThreads) void k_gn_partial(const float* __restrict__ x, int64_t L, int64_t nchunks,
                                                        float2* __restrict__ part, SegStat* __restrict__ stats,
                                                        unsigned* __restrict__ counter, float eps) {
    __shared__ float sh[4];
    __shared__ unsigned last;
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
        v[j] = idx < n4 ? dev::ld_stream(p + idx) : f4{0.f, 0.f, 0.f, 0.f};
        s += dev::hsum(v[j]);
    }
    const float sum = block_sum4(s, sh);
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
    const float M2 = block_sum4(m2, sh);
    if (threadIdx.x == 0) {
        part[seg * nchunks + chunk] = make_float2(sum, M2);
        // release our partial, then count ourselves in
        const unsigned prev =
            __hip_atomic_fetch_add(counter + seg, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = (prev == (unsigned)(nchunks - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (!last) return;
    // Last arrival for this segment: merge the chunk pairs in double, in
    // chunk order (deterministic whichever workgroup arrives last).
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __shared__ double dsh[kThreads];
    const float2* pp = part + seg * nchunks;
    double tot = 0.0;
    for (int64_t i = threadIdx.x; i < nchunks; i += kThreads) tot += (double)pp[i].x;
    dsh[threadIdx.x] = tot;
    __syncthreads();
    for (int w = kThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) dsh[threadIdx.x] += dsh[threadIdx.x + w];
        __syncthreads();
    }
    const double mean = dsh[0] / (double)L;
    __syncthreads();
    double m2t = 0.0;
    for (int64_t i = threadIdx.x; i < nchunks; i += kThreads) {
        const float2 pr = pp[i];
        const double ni = (double)(L - i * kChunk < kChunk ? L - i * kChunk : kChunk);
        const double dm = (double)pr.x / ni - mean;
        m2t += (double)pr.y + ni * dm * dm;
    }
    dsh[threadIdx.x] = m2t;
    __syncthreads();
    for (int w = kThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) dsh[threadIdx.x] += dsh[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        SegStat st;
        st.mean = mean;
        st.rstd = (float)(1.0 / sqrt(dsh[0] / (double)L + (double)eps));
        st.pad = 0.f;
        stats[seg] = st;
        counter[seg] = 0u;  // re-arm for the next call (ordered before the next kernel)
    }
}

// grid = (chunks per segment, segments), walked in reverse.
template <bool SILU>
__global__ __launch_bounds__(kThreads) void k_gn_apply(const float* __restrict__ x, float* __restrict__ y, int64_t L,
                                                      int64_t HW, int cg, int groups, int64_t nchunks,
                                                      const SegStat* __restrict__ stats,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ beta) {
    const int64_t seg = (int64_t)gridDim.y - 1 - blockIdx.y;
    const int64_t chunk = nchunks - 1 - blockIdx.x;
    const int64_t off = chunk * kChunk;
    const int64_t cnt = L - off < kChunk ? L - off : kChunk;
    const int n4 = (int)(cnt >> 2);
    const SegStat st = stats[seg];
    const float meanf = (float)st.mean;
    const int g = (int)(seg % groups);
    const f4* p = (const f4*)(x + seg * L + off);
    f4* q = (f4*)(y + seg * L + off);
    const int64_t c_first = off / HW, c_last = (off + cnt - 1) / HW;
    f4 v[kChunkV];
#pragma unroll
    for (int j = 0; j < kChunkV; ++j) {
        const int idx = threadIdx.x + kThreads * j;
        if (idx < n4) v[j] = dev::ld_stream(p + idx);
    }
    if (c_first == c_last) {
        const int ch = g * cg + (int)c_first;
        const float a = st.rstd * gamma[ch];
        const float b = beta[ch] - meanf * a;
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) {
            const int idx = threadIdx.x + kThreads * j;
            if (idx < n4) dev::st_stream(q + idx, apply4<SILU>(v[j], a, b));
        }
    } else {
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) {
            const int idx = threadIdx.x + kThreads * j;
            if (idx < n4) {
                const int ch = g * cg + (int)((off + (int64_t)idx * 4) / HW);
                const float a = st.rstd * gamma[ch];
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

template <class F>
void with_v(int v, F&& f) {
    switch (v) {
        case 1: f(std::integral_constant<int, 1>()); break;
        case 2: f(std::integral_constant<int, 2>()); break;
        case 4: f(std::integral_constant<int, 4>()); break;
        case 8: f(std::integral_constant<int, 8>()); break;
        case 16: f(std::integral_constant<int, 16>()); break;
        default: fail(SDH_ERR_INVALID, "internal: unsupported group width");
    }
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
    const int64_t cg = C / groups, L = cg * HW, nseg = N * groups;
    const bool vec = HW % 4 == 0 && aligned16(x) && aligned16(y) && L < (1LL << 31);
    if (vec && L <= (int64_t)kThreads * 4 * 16 && nseg <= 0x7fffffffLL) {
        const int64_t per_thread = (L / 4 + kThreads - 1) / kThreads;
        const int v = per_thread <= 1 ? 1 : per_thread <= 2 ? 2 : per_thread <= 4 ? 4 : per_thread <= 8 ? 8 : 16;
        with_v(v, [&](auto vc) {
            constexpr int V = decltype(vc)::value;
            if (silu)
                k_gn_single<V, true><<<(unsigned)nseg, kThreads, 0, stream()>>>(x, y, (int)C, (int)HW, groups, gamma,
                                                                               beta, eps);
            else
                k_gn_single<V, false><<<(unsigned)nseg, kThreads, 0, stream()>>>(x, y, (int)C, (int)HW, groups, gamma,
                                                                                beta, eps);
        });
    } else if (vec && nseg <= 65535) {
        const int64_t nchunks = (L + kChunk - 1) / kChunk;
        need(nchunks <= 0x7fffffffLL, op, "segment too large");
        const size_t part_bytes = (size_t)(nseg * nchunks) * sizeof(float2);
        const size_t stat_off = (part_bytes + 255) / 256 * 256;
        char* scr = (char*)scratch(stat_off + (size_t)nseg * sizeof(SegStat));
        float2* part = (float2*)scr;
        SegStat* stats = (SegStat*)(scr + stat_off);
        unsigned* cnt = counters((size_t)nseg);
        const dim3 grid((unsigned)nchunks, (unsigned)nseg);
        k_gn_partial<<<grid, kThreads, 0, stream()>>>(x, L, nchunks, part, stats, cnt, eps);
        launched(op);
        if (silu)
            k_gn_apply<true><<<grid, kThreads, 0, stream()>>>(x, y, L, HW, (int)cg, groups, nchunks, stats, gamma,
                                                            beta);
        else
            k_gn_apply<false><<<grid, kThreads, 0, stream()>>>(x, y, L, HW, (int)cg, groups, nchunks, stats, gamma,
                                                             beta);
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

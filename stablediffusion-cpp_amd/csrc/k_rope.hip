// k_rope.hip - in-place rotary embedding (tensor.cpp:698-730), for one
// tensor or for Q and K in one launch.
//
// x is [N, S, inner] with inner = heads * dim; the tables are [S, dim].
// A workgroup owns one token row (one (n, s)) of one tensor: blockIdx.x is the
// row, blockIdx.y picks Q or K. Its threads cover the row in float4 steps, so
// every HBM access is a coalesced 128-bit load/store and each table row is
// fetched once per token and reused from cache by all heads. Rows of up to
// 8 float4 per thread (16 interleaved / 4 rotate_half pairs when the head size
// divides the workgroup, 2 pairs otherwise) are held in registers, all loads
// before any store; wider rows use the looping kernels.
//   interleaved: float4 (a0, b0, a1, b1) holds pairs (2i, 2i+1), (2i+2, 2i+3),
//                rotated by cos/sin[s, 2i] and [s, 2i+2] (the even entries, as
//                tensor.cpp:717-718 uses c[i] and sn[i] for both outputs).
//   rotate_half: the float4 at head offset i < dim/2 pairs with the float4 at
//                i + dim/2 (tensor.cpp:722-724); one thread updates both.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "sdh_internal.hpp"

namespace sdh {
namespace {

using dev::f4;

constexpr int kThreads = 256;

struct RopeArgs {
    float* x[2];
    int64_t inner[2];
};

// Row in registers: RV float4 per thread, every load of the row issued before
// any store (the in-place stores would otherwise order each step's loads
// behind the previous step's stores). HINV: the head size divides the
// workgroup, so a thread's position inside the head, and with it its table
// entries, is the same at every step and the table is loaded once.
template <int RV, bool HINV>
__global__ __launch_bounds__(kThreads) void k_rope_il_reg(RopeArgs a, int64_t S, int dim,
                                                         const float* __restrict__ cs,
                                                         const float* __restrict__ sn) {
    const int t = blockIdx.y;
    const int64_t ns = blockIdx.x;
    const int64_t inner = a.inner[t];
    const int64_t s = ns % S;
    f4* row = (f4*)(a.x[t] + ns * inner);
    const f4* c4 = (const f4*)(cs + s * dim);
    const f4* s4 = (const f4*)(sn + s * dim);
    const int n4 = (int)(inner >> 2), d4 = dim >> 2;
    f4 v[RV], c[HINV ? 1 : RV], sv[HINV ? 1 : RV];
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        if (i < n4) v[j] = dev::ld_stream(row + i);
    }
    if constexpr (HINV) {
        const int h = threadIdx.x % d4;
        c[0] = c4[h];
        sv[0] = s4[h];
    } else {
#pragma unroll
        for (int j = 0; j < RV; ++j) {
            const int i = threadIdx.x + kThreads * j;
            if (i < n4) {
                c[j] = c4[i % d4];
                sv[j] = s4[i % d4];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        if (i < n4) {
            const f4 cc = c[HINV ? 0 : j], ss = sv[HINV ? 0 : j];
            f4 o;
            o.x = v[j].x * cc.x - v[j].y * ss.x;
            o.y = v[j].y * cc.x + v[j].x * ss.x;
            o.z = v[j].z * cc.z - v[j].w * ss.z;
            o.w = v[j].w * cc.z + v[j].z * ss.z;
            dev::st_stream(row + i, o);
        }
    }
}

template <int RV, bool HINV>
__global__ __launch_bounds__(kThreads) void k_rope_half_reg(RopeArgs a, int64_t S, int dim,
                                                           const float* __restrict__ cs,
                                                           const float* __restrict__ sn) {
    const int t = blockIdx.y;
    const int64_t ns = blockIdx.x;
    const int64_t inner = a.inner[t];
    const int64_t s = ns % S;
    f4* row = (f4*)(a.x[t] + ns * inner);
    const f4* c4 = (const f4*)(cs + s * dim);
    const f4* s4 = (const f4*)(sn + s * dim);
    const int h4 = dim >> 3;                    // float4 per half head
    const int pairs = (int)(inner / dim) * h4;  // float4 pairs per row
    f4 lo[RV], hi[RV];
    constexpr int TB = HINV ? 1 : RV;
    f4 cl[TB], sl[TB], ch[TB], sh[TB];
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        if (i < pairs) {
            const int head = i / h4, k = i - head * h4;
            f4* p = row + head * (dim >> 2) + k;
            lo[j] = dev::ld_stream(p);
            hi[j] = dev::ld_stream(p + h4);
        }
    }
#pragma unroll
    for (int j = 0; j < TB; ++j) {
        const int i = threadIdx.x + kThreads * j;
        if (HINV || i < pairs) {
            const int k = i % h4;
            cl[j] = c4[k];
            sl[j] = s4[k];
            ch[j] = c4[k + h4];
            sh[j] = s4[k + h4];
        }
    }
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        if (i < pairs) {
            const int head = i / h4, k = i - head * h4;
            f4* p = row + head * (dim >> 2) + k;
            const int b = HINV ? 0 : j;
            dev::st_stream(p, lo[j] * cl[b] - hi[j] * sl[b]);
            dev::st_stream(p + h4, hi[j] * ch[b] + lo[j] * sh[b]);
        }
    }
}

__global__ __launch_bounds__(kThreads) void k_rope_interleaved(RopeArgs a, int64_t S, int dim,
                                                              const float* __restrict__ cs,
                                                              const float* __restrict__ sn) {
    const int t = blockIdx.y;
    const int64_t ns = blockIdx.x;
    const int64_t inner = a.inner[t];
    const int64_t s = ns % S;
    f4* row = (f4*)(a.x[t] + ns * inner);
    const f4* c4 = (const f4*)(cs + s * dim);
    const f4* s4 = (const f4*)(sn + s * dim);
    const int n4 = (int)(inner >> 2), d4 = dim >> 2;
    for (int i = threadIdx.x; i < n4; i += kThreads) {
        const int h = i % d4;  // float4 index inside the head
        const f4 v = dev::ld_stream(row + i);
        const f4 c = c4[h], sv = s4[h];
        f4 o;
        o.x = v.x * c.x - v.y * sv.x;
        o.y = v.y * c.x + v.x * sv.x;
        o.z = v.z * c.z - v.w * sv.z;
        o.w = v.w * c.z + v.z * sv.z;
        dev::st_stream(row + i, o);
    }
}

__global__ __launch_bounds__(kThreads) void k_rope_half(RopeArgs a, int64_t S, int dim, const float* __restrict__ cs,
                                                       const float* __restrict__ sn) {
    const int t = blockIdx.y;
    const int64_t ns = blockIdx.x;
    const int64_t inner = a.inner[t];
    const int64_t s = ns % S;
    f4* row = (f4*)(a.x[t] + ns * inner);
    const f4* c4 = (const f4*)(cs + s * dim);
    const f4* s4 = (const f4*)(sn + s * dim);
    const int h4 = dim >> 3;                    // float4 per half head
    const int pairs = (int)(inner / dim) * h4;  // float4 pairs per row
    for (int i = threadIdx.x; i < pairs; i += kThreads) {
        const int head = i / h4, k = i - head * h4;
        f4* lo = row + head * (dim >> 2) + k;
        f4* hi = lo + h4;
        const f4 a0 = dev::ld_stream(lo), b0 = dev::ld_stream(hi);
        const f4 cl = c4[k], sl = s4[k], ch = c4[k + h4], shh = s4[k + h4];
        dev::st_stream(lo, a0 * cl - b0 * sl);
        dev::st_stream(hi, b0 * ch + a0 * shh);
    }
}

// Scalar fallback for any shape/alignment: one thread per pair.
__global__ __launch_bounds__(kThreads) void k_rope_scalar(RopeArgs a, int64_t NS, int64_t S, int64_t dim,
                                                         const float* __restrict__ cs, const float* __restrict__ sn,
                                                         int interleaved) {
    const int t = blockIdx.y;
    const int64_t inner = a.inner[t];
    const int64_t half = dim / 2, heads = inner / dim;
    const int64_t total = NS * heads * half;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t i = idx % half, h = (idx / half) % heads, ns = idx / (half * heads), s = ns % S;
        float* p = a.x[t] + ns * inner + h * dim;
        const float* c = cs + s * dim;
        const float* sv = sn + s * dim;
        if (interleaved) {
            const float x0 = p[2 * i], x1 = p[2 * i + 1];
            p[2 * i] = x0 * c[2 * i] - x1 * sv[2 * i];
            p[2 * i + 1] = x1 * c[2 * i] + x0 * sv[2 * i];
        } else {
            const float x0 = p[i], x1 = p[i + half];
            p[i] = x0 * c[i] - x1 * sv[i];
            p[i + half] = x1 * c[i + half] + x0 * sv[i + half];
        }
    }
}

void run_rope(const char* op, float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
              const float* cs, const float* sn, int interleaved) {
    need(N >= 0 && S >= 0 && inner_q >= 0 && inner_k >= 0, op, "negative size");
    need(dim > 0 && dim % 2 == 0, op, "dim must be positive and even");
    need(inner_q % dim == 0 && inner_k % dim == 0, op, "inner must be a multiple of dim");
    const int nt = k ? 2 : 1;
    if (N == 0 || S == 0 || (inner_q == 0 && (!k || inner_k == 0))) return;
    ensure_init();
    check_range(q, (size_t)(N * S * inner_q) * 4, op, "x/q");
    if (k) check_range(k, (size_t)(N * S * inner_k) * 4, op, "k");
    check_range(cs, (size_t)(S * dim) * 4, op, "cos");
    check_range(sn, (size_t)(S * dim) * 4, op, "sin");
    // one workgroup per token row: rows beyond what one dispatch covers go in
    // several launches, of whole sequences, or of parts of one sequence with
    // the tables offset to the part's first position
    const int64_t max_tok = units_per_launch(kThreads);
    if (N * S > max_tok) {
        if (S <= max_tok) {
            in_pieces(N, max_tok / S, [&](int64_t n0, int64_t nn) {
                run_rope(op, q + n0 * S * inner_q, inner_q, k ? k + n0 * S * inner_k : nullptr, inner_k, nn, S, dim,
                         cs, sn, interleaved);
            });
        } else {
            for (int64_t n = 0; n < N; ++n)
                in_pieces(S, max_tok, [&](int64_t s0, int64_t ns) {
                    run_rope(op, q + (n * S + s0) * inner_q, inner_q, k ? k + (n * S + s0) * inner_k : nullptr,
                             inner_k, 1, ns, dim, cs + s0 * dim, sn + s0 * dim, interleaved);
                });
        }
        return;
    }
    RopeArgs a;
    a.x[0] = q;
    a.inner[0] = inner_q;
    a.x[1] = k ? k : q;
    a.inner[1] = k ? inner_k : inner_q;
    const bool al = aligned16(q) && (!k || aligned16(k)) && aligned16(cs) && aligned16(sn);
    const dim3 grid((unsigned)(N * S), nt);
    const int64_t inner_max = std::max(inner_q, k ? inner_k : inner_q);
    if (interleaved && al && dim % 4 == 0 && inner_q % 4 == 0 && inner_k % 4 == 0) {
        // float4 per thread of the widest row
        const int64_t steps = (inner_max / 4 + kThreads - 1) / kThreads;
        const bool hinv = kThreads % (dim / 4) == 0;
        auto go = [&](auto rc) {
            constexpr int RV = decltype(rc)::value;
            if (hinv) k_rope_il_reg<RV, true><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
            else k_rope_il_reg<RV, false><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
        };
        if (steps <= 1) go(std::integral_constant<int, 1>());
        else if (steps <= 2) go(std::integral_constant<int, 2>());
        else if (steps <= 4) go(std::integral_constant<int, 4>());
        else if (steps <= 8) go(std::integral_constant<int, 8>());
        else if (steps <= 16 && hinv) k_rope_il_reg<16, true><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
        else k_rope_interleaved<<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
    } else if (!interleaved && al && dim % 8 == 0) {
        const int64_t steps = ((inner_max / dim) * (dim / 8) + kThreads - 1) / kThreads;
        const bool hinv = kThreads % (dim / 8) == 0;
        auto go = [&](auto rc) {
            constexpr int RV = decltype(rc)::value;
            if (hinv) k_rope_half_reg<RV, true><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
            else k_rope_half_reg<RV, false><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
        };
        if (steps <= 1) go(std::integral_constant<int, 1>());
        else if (steps <= 2) go(std::integral_constant<int, 2>());
        else if (steps <= 4 && hinv) k_rope_half_reg<4, true><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
        else k_rope_half<<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn);
    } else {
        const int64_t total = N * S * (std::max(inner_q, inner_k) / dim) * (dim / 2);
        const int64_t want = (total + kThreads - 1) / kThreads;
        const unsigned gx = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)num_cus() * 16));
        k_rope_scalar<<<dim3(gx, nt), kThreads, 0, stream()>>>(a, N * S, S, dim, cs, sn, interleaved);
    }
    launched(op);
}

// ---- interleaved RoPE with the angles formed on the device ----------------------------
// The tables of zimage.cpp:71-88 come from positions: pair k of a head turns
// with position axis a(k) (the concatenated axes) by the float angle
// (float)((double)pos[s, a(k)] * freq(k)), freq(k) = theta^(-2j/d_a) in
// double for index j of the pair within its axis. The host forms the
// frequencies (with the same double pow as the reference) and passes them as
// kernel arguments; each workgroup turns its token's dim/2 angles into cos and
// sin in LDS while its row loads are in flight, so no table crosses HBM. The
// positions are [S, 3] int32 on the device; the rotation is k_rope_il_reg's.
constexpr int kMaxAxisPairs = 128;  // dim <= 256

struct RopeAxes {
    double freq[kMaxAxisPairs];
    unsigned char axis[kMaxAxisPairs];
};

// WAVE: dim <= 128, so the token's dim/2 pairs fit one per lane: every wave
// forms them itself (lane k, pair k) and fetches the two pairs of each of
// its float4 by cross-lane reads, with no LDS and no workgroup barrier
// (measured: the barrier behind one wave's 64 sin/cos cost 2 us at config 3).
// Otherwise the pairs go through LDS.
template <int RV, bool WAVE>
__global__ __launch_bounds__(kThreads) void k_rope_il_axes(RopeArgs a, int64_t S, int dim, int64_t s0,
                                                          const int* __restrict__ pos, RopeAxes ax) {
    __shared__ float cl[WAVE ? 1 : kMaxAxisPairs], sl[WAVE ? 1 : kMaxAxisPairs];
    const int t = blockIdx.y;
    const int64_t ns = blockIdx.x;
    const int64_t inner = a.inner[t];
    const int64_t s = ns % S;
    f4* row = (f4*)(a.x[t] + ns * inner);
    const int n4 = (int)(inner >> 2), d4 = dim >> 2;
    f4 v[RV];
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        if (i < n4) v[j] = dev::ld_stream(row + i);
    }
    const int* ps = pos + (s0 + s) * 3;
    float cw = 1.0f, sw = 0.0f;
    if constexpr (WAVE) {
        const int k = threadIdx.x & 63;
        if (k < (dim >> 1)) {
            const float ang = (float)((double)ps[ax.axis[k]] * ax.freq[k]);
            cw = cosf(ang);
            sw = sinf(ang);
        }
    } else {
        if ((int)threadIdx.x < (dim >> 1)) {
            const int k = threadIdx.x;
            const float ang = (float)((double)ps[ax.axis[k]] * ax.freq[k]);
            cl[k] = cosf(ang);
            sl[k] = sinf(ang);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        const int h = 2 * (i % d4);  // first of the float4's two pairs
        float c0, s0v, c1, s1v;
        if constexpr (WAVE) {
            c0 = __shfl(cw, h, 64);
            s0v = __shfl(sw, h, 64);
            c1 = __shfl(cw, h + 1, 64);
            s1v = __shfl(sw, h + 1, 64);
        } else {
            c0 = cl[h];
            s0v = sl[h];
            c1 = cl[h + 1];
            s1v = sl[h + 1];
        }
        if (i < n4) {
            f4 o;
            o.x = v[j].x * c0 - v[j].y * s0v;
            o.y = v[j].y * c0 + v[j].x * s0v;
            o.z = v[j].z * c1 - v[j].w * s1v;
            o.w = v[j].w * c1 + v[j].z * s1v;
            dev::st_stream(row + i, o);
        }
    }
}

void run_rope_axes(const char* op, float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S,
                   int64_t dim, const int* pos, int64_t s0, const RopeAxes& ax) {
    const int64_t max_tok = units_per_launch(kThreads);
    if (N * S > max_tok) {
        if (S <= max_tok) {
            in_pieces(N, max_tok / S, [&](int64_t n0, int64_t nn) {
                run_rope_axes(op, q + n0 * S * inner_q, inner_q, k + n0 * S * inner_k, inner_k, nn, S, dim, pos, s0, ax);
            });
        } else {
            for (int64_t n = 0; n < N; ++n)
                in_pieces(S, max_tok, [&](int64_t p0, int64_t ns) {
                    run_rope_axes(op, q + (n * S + p0) * inner_q, inner_q, k + (n * S + p0) * inner_k, inner_k, 1, ns,
                                  dim, pos, s0 + p0, ax);
                });
        }
        return;
    }
    RopeArgs a;
    a.x[0] = q;
    a.inner[0] = inner_q;
    a.x[1] = k;
    a.inner[1] = inner_k;
    const dim3 grid((unsigned)(N * S), 2);
    const int64_t steps = (std::max(inner_q, inner_k) / 4 + kThreads - 1) / kThreads;
    const bool wave = dim <= 128;
    auto go = [&](auto rc) {
        constexpr int RV = decltype(rc)::value;
        if (wave) k_rope_il_axes<RV, true><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, s0, pos, ax);
        else k_rope_il_axes<RV, false><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, s0, pos, ax);
    };
    if (steps <= 1) go(std::integral_constant<int, 1>());
    else if (steps <= 2) go(std::integral_constant<int, 2>());
    else if (steps <= 4) go(std::integral_constant<int, 4>());
    else go(std::integral_constant<int, 8>());
    launched(op);
}

// ---- fused QK-norm + RoPE (zimage.cpp:117-120) ---------------------------------------
// rms_norm_heads_ then rope_, for Q and K in one launch: each row is read and
// written once instead of twice. A workgroup owns one token row of one tensor
// (blockIdx.y = Q or K), in registers (RV float4 per thread). Interleaved: a
// head of dim = 4 L floats is L consecutive float4, so every aligned group of
// L lanes holds one head at every step (L divides 256): group_sum<L> gives the
// head's sum of squares, and a lane's position in the head -- hence its gamma
// and table entries -- is the same at every step. Per element it applies
// k_heads' operations (o = x * rstd, then * gamma, with the fp32 rstd_fast)
// and then k_rope_il_reg's, each product and difference rounded on its own
// (dev::qk_norm_rope4, shared with the attention's fused Q/K preparation);
// where the compiler contracts the unfused kernels differently the results
// differ from them by an ulp or two.
// rotate_half: a lane holds the pair (k, k + dim/8) of float4, L = dim / 8
// lanes per head. All lanes join the reductions (rows outside the tensor are
// zeros); only the loads and stores are guarded.
struct QKArgs {
    float* x[2];
    int64_t inner[2];
    const float* gamma[2];
};

__device__ __forceinline__ f4 zero_f4() { return f4{0.f, 0.f, 0.f, 0.f}; }

template <int RV, int L>
__global__ __launch_bounds__(kThreads) void k_qknorm_rope_il(QKArgs a, int64_t S, int dim, const float* __restrict__ cs,
                                                            const float* __restrict__ sn, float eps) {
    const int t = blockIdx.y;
    const int64_t ns = blockIdx.x;
    const int64_t inner = a.inner[t];
    const int64_t s = ns % S;
    f4* row = (f4*)(a.x[t] + ns * inner);
    const int n4 = (int)(inner >> 2);
    const int h = threadIdx.x % L;
    f4 v[RV];
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        v[j] = i < n4 ? dev::ld_stream(row + i) : zero_f4();
    }
    const f4 c = ((const f4*)(cs + s * dim))[h];
    const f4 sv = ((const f4*)(sn + s * dim))[h];
    const float* gp = a.gamma[t];
    const f4 g = gp ? ((const f4*)gp)[h] : f4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const float q = dev::group_sum<L>(dev::sumsq4(v[j]));
        const float rstd = dev::rstd_fast(q, 1.0f / (4 * L), eps);  // dim = 4 L
        const f4 r = dev::qk_norm_rope4(v[j], rstd, gp != nullptr, g, c, sv);
        const int i = threadIdx.x + kThreads * j;
        if (i < n4) dev::st_stream(row + i, r);
    }
}

template <int RV, int L>
__global__ __launch_bounds__(kThreads) void k_qknorm_rope_half(QKArgs a, int64_t S, int dim,
                                                              const float* __restrict__ cs,
                                                              const float* __restrict__ sn, float eps) {
    const int t = blockIdx.y;
    const int64_t ns = blockIdx.x;
    const int64_t inner = a.inner[t];
    const int64_t s = ns % S;
    f4* row = (f4*)(a.x[t] + ns * inner);
    const f4* c4 = (const f4*)(cs + s * dim);
    const f4* s4 = (const f4*)(sn + s * dim);
    const int pairs = (int)(inner / dim) * L;
    const int k = threadIdx.x % L;
    f4 lo[RV], hi[RV];
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const int i = threadIdx.x + kThreads * j;
        if (i < pairs) {
            f4* p = row + (i / L) * (2 * L) + k;
            lo[j] = dev::ld_stream(p);
            hi[j] = dev::ld_stream(p + L);
        } else {
            lo[j] = hi[j] = zero_f4();
        }
    }
    const f4 cl = c4[k], sl = s4[k], ch = c4[k + L], sh = s4[k + L];
    const float* gp = a.gamma[t];
    const f4 glo = gp ? ((const f4*)gp)[k] : f4{1.f, 1.f, 1.f, 1.f};
    const f4 ghi = gp ? ((const f4*)gp)[k + L] : f4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int j = 0; j < RV; ++j) {
        const float q = dev::group_sum<L>(dev::sumsq4(lo[j]) + dev::sumsq4(hi[j]));
        const float rstd = dev::rstd_fast(q, 1.0f / (8 * L), eps);  // dim = 8 L
        f4 a0 = lo[j] * rstd, b0 = hi[j] * rstd;
        if (gp) {
            a0 = a0 * glo;
            b0 = b0 * ghi;
        }
        const int i = threadIdx.x + kThreads * j;
        if (i < pairs) {
            f4* p = row + (i / L) * (2 * L) + k;
            dev::st_stream(p, a0 * cl - b0 * sl);
            dev::st_stream(p + L, b0 * ch + a0 * sh);
        }
    }
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + nb && y < x + na;
}

// Returns false when no fused kernel covers the shape (the caller then runs
// the two ops one after the other).
bool run_qknorm_rope_fused(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                           const float* gq, const float* gk, float eps, const float* cs, const float* sn,
                           int interleaved) {
    const bool al = aligned16(q) && aligned16(k) && aligned16(cs) && aligned16(sn) && (!gq || aligned16(gq)) &&
                    (!gk || aligned16(gk));
    if (!al || dim % 8 != 0 || N * S * kThreads > kMaxGridItems) return false;
    const int64_t L = interleaved ? dim / 4 : dim / 8;
    if (!(L == 4 || L == 8 || L == 16 || L == 32 || L == 64)) return false;
    const int64_t inner_max = std::max(inner_q, inner_k);
    const int64_t units = interleaved ? inner_max / 4 : (inner_max / dim) * L;
    const int64_t steps = (units + kThreads - 1) / kThreads;
    if (steps > (interleaved ? 8 : 4)) return false;
    QKArgs a;
    a.x[0] = q;
    a.x[1] = k;
    a.inner[0] = inner_q;
    a.inner[1] = inner_k;
    a.gamma[0] = gq;
    a.gamma[1] = gk;
    const dim3 grid((unsigned)(N * S), 2);
    auto go = [&](auto rc, auto lc) {
        constexpr int RV = decltype(rc)::value, LL = decltype(lc)::value;
        if (interleaved)
            k_qknorm_rope_il<RV, LL><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn, eps);
        else if constexpr (RV <= 4)
            k_qknorm_rope_half<RV, LL><<<grid, kThreads, 0, stream()>>>(a, S, (int)dim, cs, sn, eps);
    };
    auto by_steps = [&](auto lc) {
        if (steps <= 1) go(std::integral_constant<int, 1>(), lc);
        else if (steps <= 2) go(std::integral_constant<int, 2>(), lc);
        else if (steps <= 4) go(std::integral_constant<int, 4>(), lc);
        else go(std::integral_constant<int, 8>(), lc);
    };
    switch (L) {
        case 4: by_steps(std::integral_constant<int, 4>()); break;
        case 8: by_steps(std::integral_constant<int, 8>()); break;
        case 16: by_steps(std::integral_constant<int, 16>()); break;
        case 32: by_steps(std::integral_constant<int, 32>()); break;
        default: by_steps(std::integral_constant<int, 64>()); break;
    }
    return true;
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_rope(float* x, int64_t N, int64_t S, int64_t inner, int64_t dim, const float* cos, const float* sin,
             int interleaved) {
    return guarded([&] { run_rope("sdh_rope", x, inner, nullptr, 0, N, S, dim, cos, sin, interleaved); });
}

int sdh_rope_qk(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                const float* cos, const float* sin, int interleaved) {
    return guarded([&] {
        need(k != nullptr, "sdh_rope_qk", "k is NULL");
        need(k != q, "sdh_rope_qk", "q and k must be distinct tensors");
        run_rope("sdh_rope_qk", q, inner_q, k, inner_k, N, S, dim, cos, sin, interleaved);
    });
}

int sdh_rope_qk_axes(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                     const int32_t* pos, int axis0, int axis1, int axis2, float theta) {
    return guarded([&] {
        const char* op = "sdh_rope_qk_axes";
        need(q != nullptr && k != nullptr && k != q, op, "q and k must be two distinct tensors");
        need(N >= 0 && S >= 0 && inner_q >= 0 && inner_k >= 0, op, "negative size");
        const int axes[3] = {axis0, axis1, axis2};
        need(axis0 >= 0 && axis1 >= 0 && axis2 >= 0 && axis0 % 2 == 0 && axis1 % 2 == 0 && axis2 % 2 == 0, op,
             "axis sizes must be even and non-negative");
        need((int64_t)axis0 + axis1 + axis2 == dim, op, "the axis sizes must add up to dim");
        need(dim > 0 && dim % 4 == 0 && dim / 2 <= kMaxAxisPairs, op, "dim must be a positive multiple of 4, at most 256");
        need(inner_q % dim == 0 && inner_k % dim == 0, op, "inner must be a multiple of dim");
        need(inner_q <= (int64_t)kThreads * 4 * 8 && inner_k <= (int64_t)kThreads * 4 * 8, op,
             "rows of at most 8192 floats");
        need(theta > 0.0f, op, "theta must be positive");
        if (N == 0 || S == 0) return;
        ensure_init();
        check_range(q, (size_t)(N * S * inner_q) * 4, op, "q");
        check_range(k, (size_t)(N * S * inner_k) * 4, op, "k");
        check_range(pos, (size_t)(S * 3) * 4, op, "pos");
        need(aligned16(q) && aligned16(k) && inner_q % 4 == 0 && inner_k % 4 == 0, op,
             "q and k must be 16-byte aligned with rows of whole float4");
        RopeAxes ax;
        int kk = 0;
        for (int a = 0; a < 3; ++a)
            for (int j = 0; j < axes[a] / 2; ++j, ++kk) {
                ax.freq[kk] = 1.0 / std::pow((double)theta, (double)(2 * j) / (double)axes[a]);
                ax.axis[kk] = (unsigned char)a;
            }
        run_rope_axes(op, q, inner_q, k, inner_k, N, S, dim, pos, 0, ax);
    });
}

int sdh_qknorm_rope(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                    const float* gamma_q, const float* gamma_k, float eps, const float* cos, const float* sin,
                    int interleaved) {
    return guarded([&] {
        const char* op = "sdh_qknorm_rope";
        need(q != nullptr && k != nullptr, op, "q and k are required");
        need(N >= 0 && S >= 0 && inner_q >= 0 && inner_k >= 0, op, "negative size");
        need(dim > 0 && dim % 2 == 0, op, "dim must be positive and even");
        need(inner_q % dim == 0 && inner_k % dim == 0, op, "inner must be a multiple of dim");
        if (N == 0 || S == 0) return;
        ensure_init();
        const size_t bq = (size_t)(N * S * inner_q) * 4, bk = (size_t)(N * S * inner_k) * 4;
        if (bq) check_range(q, bq, op, "q");
        if (bk) check_range(k, bk, op, "k");
        need(!(bq && bk && overlaps(q, bq, k, bk)), op, "q and k overlap");
        if (gamma_q) check_range(gamma_q, (size_t)dim * 4, op, "gamma_q");
        if (gamma_k) check_range(gamma_k, (size_t)dim * 4, op, "gamma_k");
        check_range(cos, (size_t)(S * dim) * 4, op, "cos");
        check_range(sin, (size_t)(S * dim) * 4, op, "sin");
        if (bq && bk && run_qknorm_rope_fused(q, inner_q, k, inner_k, N, S, dim, gamma_q, gamma_k, eps, cos, sin,
                                              interleaved)) {
            launched(op);
            return;
        }
        // shapes without a fused kernel: the reference's sequence, op by op
        auto ok = [&](int st) {
            if (st != SDH_OK) fail(st, sdh_last_error());
        };
        if (bq) ok(sdh_rms_norm_heads(q, N * S * inner_q / dim, dim, gamma_q, eps));
        if (bk) ok(sdh_rms_norm_heads(k, N * S * inner_k / dim, dim, gamma_k, eps));
        if (bq) ok(sdh_rope(q, N, S, inner_q, dim, cos, sin, interleaved));
        if (bk) ok(sdh_rope(k, N, S, inner_k, dim, cos, sin, interleaved));
    });
}

}  // extern "C"

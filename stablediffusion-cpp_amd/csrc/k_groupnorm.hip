// k_groupnorm.hip - GroupNorm and the fused GroupNorm + SiLU
// (tensor.cpp:592-625 then :843-849).
//
// A "segment" is one (sample, group): cg * HW contiguous floats, channels
// g*cg .. g*cg+cg-1 of sample n. Statistics follow the reference's two-pass
// definition (mean, then the sum of squared deviations M2 around it); the
// apply step uses the reference's folded form y = x * a + (beta - mean * a),
// a = rstd * gamma[c], then SiLU as x / (1 + exp(-x)).
//
// Four schedules:
//   * pipelined (segments of 4096-float chunks, at most 64 of them, each in
//     one channel): the split schedule's two passes in one launch, the apply
//     workgroups a round behind the stats workgroups. Described at k_gn_pipe.
//   * single: one workgroup (256 or 1024 threads) per segment of at most
//     24576 floats, held in its registers. One HBM read, one write. Longer
//     segments that the pipelined schedule does not take: the split schedule
//     below 64 MB of x, the resident one above.
//   * resident (larger segments, large tensors): teams of workgroups hold a
//     segment in registers across a team wait, so x is read once (two
//     streams); pipelined over two register buffers when a team has several
//     rounds. Described at k_gn_resident; run_gn_resident says when it is
//     chosen.
//   * split: the segment is cut into chunks of 8192, 4096 or 2048 floats
//     (split_chunk: the largest that gives the pass enough workgroups).
//     SDH_GN_SPLIT=1 takes it for every aligned shape (a test knob).
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
//     y) against the two of the algorithmic minimum: the resident schedule
//     takes those.
#include <algorithm>
#include <cstdlib>
#include <string>

#include "sdh_internal.hpp"

// Device scratch of the allocation-free entry point
// (sdh_group_norm_silu_noalloc): the resident schedule's team slots and
// counters in its first kFixedCtlBytes, the split schedule's chunk pairs and
// statistics after them. Each GPU the library runs on holds its own copy
// until the process ends. In host code this name is a stand-in, not a device
// address: host code uses the address hipGetSymbolAddress returns for the
// current device (sdh::gn_fixed_scratch_setup), never the name.
static constexpr size_t kFixedScratchBytes = size_t(1) << 20;
static __device__ __align__(256) unsigned char scratch[kFixedScratchBytes];

// Exchange area of the pipelined schedule (k_gn_pipe), used by both
// GroupNorm entry points (one stream keeps their launches in order): the
// tagged chunk pairs (2 words per chunk, at most kPipeMaxChunks chunks a
// launch), then
// the captured launches' counter and an error word. A file-scope array like
// `scratch`, so the allocation-free entry point allocates nothing for it;
// zeroed at set-up. Host code uses the address hipGetSymbolAddress returns
// (sdh::gn_fixed_scratch_setup).
static constexpr int kPipeMaxChunks = 1 << 17;  // 2 GB of x per launch
static __device__ __align__(256) unsigned long long pipe_area[2 * kPipeMaxChunks + 32];

namespace sdh {
namespace {

using dev::f4;

constexpr size_t kFixedCtlBytes = size_t(64) << 10;
constexpr int kMaxDevices = 64;
// Device address of `scratch` per device, from gn_fixed_scratch_setup.
unsigned char* g_fixed_scratch[kMaxDevices] = {};
// Device address of `pipe_area` per device, likewise, and the tag of the
// last pipelined launch made directly (not captured) on that device.
unsigned long long* g_pipe_area[kMaxDevices] = {};
unsigned g_pipe_tag[kMaxDevices] = {};
// The capture (capture_generation) the last captured pipelined call was
// recorded in, and how many such calls it has recorded.
unsigned g_pipe_cap_gen[kMaxDevices] = {};
unsigned g_pipe_cap_calls[kMaxDevices] = {};

constexpr int kThreads = 256;
// Split schedule chunks: TPB work-items x CV float4 each. The largest chunk
// is 8192 floats (256 x 8); smaller ones (4096 = 64 x 16, 2048 = 64 x 8)
// give shapes with few segments more workgroups (split_chunk).
constexpr int64_t kGnBlockMB = 0;
// Segments up to this many floats take the single-workgroup schedule
// (measured: [2,640,32,32], 20480 floats, 7.6 us single, 7.5-7.7 split;
// [2,320,32,32] 5.6 single, 9.8 split); longer ones the split or resident.
constexpr int64_t kSmallResidentMin = 24576;

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
template <int TPB, int CV>
__global__ __launch_bounds__(TPB) void k_gn_partial(const float* __restrict__ x, int64_t L, int64_t nchunks,
                                                   float2* __restrict__ part) {
    constexpr int64_t CH = (int64_t)TPB * 4 * CV;  // floats per chunk
    __shared__ float sh[TPB / 64];
    const int64_t seg = blockIdx.y, chunk = blockIdx.x;
    const int64_t off = chunk * CH;
    const int64_t cnt = L - off < CH ? L - off : CH;
    const f4* p = (const f4*)(x + seg * L + off);
    const int n4 = (int)(cnt >> 2);
    f4 v[CV];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CV; ++j) {
        const int idx = threadIdx.x + TPB * j;
        v[j] = idx < n4 ? p[idx] : f4{0.f, 0.f, 0.f, 0.f};
        s += dev::hsum(v[j]);
    }
    const float sum = block_sum<TPB>(s, sh);
    const float mc = sum / (float)cnt;
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < CV; ++j) {
        const int idx = threadIdx.x + TPB * j;
        if (idx < n4) {
            const f4 d = v[j] - mc;
            m2 += dev::hsum(d * d);
        }
    }
    const float M2 = block_sum<TPB>(m2, sh);
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
                                                   int64_t chunk, float2* __restrict__ stats, float eps) {
    const int64_t seg = blockIdx.x;
    const float2* pp = part + seg * nchunks;
    double tot = 0.0;
    for (int64_t i = threadIdx.x; i < nchunks; i += 64) tot += (double)pp[i].x;
    const double mean = wave_dsum(tot) / (double)L;
    double m2t = 0.0;
    for (int64_t i = threadIdx.x; i < nchunks; i += 64) {
        const float2 pr = pp[i];
        const double ni = (double)(L - i * chunk < chunk ? L - i * chunk : chunk);
        const double dm = (double)pr.x / ni - mean;
        m2t += (double)pr.y + ni * dm * dm;
    }
    const double m2 = wave_dsum(m2t);
    if (threadIdx.x == 0) stats[seg] = make_float2((float)mean, (float)(1.0 / sqrt(m2 / (double)L + (double)eps)));
}

// Pass B. grid = (chunks per segment, segments), same mapping as pass A.
// UNIFORM: HW is a multiple of the chunk size CH, so every chunk is full
// and lies inside one channel (channel = chunk index / (HW / CH)): no
// masks, one set of affine coefficients per workgroup. Otherwise each
// vector finds its channel with 32-bit arithmetic (a vector never
// straddles channels since HW % 4 == 0; segments are < 2^31 floats on this
// path). Index math stays 32-bit: a
// 64-bit division here expands into a software routine that doubled the
// kernel's VGPR count and cost a third of its bandwidth.
// MERGE (segments of at most 64 chunks): no finalize launch; every wave
// merges its segment's chunk pairs itself with k_gn_finalize's arithmetic
// (one pair per lane) and takes lane 0's result, the value the finalize
// kernel would store. The pair loads are issued before the x loads: loads
// complete in order, so the merge runs while the x loads are in flight
// instead of after them.
template <int TPB, int CV, bool SILU, bool UNIFORM, bool MERGE>
__global__ __launch_bounds__(TPB) void k_gn_apply(const float* __restrict__ x, float* __restrict__ y, int64_t L,
                                                 int HW, int chunks_per_ch, int cg, int groups, int seg0,
                                                 const float2* __restrict__ stats, const float2* __restrict__ part,
                                                 int nchunks, float eps, const float* __restrict__ gamma,
                                                 const float* __restrict__ beta) {
    constexpr int64_t CH = (int64_t)TPB * 4 * CV;  // floats per chunk
    const int seg = blockIdx.y, chunk = blockIdx.x;
    const int off = chunk * (int)CH;
    const f4* p = (const f4*)(x + (int64_t)seg * L + off);
    f4* q = (f4*)(y + (int64_t)seg * L + off);
    const int lane = threadIdx.x & 63;
    float2 st = make_float2(0.f, 0.f);
    if constexpr (MERGE) st = lane < nchunks ? part[(int64_t)seg * nchunks + lane] : make_float2(0.f, 0.f);
    else st = stats[seg];
    const int cnt = UNIFORM ? (int)CH : (int)(L - off < CH ? L - off : CH);
    const int n4 = cnt >> 2;
    const int gc = ((seg0 + seg) % groups) * cg;
    // chunks that cross channels: each float4's channel pair, loaded with
    // the chunk pairs ahead of the x loads (after the merge its latency
    // would follow the merge); a lane past the chunk reads the pair of the
    // chunk's last float4
    float gj[UNIFORM ? 1 : CV], bj[UNIFORM ? 1 : CV];
    if constexpr (!UNIFORM) {
#pragma unroll
        for (int j = 0; j < CV; ++j) {
            const int idx = min((int)threadIdx.x + TPB * j, n4 - 1);
            const int ch = gc + (int)((unsigned)(off + idx * 4) / (unsigned)HW);
            gj[j] = gamma[ch];
            bj[j] = beta[ch];
        }
    }
    // unconditional loads (a lane past the chunk re-reads its last float4):
    // loads under a mask split the kernel into blocks between which the
    // compiler shuffled the row through 200+ VGPRs. Ordinary loads, like
    // pass A's: the chunk is re-read from the caches (4a 14.80 against 14.92
    // us with non-temporal ones)
    f4 v[CV];
#pragma unroll
    for (int j = 0; j < CV; ++j) {
        const int idx = threadIdx.x + TPB * j;
        v[j] = p[UNIFORM ? idx : min(idx, n4 - 1)];
    }
    float meanf, rstd;
    if constexpr (MERGE) {
        const double tot = lane < nchunks ? (double)st.x : 0.0;
        const double mean = wave_dsum(tot) / (double)L;
        double m2t = 0.0;
        if (lane < nchunks) {
            const int64_t o = (int64_t)lane * CH;
            const double ni = (double)(L - o < CH ? L - o : CH);
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
    if constexpr (UNIFORM) {
        const int ch = gc + chunk / chunks_per_ch;
        const float a = rstd * gamma[ch];
        const float b = beta[ch] - meanf * a;
#pragma unroll
        for (int j = 0; j < CV; ++j) dev::st_stream(q + threadIdx.x + TPB * j, apply4<SILU>(v[j], a, b));
    } else {
#pragma unroll
        for (int j = 0; j < CV; ++j) {
            const int idx = threadIdx.x + TPB * j;
            if (idx < n4) {
                const float a = rstd * gj[j];
                const float b = bj[j] - meanf * a;
                dev::st_stream(q + idx, apply4<SILU>(v[j], a, b));
            }
        }
    }
}

// ---- resident schedule -------------------------------------------------------
// One launch of at most as many 1024-thread workgroups as the GPU holds at
// once (occupancy x CUs). A team of P consecutive workgroups owns one segment at a time
// (segments team, team + T, ...; T = teams), each workgroup a share of
// 4096 * V floats kept in registers: it loads its share once, publishes the
// share's (sum, M2 around the share mean), waits for its team's P pairs,
// merges them in double (the split schedule's finalize arithmetic, in the
// same fixed order in every workgroup of the team) and writes y from its
// registers. x is read once: two streams, the algorithmic minimum.
//
// Publication without fences: each value travels in one 64-bit agent-scope
// atomic store together with a 32-bit tag (round + 1), so a reader that sees
// the tag sees the value, and no device-scope release (which would write
// back the per-XCD L2s) is needed. Slots alternate between two parities by
// round: a workgroup's round r + 2 store, the next into round r's slot,
// follows its own wait for every teammate's round r + 1 value, which each
// teammate publishes only after its round r reads. The last workgroup to
// finish clears the slots and the finish counter, so every launch starts
// from zeroed slots and tags 1, 2, ... never match a stale value.
//
// Teams are formed by arrival, not by blockIdx: each workgroup takes a
// ticket (ctl[2]) when it starts and ticket / P is its team, ticket % P its
// share. Workgroups that have started hold tickets 0 .. k-1, so every team
// but the one holding ticket k-1 is complete and running, and at most one
// team per launch waits on members that are not yet on the GPU. Teams fixed
// by blockIdx could all be incomplete at once: the dispatcher fills each
// XCD in blockIdx order on its own, so when another process's kernel holds
// one XCD's CUs, every team with a member there waits, and two such
// launches can hold every slot. With tickets, a launch's complete teams
// always finish and free their CUs for the incomplete one. The ticket costs
// one atomic round trip before the first load (about 0.5 us at a 32 MB
// tensor, measured). (Not a cooperative launch: measured, a cooperative
// launch fails with hipErrorIllegalState in a second process while another
// process that made one is alive.) Each wait is still bounded (spin_limit
// polls): on expiry the workgroup sets ctl[1], writes NaN for its share and
// goes on, so the kernel always drains; the host reports ctl[1] at the next
// synchronisation, and from then on this process runs the split schedule
// instead (an in-place call, y == x, has then lost the expired shares of x).
constexpr int kResThreads = 1024;

constexpr int kResMaxTeam = 64;  // workgroups per segment per slot of a polling lane
constexpr int kCtlWords = 64;     // ctl[0] finished workgroups, ctl[1] error word, ctl[2] ticket; slots from ctl + 64
constexpr unsigned kSpinLimit = 1u << 20;  // polls of about 1 us: a wait ends within about a second

using u64 = unsigned long long;

__device__ __forceinline__ void put_slot(u64* s, float v, unsigned tag) {
    __hip_atomic_store(s, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 get_slot(const u64* s) {
    return __hip_atomic_load(s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct ResArgs {
    const float* x;
    float* y;
    const float* gamma;
    const float* beta;
    unsigned* ctl;  // ctl[0] finished workgroups, ctl[1] error word, ctl[2] ticket
    u64* slots;     // the team slots: [parity][workgroup] (sum, M2); uncached for scalar polls
    int L, HW, cg, groups, nseg, P;
    unsigned spin_limit;
    float eps;
};

// UNIFORM: every share is full and lies in one channel (HW % (4096 V) ==
// 0), so one (a, b) per workgroup.
// A share's loads go through a buffer descriptor that covers exactly the
// share's n4 float4 (x + base .. + 16 n4 bytes): one 32-bit offset register
// per lane instead of a 64-bit address per load (the two register buffers
// of the pipelined kernel leave no room for eight), and the descriptor's
// range check returns zeros for the lanes past a short share's end without
// a branch, and for a whole empty range without touching memory.
// Non-temporal, like the other streaming kernels.
//
// The stores stay ordinary global stores. Measured on MI355X: buffer stores
// issued while the wave's loads were still outstanding, with the compiler
// rewriting their offset registers right after them, wrote some lanes'
// values to the wrong place (lanes 12-15 of every row of 16 in some waves;
// correct once the stores waited for every load, or as global stores).
constexpr int kBufWord3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr int kNonTemporal = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t share_rsrc(const float* base, int n4) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, n4 * 16, kBufWord3);
}

template <int V, bool UNIFORM, int TPB = kResThreads>
__device__ __forceinline__ void res_load(f4 (&v)[V], const float* x, int64_t base, int n4) {
    const __amdgpu_buffer_rsrc_t r = share_rsrc(x + base, n4);
#pragma unroll
    for (int j = 0; j < V; ++j)
        v[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)threadIdx.x * 16, TPB * 16 * j,
                                                                           kNonTemporal));
}

// gamma[ch] or beta[ch] through a buffer load (ch uniform; range: ch + 1 floats).
__device__ __forceinline__ float coef_load(const float* v, int ch) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(v), (short)0, (ch + 1) * 4, kBufWord3);
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, ch * 4, 0, 0));
}


// The team's merge of this round's pairs, in wave 0: lane i holds parts i,
// i + 64, ... (KS per lane) as (sv, mv); the pairs merge in double in a
// fixed order (the split schedule's finalize arithmetic) into (mean, rstd)
// at *stat. timed_out: a wait expired; the statistics become NaN and the
// error word is set.
template <int KS>
__device__ __forceinline__ void res_merge(const ResArgs& a, const float (&sv)[KS], const float (&mv)[KS], int share,
                                          bool timed_out, float2* stat) {
    const int lane = threadIdx.x;
    double tot = 0.0;
#pragma unroll
    for (int k = 0; k < KS; ++k) tot += (double)sv[k];
    const double mean = wave_dsum(tot) / (double)a.L;
    double m2t = 0.0;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        const int i = lane + 64 * k;
        if (i < a.P) {
            const double ni = (double)min(share, a.L - i * share);
            const double dm = (double)sv[k] / ni - mean;
            m2t += (double)mv[k] + ni * dm * dm;
        }
    }
    const double m2s = wave_dsum(m2t);
    if (lane == 0) {
        float meanf = (float)mean, rstd = (float)(1.0 / sqrt(m2s / (double)a.L + (double)a.eps));
        if (timed_out) {
            __hip_atomic_store(a.ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            meanf = rstd = __builtin_nanf("");
        }
        *stat = make_float2(meanf, rstd);
    }
}

// Wave 0: waits for the team's pairs of this round with agent-scope vector
// loads (ts: part i's sum and M2 at ts[2 i], ts[2 i + 1]; lane i holds
// parts i, i + 64, ...) and merges them. These loads complete in order
// behind every vector load the wave issued before them.
template <int KS>
__device__ __forceinline__ void res_team_stats(const ResArgs& a, const u64* ts, unsigned tag, int share,
                                               float2* stat) {
    const int lane = threadIdx.x;
    float sv[KS], mv[KS];
    unsigned pending = 0;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        sv[k] = 0.f;
        mv[k] = 0.f;
        if (lane + 64 * k < a.P) pending |= 1u << k;
    }
    bool timed_out = false;
    for (unsigned it = 0;; ++it) {
        if (it >= a.spin_limit) {
            timed_out = true;
            break;
        }
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            if (pending & (1u << k)) {
                const u64* q = ts + (size_t)(lane + 64 * k) * 2;
                const u64 u = get_slot(q), w = get_slot(q + 1);
                if ((unsigned)(u >> 32) == tag && (unsigned)(w >> 32) == tag) {
                    sv[k] = __uint_as_float((unsigned)u);
                    mv[k] = __uint_as_float((unsigned)w);
                    pending &= ~(1u << k);
                }
            }
        }
        if (!__any(pending != 0)) break;
        __builtin_amdgcn_s_sleep(2);
    }
    res_merge<KS>(a, sv, mv, share, timed_out, stat);
}

typedef unsigned su16 __attribute__((ext_vector_type(16)));

// 8 tagged (sum, M2) pairs, 128 bytes at the uniform address p, by two
// scalar loads that miss the scalar cache. Scalar loads have their own
// queue and counter (lgkmcnt), so they do not wait behind the CU's
// outstanding vector loads.
__device__ __forceinline__ void sload_pairs8(const u64* p, su16& d0, su16& d1) {
    asm volatile(
        "s_load_dwordx16 %0, %2, 0x0 glc\n\t"
        "s_load_dwordx16 %1, %2, 0x40 glc\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(d0), "=&s"(d1)
        : "s"(p)
        : "memory");
}

// Every wave: the team's pairs of this round (layout as res_team_stats)
// through the scalar path, wave w polling parts 8 w .. 8 w + 7, into
// pairs[0 .. P) in LDS; an expired wait leaves NaN there and sets the error
// word. Needs the slots in uncached memory: the L2 keeps no copy of it, so
// a load that misses the scalar cache sees another XCD's latest store. The
// caller's barrier publishes pairs[].
__device__ __forceinline__ void res_gather_scalar(const ResArgs& a, const u64* ts, unsigned tag, float2* pairs) {
    // the wave index is uniform; readfirstlane lets the compiler keep the
    // poll address in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int np = min(8, a.P - 8 * wave);
    if (np <= 0) return;
    const u64* gp = ts + (size_t)wave * 16;
    su16 d0, d1;
    bool timed_out = false;
    for (unsigned it = 0;; ++it) {
        if (it >= a.spin_limit) {
            timed_out = true;
            break;
        }
        sload_pairs8(gp, d0, d1);
        bool ok = true;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const unsigned t0 = j < 4 ? d0[4 * j + 1] : d1[4 * (j - 4) + 1];
            const unsigned t1 = j < 4 ? d0[4 * j + 3] : d1[4 * (j - 4) + 3];
            if (j < np) ok = ok && t0 == tag && t1 == tag;
        }
        if (ok) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane < np) {
        unsigned sb = 0, mb = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const unsigned s0 = j < 4 ? d0[4 * j] : d1[4 * (j - 4)];
            const unsigned m0 = j < 4 ? d0[4 * j + 2] : d1[4 * (j - 4) + 2];
            sb = lane == j ? s0 : sb;
            mb = lane == j ? m0 : mb;
        }
        pairs[8 * wave + lane] = timed_out ? make_float2(__builtin_nanf(""), __builtin_nanf(""))
                                           : make_float2(__uint_as_float(sb), __uint_as_float(mb));
    }
    if (timed_out && lane == 0) __hip_atomic_store(a.ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One round of one workgroup: share statistics from registers, publication,
// (PREFETCH: the next round's loads into nxt, issued before the wait so
// they run under it; the caller passes a next segment that exists, so the
// loads are unconditional and the compiler can wait for this round's
// channel coefficients without waiting for them), the team wait, and y
// from registers. SPOLL: the wait reads the slots through the scalar path
// (res_gather_scalar), so neither the wait nor the stores after it queue
// behind the prefetch.
template <int V, bool SILU, bool UNIFORM, int KS, bool PREFETCH, bool SPOLL, int TPB = kResThreads>
__device__ __forceinline__ void res_round(const ResArgs& a, f4 (&cur)[V], f4 (&nxt)[V], int seg, int next_seg,
                                          int round, int team, int ticket, int off, int n4, float* sh,
                                          float2* stat, float2* pairs) {
    constexpr int kShare = TPB * V * 4;
    u64* slots = a.slots;
    const int G = (int)gridDim.x;
    const int gc = (seg % a.groups) * a.cg;
    // UNIFORM: the share's one channel coefficient pair, loaded ahead of the
    // prefetch so that waiting for it does not wait for the prefetch (the
    // compiler counts a wave's vector loads down in issue order), through
    // the same buffer path as the shares.
    float g_ch = 0.f, b_ch = 0.f;
    if constexpr (UNIFORM) {
        const int ch = gc + off / a.HW;
        g_ch = coef_load(a.gamma, ch);
        b_ch = coef_load(a.beta, ch);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += dev::hsum(cur[j]);  // masked entries are zero
    const float sum = block_sum<TPB>(s, sh);
    const float mc = sum / (float)(n4 * 4);
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int idx = threadIdx.x + TPB * j;
        if (UNIFORM || idx < n4) {
            const f4 d = cur[j] - mc;
            m2 += dev::hsum(d * d);
        }
    }
    const float M2 = block_sum<TPB>(m2, sh);
    const unsigned tag = (unsigned)round + 1;
    const int par = round & 1;
    // slots: [parity][ticket] (sum, M2); a team's parts are consecutive
    if (threadIdx.x == 0) {
        u64* mine = slots + ((size_t)par * G + ticket) * 2;
        put_slot(mine, sum, tag);
        put_slot(mine + 1, M2, tag);
    }
    if constexpr (PREFETCH) {
        // past the team's last segment: an empty range, so no memory access
        const bool more = next_seg < a.nseg;
        res_load<V, UNIFORM, TPB>(nxt, a.x, (int64_t)(more ? next_seg : seg) * a.L + off, more ? n4 : 0);
    }
    const u64* ts = slots + ((size_t)par * G + (size_t)team * a.P) * 2;
    if constexpr (SPOLL) {
        res_gather_scalar(a, ts, tag, pairs);
        __syncthreads();
        if (threadIdx.x < 64) {
            float sv[KS], mv[KS];
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const int i = threadIdx.x + 64 * k;
                const float2 pr = i < a.P ? pairs[i] : make_float2(0.f, 0.f);
                sv[k] = pr.x;
                mv[k] = pr.y;
            }
            res_merge<KS>(a, sv, mv, kShare, false, stat);  // an expiry left NaN pairs and set the word
        }
    } else {
        if (threadIdx.x < 64) res_team_stats<KS>(a, ts, tag, kShare, stat);
    }
    __syncthreads();
    const float meanf = stat->x, rstd = stat->y;
    f4* q = (f4*)(a.y + (int64_t)seg * a.L + off);
    if constexpr (UNIFORM) {
        const float ca = rstd * g_ch;
        const float cb = b_ch - meanf * ca;
#pragma unroll
        for (int j = 0; j < V; ++j) dev::st_stream(q + threadIdx.x + TPB * j, apply4<SILU>(cur[j], ca, cb));
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int idx = threadIdx.x + TPB * j;
            if (idx < n4) {
                const int ch = gc + (int)((unsigned)(off + idx * 4) / (unsigned)a.HW);
                const float ca = rstd * a.gamma[ch];
                const float cb = a.beta[ch] - meanf * ca;
                dev::st_stream(q + idx, apply4<SILU>(cur[j], ca, cb));
            }
        }
    }
}

// Every workgroup has taken its ticket and finished its reads of the slots
// before it counts itself finished; the last one clears the slots of this
// launch, the ticket and the counter.
__device__ __forceinline__ void res_finish(unsigned* ctl, u64* slots, unsigned* last) {
    if (threadIdx.x == 0)
        *last = __hip_atomic_fetch_add(ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (*last) {
        for (unsigned i = threadIdx.x; i < gridDim.x * 4; i += blockDim.x)
            __hip_atomic_store(slots + i, (u64)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x == 0 || threadIdx.x == 2)
            __hip_atomic_store(ctl + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// This workgroup's ticket: its place in arrival order (see above).
__device__ __forceinline__ int res_ticket(unsigned* ctl, int* sh_ticket) {
    if (threadIdx.x == 0)
        *sh_ticket = (int)__hip_atomic_fetch_add(ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return *sh_ticket;
}

// grid = T * P workgroups of kResThreads; segments team, team + T, ... one
// round each; P <= 64.
template <int V, bool SILU, bool UNIFORM, bool SPOLL>
__global__ __launch_bounds__(kResThreads) void k_gn_resident(ResArgs a) {
    constexpr int kShare4 = kResThreads * V;
    __shared__ float sh[kResThreads / 64];
    __shared__ float2 stat;
    __shared__ float2 pairs[SPOLL ? kResMaxTeam : 1];
    __shared__ unsigned last;
    __shared__ int sh_ticket;
    const int ticket = __builtin_amdgcn_readfirstlane(res_ticket(a.ctl, &sh_ticket));
    const int team = ticket / a.P, part = ticket - team * a.P, T = gridDim.x / a.P;
    const int off = part * kShare4 * 4;
    const int n4 = UNIFORM ? kShare4 : min(kShare4, (a.L - off) >> 2);
    int round = 0;
    for (int seg = team; seg < a.nseg; seg += T, ++round) {
        f4 v[V];
        res_load<V, UNIFORM>(v, a.x, (int64_t)seg * a.L + off, n4);
        res_round<V, SILU, UNIFORM, 1, false, SPOLL>(a, v, v, seg, 0, round, team, ticket, off, n4, sh, &stat,
                                                     pairs);
    }
    res_finish(a.ctl, a.slots, &last);
}

// The same schedule software-pipelined over two register buffers: round
// r + 1's share is loaded while round r waits for its team, so the waits
// (and the share reductions) overlap HBM traffic. P <= 128 (two slots per
// polling lane). A team's last round prefetches through an empty buffer
// range (no memory access), so every prefetch is issued unconditionally.
template <int V, bool SILU, bool UNIFORM, bool SPOLL>
__global__ __launch_bounds__(kResThreads) void k_gn_resident_pipe(ResArgs a) {
    constexpr int kShare4 = kResThreads * V;
    __shared__ float sh[kResThreads / 64];
    __shared__ float2 stat;
    __shared__ float2 pairs[SPOLL ? 2 * kResMaxTeam : 1];
    __shared__ unsigned last;
    __shared__ int sh_ticket;
    const int ticket = __builtin_amdgcn_readfirstlane(res_ticket(a.ctl, &sh_ticket));
    const int team = ticket / a.P, part = ticket - team * a.P, T = gridDim.x / a.P;
    const int off = part * kShare4 * 4;
    const int n4 = UNIFORM ? kShare4 : min(kShare4, (a.L - off) >> 2);
    f4 va[V], vb[V];
    int seg = team;
    if (seg < a.nseg) res_load<V, UNIFORM>(va, a.x, (int64_t)seg * a.L + off, n4);
    for (int round = 0; seg < a.nseg; round += 2) {
        const int s1 = seg + T;
        res_round<V, SILU, UNIFORM, 2, true, SPOLL>(a, va, vb, seg, s1, round, team, ticket, off, n4, sh, &stat,
                                                    pairs);
        if (s1 >= a.nseg) break;
        const int s2 = s1 + T;
        res_round<V, SILU, UNIFORM, 2, true, SPOLL>(a, vb, va, s1, s2, round + 1, team, ticket, off, n4, sh, &stat,
                                                    pairs);
        seg = s2;
    }
    res_finish(a.ctl, a.slots, &last);
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

// ---- pipelined schedule --------------------------------------------------------
// Segments that are whole 4096-float chunks lying in one channel (HW % 4096
// == 0, at most 64 chunks per segment), any tensor size: the split
// schedule's two passes in ONE launch (per kPipeMaxChunks chunks). Workgroups come in units of gsz
// segments: a stats unit (one workgroup per chunk: the chunk's sum and M2
// around its mean, published as two tagged 64-bit words) and, later in
// blockIdx order, the same segments' apply unit (merges the segment's pairs
// in double in chunk order, then y = silu(x a + b) for its chunk). The order
// is S(0) .. S(lag-1), then S(g + lag), A(g) alternating, then the last A
// units: with lag units of stats ahead of each apply unit, about one round
// of resident workgroups, an apply workgroup is dispatched when a stats
// workgroup of the round before ends, by which time its segment's pairs are
// out, and it re-reads its chunk from the caches while later chunks stream
// in from HBM. Reads and writes overlap as in a copy, where the split
// schedule's second pass starts only after its first has drained. Dynamic
// LDS the kernel never touches holds the GPU to kPipeOcc workgroups per CU:
// with more, apply workgroups dispatched beside their own stats workgroups
// wait, and re-read x from HBM. Measured at config 4a ([1,512,128,128]): 6
// per CU 12.1-12.3 us, 5 per CU 12.8, 7 per CU 13.3-14.9, the split schedule
// 14.4-14.8; lag 4 / 5 / 6 / 7 units of 256 chunks: 13.1 / 12.4 / 12.2-12.5 /
// 13.0 us. Larger tensors keep the re-read distance (lag units) and so the
// cache hits: [4,512,128,128] 46.8 us against 53.5 (split), [8,512,128,128]
// 90.7 against 97.1 (resident). Longer segments were tried with a finalize
// workgroup per segment between the stats and apply units and measured
// slower than the resident schedule ([1,128,512,512] 66 against 50 us,
// [1,128,1024,1024] 272 against 183), so they are not taken here.
//
// Tags. Every launch tags its pairs with a value no earlier launch used, so
// pairs left by earlier launches never match: a direct call takes the next
// value of a host counter (1 .. 2^31 - 1; the pairs are cleared when it
// wraps), passed as an argument. A captured call's arguments are replayed
// unchanged, so its tag is 2^31 + 64 E + k: E a device counter that a
// one-workgroup kernel advances before the first pipelined call of each
// capture (and before every 64th), k the call's place among them. Each
// replay thus advances E once per 64 calls. (A counter advanced within the
// launch itself would need every workgroup to have read it before it moves:
// a word per workgroup and one reader of them all, measured 2.4 us more at
// 4a; an atomic load or store per workgroup alone costs 0.6 us; the separate
// kernel costs about 2 us per replay.)
//
// Waits. An apply workgroup's wave 0 polls the segment's pairs (one pair
// per lane). When x and y do not overlap, a pair still missing after
// `polls` polls is computed by the apply workgroup itself from x, with the
// same function the stats workgroup uses (pipe_pair), so the bits are the
// same; no apply workgroup then waits on another for long, whatever order
// the dispatcher or another process's work imposes. In place (y == x) the
// chunk may already be overwritten, so the wait is bounded (polls) and on
// expiry the workgroup writes NaN and sets ctl[1], which the host reports at
// the next synchronisation (and then leaves this schedule for the rest of
// the process), as for the resident schedule.
constexpr int kPipeTPB = 256, kPipeCV = 4;
constexpr int kPipeChunk = kPipeTPB * 4 * kPipeCV;  // 4096 floats
constexpr int kPipeOcc = 6;                         // workgroups per CU
constexpr unsigned kPipePolls = 256;                // polls before a missing pair is computed here
constexpr int kPipeUnitChunks = 256;                // chunks per unit, at most

struct PipeArgs {
    const float* x;
    float* y;
    const float* gamma;
    const float* beta;
    u64* slots;          // [segment][chunk][sum, M2], tagged
    unsigned* ctl;       // ctl[0] captured launches' counter, ctl[1] error word
    unsigned tag;        // this launch's tag, or 0: 2^31 + 64 ctl[0] + k (captured)
    unsigned k;          // a captured call's place among those sharing ctl[0]
    int L, HW, cg, groups, seg0, cps, gsz, ngroups, lag;  // seg0: the group of the launch's first segment
    unsigned polls;      // polls before a missing pair is computed here (in place: before the wait fails)
    int selfhelp;        // x and y do not overlap
    float eps;
};

// Before the first of up to 64 captured launches: advances the counter their
// tags are formed from.
__global__ void k_gn_pipe_epoch(unsigned* ctl) {
    if (threadIdx.x == 0) ctl[0] = (ctl[0] + 1u) & 0x1ffffffu;
}

// A chunk's float4 for this thread (t + 256 j), and its (sum, M2 around the
// chunk mean). Stats workgroups and apply workgroups computing a missing
// pair both use these, so a pair has the same bits whoever forms it.
__device__ __forceinline__ void pipe_load(const float* c, f4 (&v)[kPipeCV]) {
    const f4* p = (const f4*)c;
#pragma unroll
    for (int j = 0; j < kPipeCV; ++j) v[j] = p[threadIdx.x + kPipeTPB * j];
}
// The chunk's (sum, M2) in one reduction: each thread forms the mean and M2
// of its 16 floats from registers, then pairs of equal counts merge, over
// shuffles within a wave (M2 = M2_a + M2_b + (mean_b - mean_a)^2 n / 2, n
// floats on each side; every lane gets the same bits: the sums commute) and
// through LDS across the four waves. One barrier pair instead of the two of
// a sum and then a sum of squares around it (4a: 11.9-12.1 against
// 12.3-12.4 us, interleaved; the DPP tree of block_sum measured 0.3 us slower
// again).
__device__ __forceinline__ void pipe_pair(const f4 (&v)[kPipeCV], float* sh, float& sum, float& m2) {
    static_assert(kPipeTPB == 256, "four waves");
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kPipeCV; ++j) s += dev::hsum(v[j]);
    float m = s * (1.f / (4 * kPipeCV));
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < kPipeCV; ++j) q += dev::sumsq4(v[j] - m);
    float n = 4.f * kPipeCV;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float mo = __shfl_xor(m, o, 64), qo = __shfl_xor(q, o, 64);
        const float d = mo - m;
        m = (m + mo) * 0.5f;
        q = (q + qo) + d * d * (n * 0.5f);
        n *= 2.f;
    }
    __syncthreads();  // sh may still be read by the previous pair
    if ((threadIdx.x & 63) == 0) {
        sh[(threadIdx.x >> 6) * 2] = m;
        sh[(threadIdx.x >> 6) * 2 + 1] = q;
    }
    __syncthreads();
    const float h = 64.f * 4 * kPipeCV * 0.5f;  // floats a wave holds, halved
    const float d01 = sh[2] - sh[0], d23 = sh[6] - sh[4];
    const float m01 = (sh[0] + sh[2]) * 0.5f, m23 = (sh[4] + sh[6]) * 0.5f;
    const float q01 = (sh[1] + sh[3]) + d01 * d01 * h, q23 = (sh[5] + sh[7]) + d23 * d23 * h;
    const float d = m23 - m01;
    sum = (m01 + m23) * 0.5f * (float)kPipeChunk;
    m2 = (q01 + q23) + d * d * (h * 2.f);
}

template <bool SILU>
__global__ __launch_bounds__(kPipeTPB) void k_gn_pipe(PipeArgs a) {
    __shared__ float sh[2 * kPipeTPB / 64];
    __shared__ float fix[2][64];
    __shared__ float stat[2];
    __shared__ unsigned long long miss;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    // the kernel before a captured launch wrote ctl[0]; kernel boundaries make it visible
    const unsigned tag = a.tag ? a.tag : 0x80000000u | (*(volatile const unsigned*)a.ctl << 6) | a.k;
    // unit u of the order S(0) .. S(lg-1), {S(g + lg), A(g)} ..., A(ngroups-lg) .. A(ngroups-1)
    const int per = a.gsz * a.cps;
    const int u = (int)blockIdx.x / per, r = (int)blockIdx.x - u * per;
    const int lg = min(a.lag, a.ngroups), mid = lg + 2 * (a.ngroups - lg);
    bool apply;
    int grp;
    if (u < lg) {
        apply = false;
        grp = u;
    } else if (u < mid) {
        const int k = u - lg;
        apply = k & 1;
        grp = (k >> 1) + (apply ? 0 : lg);
    } else {
        apply = true;
        grp = a.ngroups - lg + (u - mid);
    }
    const int sseg = r / a.cps, chunk = r - sseg * a.cps, seg = grp * a.gsz + sseg;
    const float* xs = a.x + (int64_t)seg * a.L;
    u64* sl = a.slots + (int64_t)seg * a.cps * 2;
    f4 v[kPipeCV];
    if (!apply) {
        pipe_load(xs + (int64_t)chunk * kPipeChunk, v);
        float s, q;
        pipe_pair(v, sh, s, q);
        if (threadIdx.x == 0) {
            put_slot(sl + 2 * chunk, s, tag);
            put_slot(sl + 2 * chunk + 1, q, tag);
        }
        return;
    }
    u64 ps = 0, pm = 0;
    if (w == 0 && lane < a.cps) {
        ps = get_slot(sl + 2 * lane);
        pm = get_slot(sl + 2 * lane + 1);
    }
    {
        const f4* p = (const f4*)(xs + (int64_t)chunk * kPipeChunk);
#pragma unroll
        for (int j = 0; j < kPipeCV; ++j) v[j] = dev::ld_stream(p + threadIdx.x + kPipeTPB * j);
    }
    if (w == 0) {
        auto missing = [&] {
            return __ballot(lane < a.cps && ((unsigned)(ps >> 32) != tag || (unsigned)(pm >> 32) != tag));
        };
        u64 m = missing();
        for (unsigned n = 0; m && n < a.polls; ++n) {
            __builtin_amdgcn_s_sleep(2);
            if (lane < a.cps) {
                ps = get_slot(sl + 2 * lane);
                pm = get_slot(sl + 2 * lane + 1);
            }
            m = missing();
        }
        if (lane == 0) miss = m;
    }
    __syncthreads();
    const u64 m = miss;
    bool failed = false;
    if (m) {
        if (a.selfhelp) {
            for (u64 mm = m; mm; mm &= mm - 1) {
                const int c = __builtin_ctzll(mm);
                f4 vc[kPipeCV];
                pipe_load(xs + (int64_t)c * kPipeChunk, vc);
                float s, q;
                pipe_pair(vc, sh, s, q);
                if (threadIdx.x == 0) {
                    fix[0][c] = s;
                    fix[1][c] = q;
                }
            }
            __syncthreads();
        } else {
            failed = true;
            if (threadIdx.x == 0) __hip_atomic_store(a.ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (w == 0) {
        // k_gn_finalize's merge, one pair per lane
        float s = 0.f, q = 0.f;
        if (lane < a.cps) {
            const bool f = (m >> lane) & 1;
            s = f ? fix[0][lane] : __uint_as_float((unsigned)ps);
            q = f ? fix[1][lane] : __uint_as_float((unsigned)pm);
        }
        const double mean = wave_dsum(lane < a.cps ? (double)s : 0.0) / (double)a.L;
        double m2t = 0.0;
        if (lane < a.cps) {
            const double dm = (double)s / (double)kPipeChunk - mean;
            m2t = (double)q + (double)kPipeChunk * dm * dm;
        }
        const double m2 = wave_dsum(m2t);
        if (lane == 0) {
            stat[0] = (float)mean;
            stat[1] = failed ? __builtin_nanf("") : (float)(1.0 / sqrt(m2 / (double)a.L + (double)a.eps));
        }
    }
    __syncthreads();
    const float meanf = stat[0], rstd = stat[1];
    const int ch = ((a.seg0 + seg) % a.groups) * a.cg + (chunk * kPipeChunk) / a.HW;
    const float ga = rstd * a.gamma[ch];
    const float gb = a.beta[ch] - meanf * ga;
    f4* q = (f4*)(a.y + (int64_t)seg * a.L + (int64_t)chunk * kPipeChunk);
#pragma unroll
    for (int j = 0; j < kPipeCV; ++j) dev::st_stream(q + threadIdx.x + kPipeTPB * j, apply4<SILU>(v[j], ga, gb));
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

long env_long(const char* name, long dflt) {
    const char* e = std::getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    const long v = std::strtol(e, &end, 10);
    return (end && *end == 0 && v >= 0) ? v : dflt;
}

// The split schedule's chunk for nseg segments of L floats: the largest of
// 8192, 4096 and 2048 floats that still gives 768 workgroups per pass, else
// 2048. Measured (graph replays, GroupNorm + SiLU, 32 groups), chunk 8192
// against the one chosen: [2,320,64,64] 9.6 vs 8.6 us (2048),
// [2,640,64,64] 12.3 vs 11.8 us (4096), [2,1280,32,32] 9.5 vs 9.3 us (2048);
// [1,512,120,120] keeps 8192 (928 workgroups): 14.6 us, against 16.7 with
// 4096. SDH_GN_CHUNK forces one of them.
int64_t split_chunk(int64_t nseg, int64_t L) {
    static const long force = env_long("SDH_GN_CHUNK", 0);
    if (force == 2048 || force == 4096 || force == 8192) return force;
    for (int64_t c : {int64_t(8192), int64_t(4096)})
        if (nseg * ((L + c - 1) / c) >= 768) return c;
    return 2048;
}

// One resident kernel: pipelined or not, V float4 per thread.
struct ResKind {
    bool pipe;
    int V;
};

// Calls f with the instantiation for (kind, silu, uniform, spoll).
// Instantiated: k_gn_resident V = 4, 8, 16 (16 only uniform: the per-vector
// channel lookup would spill) and k_gn_resident_pipe V = 4, 8; each with
// scalar (spoll) or vector polls.
template <class F>
void with_resident(ResKind k, bool silu, bool uniform, bool spoll, F&& f) {
    auto go = [&](auto vc, auto pc, auto sc) {
        constexpr int VV = decltype(vc)::value;
        constexpr bool PP = decltype(pc)::value;
        constexpr bool SP = decltype(sc)::value;
        if constexpr (PP) {
            if (silu) uniform ? f(k_gn_resident_pipe<VV, true, true, SP>) : f(k_gn_resident_pipe<VV, true, false, SP>);
            else uniform ? f(k_gn_resident_pipe<VV, false, true, SP>) : f(k_gn_resident_pipe<VV, false, false, SP>);
        } else if constexpr (VV == 16) {
            if (silu) f(k_gn_resident<16, true, true, SP>);
            else f(k_gn_resident<16, false, true, SP>);
        } else {
            if (silu) uniform ? f(k_gn_resident<VV, true, true, SP>) : f(k_gn_resident<VV, true, false, SP>);
            else uniform ? f(k_gn_resident<VV, false, true, SP>) : f(k_gn_resident<VV, false, false, SP>);
        }
    };
    auto go2 = [&](auto vc, auto pc) {
        if (spoll) go(vc, pc, std::true_type());
        else go(vc, pc, std::false_type());
    };
    using P1 = std::true_type;
    using P0 = std::false_type;
    if (k.V == 4) k.pipe ? go2(std::integral_constant<int, 4>(), P1()) : go2(std::integral_constant<int, 4>(), P0());
    else if (k.V == 8) k.pipe ? go2(std::integral_constant<int, 8>(), P1()) : go2(std::integral_constant<int, 8>(), P0());
    else if (k.V == 16 && !k.pipe && uniform) go2(std::integral_constant<int, 16>(), P0());
    else fail(SDH_ERR_INVALID, "k_gn_resident: no such instantiation");
}

bool instantiated(ResKind k, bool uniform) { return k.pipe ? (k.V == 4 || k.V == 8) : (k.V != 16 || uniform); }

// Resident workgroups per CU of one instantiation (0 if none); cached (calls
// are serialised by the op lock).
int resident_occupancy(ResKind k, bool silu, bool uniform, bool spoll = false) {
    static int cache[2][3][2][2][2];
    static bool filled = false;
    if (!filled) {
        for (auto& a : cache)
            for (auto& b : a)
                for (auto& c : b)
                    for (auto& d : c)
                        for (int& e : d) e = -1;
        filled = true;
    }
    if (!instantiated(k, uniform)) return 0;
    int& c = cache[k.pipe][k.V == 4 ? 0 : k.V == 8 ? 1 : 2][silu][uniform][spoll];
    if (c < 0) {
        c = 0;
        with_resident(k, silu, uniform, spoll, [&](auto kern) {
            int nb = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), kResThreads, 0) ==
                hipSuccess)
                c = nb;
            else
                (void)hipGetLastError();
        });
    }
    return c;
}

// The resident schedule for segments of L floats (HW % 4 == 0, 16-byte
// aligned, L < 2^31), when it is expected to beat the split schedule
// (measured on MI355X, GroupNorm + SiLU, 32 groups): x of at least 64 MB,
// where the split schedule's re-read comes from HBM; the
// k_gn_resident_pipe plan with the fewest rounds (smaller share on ties;
// else k_gn_resident's), e.g. [1,128,1024,1024] 247 -> 181 us,
// [1,256,256,256] 29.6 -> 25.8 us. Below 64 MB the split schedule with
// chunks sized to the tensor (split_chunk) measured as fast or faster than
// one resident round, which an earlier, slower split took: [2,320,64,64]
// 10.9 -> 8.6 us, [2,640,64,64] 14.1 -> 11.8 us, [2,1280,32,32] 10.7 -> 9.3
// us, [2,960,32,32] 9.5 -> 8.2 us (graph replays); [2,1280,64,64] (84 MB)
// 18.4 resident against 18.5 split.
// False: use the split schedule. Knobs for tests and tuning:
// SDH_GN_RESIDENT=0 never, =2 always when a plan exists (one round for
// segments of 24577-65536 floats, else the plan chosen as for large x);
// SDH_GN_RESIDENT_V=4|8|16 fixes the share;
// SDH_GN_RESIDENT_PIPE=0|1 allows only the plain or only the pipelined
// kernel; SDH_GN_ONE_ROUND_PIPE=0 keeps the plain kernel's plan for one
// round (the pipelined plan measured 2-7 % faster there: [2,640,64,64]
// 12.65 -> 11.9 us, [2,320,64,64] 9.31 -> 9.09 us); SDH_GN_SPIN_LIMIT
// bounds each wait (polls; 0 expires every wait at once).
// Set when a resident launch's bounded wait expired (the host learns it at
// the next synchronisation): later calls in this process take the other
// schedules, which never wait across workgroups.
bool g_resident_off = false;
void resident_expired() { g_resident_off = true; }

// fixed: the allocation-free entry point's scratch (slots and counters at
// its start), or null for the library's counters.
bool run_gn_resident(const char* op, bool silu, const float* x, float* y, int64_t L, int64_t HW, int64_t cg,
                     int groups, int64_t nseg, const float* gamma, const float* beta, float eps,
                     bool one_round_only, unsigned char* fixed) {
    if (g_resident_off) return false;
    static const long mode = env_long("SDH_GN_RESIDENT", 1);
    static const long force_v = env_long("SDH_GN_RESIDENT_V", 0);
    static const long force_pipe = env_long("SDH_GN_RESIDENT_PIPE", -1);
    static const unsigned spin = (unsigned)std::min<long>(env_long("SDH_GN_SPIN_LIMIT", kSpinLimit), 0x7fffffffL);
    static const bool scalar_poll = env_long("SDH_GN_SCALAR_POLL", 1) != 0;
    if (mode == 0 || nseg > 0x7fffffffLL) return false;
    struct Plan {
        ResKind k{false, 0};
        int64_t P = 0, T = 0, rounds = INT64_MAX;
    };
    Plan best_pipe, best_plain, best_one;
    for (bool pipe : {false, true}) {
        if (force_pipe >= 0 && pipe != (force_pipe != 0)) continue;
        for (int V : {4, 8, 16}) {
            if (force_v && V != force_v) continue;
            const int64_t share = (int64_t)kResThreads * 4 * V;
            const int64_t P = (L + share - 1) / share;
            if (P > (pipe ? 2 : 1) * kResMaxTeam) continue;
            const ResKind k{pipe, V};
            const int64_t T = (int64_t)resident_occupancy(k, silu, HW % share == 0) * num_cus() / P;
            if (T == 0) continue;
            const Plan pl{k, P, T, (nseg + T - 1) / T};
            Plan& slot = pipe ? best_pipe : best_plain;
            if (pl.rounds < slot.rounds) slot = pl;
            if (!pipe && pl.rounds == 1 && !best_one.k.V) best_one = pl;
        }
    }
    const bool large = nseg * L * 4 >= (int64_t(64) << 20);
    // one round: the pipelined kernel's plan when it also covers the tensor
    // in one round (shares of 8 float4 where the plain one has 4: fewer
    // workgroups, each holding more in flight), else the plain kernel's
    if (best_pipe.k.V && best_pipe.rounds == 1 && env_long("SDH_GN_ONE_ROUND_PIPE", 1)) best_one = best_pipe;
    Plan pl;
    if (one_round_only) {
        if (best_one.k.V && mode == 2) pl = best_one;
    } else if (large || mode == 2) pl = best_pipe.k.V ? best_pipe : best_plain;
    if (!pl.k.V) return false;
    const bool uniform = HW % ((int64_t)kResThreads * 4 * pl.k.V) == 0;
    const int64_t grid = std::min(pl.T, nseg) * pl.P;
    ResArgs args{x, y, gamma, beta, nullptr, nullptr, (int)L, (int)HW, (int)cg, groups, (int)nseg, (int)pl.P,
                 spin, eps};
    const size_t ctl_words = (size_t)kCtlWords + (size_t)grid * 8;
    // scalar polls (plans of several rounds) need the slots in the library's
    // uncached words (the last poll of a team reads up to 7 parts past its
    // own: 32 words of slack); the allocation-free entry point's fixed
    // scratch is ordinary memory, so it keeps the vector polls.
    // SDH_GN_SCALAR_POLL=0 turns the scalar polls off.
    bool spoll = false;
    if (fixed) {
        if (ctl_words * sizeof(unsigned) > kFixedCtlBytes)
            fail(SDH_ERR_INVALID, std::string(op) + ": " + std::to_string(grid) +
                                      " resident workgroups need more team slots than the fixed scratch holds");
        args.ctl = (unsigned*)fixed;  // zero at set-up; every launch leaves it zero when it ends
        args.slots = (u64*)(args.ctl + kCtlWords);
    } else {
        // the counters (ticket, finish, error word) in ordinary memory: an
        // atomic on uncached memory goes to the memory controller, and one
        // per workgroup on one word serialises there
        args.ctl = counters(ctl_words);
        args.slots = (u64*)(args.ctl + kCtlWords);
        // plans are made with the vector-poll kernels' occupancy; the scalar
        // one must hold as many workgroups per CU (its grid is the same)
        if (scalar_poll && pl.rounds > 1 &&
            resident_occupancy(pl.k, silu, uniform, true) >= resident_occupancy(pl.k, silu, uniform)) {
            // one round has no prefetch for the wait to pass: the vector
            // poll, without the scalar path's extra barrier, measured faster
            if (unsigned* w = uncached_words((size_t)grid * 8 + 32)) {
                args.slots = (u64*)w;
                spoll = true;
            }
        }
    }
    void* argv[] = {&args};
    with_resident(pl.k, silu, uniform, spoll, [&](auto kern) {
        const std::string what = std::string(op) + ": launch of " + std::to_string(grid) + " resident workgroups (" +
                                 (pl.k.pipe ? "pipelined, " : "") + (spoll ? "scalar polls, " : "") + "V " +
                                 std::to_string(pl.k.V) + ", " +
                                 std::to_string(resident_occupancy(pl.k, silu, uniform, spoll)) + " per CU)";
        hip_check(hipLaunchKernel(reinterpret_cast<const void*>(kern), dim3((unsigned)grid), dim3(kResThreads), argv,
                                  0, stream()),
                  what.c_str());
    });
    arm_device_check(args.ctl + 1, op, resident_expired);
    return true;
}

// Set when a pipelined launch's bounded wait expired (in place only): later
// calls in this process take the other schedules.
bool g_pipe_off = false;
void pipe_expired() { g_pipe_off = true; }

// Dynamic LDS that holds k_gn_pipe to kPipeOcc workgroups per CU (0: its
// natural occupancy is already at most that), or -1 when it fits fewer than
// four (the schedule is then not used); cached.
int pipe_lds_bytes(bool silu) {
    static int cache[2] = {-2, -2};
    static const int occ_want = (int)std::max<long>(1, std::min<long>(env_long("SDH_GN_PIPE_OCC", kPipeOcc), 16));
    int& c = cache[silu];
    if (c == -2) {
        c = -1;
        int dev = 0, lds = 0;
        const void* k = silu ? reinterpret_cast<const void*>(k_gn_pipe<true>) : reinterpret_cast<const void*>(k_gn_pipe<false>);
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) == hipSuccess &&
            lds > 0) {
            for (int dyn = 0; dyn <= lds; dyn += 256) {
                int n = 0;
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kPipeTPB, (size_t)dyn) != hipSuccess) break;
                if (n <= occ_want) {
                    if (n >= std::min(4, occ_want)) c = dyn;
                    break;
                }
                if (dyn == 0) dyn = (lds / (occ_want + 1)) & ~255;  // skip ahead; the loop adds 256
            }
        }
        (void)hipGetLastError();
    }
    return c;
}

bool run_gn_pipe(const char* op, bool silu, const float* x, float* y, int64_t L, int64_t HW, int64_t cg, int groups,
                 int64_t nseg, const float* gamma, const float* beta, float eps) {
    static const bool on = env_long("SDH_GN_PIPE", 1) != 0;
    static const long resident_mode = env_long("SDH_GN_RESIDENT", 1);
    static const unsigned spin = (unsigned)std::min<long>(env_long("SDH_GN_SPIN_LIMIT", kSpinLimit), 0x7fffffffL);
    if (!on || g_pipe_off || resident_mode == 2 || gn_block_bytes() != 0) return false;
    if (HW % kPipeChunk != 0 || L % kPipeChunk != 0) return false;
    const int64_t cps = L / kPipeChunk;
    // segments of more than 64 chunks: the resident or split schedule
    if (cps < 1 || cps > 64) return false;
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    u64* area = dev >= 0 && dev < kMaxDevices ? g_pipe_area[dev] : nullptr;
    if (!area) return false;
    const int dyn = pipe_lds_bytes(silu);
    if (dyn < 0) return false;
    int occ = 0;
    const void* kern = silu ? reinterpret_cast<const void*>(k_gn_pipe<true>) : reinterpret_cast<const void*>(k_gn_pipe<false>);
    hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, kPipeTPB, (size_t)dyn), "occupancy");
    const int64_t rounds = (int64_t)std::max(occ, 1) * num_cus();
    static const long force_lag = env_long("SDH_GN_PIPE_LAG", 0);
    const size_t bytes = (size_t)(nseg * L) * 4;
    const uintptr_t xa = (uintptr_t)x, ya = (uintptr_t)y;
    const bool disjoint = xa + bytes <= ya || ya + bytes <= xa;
    unsigned* ctl = (unsigned*)(area + 2 * kPipeMaxChunks);
    // segments per launch: as many as the exchange area holds
    const int64_t sb_max = kPipeMaxChunks / cps;
    for (int64_t s0 = 0; s0 < nseg; s0 += sb_max) {
        const int64_t sb = std::min(sb_max, nseg - s0);
        // units: the most segments whose chunks stay within kPipeUnitChunks;
        // lag: about one round of resident workgroups, in units
        int64_t gsz = 1;
        for (int64_t d = 2; d <= sb && d * cps <= kPipeUnitChunks; ++d)
            if (sb % d == 0) gsz = d;
        const int64_t unit = gsz * cps, ngroups = sb / gsz;
        const int64_t lag = force_lag > 0 ? force_lag : std::max<int64_t>(1, (rounds + unit / 2) / unit);
        unsigned tag = 0, k = 0;
        if (capturing()) {
            const unsigned gen = capture_generation();
            if (g_pipe_cap_gen[dev] != gen) {
                g_pipe_cap_gen[dev] = gen;
                g_pipe_cap_calls[dev] = 0;
            }
            k = g_pipe_cap_calls[dev]++ % 64;
            if (k == 0) {
                k_gn_pipe_epoch<<<1, 64, 0, stream()>>>(ctl);
                launched(op);
            }
        } else {
            unsigned& t = g_pipe_tag[dev];
            if (t == 0x7fffffffu) {  // every tag used: no pair may match a reused one
                zero_device(area, 2 * kPipeMaxChunks * sizeof(u64));
                t = 0;
            }
            tag = ++t;
        }
        PipeArgs args{x + s0 * L, y + s0 * L, gamma, beta, area, ctl, tag, k, (int)L, (int)HW, (int)cg, groups,
                      (int)(s0 % groups), (int)cps, (int)gsz, (int)ngroups, (int)std::min<int64_t>(lag, ngroups),
                      disjoint ? std::min(kPipePolls, spin) : spin, disjoint ? 1 : 0, eps};
        const unsigned grid = (unsigned)(2 * sb * cps);
        void* argv[] = {&args};
        hip_check(hipLaunchKernel(kern, dim3(grid), dim3(kPipeTPB), argv, (size_t)dyn, stream()),
                  (std::string(op) + ": pipelined launch of " + std::to_string(grid) + " workgroups").c_str());
        if (s0 + sb < nseg) launched(op);
    }
    arm_device_check(ctl + 1, op, pipe_expired);
    return true;
}

// fixed: the allocation-free entry point's scratch, or null for the
// library's scratch and counters (which may allocate from the arena).
void run_gn(const char* op, bool silu, const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups,
            const float* gamma, const float* beta, float eps, unsigned char* fixed = nullptr) {
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
            run_gn(op, silu, x + n0 * C * HW, y + n0 * C * HW, nn, C, HW, groups, gamma, beta, eps, fixed);
        });
        return;
    }
    const int64_t cg = C / groups, L = cg * HW, nseg = N * groups;
    const bool vec = HW % 4 == 0 && aligned16(x) && aligned16(y) && L < (1LL << 31);
    static const bool force_split = env_long("SDH_GN_SPLIT", 0) != 0;
    // segments of 24577-65536 floats: one resident round only when forced
    // (SDH_GN_RESIDENT=2); the split schedule otherwise
    if (!force_split && vec && L > kSmallResidentMin && L <= (int64_t)1024 * 4 * 16 && gn_block_bytes() == 0 &&
        run_gn_resident(op, silu, x, y, L, HW, cg, groups, nseg, gamma, beta, eps, true, fixed))
        return;
    if (!force_split && vec && L > kSmallResidentMin &&
        run_gn_pipe(op, silu, x, y, L, HW, cg, groups, nseg, gamma, beta, eps)) {
        launched(op);
        return;
    }
    if (!force_split && vec && L <= kSmallResidentMin && nseg <= 0x7fffffffLL) {
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
        else go(K(), std::integral_constant<int, 8>());  // n4 <= 6144
    } else if (!force_split && vec && gn_block_bytes() == 0 &&
               run_gn_resident(op, silu, x, y, L, HW, cg, groups, nseg, gamma, beta, eps, false, fixed)) {
        return;
    } else if (vec) {
        const int64_t chunk = split_chunk(nseg, L);
        const int64_t nchunks = (L + chunk - 1) / chunk;
        // segments per block: the apply pass re-reads a block right after
        // the partial pass read it, while it is still cached
        int64_t sb = nseg;
        const int64_t budget = gn_block_bytes();
        if (budget > 0) sb = std::max<int64_t>(1, std::min<int64_t>(nseg, budget / (L * 4)));
        sb = std::min<int64_t>(sb, 65535);
        if (fixed) {
            // the fixed scratch holds the chunk pairs and statistics of this
            // many segments at once; larger tensors run in more blocks
            const int64_t room = (int64_t)(kFixedScratchBytes - kFixedCtlBytes - 256) /
                                 ((nchunks + 1) * (int64_t)sizeof(float2));
            if (room < 1)
                fail(SDH_ERR_INVALID, std::string(op) + ": a segment of " + std::to_string(L) + " floats needs " +
                                          std::to_string((nchunks + 1) * (int64_t)sizeof(float2)) +
                                          " bytes of scratch for its chunk statistics; this entry point holds " +
                                          std::to_string(kFixedScratchBytes - kFixedCtlBytes));
            sb = std::min<int64_t>(sb, room);
        }
        const size_t part_bytes = ((size_t)(sb * nchunks) * sizeof(float2) + 255) / 256 * 256;
        const size_t scr_bytes = part_bytes + (size_t)sb * sizeof(float2);
        char* scr = nullptr;
        if (fixed) {
            // every pair and statistic is written before it is read: nothing here must start at zero
            if (scr_bytes > kFixedScratchBytes - kFixedCtlBytes)
                fail(SDH_ERR_INVALID, std::string(op) + ": block of " + std::to_string(sb) +
                                           " segments exceeds the fixed scratch");
            scr = (char*)fixed + kFixedCtlBytes;
        } else {
            scr = (char*)scratch(scr_bytes);
        }
        float2* part = (float2*)scr;
        float2* stats = (float2*)(scr + part_bytes);
        const bool uniform = HW % chunk == 0;
        const int cpc = uniform ? (int)(HW / chunk) : 1;
        const bool merge = nchunks <= 64;  // one chunk pair per lane: merged inside pass B
        auto passes = [&](auto tc, auto vc) {
            constexpr int TPB = decltype(tc)::value, CV = decltype(vc)::value;
            for (int64_t s0 = 0; s0 < nseg; s0 += sb) {
                const int64_t k = std::min<int64_t>(sb, nseg - s0);
                const float* xb = x + s0 * L;
                float* yb = y + s0 * L;
                const dim3 grid((unsigned)nchunks, (unsigned)k);
                k_gn_partial<TPB, CV><<<grid, TPB, 0, stream()>>>(xb, L, nchunks, part);
                launched(op);
                if (!merge) {
                    k_gn_finalize<<<(unsigned)k, 64, 0, stream()>>>(part, L, nchunks, chunk, stats, eps);
                    launched(op);
                }
                const int seg0 = (int)(s0 % groups);
                auto apply = [&](auto sc, auto uc) {
                    constexpr bool S = decltype(sc)::value, U = decltype(uc)::value;
                    if (merge)
                        k_gn_apply<TPB, CV, S, U, true><<<grid, TPB, 0, stream()>>>(
                            xb, yb, L, (int)HW, cpc, (int)cg, groups, seg0, stats, part, (int)nchunks, eps, gamma, beta);
                    else
                        k_gn_apply<TPB, CV, S, U, false><<<grid, TPB, 0, stream()>>>(
                            xb, yb, L, (int)HW, cpc, (int)cg, groups, seg0, stats, part, (int)nchunks, eps, gamma, beta);
                };
                using T_ = std::true_type;
                using F_ = std::false_type;
                if (silu) uniform ? apply(T_(), T_()) : apply(T_(), F_());
                else uniform ? apply(F_(), T_()) : apply(F_(), F_());
                if (s0 + sb < nseg) launched(op);
            }
        };
        using I = std::integral_constant<int, 64>;
        if (chunk == 8192) passes(std::integral_constant<int, 256>(), std::integral_constant<int, 8>());
        else if (chunk == 4096) passes(I(), std::integral_constant<int, 16>());
        else passes(I(), std::integral_constant<int, 8>());
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

void gn_fixed_scratch_setup() {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) fail(SDH_ERR_INVALID, "backend_hip: device index out of range");
    void* p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch)), "hipGetSymbolAddress(scratch)");
    zero_device(p, kFixedScratchBytes);
    g_fixed_scratch[dev] = (unsigned char*)p;
    void* q = nullptr;
    hip_check(hipGetSymbolAddress(&q, HIP_SYMBOL(::pipe_area)), "hipGetSymbolAddress(pipe_area)");
    zero_device(q, sizeof(::pipe_area));
    g_pipe_area[dev] = (unsigned long long*)q;
}

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

// The kernels and schedules of sdh_group_norm_silu, with their scratch in
// the file-scope `scratch` array instead of the arena: no allocation of any
// kind, the library's set-up included (which is why it requires sdh_init
// first). Calls that overlap on one GPU would share the array and race; the
// library's lock and single stream keep its own calls in order.
int sdh_group_norm_silu_noalloc(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups,
                                const float* gamma, const float* beta, float eps) {
    return guarded([&] {
        const char* op = "sdh_group_norm_silu_noalloc";
        need(initialized(), op, "call sdh_init first (this entry point allocates nothing, set-up included)");
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        unsigned char* f = dev >= 0 && dev < kMaxDevices ? g_fixed_scratch[dev] : nullptr;
        need(f != nullptr, op, "the current device has no scratch address (it was not set up by sdh_init)");
        run_gn(op, true, x, y, N, C, HW, groups, gamma, beta, eps, f);
    });
}

}  // extern "C"

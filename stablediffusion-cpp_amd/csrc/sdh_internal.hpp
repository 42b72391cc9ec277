// sdh_internal.hpp - shared internals of backend_hip: error plumbing, the
// runtime singleton's interface, launch helpers and wave64 device primitives
// for gfx950 (CDNA4).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <mutex>
#include <string>

#include "sdh_backend.h"

namespace sdh {

// ---------------------------------------------------------------------------
// Errors: internal code throws Error; every extern "C" entry point catches it
// (and any std::exception), records the message for sdh_last_error() and
// returns the status. Nothing crosses the C ABI as an exception.
// ---------------------------------------------------------------------------
struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string& m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] void fail(int status, const std::string& msg);
void hip_check(hipError_t e, const char* what);
void set_last_error(const char* msg);
// Held by every C entry point while it checks arguments and queues its
// work, so an op's launches reach the stream together: ops that run several
// kernels through the shared scratch buffer (GroupNorm's split schedule,
// attention, the bf16 GEMM's packed A, conv2d) cannot interleave with
// another thread's. Recursive: entry points call entry points.
std::recursive_mutex& op_mutex();

template <class F>
int guarded(F&& f) noexcept {
    std::lock_guard<std::recursive_mutex> lk(op_mutex());
    try {
        f();
        set_last_error("");
        return SDH_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.status;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return SDH_ERR_HIP;
    } catch (...) {
        set_last_error("unknown error");
        return SDH_ERR_HIP;
    }
}

// ---------------------------------------------------------------------------
// Runtime (runtime.hip)
// ---------------------------------------------------------------------------
void ensure_init();
// True once sdh_init (or any entry point's implicit set-up) has run.
bool initialized();
// Looks up, for the current device, the address of the allocation-free
// GroupNorm entry point's fixed scratch and zeroes it (k_groupnorm.hip);
// called by the library's set-up.
void gn_fixed_scratch_setup();
hipStream_t stream();
// True between sdh_capture_begin and sdh_capture_end: launches are being
// recorded into a graph, to be replayed later.
bool capturing();
// Counts the captures begun so far (sdh_capture_begin).
unsigned capture_generation();
int num_cus();
// Throws SDH_ERR_INVALID unless [p, p + bytes) lies inside one live arena
// block or one registered external range. `what` names the argument.
void check_range(const void* p, size_t bytes, const char* op, const char* what);
// Per-call device scratch of at least `bytes`, owned by the library, valid
// until the next call that asks for scratch (ops are serialised on one stream).
void* scratch(size_t bytes);
// A persistent library-owned device block of at least `bytes` for a library
// routine's workspace (the BLAS GEMM), distinct from scratch().
void* workspace(size_t bytes);
// C[M,N] = P[M,K] B[N,K]^T (+ bias[N]) (+ C) on hipBLASLt, fp32 accumulation;
// P and B bf16 (f32 false) or fp32 (f32 true), leading dimensions in elements
// (k_gemm.hip). False when hipBLASLt has no algorithm for the shape.
bool blaslt_gemm(bool f32, int64_t M, int64_t N, int64_t K, const void* P, int64_t ldp, const void* B, int64_t ldb,
                 float* C, int64_t ldc, const float* bias, bool accumulate);
// y = silu(gate) * up over n floats (the SwiGLU kernel of sdh_swiglu, no checks).
void launch_swiglu(const float* gate, const float* up, float* y, int64_t n);
// sdh_softmax_rows on [rows, cols] (k_softmax.hip), errors named after `op`.
void softmax_rows_device(const char* op, float* x, int64_t rows, int64_t cols, float scale, bool causal);
// [B, R, K] -> [B, K, R] (k_layout.hip), errors named after `op`.
void transpose_device(const char* op, const float* x, float* y, int64_t B, int64_t R, int64_t K);
// y[i] = bf16 bits of x[i], the rounding of gemm_nt_bf16's A (k_gemm_f32.hip).
void to_bf16_device(const char* op, const float* x, uint16_t* y, int64_t n);
// Zero-initialised per-library device counters (uint32), persistent across
// calls; kernels that use them leave them at zero when they finish.
unsigned* counters(size_t count);
// Zero-initialised device words in uncached memory (the L2 keeps no copy,
// so a scalar load that misses the scalar cache reads what another XCD
// stored last), persistent across calls and never freed; kernels that use
// them leave them at zero when they finish. Null if the block holds fewer
// than `count` words.
unsigned* uncached_words(size_t count);
// At least n floats of 1.0f on the device, library-owned and persistent (for
// kernels that take a missing column vector as ones).
const float* ones_vector(size_t n);
void launched(const char* op);
// Registers a device word that the kernel just queued sets nonzero on a
// failure it cannot return as a status (a bounded wait that expired). The
// next sdh_synchronize or sdh_download reads the word after its stream
// synchronisation, clears it, calls on_failure (if given) and fails with
// SDH_ERR_HIP naming `what`.
void arm_device_check(unsigned* word, const char* what, void (*on_failure)() = nullptr);
// Queues a zero fill of [p, p + bytes) on the library stream (a kernel, not a memset).
void zero_device(void* p, size_t bytes);

// Argument helpers shared by the op entry points.
inline void need(bool ok, const char* op, const char* msg) {
    if (!ok) fail(SDH_ERR_INVALID, std::string(op) + ": " + msg);
}
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline unsigned blocks_for(int64_t items, int64_t per_block) {
    int64_t b = (items + per_block - 1) / per_block;
    return (unsigned)(b < 1 ? 1 : b);
}

// A dispatch covers at most 2^32 - 1 work-items per grid dimension (the
// dispatch packet holds the grid size in work-items as a uint32); a larger
// grid is not rejected, it wraps and covers less than asked. Launchers whose
// grid grows with the tensor keep each launch at or below kMaxGridItems
// work-items and cover larger tensors in several launches.
constexpr int64_t kMaxGridItems = int64_t(1) << 31;
// The work-items per launch the splitting launchers aim for: kMaxGridItems,
// or less when the environment variable SDH_LAUNCH_ITEMS asks for less (at
// least 1024; a test knob that sends small tensors through the split path).
int64_t launch_items();

// Calls launch(first, count) for consecutive pieces of [0, units) of at most
// per_launch units each.
template <class F>
inline void in_pieces(int64_t units, int64_t per_launch, F&& launch) {
    if (per_launch < 1) per_launch = 1;
    for (int64_t first = 0; first < units; first += per_launch)
        launch(first, units - first < per_launch ? units - first : per_launch);
}

// Rows (or other units) one launch may cover when each takes items_per_unit
// work-items; at least 1.
inline int64_t units_per_launch(int64_t items_per_unit) {
    const int64_t u = launch_items() / (items_per_unit < 1 ? 1 : items_per_unit);
    return u < 1 ? 1 : u;
}

}  // namespace sdh

// ---------------------------------------------------------------------------
// Device primitives (wave64)
// ---------------------------------------------------------------------------
namespace sdh {
namespace dev {

constexpr int kWave = 64;

// Native 128-bit vector of 4 floats (one global_load_dwordx4 per lane).
typedef float f4 __attribute__((ext_vector_type(4)));

// DPP lane moves within a row of 16 lanes. Controls (GCN/CDNA DPP encoding):
// quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_half_mirror =
// 0x141, row_mirror = 0x140. Every lane reads a valid lane for these.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over aligned groups of W lanes (W = 4, 8, 16, 32, 64); every lane of a
// group receives the group's sum. All 64 lanes must be active.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    if constexpr (W >= 8) v += dpp<0x141>(v);
    if constexpr (W >= 16) v += dpp<0x140>(v);
    if constexpr (W == 32) v += __shfl_xor(v, 16, 64);
    if constexpr (W == 64) {
        // Row sums are uniform within each row of 16; combine the 4 rows
        // through scalar reads so the result is bitwise identical in all lanes.
        const float a = readlane(v, 0), b = readlane(v, 16), c = readlane(v, 32), d = readlane(v, 48);
        v = (a + b) + (c + d);
    }
    return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
    static_assert(W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    if constexpr (W >= 8) v = fmaxf(v, dpp<0x141>(v));
    if constexpr (W >= 16) v = fmaxf(v, dpp<0x140>(v));
    if constexpr (W == 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if constexpr (W == 64) {
        const float a = readlane(v, 0), b = readlane(v, 16), c = readlane(v, 32), d = readlane(v, 48);
        v = fmaxf(fmaxf(a, b), fmaxf(c, d));
    }
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// Double-precision wave sum: the same DPP tree on both 32-bit halves; every
// lane receives the bitwise same total.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, lane);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }

__device__ __forceinline__ float hsum(const f4& v) { return (v.x + v.y) + (v.z + v.w); }
// Sum of the squares of a float4 with its rounding fixed: x^2 + y^2 and
// z^2 + w^2 each as one fused multiply-add, then their sum. The kernels whose
// results are claimed bit-equal to one another (the RMS norms, their fused
// forms, QK-norm) form their sums of squares with it, so the compiler's
// contraction of hsum(v * v), which changes with the surrounding control flow,
// cannot change their bits.
__device__ __forceinline__ float sumsq4(const f4& v) { return fmaf(v.x, v.x, v.y * v.y) + fmaf(v.z, v.z, v.w * v.w); }

// Streaming accesses: data touched exactly once per launch is loaded and
// stored non-temporally so it does not displace reusable lines in L2/MALL.
__device__ __forceinline__ f4 ld_stream(const f4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(f4* p, f4 v) { __builtin_nontemporal_store(v, p); }
typedef unsigned u2v __attribute__((ext_vector_type(2)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st_stream(uint2* p, uint2 v) {
    __builtin_nontemporal_store(u2v{v.x, v.y}, reinterpret_cast<u2v*>(p));
}

// exp(x) as 2^(x log2 e) on the hardware exp2 (v_exp_f32). Relative error
// about |x| 2^-24 (from rounding x log2 e) plus 1 ulp; for ops whose bound
// is relative 1e-4, not for the max-abs 1e-5 elementwise ops.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
// x / (1 + exp(-x)) with the hardware reciprocal (v_rcp_f32, 1 ulp).
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.0f + exp_fast(-x)); }

// rstd as the reference forms it: (float)(1 / sqrt(stat / C + eps)) in double
// (tensor.cpp:648, :674, :692).
__device__ __forceinline__ float rstd_of(float stat, int64_t C, float eps) {
    return (float)(1.0 / sqrt((double)stat / (double)C + (double)eps));
}
// rstd for per-head statistics (one per few float4 per lane, as in QK-norm):
// stat * (1/C) + eps in fp32, then the hardware reciprocal square root
// (v_rsq_f32, 1 ulp). A few ulp from rstd_of's double form, far inside the
// 1e-4 bound of the norms; the double divide and square root per head
// measured 6 of 46 us in the fused QK-norm + RoPE kernel on MI355X.
__device__ __forceinline__ float rstd_fast(float stat, float inv_c, float eps) {
    return __builtin_amdgcn_rsqf(stat * inv_c + eps);
}

// float -> bf16 bits, nearest even; inf and NaN keep their top 16 bits
// (tensor.cpp:114-121, the rounding of gemm_nt_bf16's A on the device).
__device__ __forceinline__ unsigned short bf16_rne(float f) {
    const unsigned b = __float_as_uint(f);
    if ((b & 0x7F800000u) == 0x7F800000u) return (unsigned short)(b >> 16);
    return (unsigned short)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}
// four floats -> four bf16 in one 8-byte word (element 0 in the low half)
__device__ __forceinline__ uint2 bf16x4(const f4& v) {
    return uint2{(unsigned)bf16_rne(v.x) | ((unsigned)bf16_rne(v.y) << 16),
                 (unsigned)bf16_rne(v.z) | ((unsigned)bf16_rne(v.w) << 16)};
}

// Reference-order activations (tensor.cpp:745, :847, :859, :866, :830).
__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float gelu_erf(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f)); }
__device__ __forceinline__ float quick_gelu(float v) { return v / (1.0f + expf(-1.702f * v)); }

// QK-norm then interleaved RoPE of one float4 of a head: o = (v * rstd), then
// * g when has_g, rotated pairwise, (x, y) by (c.x, s.x) and (z, w) by (c.z, s.z)
// (the even table entries, tensor.cpp:717-718). Every product and difference
// is rounded on its own, so each kernel that applies it gives the same bits.
__device__ __forceinline__ f4 qk_norm_rope4(const f4& v, float rstd, bool has_g, const f4& g, const f4& c,
                                            const f4& s) {
#pragma clang fp contract(off)
    f4 o = v * rstd;
    if (has_g) o = o * g;
    f4 r;
    r.x = o.x * c.x - o.y * s.x;
    r.y = o.y * c.x + o.x * s.x;
    r.z = o.z * c.z - o.w * s.z;
    r.w = o.w * c.z + o.z * s.z;
    return r;
}
}  // namespace dev
}  // namespace sdh

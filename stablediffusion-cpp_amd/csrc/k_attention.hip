// k_attention.hip - multi-head scaled dot-product attention, fused (flash
// style) on the MFMA units: out = softmax(q k^T / sqrt(d)) v per head, with
// grouped-query heads and the causal mask (backend_cuda.h:57-59; tensor.cpp:
// 776-810; the reference's GPU path backend_cuda.cu:550-586 materialises the
// [Sq, Skv] scores and runs them through softmax_rows, tensor.cpp:752-769).
//
// Numerics: the reference computes scores, softmax and the weighted sum in
// fp32. Here the operands are put in block floating point and split into two
// fp16 halves: a block (one query row of q; one 64-key tile of k, of v) is
// scaled by a power of two 2^-e that brings its largest magnitude into
// [2^13, 2^14), and each scaled value x becomes hi = rne16(x), lo =
// rne16(x - hi) (|x - hi - lo| <= 2^-22 |x| for normal lo). A product is
// formed as hi_a hi_b + hi_a lo_b + lo_a hi_b on the fp16 MFMA units with
// fp32 accumulation: about 2^-21 relative per product, three dense-fp16
// MFMAs per product (fp32 MFMA has 1/16 of the fp16 rate). The exponents
// are exact and fold into per-lane constants: the score scale becomes
// c = log2(e) / sqrt(d) * 2^(e_q + e_k) per query and tile; softmax weights
// are formed as 2^(s c - m + 14 + e_v - E) (E = the largest e_v of the head,
// m a running reference at most 1.5 below the row max, so they stay below
// 2^15.5, inside fp16) against values scaled by 2^-e_v, which keeps every
// tile's P V on the common scale 2^(14 - E); the sum of the weights is
// carried as 2^14 sum(p), and the output is divided by it (and scaled by 2^E)
// once at the end. The softmax is the online form (running row max m and
// sum); masked scores (kv > q when causal, kv past the keys) contribute
// exactly zero.
//
// sdh_attention_fp16 (opt-in, no counterpart in the reference) keeps the
// block scaling but forms each product once, hi_a hi_b: every operand
// rounded to 11 significant bits relative to its block's largest magnitude,
// one MFMA per product, half the packed bytes. Its error is that of fp16
// operands (about 2^-12 relative per element), not the reference's fp32.
//
// Layout. A pack kernel splits k and v of each key/value head into 64-key
// tiles of library scratch, each one contiguous block:
//   [K hi: 64 keys x DP][K lo][V^T hi: DP x 64 keys][V^T lo]   (fp16)
// plus the tile's two exponents (e_k, e_v) in a side array,
// with the head dimension zero-padded to DP (64 or 128) and keys past Skv
// zero (the fp16 variant packs [K][V^T] only). Rows sit in the order the
// MFMA fragment reads want them in LDS (16-B
// chunk c of row r at c ^ swz(r)), so the attention kernel copies a tile from
// global memory to LDS as one contiguous block (buffer_load_dwordx4 ... lds).
// The kernel computes S^T = K Q^T (v_mfma_f32_32x32x16_f16: K tile as the A
// operand, rows = keys; Q in registers as the B operand, columns = queries),
// so lane l holds scores of query l%32 only: the softmax statistics are
// per-lane values (one cross-lane max per tile, lanes l and l^32), and
// O^T = V^T P^T takes P straight from the score registers as its B operand.
// The accumulator gives lane l the keys 8(i/4) + 4(l/32) + i%4 of a 32-key
// block (i = 0..15); the pack kernel stores V^T with the keys of every
// 16-key group in the matching order (positions 8h + 4a + b hold key
// 8a + 4h + b), so the A operand of O^T is again one 16-B LDS read per lane.
// Workgroup: 8 waves x 32 queries of one head, in two groups that run half
// a tile apart (see k_attn_fwd); K and V tiles double-buffered in LDS; the
// running max a weight is taken against is raised only when a tile's max
// passes it by 2^1.5 (weights stay below 2^15.5), so O is rescaled on few
// tiles, and then by exactly the factor between the old and new reference.
// Head dimensions above 128 take a plain fp32 kernel (one wave per query).
// Both kernels can store the output rounded to bf16 (sdh_attention_bf16):
// the operand rounding of the projection that follows (to_out), applied to
// the same fp32 values, so the next GEMM reads half the bytes and no
// separate rounding pass runs.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "sdh_internal.hpp"

namespace sdh {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
using dev::f4;

constexpr int kKT = 64;                     // keys per tile
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kBM = 32 * kWaves;            // queries per workgroup
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kNoMax = -1e30f;            // running max before any key: finite, so 2^(m - m') never sees inf - inf
// The running reference m is raised only when a tile's max passes it by
// kLazy or more: weights then stay below 2^(14 + kLazy) (fp16 holds < 2^16),
// and O is rescaled only on those tiles.
constexpr float kLazy = 1.5f;
// LDS fragment reads of the MFMA loops run kPipe - 1 steps ahead
constexpr int kPipe = 2;
// s_waitcnt immediate (gfx9 encoding) that waits on vmcnt only: expcnt and
// lgkmcnt at their maxima; OR in a vmcnt below 16.
constexpr int kWaitVmBase = 0x0F70;
// Word 3 of a raw buffer resource (gfx9: 32-bit data format, no swizzle)
constexpr int kBufferWord3 = 0x00020000;

// 16-B chunk c of row r of a K tile (rows of DP fp16) sits at c ^ swz_k(r):
// for 256-B rows (DP = 128) 16 consecutive rows map one logical chunk to 16
// distinct chunks of LDS; for 128-B rows (DP = 64, and the 64-key rows of the
// V^T tile) the same holds per pair of rows.
template <int DP>
__device__ __host__ __forceinline__ int swz_k(int r) {
    return DP == 128 ? (r & 15) : ((r >> 1) & 7);
}
__device__ __host__ __forceinline__ int swz_v(int r) { return (r >> 1) & 7; }
// Key stored at position p of a V^T row (an involution on 0..63: bits 2 and 3 swap).
__device__ __host__ __forceinline__ int key_at(int p) { return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1); }

__device__ __forceinline__ void split(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}
// Softmax weight p in [0, 2^16) into hi + lo: hi keeps p's leading 11 bits
// (truncated: exact in fp16 for p >= 2^-14), lo = p - hi exactly in fp32,
// then rounded to fp16 (|lo| < 2^-10 p, so the pair is within 2^-21 p; below
// 2^-14, where fp16 is subnormal, within 2^-24 absolutely).
__device__ __forceinline__ void split_weight(float p, _Float16& hi, _Float16& lo) {
    const float h = __uint_as_float(__float_as_uint(p) & 0xFFFFE000u);
    hi = (_Float16)h;
    lo = (_Float16)(p - h);
}

// Exponent e of a block whose largest magnitude is amax: amax 2^-e lies in
// [2^13, 2^14). Zero, subnormal, inf and NaN maxima give 0 (no scaling).
__device__ __forceinline__ int block_exp(float amax) {
    const int f = (int)((__float_as_uint(amax) >> 23) & 0xFFu);
    if (f == 0 || f == 255) return 0;
    return min(max(f - 140, -126), 126);
}
// 2^e for e in [-126, 127]
__device__ __forceinline__ float pow2(int e) { return __uint_as_float((unsigned)(127 + e) << 23); }

// ---------------------------------------------------------------------------
// Pack: k, v [N, Skv, kv_heads * d] (fp32) -> tiles as described above, and
// the exponents (e_k, e_v) of every tile. One workgroup per (tile, kv head,
// batch); 256 threads. VEC: d == DP and 16-B aligned rows (float4 loads).
// ---------------------------------------------------------------------------
template <int DP, bool VEC, bool SPLIT>
__global__ __launch_bounds__(256) void k_attn_pack(const float* __restrict__ K, const float* __restrict__ V,
                                                   u16* __restrict__ tiles, int2* __restrict__ exps, int Skv,
                                                   int kv_inner, int d, int ntiles, int kv_heads) {
    constexpr int CPR = DP / 8;              // 16-B chunks per K row
    constexpr int KCH = kKT * CPR / 256;     // K chunks per thread
    constexpr int VCH = kKT * DP / 4 / 256;  // V float4 per thread
    __shared__ float sv[kKT][DP + 4];
    __shared__ float red[2][4];
    const int t = blockIdx.x, kh = blockIdx.y, nb = blockIdx.z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t row0 = (int64_t)nb * Skv + (int64_t)t * kKT;
    const int64_t col0 = (int64_t)kh * d;
    const int64_t tile = ((int64_t)nb * kv_heads + kh) * ntiles + t;
    constexpr int PARTS = SPLIT ? 4 : 2;  // [K hi][K lo][V^T hi][V^T lo], or [K][V^T] rounded to fp16
    u16* out = tiles + tile * PARTS * (kKT * DP);
    const int nrows = min(kKT, Skv - t * kKT);
    // K chunks into registers: slot i holds logical chunk (i % CPR) ^ swz of row i / CPR
    float kx[KCH][8];
    float kmax = 0.f, vmax = 0.f;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
        const int i = threadIdx.x + j * 256, r = i / CPR, c = (i % CPR) ^ swz_k<DP>(r);
        if constexpr (VEC) {
            // unconditional loads (rows past the keys re-read the last row,
            // zeroed after the load): a load under a mask splits the kernel
            // into blocks that cost registers
            const f4* p = (const f4*)(K + (row0 + min(r, nrows - 1)) * kv_inner + col0 + c * 8);
            f4 a = dev::ld_stream(p), b = dev::ld_stream(p + 1);
            if (r >= nrows) a = b = f4{0.f, 0.f, 0.f, 0.f};
            kx[j][0] = a.x; kx[j][1] = a.y; kx[j][2] = a.z; kx[j][3] = a.w;
            kx[j][4] = b.x; kx[j][5] = b.y; kx[j][6] = b.z; kx[j][7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int col = c * 8 + e;
                kx[j][e] = (r < nrows && col < d) ? K[(row0 + r) * kv_inner + col0 + col] : 0.f;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) kmax = fmaxf(kmax, fabsf(kx[j][e]));
    }
    // V tile into LDS (zero beyond the keys and the head dimension)
#pragma unroll
    for (int j = 0; j < VCH; ++j) {
        const int i = threadIdx.x + j * 256, r = i / (DP / 4), c = (i % (DP / 4)) * 4;
        f4 x = {0.f, 0.f, 0.f, 0.f};
        if constexpr (VEC) {
            x = dev::ld_stream((const f4*)(V + (row0 + min(r, nrows - 1)) * kv_inner + col0 + c));
            if (r >= nrows) x = f4{0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (r < nrows && c + e < d) x[e] = V[(row0 + r) * kv_inner + col0 + c + e];
        }
        *(f4*)&sv[r][c] = x;
        vmax = fmaxf(vmax, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
    }
    kmax = dev::wave_max(kmax);
    vmax = dev::wave_max(vmax);
    if (lane == 0) {
        red[0][w] = kmax;
        red[1][w] = vmax;
    }
    __syncthreads();
    kmax = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    vmax = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const int ek = block_exp(kmax), ev = block_exp(vmax);
    if (threadIdx.x == 0) exps[tile] = make_int2(ek, ev);
    const float sk = pow2(-ek), svs = pow2(-ev);
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
        const int i = threadIdx.x + j * 256, r = i / CPR, p = i % CPR;
        h8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            _Float16 a, b;
            split(kx[j][e] * sk, a, b);
            hi[e] = a;
            lo[e] = b;
        }
        *(h8*)(out + r * DP + p * 8) = hi;
        if constexpr (SPLIT) *(h8*)(out + kKT * DP + r * DP + p * 8) = lo;
    }
    // V^T: row = head-dim index, 8 chunks of 8 key positions
    u16* vt = out + (PARTS / 2) * kKT * DP;
    for (int i = threadIdx.x; i < DP * 8; i += 256) {
        const int r = i / 8, p = i % 8, c = p ^ swz_v(r);
        h8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            _Float16 a, b;
            split(sv[key_at(c * 8 + e)][r] * svs, a, b);
            hi[e] = a;
            lo[e] = b;
        }
        *(h8*)(vt + r * kKT + p * 8) = hi;
        if constexpr (SPLIT) *(h8*)(vt + DP * kKT + r * kKT + p * 8) = lo;
    }
}

// ---------------------------------------------------------------------------
// QK-norm + RoPE with the pack (zimage.cpp:117-121: rms_norm_heads_ and rope_
// on q and k, then attention): for one 64-token tile and one head, q is
// normalised and rotated in place and written back, k normalised and rotated
// in registers and packed from there (never written back as fp32), v packed
// as k_attn_pack packs it. Heads == kv_heads, head dim 128, interleaved
// rotation with [S, 128] tables. 32 lanes hold a head (lane i: float4 i), so
// the sum of squares is k_qknorm_rope_il's group_sum<32> and the element
// math its dev::qk_norm_rope4: q, the tiles and their exponents equal those of
// sdh_qknorm_rope followed by the pack. k's rows go from registers through
// LDS into the pack's chunk order.
template <bool SPLIT>
__global__ __launch_bounds__(256) void k_qkv_prep(float* __restrict__ Q, const float* __restrict__ K,
                                                  const float* __restrict__ V, u16* __restrict__ tiles,
                                                  int2* __restrict__ exps, int S, int inner, int ntiles, int heads,
                                                  const float* __restrict__ gq, const float* __restrict__ gk,
                                                  float eps, const float* __restrict__ cs,
                                                  const float* __restrict__ sn) {
    constexpr int DP = 128, L = 32;
    constexpr int RS = 256 / L;              // rows per step (8)
    constexpr int NS = kKT / RS;             // steps (8)
    constexpr int CPR = DP / 8;              // 16-B chunks per K row
    constexpr int KCH = kKT * CPR / 256;     // K chunks per thread
    constexpr int VCH = kKT * DP / 4 / 256;  // V float4 per thread
    __shared__ float tl[kKT][DP + 4];        // the normalised K tile, then the V tile
    __shared__ float red[2][4];
    const int t = blockIdx.x, h = blockIdx.y, nb = blockIdx.z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int hl = threadIdx.x % L, rs = threadIdx.x / L;
    const int64_t row0 = (int64_t)nb * S + (int64_t)t * kKT;
    const int64_t col0 = (int64_t)h * DP;
    const int nrows = min(kKT, S - t * kKT);
    const f4 one = {1.f, 1.f, 1.f, 1.f}, zero = {0.f, 0.f, 0.f, 0.f};
    const f4 gq4 = gq ? ((const f4*)gq)[hl] : one;
    const f4 gk4 = gk ? ((const f4*)gk)[hl] : one;
    // Loads are unconditional: rows past the sequence end (the last tile)
    // re-read its last row, and only what is stored or packed is masked
    // (a load under a mask splits the kernel into blocks that cost
    // registers).
    f4 kq[NS], kk[NS], vv[VCH];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int r = min(rs + RS * j, nrows - 1);
        kq[j] = dev::ld_stream((const f4*)(Q + (row0 + r) * inner + col0) + hl);
        kk[j] = dev::ld_stream((const f4*)(K + (row0 + r) * inner + col0) + hl);
    }
#pragma unroll
    for (int j = 0; j < VCH; ++j) {
        const int i = threadIdx.x + j * 256, r = i / (DP / 4), c = (i % (DP / 4)) * 4;
        const f4 a = dev::ld_stream((const f4*)(V + (row0 + min(r, nrows - 1)) * inner + col0 + c));
        vv[j] = r < nrows ? a : zero;  // keys past the sequence pack as zero
    }
    float kmax = 0.f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int r = rs + RS * j;
        const int64_t s = (int64_t)t * kKT + min(r, nrows - 1);  // position in the sequence
        const f4 c = ((const f4*)(cs + s * DP))[hl], sw = ((const f4*)(sn + s * DP))[hl];
        const float rq = dev::rstd_fast(dev::group_sum<L>(dev::sumsq4(kq[j])), 1.0f / DP, eps);
        const float rk = dev::rstd_fast(dev::group_sum<L>(dev::sumsq4(kk[j])), 1.0f / DP, eps);
        f4 o = zero;
        if (r < nrows) {
            dev::st_stream((f4*)(Q + (row0 + r) * inner + col0) + hl,
                           dev::qk_norm_rope4(kq[j], rq, gq != nullptr, gq4, c, sw));
            o = dev::qk_norm_rope4(kk[j], rk, gk != nullptr, gk4, c, sw);
            kmax = fmaxf(kmax, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
        }
        *(f4*)&tl[r][hl * 4] = o;
    }
    float vmax = 0.f;
#pragma unroll
    for (int j = 0; j < VCH; ++j)
        vmax = fmaxf(vmax, fmaxf(fmaxf(fabsf(vv[j].x), fabsf(vv[j].y)), fmaxf(fabsf(vv[j].z), fabsf(vv[j].w))));
    kmax = dev::wave_max(kmax);
    vmax = dev::wave_max(vmax);
    if (lane == 0) {
        red[0][w] = kmax;
        red[1][w] = vmax;
    }
    __syncthreads();
    kmax = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    vmax = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const int ek = block_exp(kmax), ev = block_exp(vmax);
    const int64_t tile = ((int64_t)nb * heads + h) * ntiles + t;
    if (threadIdx.x == 0) exps[tile] = make_int2(ek, ev);
    const float sk2 = pow2(-ek), svs = pow2(-ev);
    constexpr int PARTS = SPLIT ? 4 : 2;
    u16* out = tiles + tile * PARTS * (kKT * DP);
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
        const int i = threadIdx.x + j * 256, r = i / CPR, p = i % CPR, c = p ^ swz_k<DP>(r);
        h8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            _Float16 a, b;
            split(tl[r][c * 8 + e] * sk2, a, b);
            hi[e] = a;
            lo[e] = b;
        }
        *(h8*)(out + r * DP + p * 8) = hi;
        if constexpr (SPLIT) *(h8*)(out + kKT * DP + r * DP + p * 8) = lo;
    }
    __syncthreads();  // every K chunk read: the tile now takes V
#pragma unroll
    for (int j = 0; j < VCH; ++j) {
        const int i = threadIdx.x + j * 256, r = i / (DP / 4), c = (i % (DP / 4)) * 4;
        *(f4*)&tl[r][c] = vv[j];
    }
    __syncthreads();
    u16* vt = out + (PARTS / 2) * kKT * DP;
    for (int i = threadIdx.x; i < DP * 8; i += 256) {
        const int r = i / 8, p = i % 8, c = p ^ swz_v(r);
        h8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            _Float16 a, b;
            split(tl[key_at(c * 8 + e)][r] * svs, a, b);
            hi[e] = a;
            lo[e] = b;
        }
        *(h8*)(vt + r * kKT + p * 8) = hi;
        if constexpr (SPLIT) *(h8*)(vt + DP * kKT + r * kKT + p * 8) = lo;
    }
}

// ---------------------------------------------------------------------------
// Fused attention, head dimension padded to DP (64 or 128).
// 1-D grid of ceil(Sq / 256) * heads * N workgroups; 512 threads = 8 waves of 32 queries.
// Each wave alternates an MFMA phase (O += V(t-1) P(t-1), then S^T(t) =
// K(t) Q^T: 96 MFMAs) with a VALU phase (softmax(t)); waves 0-3 (X) and 4-7
// (Y) run half an iteration apart (waves w and w + 4 share a SIMD), so one
// wave's MFMAs run while the other computes its softmax. One barrier per
// iteration; K and V have separate double buffers (see the loop). Measured on
// the [1,4096,30x128] layer: 7680 cycles per 64-key tile against the 6144 of
// the MFMA work alone (the earlier two-barrier schedule, softmax and O += V P
// in one segment against S^T in the other, took 8960).
// ---------------------------------------------------------------------------
template <int DP, bool CAUSAL, bool OUT16, bool SPLIT>
__global__ __launch_bounds__(kThreads, 1) void k_attn_fwd(const float* __restrict__ Q, const u16* __restrict__ tiles,
                                                          const int2* __restrict__ exps, void* __restrict__ O, int Sq,
                                                          int Skv, int inner, int d, int group, int kv_heads,
                                                          int ntiles, float c2, int qvec, int nqb, int heads) {
    constexpr int DS = DP / 16;                    // 16-wide head-dim steps of S^T = K Q^T
    constexpr int DT = DP / 32;                    // 32-row head-dim tiles of O^T
    constexpr int TILE = (SPLIT ? 4 : 2) * kKT * DP, HALF = TILE / 2;  // fp16 values per packed tile, per K or V part
    constexpr int NLD = HALF * 2 / 16 / kThreads;  // 16-B loads per thread per part
    // Four separate LDS objects, each named statically where it is read or
    // filled (the loop below is unrolled by two): the compiler then knows
    // which LDS-DMA writes a read can alias, and does not make the read of
    // one buffer wait for the copy into the other.
    __shared__ __attribute__((aligned(1024))) u16 kbuf0[HALF];
    __shared__ __attribute__((aligned(1024))) u16 kbuf1[HALF];
    __shared__ __attribute__((aligned(1024))) u16 vbuf0[HALF];
    __shared__ __attribute__((aligned(1024))) u16 vbuf1[HALF];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const bool isY = w >= kWaves / 2;
    const int fr = lane & 31, fh = lane >> 5;
    // Workgroups are dealt to the 8 XCDs round robin (id % 8). Logical blocks
    // (query block fastest, then head, then batch) are renumbered so that each
    // XCD runs one contiguous range of them: the query blocks of a head share
    // one L2, which then fetches each K/V tile once instead of once per XCD.
    const int nblk = gridDim.x, xcd = blockIdx.x & 7, per = nblk >> 3, rem = nblk & 7;
    const int lb = xcd * per + min(xcd, rem) + (blockIdx.x >> 3);
    const int qb = lb % nqb, h = (lb / nqb) % heads, nb = lb / (nqb * heads), kh = h / group;
    const int q0 = qb * kBM, qw0 = q0 + w * 32;
    const int qlane = qw0 + fr;
    const int qend = min(q0 + kBM, Sq);
    const int T = CAUSAL ? min(ntiles, (qend - 1) / kKT + 1) : ntiles;
    const u16* src = tiles + ((int64_t)nb * kv_heads + kh) * ntiles * TILE;
    const int2* ex = exps + ((int64_t)nb * kv_heads + kh) * ntiles;
    // The head's tiles as one buffer (the host checks that they span less
    // than 2^31 bytes). Tiles are copied to LDS with buffer loads, not
    // global_load_lds: the compiler counts a FLAT-encoded copy into LDS as
    // pending on both the vector-memory and the LDS counters, and then waits
    // for every LDS read in full (lgkmcnt(0)) until the copy has landed.
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, ntiles * TILE * 2, kBufferWord3);
    auto issue = [&](int t, int part, u16* dst) __attribute__((always_inline)) {
        const int off = (t * TILE + part * HALF) * 2;  // bytes
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
            const int chunk = (j * kWaves + __builtin_amdgcn_readfirstlane(w)) * 64;  // wave-uniform
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(dst + chunk * 8),
                                                     16, lane * 16, off + chunk * 16, 0, 0);
        }
    };
    issue(0, 0, kbuf0);

    // Q fragments (B operand of S^T): query qlane, head dims ds*16 + fh*8 .. +7,
    // scaled by 2^-eq for the query's largest magnitude (lanes l and l^32 hold its two halves)
    h8 qh[DS], ql[DS];
    int eq;
    {
        const float* qp = Q + ((int64_t)nb * Sq + min(qlane, Sq - 1)) * inner + (int64_t)h * d;
        float x[DS][8];
        float qmax = 0.f;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const int c0 = ds * 16 + fh * 8;
            if (qvec) {
                const f4 a = *(const f4*)(qp + c0), b = *(const f4*)(qp + c0 + 4);
                x[ds][0] = a.x; x[ds][1] = a.y; x[ds][2] = a.z; x[ds][3] = a.w;
                x[ds][4] = b.x; x[ds][5] = b.y; x[ds][6] = b.z; x[ds][7] = b.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[ds][e] = c0 + e < d ? qp[c0 + e] : 0.f;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) qmax = fmaxf(qmax, fabsf(x[ds][e]));
        }
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
        eq = block_exp(qmax);
        const float sc = pow2(-eq);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 hi, lo;
                split(x[ds][e] * sc, hi, lo);
                qh[ds][e] = hi;
                ql[ds][e] = lo;  // unused without SPLIT
            }
    }
    // E: the largest value exponent among the tiles this workgroup reads
    int E;
    {
        float em = -1e30f;
        for (int t = lane; t < T; t += 64) em = fmaxf(em, (float)ex[t].y);
        E = (int)dev::wave_max(em);
    }

    f32x16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
    float m = kNoMax, lsum = 0.f;
    f32x16 s[2];      // S^T of the newest tile
    h8 ph[4], pl[4];  // its softmax weights, split (B operands of O^T += V^T P^T, one per 16-key step)

    auto scores = [&](const u16* Kh) __attribute__((always_inline)) {
        const u16* Kl = Kh + kKT * DP;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[j][i] = 0.f;
        // DS steps; step ds reads the hi/lo K fragments of both 32-key halves
        // j, kPipe - 1 steps ahead of its MFMAs, and interleaves the two
        // accumulator chains (each MFMA's predecessor is two issues back)
        h8 kf[kPipe][2][2];  // [slot][j][hi, lo]
        auto fetch = [&](int ds) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r = j * 32 + fr;
                const int off = r * DP + (((ds * 2 + fh) ^ swz_k<DP>(r)) << 3);
                kf[ds % kPipe][j][0] = *(const h8*)(Kh + off);
                if constexpr (SPLIT) kf[ds % kPipe][j][1] = *(const h8*)(Kl + off);
            }
        };
#pragma unroll
        for (int i = 0; i < kPipe - 1; ++i) fetch(i);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            if (ds + kPipe - 1 < DS) fetch(ds + kPipe - 1);
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
            const int sl = ds % kPipe;
#pragma unroll
            for (int j = 0; j < 2; ++j) s[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[sl][j][0], qh[ds], s[j], 0, 0, 0);
            if constexpr (SPLIT) {
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    s[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[sl][j][0], ql[ds], s[j], 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    s[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[sl][j][1], qh[ds], s[j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // softmax of tile t: s -> weights (ph, pl); running max and sum; O rescaled
    auto softmax = [&](int t) __attribute__((always_inline)) {
        const int k0 = t * kKT;
        const int2 et = ex[t];
        // mask: keys past Skv, and (causal) keys after the query
        if (k0 + kKT > Skv || (CAUSAL && k0 + kKT - 1 > qw0)) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kv = k0 + j * 32 + (i >> 2) * 8 + fh * 4 + (i & 3);
                    if (kv >= Skv || (CAUSAL && kv > qlane)) s[j][i] = -INFINITY;
                }
        }
        // log2(e)/sqrt(d) on the unscaled scores; kept normal so that a masked -inf stays -inf
        const float ct = fmaxf(ldexpf(c2, eq + et.x), 1.17549435e-38f);
        float mx = s[0][0];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[j][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mt = mx * ct;
        const float mnew = mt > m + kLazy ? mt : m;
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);  // exactly 1 when m is kept
        m = mnew;
        // weights 2^(s ct - m) times 2^(14 + e_v - E), < 2^(14 + kLazy)
        const float shift = (float)(14 + et.y - E) - mnew;
        float rs = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[j][i], ct, shift));
                s[j][i] = p;
                rs += p;
            }
        lsum = lsum * alpha + ldexpf(rs, E - et.y);  // 2^14 sum(p)
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if constexpr (SPLIT) {
                    _Float16 hi, lo;
                    split_weight(s[ks >> 1][(ks & 1) * 8 + e], hi, lo);
                    ph[ks][e] = hi;
                    pl[ks][e] = lo;
                } else {
                    ph[ks][e] = (_Float16)s[ks >> 1][(ks & 1) * 8 + e];
                }
            }
    };
    // O^T += V^T P^T in 2 DT steps of (16-key step ks, pair of 32-row tiles
    // dt, dt + 1): step i reads the pair's hi/lo V fragments kPipe - 1 steps
    // ahead of its MFMAs, and interleaves the two accumulator chains
    auto pv = [&](const u16* Vh) __attribute__((always_inline)) {
        const u16* Vl = Vh + DP * kKT;
        constexpr int NS = 2 * DT;
        h8 vf[kPipe][2][2];  // [slot][dt of the pair][hi, lo]
        auto fetch = [&](int i) __attribute__((always_inline)) {
            const int ks = i / (DT / 2), d0 = (i % (DT / 2)) * 2;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int r = (d0 + u) * 32 + fr;
                const int off = r * kKT + (((ks * 2 + fh) ^ swz_v(r)) << 3);
                vf[i % kPipe][u][0] = *(const h8*)(Vh + off);
                if constexpr (SPLIT) vf[i % kPipe][u][1] = *(const h8*)(Vl + off);
            }
        };
#pragma unroll
        for (int i = 0; i < kPipe - 1; ++i) fetch(i);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + kPipe - 1 < NS) fetch(i + kPipe - 1);
            __builtin_amdgcn_sched_barrier(0);
            const int ks = i / (DT / 2), d0 = (i % (DT / 2)) * 2, sl = i % kPipe;
#pragma unroll
            for (int u = 0; u < 2; ++u)
                o[d0 + u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[sl][u][0], ph[ks], o[d0 + u], 0, 0, 0);
            if constexpr (SPLIT) {
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    o[d0 + u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[sl][u][0], pl[ks], o[d0 + u], 0, 0, 0);
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    o[d0 + u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[sl][u][1], ph[ks], o[d0 + u], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // a wave with no real query, or (causal) whose queries all precede tile t, skips it
    const bool active = qw0 < Sq;
    auto wants = [&](int t) { return active && !(CAUSAL && qw0 + 31 < t * kKT); };

    // Iteration t, one barrier: K(t) and V(t-1) have landed, and no wave
    // reads K(t-1) or V(t-2) any more, whose buffers then take K(t+1) and
    // V(t). Each wave alternates an MFMA phase, O += V(t-1) P(t-1) then
    // S(t) = K(t) Q^T, with a VALU phase, softmax(t); the two waves of a SIMD
    // (w and w + 4) run half an iteration apart:
    //   X (waves 0-3):  [O += V P(t-1); S(t)]   softmax(t)
    //   Y (waves 4-7):  softmax(t-1)            [O += V P(t-1); S(t)]
    // so one wave's MFMAs run while the other computes its softmax.
    // Every part is copied unconditionally (past the last tile, a second copy
    // of tile T-1 into the free buffer): with no branch around the copies
    // the compiler tracks which buffer each one writes, and an LDS read waits
    // only for copies into its own buffer. The barrier is a bare s_barrier (a
    // compiler memory barrier too); the copies of an iteration have a whole
    // iteration to land.
    auto land = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(kWaitVmBase);
        asm volatile("s_barrier" ::: "memory");
    };
    // kc: K(t); vp: V(t-1); kn: K(t-1), to take K(t+1); vn: V(t-2), to take V(t)
    auto iteration = [&](int t, const u16* kc, const u16* vp, u16* kn, u16* vn) __attribute__((always_inline)) {
        land();
        issue(min(t + 1, T - 1), 0, kn);
        issue(min(t, T - 1), 1, vn);
        if (!isY) {
            if (t >= 1 && wants(t - 1)) pv(vp);
            if (t < T && wants(t)) {
                scores(kc);
                softmax(t);
            }
        } else {
            if (t >= 1 && wants(t - 1)) {
                softmax(t - 1);
                pv(vp);
            }
            if (t < T && wants(t)) scores(kc);
        }
    };
    for (int t = 0; t <= T; t += 2) {
        iteration(t, kbuf0, vbuf1, kbuf1, vbuf0);
        if (t + 1 <= T) iteration(t + 1, kbuf1, vbuf0, kbuf0, vbuf1);
    }
    // the surplus copies must land before the workgroup's LDS is released
    __builtin_amdgcn_s_waitcnt(kWaitVmBase);
    if (qlane >= Sq) return;
    lsum += __shfl_xor(lsum, 32, 64);
    // the reference scales P by 1/sum (tensor.cpp:761-764); O^T carries 2^(14-E) sum(p v), lsum 2^14 sum(p)
    const float inv = ldexpf(1.0f / lsum, E);
    const int64_t obase = ((int64_t)nb * Sq + qlane) * inner + (int64_t)h * d;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c0 = dt * 32 + g * 8 + fh * 4;
            const f4 v = {o[dt][g * 4] * inv, o[dt][g * 4 + 1] * inv, o[dt][g * 4 + 2] * inv, o[dt][g * 4 + 3] * inv};
            if constexpr (OUT16) {
                // the rounding gemm_nt_bf16 gives its A, applied to the fp32 value above
                u16* op = (u16*)O + obase;
                if (qvec) {
                    *(uint2*)(op + c0) = dev::bf16x4(v);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c0 + e < d) op[c0 + e] = dev::bf16_rne(v[e]);
                }
            } else {
                float* op = (float*)O + obase;
                if (qvec) {
                    *(f4*)(op + c0) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c0 + e < d) op[c0 + e] = v[e];
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Any head dimension: fp32 online softmax, one wave per (query, head, batch).
// Lanes take 64 keys at a time for the scores, then 64 head-dim columns at a
// time for the weighted sum. The query row and the scores pass through LDS.
// ---------------------------------------------------------------------------
constexpr int kGenWaves = 4, kGenMaxD = 1024;

template <bool CAUSAL, bool OUT16>
__global__ __launch_bounds__(64 * kGenWaves) void k_attn_generic(const float* __restrict__ Q, const float* __restrict__ K,
                                                                 const float* __restrict__ V, void* __restrict__ O,
                                                                 int Sq, int Skv, int inner, int kv_inner, int d,
                                                                 int group, float c2) {
    __shared__ float sq[kGenWaves][kGenMaxD];
    __shared__ float sp[kGenWaves][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int q = blockIdx.x * kGenWaves + w, h = blockIdx.y, nb = blockIdx.z;
    if (q >= Sq) return;  // whole wave; no block-level barrier below
    const float* qp = Q + ((int64_t)nb * Sq + q) * inner + (int64_t)h * d;
    const float* kb = K + (int64_t)nb * Skv * kv_inner + (int64_t)(h / group) * d;
    const float* vb = V + (int64_t)nb * Skv * kv_inner + (int64_t)(h / group) * d;
    for (int c = lane; c < d; c += 64) sq[w][c] = qp[c];
    __builtin_amdgcn_wave_barrier();
    constexpr int kAcc = kGenMaxD / 64;
    float acc[kAcc];
#pragma unroll
    for (int i = 0; i < kAcc; ++i) acc[i] = 0.f;
    float m = kNoMax, lsum = 0.f;
    const int kend = CAUSAL ? min(Skv, q + 1) : Skv;
    for (int k0 = 0; k0 < kend; k0 += 64) {
        const int kv = k0 + lane;
        float s = -INFINITY;
        if (kv < kend) {
            const float* kp = kb + (int64_t)kv * kv_inner;
            float a = 0.f;
            for (int c = 0; c < d; ++c) a = fmaf(sq[w][c], kp[c], a);
            s = a;
        }
        const float mnew = fmaxf(m, dev::wave_max(s) * c2);
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);
        m = mnew;
        const float p = __builtin_amdgcn_exp2f(fmaf(s, c2, -mnew));
        lsum = lsum * alpha + dev::wave_sum(p);
        __builtin_amdgcn_wave_barrier();
        sp[w][lane] = p;
        __builtin_amdgcn_wave_barrier();
        const int nk = min(64, kend - k0);
#pragma unroll
        for (int i = 0; i < kAcc; ++i) {
            const int c = i * 64 + lane;
            if (i * 64 >= d) break;
            float a = acc[i] * alpha;
            if (c < d)
                for (int j = 0; j < nk; ++j) a = fmaf(sp[w][j], vb[(int64_t)(k0 + j) * kv_inner + c], a);
            acc[i] = a;
        }
    }
    const float inv = 1.0f / lsum;
    const int64_t obase = ((int64_t)nb * Sq + q) * inner + (int64_t)h * d;
#pragma unroll
    for (int i = 0; i < kAcc; ++i) {
        const int c = i * 64 + lane;
        if (i * 64 >= d) break;
        if (c < d) {
            if constexpr (OUT16) ((u16*)O)[obase + c] = dev::bf16_rne(acc[i] * inv);
            else ((float*)O)[obase + c] = acc[i] * inv;
        }
    }
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + nb && y < x + na;
}

// QK-norm + RoPE folded into the pack (k_qkv_prep); q is written back.
struct QKPrep {
    float* q;
    const float* gq;
    const float* gk;
    const float* cs;
    const float* sn;
    float eps;
};

template <int DP, bool OUT16, bool SPLIT>
void run_mfma(const float* q, const float* k, const float* v, void* out, int64_t N, int64_t Sq, int64_t Skv,
              int heads, int kv_heads, int64_t d, bool causal, float c2, const QKPrep* prep = nullptr) {
    const int64_t ntiles = (Skv + kKT - 1) / kKT;
    const int64_t ntot = N * kv_heads * ntiles;
    const size_t tile_bytes = (size_t)(SPLIT ? 4 : 2) * kKT * DP * 2;
    char* base = (char*)scratch((size_t)ntot * (tile_bytes + sizeof(int2)));
    u16* tiles = (u16*)base;
    int2* exps = (int2*)(base + (size_t)ntot * tile_bytes);
    const int64_t inner = heads * d, kv_inner = (int64_t)kv_heads * d;
    need(ntiles * 256 <= kMaxGridItems, "sdh_attention", "too many keys for one launch");
    need(ntiles * (int64_t)tile_bytes < (int64_t(1) << 31), "sdh_attention", "too many keys per head for one launch");
    const dim3 pgrid((unsigned)ntiles, (unsigned)kv_heads, (unsigned)N);
    if constexpr (DP == 128) {
        if (prep)
            k_qkv_prep<SPLIT><<<pgrid, 256, 0, stream()>>>(prep->q, k, v, tiles, exps, (int)Skv, (int)kv_inner,
                                                            (int)ntiles, kv_heads, prep->gq, prep->gk, prep->eps,
                                                            prep->cs, prep->sn);
    }
    if (prep) {
        need(DP == 128, "sdh_qknorm_rope_attention", "internal: fused preparation needs head dim 128");
    } else if (d == DP && kv_inner % 4 == 0 && aligned16(k) && aligned16(v))
        k_attn_pack<DP, true, SPLIT><<<pgrid, 256, 0, stream()>>>(k, v, tiles, exps, (int)Skv, (int)kv_inner, (int)d,
                                                           (int)ntiles, kv_heads);
    else
        k_attn_pack<DP, false, SPLIT><<<pgrid, 256, 0, stream()>>>(k, v, tiles, exps, (int)Skv, (int)kv_inner, (int)d,
                                                            (int)ntiles, kv_heads);
    launched("sdh_attention");
    const int qvec = d == DP && inner % 4 == 0 && aligned16(q) && (OUT16 ? ((uintptr_t)out & 7) == 0 : aligned16(out));
    const int64_t nqb = (Sq + kBM - 1) / kBM, nblk = nqb * heads * N;
    need(nblk * kThreads <= kMaxGridItems, "sdh_attention", "too many query blocks for one launch");
    if (causal)
        k_attn_fwd<DP, true, OUT16, SPLIT><<<(unsigned)nblk, kThreads, 0, stream()>>>(
            q, tiles, exps, out, (int)Sq, (int)Skv, (int)inner, (int)d, heads / kv_heads, kv_heads, (int)ntiles, c2,
            qvec, (int)nqb, heads);
    else
        k_attn_fwd<DP, false, OUT16, SPLIT><<<(unsigned)nblk, kThreads, 0, stream()>>>(
            q, tiles, exps, out, (int)Sq, (int)Skv, (int)inner, (int)d, heads / kv_heads, kv_heads, (int)ntiles, c2,
            qvec, (int)nqb, heads);
    launched("sdh_attention");
}

// Head dimensions above 128 on long sequences (the VAE's one-head attention
// over 512 channels, modules.cpp:133-141): the score matrix, as the
// reference's device path forms it (backend_cuda.cu:550-586), on the fp32
// library GEMM: per (batch, head) and block of query rows, S = q_h k_g^T,
// the scaled (causal) row softmax in place, then O_h = P v_g as a GEMM
// against v^T (v transposed once per batch). fp32 products and sums
// throughout. The score block is bounded to score_bytes() (causal: one block,
// so the mask's row index is the query's). False, with nothing queued, when
// the operands do not suit the library GEMM (alignment, Skv % 4) or the
// causal block would not fit: the caller then runs the one-wave kernel.
// The score block's budget: SD_CUDA_ATTN_MB megabytes, at least 64, 1024 when
// unset, as the reference caps its score buffer (backend_cuda.cu:558-561).
int64_t score_bytes() {
    static const int64_t v = [] {
        const char* e = std::getenv("SD_CUDA_ATTN_MB");
        return (int64_t)(e ? std::max(64, std::atoi(e)) : 1024) << 20;
    }();
    return v;
}

bool run_attention_gemm(const char* op, const float* q, const float* k, const float* v, void* out, bool out16,
                        int64_t N, int64_t Sq, int64_t Skv, int heads, int kv_heads, int64_t d, bool causal,
                        float scale) {
    const int64_t inner = heads * d, kv_inner = (int64_t)kv_heads * d;
    if (d % 4 || Skv % 4 || !aligned16(q) || !aligned16(k) || !aligned16(v) || (!out16 && !aligned16(out)))
        return false;
    const int64_t budget = score_bytes();
    const int64_t rb = causal ? Sq : std::max<int64_t>(1, std::min<int64_t>(Sq, budget / (Skv * 4)));
    if (rb * Skv * 4 > 4 * budget) return false;
    const size_t vt_n = (size_t)(Skv * kv_inner), sc_n = (size_t)(rb * Skv), o_n = out16 ? (size_t)(N * Sq * inner) : 0;
    float* vt = (float*)scratch((vt_n + sc_n + o_n) * 4 + 512);
    float* sc = vt + ((vt_n + 63) & ~size_t(63));
    float* o32 = out16 ? sc + ((sc_n + 63) & ~size_t(63)) : (float*)out;
    const int group = heads / kv_heads;
    bool first = true;
    for (int64_t n = 0; n < N; ++n) {
        transpose_device(op, v + n * Skv * kv_inner, vt, 1, Skv, kv_inner);  // [Skv, kv_inner] -> [kv_inner, Skv]
        for (int h = 0; h < heads; ++h) {
            const int g = h / group;
            for (int64_t q0 = 0; q0 < Sq; q0 += rb) {
                const int64_t m = std::min(rb, Sq - q0);
                const bool ok = blaslt_gemm(true, m, Skv, d, q + (n * Sq + q0) * inner + h * d, inner,
                                            k + n * Skv * kv_inner + g * d, kv_inner, sc, Skv, nullptr, false);
                if (!ok) {
                    need(first, op, "the library GEMM has no algorithm for a later block");
                    return false;  // nothing but the transpose queued; the one-wave kernel takes over
                }
                first = false;
                softmax_rows_device(op, sc, m, Skv, scale, causal);
                need(blaslt_gemm(true, m, d, Skv, sc, Skv, vt + g * d * Skv, Skv, o32 + (n * Sq + q0) * inner + h * d,
                                 inner, nullptr, false),
                     op, "the library GEMM has no algorithm for P v");
            }
        }
    }
    if (out16) to_bf16_device(op, o32, (uint16_t*)out, N * Sq * inner);
    launched(op);
    return true;
}

// out is float32, or bf16 (uint16) when out16
void run_attention(const float* q, const float* k, const float* v, void* out, bool out16, int64_t N, int64_t Sq,
                   int64_t Skv, int heads, int kv_heads, int64_t d, bool causal, bool fp16 = false) {
    const char* op = fp16 ? "sdh_attention_fp16" : out16 ? "sdh_attention_bf16" : "sdh_attention";
    if (kv_heads <= 0) kv_heads = heads;  // tensor.cpp:777
    need(N >= 0 && Sq >= 0 && Skv >= 0, op, "negative size");
    need(heads > 0 && d > 0, op, "heads and d must be positive");
    need(heads % kv_heads == 0, op, "heads mismatch");  // tensor.cpp:779
    need(d <= kGenMaxD, op, "head dimension above 1024");
    const int64_t inner = heads * d, kv_inner = (int64_t)kv_heads * d;
    need(N <= 65535 && heads <= 65535 && kv_heads <= 65535, op, "too many batches or heads for one launch");
    need(N * Sq * inner < (1LL << 31) && N * Skv * kv_inner < (1LL << 31), op, "tensor too large (2^31 elements)");
    if (N == 0 || Sq == 0) return;
    ensure_init();
    const size_t qb = (size_t)(N * Sq * inner) * 4, kb = (size_t)(N * Skv * kv_inner) * 4;
    const size_t ob = out16 ? qb / 2 : qb;
    check_range(q, qb, op, "q");
    check_range(out, ob, op, "out");
    if (Skv > 0) {
        check_range(k, kb, op, "k");
        check_range(v, kb, op, "v");
    }
    need(!overlaps(out, ob, q, qb) && !(Skv > 0 && (overlaps(out, ob, k, kb) || overlaps(out, ob, v, kb))), op,
         "out overlaps an input");
    if (Skv == 0) {  // empty key set: every weighted sum is empty (the reference's gemm leaves 0)
        zero_device(out, ob);
        return;
    }
    const float scale = 1.0f / std::sqrt((float)d);  // tensor.cpp:784
    const float c2 = scale * kLog2e;
    if (d <= 128) {
        auto go = [&](auto dp, auto o16, auto sp) {
            run_mfma<decltype(dp)::value, decltype(o16)::value, decltype(sp)::value>(q, k, v, out, N, Sq, Skv, heads,
                                                                                    kv_heads, d, causal, c2);
        };
        using D64 = std::integral_constant<int, 64>;
        using D128 = std::integral_constant<int, 128>;
        using T_ = std::true_type;
        using F_ = std::false_type;
        if (d <= 64) {
            if (fp16) out16 ? go(D64(), T_(), F_()) : go(D64(), F_(), F_());
            else out16 ? go(D64(), T_(), T_()) : go(D64(), F_(), T_());
        } else {
            if (fp16) out16 ? go(D128(), T_(), F_()) : go(D128(), F_(), F_());
            else out16 ? go(D128(), T_(), T_()) : go(D128(), F_(), T_());
        }
    } else if (!(Sq * Skv >= (int64_t(1) << 18) &&
                 run_attention_gemm(op, q, k, v, out, out16, N, Sq, Skv, heads, kv_heads, d, causal, scale))) {
        const int64_t gx = (Sq + kGenWaves - 1) / kGenWaves;
        need(gx * 64 * kGenWaves <= kMaxGridItems, op, "too many queries for one launch");
        const dim3 grid((unsigned)gx, (unsigned)heads, (unsigned)N);
        auto go = [&](auto cc, auto oc) {
            constexpr bool C = decltype(cc)::value, O16 = decltype(oc)::value;
            k_attn_generic<C, O16><<<grid, 64 * kGenWaves, 0, stream()>>>(
                q, k, v, out, (int)Sq, (int)Skv, (int)inner, (int)kv_inner, (int)d, heads / kv_heads, c2);
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        if (causal) out16 ? go(T_(), T_()) : go(T_(), F_());
        else out16 ? go(F_(), T_()) : go(F_(), F_());
        launched(op);
    }
}

// qknorm_rope_ of q and k (zimage.cpp:117-120) then attention (:121), with
// q left normalised and rotated as sdh_qknorm_rope leaves it, k and v read
// only. Head dim 128 with heads == kv_heads, Sq == Skv, interleaved [S, 128]
// tables and aligned operands: one launch prepares q and packs k and v
// (k_qkv_prep), then the attention kernel; otherwise the same sequence
// through the separate entry points on a copy of k.
void run_qknorm_rope_attention(float* q, const float* k, const float* v, void* out, bool out16, int64_t N,
                               int64_t S, int heads, int64_t dim, const float* gq, const float* gk, float eps,
                               const float* cs, const float* sn, bool fp16) {
    const char* op = "sdh_qknorm_rope_attention";
    need(N >= 0 && S >= 0, op, "negative size");
    need(heads > 0 && dim > 0 && dim % 2 == 0, op, "heads and dim must be positive, dim even");
    need(N * S * heads * dim < (1LL << 31), op, "tensor too large (2^31 elements)");
    need(N <= 65535 && heads <= 65535, op, "too many batches or heads for one launch");
    if (N == 0 || S == 0) return;
    ensure_init();
    const int64_t inner = heads * dim;
    const size_t bytes = (size_t)(N * S * inner) * 4;
    check_range(q, bytes, op, "q");
    check_range(k, bytes, op, "k");
    check_range(v, bytes, op, "v");
    check_range(out, out16 ? bytes / 2 : bytes, op, "out");
    check_range(cs, (size_t)(S * dim) * 4, op, "cos");
    check_range(sn, (size_t)(S * dim) * 4, op, "sin");
    if (gq) check_range(gq, (size_t)dim * 4, op, "gamma_q");
    if (gk) check_range(gk, (size_t)dim * 4, op, "gamma_k");
    const size_t ob = out16 ? bytes / 2 : bytes;
    need(!overlaps(out, ob, q, bytes) && !overlaps(out, ob, k, bytes) && !overlaps(out, ob, v, bytes) &&
             !overlaps(q, bytes, k, bytes) && !overlaps(q, bytes, v, bytes),
         op, "operands overlap");
    const bool fused = dim == 128 && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(cs) &&
                       aligned16(sn) && (!gq || aligned16(gq)) && (!gk || aligned16(gk)) &&
                       (out16 ? ((uintptr_t)out & 7) == 0 : aligned16(out));
    if (fused) {
        const QKPrep prep{q, gq, gk, cs, sn, eps};
        const float c2 = 1.0f / std::sqrt((float)dim) * kLog2e;
        if (fp16) {
            if (out16) run_mfma<128, true, false>(q, k, v, out, N, S, S, heads, heads, dim, false, c2, &prep);
            else run_mfma<128, false, false>(q, k, v, out, N, S, S, heads, heads, dim, false, c2, &prep);
        } else {
            if (out16) run_mfma<128, true, true>(q, k, v, out, N, S, S, heads, heads, dim, false, c2, &prep);
            else run_mfma<128, false, true>(q, k, v, out, N, S, S, heads, heads, dim, false, c2, &prep);
        }
        return;
    }
    // the op sequence, k normalised on a copy
    auto ok = [&](int rc) {
        if (rc != SDH_OK) fail(rc, sdh_last_error());
    };
    void* kc = nullptr;
    ok(sdh_malloc(bytes, &kc));
    try {
        ok(sdh_copy(kc, k, bytes));
        ok(sdh_qknorm_rope(q, inner, (float*)kc, inner, N, S, dim, gq, gk, eps, cs, sn, 1));
        if (fp16) ok(sdh_attention_fp16(q, (const float*)kc, v, out, out16, N, S, S, heads, heads, dim, 0));
        else if (out16) ok(sdh_attention_bf16(q, (const float*)kc, v, (uint16_t*)out, N, S, S, heads, heads, dim, 0));
        else ok(sdh_attention(q, (const float*)kc, v, (float*)out, N, S, S, heads, heads, dim, 0));
    } catch (...) {
        sdh_free(kc);
        throw;
    }
    ok(sdh_free(kc));
}

}  // namespace
}  // namespace sdh

using namespace sdh;

extern "C" {

int sdh_attention(const float* q, const float* k, const float* v, float* out, int64_t N, int64_t Sq, int64_t Skv,
                  int heads, int kv_heads, int64_t d, int causal) {
    return guarded([&] { run_attention(q, k, v, out, false, N, Sq, Skv, heads, kv_heads, d, causal != 0); });
}

int sdh_attention_bf16(const float* q, const float* k, const float* v, uint16_t* out, int64_t N, int64_t Sq,
                       int64_t Skv, int heads, int kv_heads, int64_t d, int causal) {
    return guarded([&] { run_attention(q, k, v, out, true, N, Sq, Skv, heads, kv_heads, d, causal != 0); });
}

int sdh_attention_fp16(const float* q, const float* k, const float* v, void* out, int out_bf16, int64_t N,
                       int64_t Sq, int64_t Skv, int heads, int kv_heads, int64_t d, int causal) {
    return guarded(
        [&] { run_attention(q, k, v, out, out_bf16 != 0, N, Sq, Skv, heads, kv_heads, d, causal != 0, true); });
}

int sdh_qknorm_rope_attention(float* q, const float* k, const float* v, void* out, int out_bf16, int64_t N,
                              int64_t S, int heads, int64_t dim, const float* gamma_q, const float* gamma_k,
                              float eps, const float* cos, const float* sin, int fp16) {
    return guarded([&] {
        run_qknorm_rope_attention(q, k, v, out, out_bf16 != 0, N, S, heads, dim, gamma_q, gamma_k, eps, cos, sin,
                                  fp16 != 0);
    });
}

}  // extern "C"

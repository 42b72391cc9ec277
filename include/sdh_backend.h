/*
 * sdh_backend.h - C ABI of backend_hip, the MI355X (gfx950) backend for the
 * elementwise / reduction / broadcast ops of StableDiffusion-cpp's tensor
 * library.
 *
 * It implements every function of the reference's GPU boundary,
 * src/backend_cuda.h (namespace sd::cuda, raw device pointers + int64 sizes):
 * the elementwise / reduction / broadcast ops it is built for, and the
 * GEMMs, attention and conv2d that complete the interface.
 * Each entry point keeps the parameters of the function it replaces, in the
 * same order and with the same meaning; the comment on each cites that
 * declaration. Differences, all at the ABI level:
 *   - plain C: every function returns an int status (SDH_OK = 0) instead of
 *     throwing; sdh_last_error() gives the message of the calling thread's
 *     last failure. bool parameters are int.
 *   - memory comes from a device arena owned by the library; op outputs are
 *     NOT zero-filled (the reference's Tensor(shape, Device) zero-fills,
 *     tensor.cpp:55-63; every op here writes its whole output).
 *   - every pointer argument of an op must lie, with the extent the op
 *     touches, inside one live allocation of this library (sdh_malloc) or a
 *     range registered with sdh_register_external; otherwise the call fails
 *     with SDH_ERR_INVALID before anything is launched.
 *   - all work is queued in order on one HIP stream owned by the library.
 *     Ops return as soon as the work is queued; sdh_download and
 *     sdh_synchronize wait for it (backend_cuda.h:12-13 semantics).
 *   - additive entry points (marked FUSED) have no single reference
 *     function; their comment names the reference composition they equal.
 *
 * Thread safety: calls may come from any thread. Each entry point holds
 * one library lock while it checks its arguments and queues its kernels,
 * so the launches of one op reach the single library stream together and
 * ops that run several kernels through the shared scratch buffer cannot
 * interleave; ops run in the order their calls took the lock. A call that
 * waits (sdh_download, sdh_synchronize) holds the lock while it waits.
 */
#ifndef SDH_BACKEND_H
#define SDH_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
#define SDH_OK 0
#define SDH_ERR_UNAVAILABLE 1 /* no HIP device, or the CPU-only stub library */
#define SDH_ERR_INVALID 2     /* bad argument: size, shape or pointer range */
#define SDH_ERR_OOM 3         /* device arena exhausted */
#define SDH_ERR_HIP 4         /* HIP runtime error (message has the HIP string) */

/* Message of the calling thread's last failed call ("" if none). */
const char* sdh_last_error(void);

/* ---- device ------------------------------------------------------------ */
/* backend_cuda.h:24 available(): 1 if built with HIP and a device is present. */
int sdh_available(void);
/* backend_cuda.h:26 device_name(): name of device 0, "" if unavailable. */
const char* sdh_device_name(void);
/* backend_cuda.h:27 device_memory(): bytes of device 0, 0 if unavailable. */
size_t sdh_device_memory(void);
/* No reference counterpart (the reference probes lazily, backend_cuda.cu:50-89):
 * explicit initialisation. Creates the stream, the staging buffers and a first
 * arena segment of arena_bytes (0 = SDH_ARENA_MB from the environment, else
 * 1024 MiB). Called implicitly by the first call that needs the device. */
int sdh_init(size_t arena_bytes);
/* Frees every device and pinned allocation of the library. */
int sdh_shutdown(void);

/* ---- memory (backend_cuda.h:29-36) -------------------------------------- */
/* backend_cuda.h:30 malloc(): *out = device block of `bytes` (256-byte aligned,
 * uninitialised). bytes == 0 gives *out = NULL and SDH_OK. */
int sdh_malloc(size_t bytes, void** out);
/* backend_cuda.h:31 free(): returns a block to the arena (NULL is a no-op). */
int sdh_free(void* p);
/* backend_cuda.h:32 upload(): host -> device. Staged through pinned buffers
 * with hipMemcpyAsync; the host buffer may be reused when the call returns. */
int sdh_upload(void* dst, const void* src, size_t bytes);
/* backend_cuda.h:33 download(): device -> host; waits for all queued work.
 * Also reports a failure found on the device since the last wait (an expired
 * GroupNorm team wait, see sdh_group_norm) as SDH_ERR_HIP, after the copy. */
int sdh_download(void* dst, const void* src, size_t bytes);
/* backend_cuda.h:34 copy(): device -> device, asynchronous. */
int sdh_copy(void* dst, const void* src, size_t bytes);
/* backend_cuda.h:35 zero(): fills with zero bytes, asynchronous. */
int sdh_zero(void* dst, size_t bytes);
/* backend_cuda.h:36 synchronize(): waits for all queued work; reports a
 * failure found on the device as sdh_download does. */
int sdh_synchronize(void);
/* No reference counterpart: lets ops accept device memory that the library did
 * not allocate (for example a framework's tensor). The range must stay valid
 * until sdh_unregister_external. */
int sdh_register_external(void* p, size_t bytes);
int sdh_unregister_external(void* p);
/* No reference counterpart: arena statistics (bytes reserved from HIP, bytes
 * handed out to live blocks). */
int sdh_memory_stats(size_t* reserved, size_t* in_use);

/* FUSED for the Z-Image block: a pre-rounded bf16 A (ld lda), as
 * gemm_nt_bf16 forms it on the device (backend_cuda.cu:183-188), so one
 * rounding serves several projections of the same input (to_q, to_k, to_v).
 * Otherwise as sdh_gemm_nt_bf16. */
int sdh_gemm_nt_bf16_packed(int64_t M, int64_t N, int64_t K, const uint16_t* A, int64_t lda, const uint16_t* B,
                            int64_t ldb, float* C, int64_t ldc, const float* bias, int accumulate);

/* ---- GEMM with fp32 weights --------------------------------------------- */
/* backend_cuda.h:38-40 gemm_nt_f32(): C[M,N] = A[M,K] * B[N,K]^T (+ C when
 * accumulate) (+ bias[N]), all fp32, row-major with leading dimensions in
 * elements; bias may be NULL. The linear layers whose weights stay fp32. */
int sdh_gemm_nt_f32(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B, int64_t ldb,
                    float* C, int64_t ldc, const float* bias, int accumulate);
/* backend_cuda.h:45-47 conv2d(); tensor.h:159 (tensor.cpp:520-560).
 * x [N, Cin, H, W], w [Cout, Cin, kh, kw] fp32, bias [Cout] or NULL,
 * out [N, Cout, Ho, Wo] with Ho = (H + 2 pad - kh) / stride + 1 (and Wo
 * alike); zero padding. Patches gathered per pixel chunk, then the fp32
 * GEMM: completes the reference's backend interface, not a tuned path. */
int sdh_conv2d(const float* x, int64_t N, int64_t Cin, int64_t H, int64_t W, const float* w, int64_t Cout, int64_t kh,
               int64_t kw, const float* bias, int stride, int pad, float* out, int64_t Ho, int64_t Wo);
/* Tensor::to_bf16 (tensor.cpp:131-137) on device memory: y[i] = bf16 bits of
 * x[i] (nearest even; inf and NaN keep their top 16 bits). */
int sdh_to_bf16(const float* x, uint16_t* y, int64_t n);

/* ---- GEMM (MFMA) ------------------------------------------------------- */
/* backend_cuda.h:41-43 gemm_nt_bf16(): C[M,N] = A[M,K] * B[N,K]^T (+ C when
 * accumulate) (+ bias[N]); row-major with leading dimensions in elements; A
 * fp32 (rounded to bf16 on the device, as the reference's tensor-core path),
 * B bf16, fp32 accumulation. bias may be NULL. */
int sdh_gemm_nt_bf16(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const uint16_t* B, int64_t ldb,
                     float* C, int64_t ldc, const float* bias, int accumulate);
/* FUSED: y [rows, hidden] = swiglu(x w1^T, x w3^T) with x [rows, in] fp32 and
 * w1, w3 [hidden, in] bf16 (no biases); equals swiglu(linear(x, w1),
 * linear(x, w3)) (zimage.cpp:130) without writing the two products. */
int sdh_linear_swiglu(const float* x, const uint16_t* w1, const uint16_t* w3, float* y, int64_t rows, int64_t in,
                      int64_t hidden);

/* ---- norms -------------------------------------------------------------- */
/* backend_cuda.h:48 group_norm(); tensor.h:166. x, y [N, C, HW]; gamma, beta
 * [C]; C % groups == 0. y may equal x. Large segments may run on the
 * resident schedule, whose workgroups wait for each other inside the kernel;
 * each wait is bounded, and one that expires leaves NaN in y and is reported
 * by the next sdh_synchronize or sdh_download. */
int sdh_group_norm(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                   const float* beta, float eps);
/* backend_cuda.h:50 layer_norm(); tensor.h:170. x, y [rows, C]; gamma, beta
 * [C] or NULL. y may equal x. */
int sdh_layer_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, const float* beta,
                   float eps);
/* backend_cuda.h:51 rms_norm(); tensor.h:177. x, y [rows, C]; gamma [C] or
 * NULL. y may equal x. */
int sdh_rms_norm(const float* x, float* y, int64_t rows, int64_t C, const float* gamma, float eps);
/* backend_cuda.h:52 rms_norm_heads(); tensor.h:180. In place on x
 * [groups, dim]; gamma [dim] or NULL. */
int sdh_rms_norm_heads(float* x, int64_t groups, int64_t dim, const float* gamma, float eps);

/* ---- rotary -------------------------------------------------------------- */
/* backend_cuda.h:54 rope(); tensor.h:188. In place on x [N, S, inner],
 * inner % dim == 0, dim even; cos, sin [S, dim]. interleaved = 1: pairs
 * (2i, 2i+1) rotated by cos/sin[s, 2i]; 0: pairs (i, i + dim/2) as
 * tensor.cpp:721-725. */
int sdh_rope(float* x, int64_t N, int64_t S, int64_t inner, int64_t dim, const float* cos, const float* sin,
             int interleaved);
/* FUSED: rope() on q [N, S, inner_q] and on k [N, S, inner_k] in one launch;
 * equals rope_(q, ...) then rope_(k, ...) (zimage.cpp:119-120). */
int sdh_rope_qk(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                const float* cos, const float* sin, int interleaved);
/* VARIANT of sdh_rope_qk (interleaved) with the tables formed on the device
 * from positions, as zimage.cpp:71-88 forms them on the host: pos [S, 3]
 * int32 (device); the head's dim = axis0 + axis1 + axis2 channels are the
 * concatenated axes, pair j of axis a turns by the float angle
 * (float)((double)pos[s, a] * theta^(-2j/d_a)) whose cos and sin (float)
 * rotate it. Equals building those [S, dim] tables and calling
 * sdh_rope_qk(..., interleaved = 1). q, k 16-byte aligned, rows of at most
 * 8192 floats, dim a multiple of 4 and at most 256. */
int sdh_rope_qk_axes(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                     const int32_t* pos, int axis0, int axis1, int axis2, float theta);
/* FUSED: QK-norm then RoPE on q [N, S, inner_q] and k [N, S, inner_k] in one
 * launch; equals rms_norm_heads_(q, dim, gamma_q, eps),
 * rms_norm_heads_(k, dim, gamma_k, eps), rope_(q, ...), rope_(k, ...)
 * (zimage.cpp:117-120, interleaved; qwen3.cpp:59-62, rotate_half).
 * gamma_q / gamma_k [dim] may be NULL; q and k must not overlap. */
int sdh_qknorm_rope(float* q, int64_t inner_q, float* k, int64_t inner_k, int64_t N, int64_t S, int64_t dim,
                    const float* gamma_q, const float* gamma_k, float eps, const float* cos, const float* sin,
                    int interleaved);

/* ---- softmax ------------------------------------------------------------- */
/* backend_cuda.h:56 softmax_rows(); tensor.h:236. In place on x [rows, cols]:
 * p = exp(x*scale - max) / sum over the valid columns; causal keeps columns
 * 0..r of row r and zeroes the rest. */
int sdh_softmax_rows(float* x, int64_t rows, int64_t cols, float scale, int causal);
/* As sdh_softmax_rows, with the causal row index taken modulo `period` (a
 * stack of [period, cols] score matrices, as the reference's attention launch
 * at backend_cuda.cu:578). */
int sdh_softmax_rows_batched(float* x, int64_t rows, int64_t cols, float scale, int causal, int64_t period);

/* ---- the Z-Image block's fused row ops (zimage.cpp:114-135) ---------------- */
/* FUSED: y = bf16 bits of rms_norm(x, gamma, eps) * scale, rows of C floats:
 * rms_norm then mul_rows_(., scale) then the bf16 rounding gemm_nt_bf16
 * applies to its A; the bits equal those of that sequence. gamma and scale
 * may be NULL; y must not overlap x. */
int sdh_rms_norm_modulate_bf16(const float* x, uint16_t* y, int64_t rows, int64_t C, const float* gamma,
                               const float* scale, float eps);
/* FUSED: x += gate * rms_norm(a, gamma, eps), or x += rms_norm(a, gamma, eps)
 * with gate NULL: rms_norm then add_rows_scaled_ (or add_), with the same
 * fp32 results. a is not modified; x and a must not overlap. */
int sdh_rms_norm_gated_add(float* x, const float* a, int64_t rows, int64_t C, const float* gamma, const float* gate,
                           float eps);
/* FUSED (residual add + RMSNorm + modulate; zimage.cpp:124-129, :132-135 ->
 * :114-116): x += gate * rms_norm(a, gamma_out, eps_out), then y = bf16 bits
 * of rms_norm(x, gamma_in, eps_in) * scale for the updated x: one sublayer's
 * norm + gated residual and the next sublayer's modulated input in one pass
 * over x; x and y are bit-equal to sdh_rms_norm_gated_add followed by
 * sdh_rms_norm_modulate_bf16. gamma_out, gate, gamma_in and scale may be
 * NULL; x and a must not overlap, nor y either of them. */
int sdh_rms_norm_gated_add_modulate_bf16(float* x, const float* a, uint16_t* y, int64_t rows, int64_t C,
                                         const float* gamma_out, const float* gate, const float* gamma_in,
                                         const float* scale, float eps_out, float eps_in);
/* FUSED: y = bf16 bits of swiglu(gate, up): swiglu then the bf16 rounding of
 * gemm_nt_bf16's A (the input of the FFN's w2, zimage.cpp:130). */
int sdh_swiglu_bf16(const float* gate, const float* up, uint16_t* y, int64_t n);

/* ---- attention ------------------------------------------------------------ */
/* backend_cuda.h:57-59 attention(); tensor.h:205-212 (tensor.cpp:776-810).
 * q [N, Sq, heads*d], k and v [N, Skv, kv_heads*d], out [N, Sq, heads*d]:
 * out = softmax(q k^T / sqrt(d)) v per head, query head h reading key/value
 * head h / (heads / kv_heads); causal keeps keys 0..i for query i.
 * kv_heads <= 0 means kv_heads = heads. out must not overlap the inputs.
 * Fused on the MFMA units (no score matrix in memory) for d <= 128. */
int sdh_attention(const float* q, const float* k, const float* v, float* out, int64_t N, int64_t Sq, int64_t Skv,
                  int heads, int kv_heads, int64_t d, int causal);
/* FUSED: out = bf16 bits of attention(q, k, v): sdh_attention then the bf16
 * rounding gemm_nt_bf16 applies to its A (backend_cuda.h:41-43; the input of
 * the block's to_out projection, zimage.cpp:121); the bits equal those of
 * that sequence. out [N, Sq, heads*d] uint16. */
int sdh_attention_bf16(const float* q, const float* k, const float* v, uint16_t* out, int64_t N, int64_t Sq,
                       int64_t Skv, int heads, int kv_heads, int64_t d, int causal);
/* FUSED (zimage.cpp:117-121): rms_norm_heads_(q), rms_norm_heads_(k), rope_(q),
 * rope_(k) (as sdh_qknorm_rope, interleaved tables [S, dim]) then attention
 * (self-attention, heads == kv_heads, not causal): q [N, S, heads*dim] is left
 * normalised and rotated as sdh_qknorm_rope leaves it; k and v are read only;
 * out as sdh_attention (out_bf16 == 0, float32) or sdh_attention_bf16
 * (uint16 bf16 bits), with fp16 != 0 the products of sdh_attention_fp16. For
 * dim 128 and 16-byte aligned operands one launch normalises and rotates q and
 * k and packs k and v for the attention kernel (k's normalised rows never
 * reach memory); q and out are bit-equal to the op sequence. Other shapes
 * run the sequence on a copy of k. */
int sdh_qknorm_rope_attention(float* q, const float* k, const float* v, void* out, int out_bf16, int64_t N,
                              int64_t S, int heads, int64_t dim, const float* gamma_q, const float* gamma_k,
                              float eps, const float* cos, const float* sin, int fp16);
/* OPT-IN REDUCED PRECISION, no counterpart in the reference: attention as
 * sdh_attention (out float32) or sdh_attention_bf16 (out_bf16 != 0, out the
 * uint16 bf16 bits), with every product formed once from fp16 operands: q
 * per row, k and v per 64-key tile scaled by a power of two that brings the
 * block's largest magnitude into [2^13, 2^14), then rounded to fp16 (11
 * significant bits); the softmax weights rounded to fp16 likewise; fp32
 * accumulation and softmax statistics. A third of sdh_attention's MFMA work
 * and half its packed bytes; the error is that of fp16 operands (about 2^-12
 * relative per element), for callers whose tolerance allows it (a diffusion
 * step's 2e-2). Head dimensions above 128 run the fp32 kernel. */
int sdh_attention_fp16(const float* q, const float* k, const float* v, void* out, int out_bf16, int64_t N,
                       int64_t Sq, int64_t Skv, int heads, int kv_heads, int64_t d, int causal);

/* ---- activations ----------------------------------------------------------- */
/* backend_cuda.h:61 swiglu(); tensor.h:191. y = gate / (1 + exp(-gate)) * up. */
int sdh_swiglu(const float* gate, const float* up, float* y, int64_t n);
/* backend_cuda.h:60 geglu(); tensor.h:217. x [rows, 2D] -> y [rows, D]. */
int sdh_geglu(const float* x, float* y, int64_t rows, int64_t D);
/* backend_cuda.h:64 silu(), :65 tanh(), :66 gelu(), :67 quick_gelu(): in place. */
int sdh_silu(float* x, int64_t n);
int sdh_tanh(float* x, int64_t n);
int sdh_gelu(float* x, int64_t n);
int sdh_quick_gelu(float* x, int64_t n);

/* ---- broadcasts / residual ------------------------------------------------- */
/* backend_cuda.h:68 add(): a += b. */
int sdh_add(float* a, const float* b, int64_t n);
/* backend_cuda.h:69 scale(): x *= s. */
int sdh_scale(float* x, float s, int64_t n);
/* backend_cuda.h:70 affine(): x = x * a + b. */
int sdh_affine(float* x, float a, float b, int64_t n);
/* FUSED for the Z-Image block: x [2 * pairs, dim] in place, rows 2p become
 * 1 + x (affine_(scale, 1, 1)) and rows 2p + 1 tanh(x) (tanh_(gate)), the four
 * ops of zimage.cpp:104-107 in one launch; bits equal those of the ops. */
int sdh_modulation_rows(float* x, int64_t pairs, int64_t dim);
/* backend_cuda.h:71 mul_rows(): x[r, :] *= v[:]. */
int sdh_mul_rows(float* x, const float* v, int64_t rows, int64_t dim);
/* backend_cuda.h:72 add_rows_scaled(): x[r, :] += g[:] * y[r, :]. */
int sdh_add_rows_scaled(float* x, const float* y, const float* g, int64_t rows, int64_t dim);
/* backend_cuda.h:73 add_channel_bias(): x[n, c, :] += b[n, c]. */
int sdh_add_channel_bias(float* x, const float* b, int64_t N, int64_t C, int64_t HW);
/* x[r, :] += v[:] (row-vector bias / adaLN shift). The reference has this only
 * inside linear's bias epilogue (k_add_bias_cols, backend_cuda.cu:239-241);
 * on the CPU it equals add_rows_scaled_(x, ones, v). */
int sdh_add_rows(float* x, const float* v, int64_t rows, int64_t dim);

/* ---- layout (bit-exact copies; the output must not overlap an input) --------- */
/* backend_cuda.h:74 upsample_nearest2x(); tensor.h:238. x [NC, H, W] ->
 * y [NC, 2H, 2W], each input element repeated into a 2 x 2 block. */
int sdh_upsample_nearest2x(const float* x, float* y, int64_t NC, int64_t H, int64_t W);
/* backend_cuda.h:75 concat_channels(); tensor.h:240. a [N, Ca, HW] and
 * b [N, Cb, HW] -> y [N, Ca + Cb, HW]. */
int sdh_concat_channels(const float* a, const float* b, float* y, int64_t N, int64_t Ca, int64_t Cb, int64_t HW);
/* backend_cuda.h:76 nchw_to_nlc(); tensor.h:244. x [N, C, HW] -> y [N, HW, C]. */
int sdh_nchw_to_nlc(const float* x, float* y, int64_t N, int64_t C, int64_t HW);
/* backend_cuda.h:77 nlc_to_nchw(); tensor.h:246. x [N, HW, C] -> y [N, C, HW]. */
int sdh_nlc_to_nchw(const float* x, float* y, int64_t N, int64_t C, int64_t HW);
/* backend_cuda.h:79 patchify(); tensor.h:200. x [C, H, W] -> y [(H/p)(W/p),
 * p*p*C], features ordered (ph, pw, c). H and W must be multiples of p. */
int sdh_patchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p);
/* backend_cuda.h:80 unpatchify(); tensor.h:201. The inverse of sdh_patchify:
 * x [(H/p)(W/p), p*p*C] -> y [C, H, W]. H and W must be multiples of p (the
 * reference's kernel would read past the tokens otherwise). */
int sdh_unpatchify(const float* x, float* y, int64_t C, int64_t H, int64_t W, int p);

/* ---- fused ------------------------------------------------------------------ */
/* FUSED: x += r; y = rms_norm(x, gamma, eps). Equals add_(x, r) then
 * rms_norm(x, gamma, eps) (the residual -> norm order of zimage.cpp:123-128).
 * x, r, y [rows, C]; gamma [C] or NULL. */
int sdh_add_rms_norm(float* x, const float* r, float* y, int64_t rows, int64_t C, const float* gamma, float eps);
/* FUSED: y = silu(group_norm(x)). Equals group_norm then silu_
 * (modules.cpp:34-35, vae.cpp:48-49, unet.cpp:120-121). y may equal x. */
int sdh_group_norm_silu(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups, const float* gamma,
                        const float* beta, float eps);
/* ALLOCATION-FREE: no counterpart in the reference. For callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc). The same kernels and result as
 * sdh_group_norm_silu, with the scratch they need (team slots and counters,
 * chunk statistics) in a fixed 1 MiB device array per GPU instead of the
 * arena; it calls no hipMalloc, hipFree or allocating routine, so sdh_init
 * must have run first (SDH_ERR_INVALID otherwise). The split schedule runs
 * as many segments at a time as the array's 960 KiB of chunk statistics
 * holds; a single segment whose statistics exceed it (over about 10^9
 * floats) is rejected with SDH_ERR_INVALID. The resident and
 * single-workgroup schedules need at most 17 KiB. The one-launch pipelined
 * schedule (segments of at most 64 whole 4096-float chunks) exchanges its
 * chunk statistics through a second fixed 2 MiB array that
 * sdh_group_norm_silu uses too (2^17 chunks a launch; larger tensors take
 * several launches). Calls that overlap on one GPU share the
 * arrays and would race; the library's own calls are serialised on its one
 * stream. */
int sdh_group_norm_silu_noalloc(const float* x, float* y, int64_t N, int64_t C, int64_t HW, int groups,
                                const float* gamma, const float* beta, float eps);
/* FUSED adaLN: y = layer_norm(x, no affine, eps) * (1 + scale) + shift;
 * res += tanh(gate) * y. Equals layer_norm -> affine_(scale, 1, 1) ->
 * tanh_(gate) -> mul_rows_(y, 1+scale) -> add_rows_scaled_(y, ones, shift) ->
 * add_rows_scaled_(res, y, tanh(gate)) (zimage.cpp:104-107, :221-224).
 * x, res [rows, C]; scale, gate [C]; shift [C] or NULL; y_out [rows, C] or
 * NULL (y is then not stored). */
int sdh_ln_modulate_gate(const float* x, float* res, const float* scale, const float* shift, const float* gate,
                         float* y_out, int64_t rows, int64_t C, float eps);

/* ---- measurement helpers (no reference counterpart) -------------------------- */
/* Fills x[0..n) on the device with N(mean, std) values of the library's
 * seeded counter-based generator (splitmix64 + Box-Muller); for synthetic
 * benchmark inputs. */
int sdh_fill_normal(float* x, int64_t n, uint64_t seed, float mean, float std);
/* Records timer slot `slot` (0..15) on the library stream. */
int sdh_timer_record(int slot);
/* Milliseconds between two recorded slots; waits for the second. */
int sdh_timer_elapsed(int start_slot, int end_slot, float* ms);
/* Graph capture of the library stream, for callers that replay a fixed
 * sequence of ops with no host work between launches (and for timing
 * launch-bound ops on the device). Between sdh_capture_begin and
 * sdh_capture_end the ops' launches are recorded, not run; sdh_capture_end
 * returns an instantiated graph that sdh_graph_launch queues on the library
 * stream (in order with every other call) and sdh_graph_destroy frees after
 * waiting for the stream. While capturing, everything that waits on the
 * stream (upload, download, synchronize, timer readout) and every op whose
 * scratch would have to grow is refused with SDH_ERR_INVALID: run each op
 * once before capturing it. The graph keeps the pointers it was captured
 * with. */
int sdh_capture_begin(void);
int sdh_capture_end(void** graph);
int sdh_graph_launch(void* graph);
int sdh_graph_destroy(void* graph);

#ifdef __cplusplus
}
#endif

#endif /* SDH_BACKEND_H */

// backend_stub.cpp - CPU-only stand-in for libsdh (the role
// src/backend_cuda_stub.cpp plays for the reference, :14-56): it exports every
// entry point of sdh_backend.h, sdh_available() is 0 and every other call
// fails with SDH_ERR_UNAVAILABLE and a message, so a host without a GPU can
// build and link the C++ side and a mistake is loud rather than silent.
// It computes nothing: there is no CPU fallback behind the C ABI.
#include "sdh_backend.h"

namespace {
const char* g_msg = "";
int unavailable() {
    g_msg = "backend_hip not built for this host (CPU-only stub library)";
    return SDH_ERR_UNAVAILABLE;
}
}  // namespace

#define STUB(decl) \
    decl { return unavailable(); }

extern "C" {

const char* sdh_last_error(void) { return g_msg; }
int sdh_available(void) { return 0; }
const char* sdh_device_name(void) { return ""; }
size_t sdh_device_memory(void) { return 0; }
STUB(int sdh_init(size_t))
int sdh_shutdown(void) { return SDH_OK; }

STUB(int sdh_malloc(size_t, void**))
int sdh_free(void* p) { return p ? unavailable() : SDH_OK; }
STUB(int sdh_upload(void*, const void*, size_t))
STUB(int sdh_download(void*, const void*, size_t))
STUB(int sdh_copy(void*, const void*, size_t))
STUB(int sdh_zero(void*, size_t))
int sdh_synchronize(void) { return SDH_OK; }
STUB(int sdh_register_external(void*, size_t))
STUB(int sdh_unregister_external(void*))
STUB(int sdh_memory_stats(size_t*, size_t*))

STUB(int sdh_group_norm(const float*, float*, int64_t, int64_t, int64_t, int, const float*, const float*, float))
STUB(int sdh_layer_norm(const float*, float*, int64_t, int64_t, const float*, const float*, float))
STUB(int sdh_rms_norm(const float*, float*, int64_t, int64_t, const float*, float))
STUB(int sdh_rms_norm_heads(float*, int64_t, int64_t, const float*, float))
STUB(int sdh_rope(float*, int64_t, int64_t, int64_t, int64_t, const float*, const float*, int))
STUB(int sdh_rope_qk(float*, int64_t, float*, int64_t, int64_t, int64_t, int64_t, const float*, const float*, int))
STUB(int sdh_softmax_rows(float*, int64_t, int64_t, float, int))
STUB(int sdh_softmax_rows_batched(float*, int64_t, int64_t, float, int, int64_t))
STUB(int sdh_attention(const float*, const float*, const float*, float*, int64_t, int64_t, int64_t, int, int,
                        int64_t, int))
STUB(int sdh_attention_bf16(const float*, const float*, const float*, uint16_t*, int64_t, int64_t, int64_t, int, int,
                             int64_t, int))
STUB(int sdh_attention_fp16(const float*, const float*, const float*, void*, int, int64_t, int64_t, int64_t, int, int,
                             int64_t, int))
STUB(int sdh_qknorm_rope_attention(float*, const float*, const float*, void*, int, int64_t, int64_t, int, int64_t,
                                    const float*, const float*, float, const float*, const float*, int))
STUB(int sdh_swiglu(const float*, const float*, float*, int64_t))
STUB(int sdh_geglu(const float*, float*, int64_t, int64_t))
STUB(int sdh_silu(float*, int64_t))
STUB(int sdh_tanh(float*, int64_t))
STUB(int sdh_gelu(float*, int64_t))
STUB(int sdh_quick_gelu(float*, int64_t))
STUB(int sdh_add(float*, const float*, int64_t))
STUB(int sdh_scale(float*, float, int64_t))
STUB(int sdh_modulation_rows(float*, int64_t, int64_t))
STUB(int sdh_affine(float*, float, float, int64_t))
STUB(int sdh_mul_rows(float*, const float*, int64_t, int64_t))
STUB(int sdh_add_rows_scaled(float*, const float*, const float*, int64_t, int64_t))
STUB(int sdh_add_channel_bias(float*, const float*, int64_t, int64_t, int64_t))
STUB(int sdh_add_rows(float*, const float*, int64_t, int64_t))
STUB(int sdh_add_rms_norm(float*, const float*, float*, int64_t, int64_t, const float*, float))
STUB(int sdh_group_norm_silu(const float*, float*, int64_t, int64_t, int64_t, int, const float*, const float*, float))
STUB(int sdh_group_norm_silu_noalloc(const float*, float*, int64_t, int64_t, int64_t, int, const float*, const float*, float))
STUB(int sdh_ln_modulate_gate(const float*, float*, const float*, const float*, const float*, float*, int64_t,
                              int64_t, float))
STUB(int sdh_rope_qk_axes(float*, int64_t, float*, int64_t, int64_t, int64_t, int64_t, const int32_t*, int, int, int, float))
STUB(int sdh_qknorm_rope(float*, int64_t, float*, int64_t, int64_t, int64_t, int64_t, const float*, const float*,
                         float, const float*, const float*, int))
STUB(int sdh_gemm_nt_bf16_packed(int64_t, int64_t, int64_t, const uint16_t*, int64_t, const uint16_t*, int64_t, float*,
                                 int64_t, const float*, int))
STUB(int sdh_rms_norm_modulate_bf16(const float*, uint16_t*, int64_t, int64_t, const float*, const float*, float))
STUB(int sdh_rms_norm_gated_add(float*, const float*, int64_t, int64_t, const float*, const float*, float))
STUB(int sdh_rms_norm_gated_add_modulate_bf16(float*, const float*, uint16_t*, int64_t, int64_t, const float*,
                                              const float*, const float*, const float*, float, float))
STUB(int sdh_swiglu_bf16(const float*, const float*, uint16_t*, int64_t))
STUB(int sdh_gemm_nt_f32(int64_t, int64_t, int64_t, const float*, int64_t, const float*, int64_t, float*, int64_t,
                         const float*, int))
STUB(int sdh_to_bf16(const float*, uint16_t*, int64_t))
STUB(int sdh_conv2d(const float*, int64_t, int64_t, int64_t, int64_t, const float*, int64_t, int64_t, int64_t,
                    const float*, int, int, float*, int64_t, int64_t))
STUB(int sdh_gemm_nt_bf16(int64_t, int64_t, int64_t, const float*, int64_t, const uint16_t*, int64_t, float*, int64_t,
                          const float*, int))
STUB(int sdh_linear_swiglu(const float*, const uint16_t*, const uint16_t*, float*, int64_t, int64_t, int64_t))
STUB(int sdh_upsample_nearest2x(const float*, float*, int64_t, int64_t, int64_t))
STUB(int sdh_concat_channels(const float*, const float*, float*, int64_t, int64_t, int64_t, int64_t))
STUB(int sdh_nchw_to_nlc(const float*, float*, int64_t, int64_t, int64_t))
STUB(int sdh_nlc_to_nchw(const float*, float*, int64_t, int64_t, int64_t))
STUB(int sdh_patchify(const float*, float*, int64_t, int64_t, int64_t, int))
STUB(int sdh_unpatchify(const float*, float*, int64_t, int64_t, int64_t, int))
STUB(int sdh_fill_normal(float*, int64_t, uint64_t, float, float))
STUB(int sdh_timer_record(int))
STUB(int sdh_timer_elapsed(int, int, float*))
STUB(int sdh_capture_begin(void))
STUB(int sdh_capture_end(void**))
STUB(int sdh_graph_launch(void*))
STUB(int sdh_graph_destroy(void*))

}  // extern "C"

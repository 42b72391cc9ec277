// tensor_hip.h - the reference's tensor.h operator API for HIP device tensors.
//
// sdh::Tensor mirrors sd::Tensor (src/tensor.h:48-95) for fp32 data: a shape
// plus storage that lives either on the host (std::vector<float>) or on the
// MI355X (a backend_hip arena block). The free functions below keep the
// names, parameters, return conventions (new tensor vs in-place `_` ops) and
// error messages of the tensor.h declarations they cite, and run on the
// device through backend_hip. They implement the device branch only: the
// CPU branch of every op is the reference's own tensor.cpp, so passing a host
// tensor to an op throws rather than computing anything on the CPU.
//
// Additive fused ops (add_rms_norm_, group_norm_silu, ln_modulate_gate_,
// rope_qk_) equal the reference compositions named in their comments.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace sdh {

// tensor.h:32, with HIP in place of CUDA.
enum class Device { CPU, HIP };
const char* device_name(Device d);          // "cpu" / "hip"
Device parse_device(const std::string& s);  // "cpu", "hip", or "auto" (hip if available)

struct DeviceBuffer;  // one backend_hip arena block

// tensor.h:45. Activations are F32; weights may be BF16 (the top 16 bits of a
// float32), accepted by linear.
enum class DType { F32, BF16 };

struct Tensor {
    std::vector<int64_t> shape;
    std::vector<float> data;            // F32 host storage when device == CPU
    std::vector<uint16_t> data16;       // BF16 host storage when device == CPU
    DType dtype = DType::F32;
    Device device = Device::CPU;
    std::shared_ptr<DeviceBuffer> dev;  // device storage when device == HIP
    int64_t dev_off = 0;                // first element within dev (rows_view)

    Tensor() = default;
    // Zero-filled host tensor (tensor.h:58).
    explicit Tensor(std::vector<int64_t> s);
    // Zero-filled tensor on the given device (tensor.h:60, tensor.cpp:55-63).
    Tensor(std::vector<int64_t> s, Device d);
    // Device tensor whose contents are left uninitialised; ops use it for
    // outputs they overwrite completely (no zero-fill pass).
    static Tensor empty(std::vector<int64_t> s, Device d);
    // Uninitialised BF16 device tensor (bf16 bit patterns, two bytes each).
    static Tensor empty_bf16(std::vector<int64_t> s);

    static int64_t numel_of(const std::vector<int64_t>& s);
    int64_t numel() const { return numel_of(shape); }
    bool is_hip() const { return device == Device::HIP; }
    bool is_bf16() const { return dtype == DType::BF16; }
    const uint16_t* dptr16() const;  // BF16 device storage
    uint16_t* dptr16();
    // F32 host storage -> BF16, rounding to nearest even (tensor.h:86-87).
    void to_bf16();
    Tensor to(Device d) const;  // tensor.cpp:72-93
    float* dptr();
    const float* dptr() const;
    int ndim() const { return (int)shape.size(); }
    int64_t dim(int i) const { return shape[i < 0 ? i + ndim() : i]; }
    float* ptr();  // host only
    const float* ptr() const;
    Tensor& reshape(std::vector<int64_t> s);
    std::string shape_str() const;
};

// ---- norms (tensor.h:166-180) ----
Tensor group_norm(const Tensor& x, int groups, const Tensor& gamma, const Tensor& beta, float eps);
Tensor layer_norm(const Tensor& x, const Tensor* gamma, const Tensor* beta, float eps);
inline Tensor layer_norm(const Tensor& x, const Tensor& gamma, const Tensor& beta, float eps) {
    return layer_norm(x, &gamma, &beta, eps);
}
Tensor rms_norm(const Tensor& x, const Tensor* gamma, float eps);
void rms_norm_heads_(Tensor& x, int64_t dim, const Tensor* gamma, float eps);

// ---- rotary, activations (tensor.h:188-191, :217-228) ----
void rope_(Tensor& x, int64_t dim, const Tensor& cos, const Tensor& sin, bool interleaved);
Tensor swiglu(const Tensor& gate, const Tensor& up);
Tensor geglu(const Tensor& x);
void silu_(Tensor& x);
void tanh_(Tensor& x);
void gelu_(Tensor& x);
void quick_gelu_(Tensor& x);

// ---- broadcasts / residual (tensor.h:195-198, :230-232) ----
void affine_(Tensor& x, float a, float b);
// x [2 P, D] in place: rows 2p -> 1 + x (affine_(x, 1, 1)), rows 2p + 1 ->
// tanh(x) (tanh_), one launch (the adaLN modulation of a Z-Image block).
void modulation_rows_(Tensor& x);
void mul_rows_(Tensor& x, const Tensor& v);
void add_rows_scaled_(Tensor& x, const Tensor& y, const Tensor& g);
void add_channel_bias_(Tensor& x, const Tensor& b);
void add_(Tensor& a, const Tensor& b);
void scale_(Tensor& x, float s);

// ---- layout (tensor.h:200-203, :238-250); outputs are new device tensors ----
Tensor patchify2d(const Tensor& x, int p);  // x [1, C, H, W] -> [(H/p)(W/p), p*p*C]
Tensor unpatchify2d(const Tensor& tokens, int64_t C, int64_t H, int64_t W, int p);
Tensor slice_rows(const Tensor& x, int64_t from, int64_t to);
// Rows [from, to) of a device tensor as a tensor that shares x's storage (no
// copy; in-place ops on it change x). No counterpart in tensor.h, whose
// slice_rows copies; used where a copy would only feed in-place ops.
Tensor rows_view(const Tensor& x, int64_t from, int64_t to);
Tensor upsample_nearest2x(const Tensor& x);
Tensor concat_channels(const Tensor& a, const Tensor& b);
Tensor concat_batch(const Tensor& a, const Tensor& b);
Tensor nchw_to_nlc(const Tensor& x);
Tensor nlc_to_nchw(const Tensor& x, int64_t H, int64_t W);
Tensor slice_batch(const Tensor& x, int64_t b);
Tensor repeat_batch(const Tensor& x, int64_t times);

// ---- linear (tensor.h:146): y = x W^T (+ b), W [out, in] ----
// The reference's device branch (tensor.cpp:489-494): with BF16 weights x is
// rounded to bf16 and products accumulate in fp32 (MFMA); F32 weights take
// the fp32 GEMM. A BF16 x (from rms_norm_modulate_bf16 / swiglu_bf16) is
// already rounded and is used as is (BF16 weights only).
Tensor linear(const Tensor& x, const Tensor& W, const Tensor* b);
// swiglu(linear(x, w1), linear(x, w3)) in one GEMM (zimage.cpp:130)
Tensor linear_swiglu(const Tensor& x, const Tensor& w1, const Tensor& w3);
// tensor.h:159: x [N, Cin, H, W], W [Cout, Cin, kh, kw] (F32), b [Cout] or null
Tensor conv2d(const Tensor& x, const Tensor& W, const Tensor* b, int stride, int pad);

// ---- the Z-Image block's fused ops (zimage.cpp:114-135); results equal the
// op sequences named, bit for bit ----
// rms_norm(x, gamma, eps), then mul_rows_(., *scale) when scale is given, rounded
// to BF16: the A operand linear() takes for BF16 weights (no second rounding).
Tensor rms_norm_modulate_bf16(const Tensor& x, const Tensor* gamma, const Tensor* scale, float eps);
// x += *gate * rms_norm(a, gamma, eps), or x += rms_norm(a, gamma, eps) without a gate
void rms_norm_gated_add_(Tensor& x, const Tensor& a, const Tensor* gamma, const Tensor* gate, float eps);
// rms_norm_gated_add_(x, a, gamma_out, gate, eps), then
// rms_norm_modulate_bf16(x, gamma_in, scale, eps) of the updated x, in one pass
Tensor rms_norm_gated_add_modulate_bf16_(Tensor& x, const Tensor& a, const Tensor* gamma_out, const Tensor* gate,
                                         const Tensor* gamma_in, const Tensor* scale, float eps);
// swiglu(gate, up) rounded to BF16 (the input of the FFN's w2)
Tensor swiglu_bf16(const Tensor& gate, const Tensor& up);

// ---- attention (tensor.h:205-212) ----
// q [N, Sq, heads*d], k and v [N, Skv, kv_heads*d] -> [N, Sq, heads*d];
// query head h reads key/value head h / (heads / kv_heads); kv_heads 0 = heads.
Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal = false, int kv_heads = 0);
// attention rounded to BF16 (the input of the block's to_out projection)
Tensor attention_bf16(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal = false,
                      int kv_heads = 0);
// opt-in, no counterpart in the reference: attention from block-scaled fp16
// operands (sdh_attention_fp16), FP32 or (out_bf16) BF16 result
// qknorm_rope_(q, k, ...) (interleaved) then attention(q, k, v, heads): q is
// left normalised and rotated, k is not modified. BF16 result with out_bf16,
// the products of attention_fp16 with fp16_products.
Tensor qknorm_rope_attention_(Tensor& q, const Tensor& k, const Tensor& v, int heads, int64_t dim,
                              const Tensor* gamma_q, const Tensor* gamma_k, float eps, const Tensor& cos,
                              const Tensor& sin, bool out_bf16, bool fp16_products = false);
Tensor attention_fp16(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal = false,
                      int kv_heads = 0, bool out_bf16 = false);

// ---- softmax (tensor.h:236) ----
// Same parameters as the reference; x is a DEVICE pointer here (rows x cols
// floats inside a backend_hip block).
void softmax_rows_(float* x, int64_t rows, int64_t cols, float scale, bool causal);
// Convenience: the whole tensor viewed as [numel / last dim, last dim].
void softmax_rows_(Tensor& x, float scale, bool causal);

// ---- fused (no single tensor.h counterpart) ----
// add_(x, r); return rms_norm(x, gamma, eps)   (zimage.cpp:123-128 order)
Tensor add_rms_norm_(Tensor& x, const Tensor& r, const Tensor* gamma, float eps);
// group_norm then silu_   (modules.cpp:34-35, vae.cpp:48-49)
Tensor group_norm_silu(const Tensor& x, int groups, const Tensor& gamma, const Tensor& beta, float eps);
// y = layer_norm(x, no affine) * (1 + scale) + shift; res += tanh(gate) * y
// (zimage.cpp:104-107, :221-224). shift and y_out may be null.
void ln_modulate_gate_(const Tensor& x, Tensor& res, const Tensor& scale, const Tensor* shift, const Tensor& gate,
                       float eps, Tensor* y_out = nullptr);
// rope_(q, ...) then rope_(k, ...) in one launch (zimage.cpp:119-120)
void rope_qk_(Tensor& q, Tensor& k, int64_t dim, const Tensor& cos, const Tensor& sin, bool interleaved);
// rms_norm_heads_(q, dim, gamma_q, eps); rms_norm_heads_(k, dim, gamma_k, eps);
// rope_(q, ...); rope_(k, ...) in one launch (zimage.cpp:117-120)
void qknorm_rope_(Tensor& q, Tensor& k, int64_t dim, const Tensor* gamma_q, const Tensor* gamma_k, float eps,
                  const Tensor& cos, const Tensor& sin, bool interleaved);

}  // namespace sdh

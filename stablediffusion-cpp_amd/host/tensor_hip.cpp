// tensor_hip.cpp - device branch of the tensor.h operators over backend_hip.
// Shape checks and their messages follow src/tensor.cpp (lines cited per op);
// the arithmetic is backend_hip's (include/sdh_backend.h).
#include "tensor_hip.h"

#include <algorithm>
#include <cstring>
#include <sstream>
#include <stdexcept>

#include "sd_hip.hpp"

namespace sdh {

struct DeviceBuffer {
    void* p = nullptr;
    size_t bytes = 0;
    explicit DeviceBuffer(size_t n) : bytes(n) { p = n ? sd::hip::malloc(n) : nullptr; }
    ~DeviceBuffer() {
        if (p) sdh_free(p);  // never throws from a destructor
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
};

const char* device_name(Device d) { return d == Device::HIP ? "hip" : "cpu"; }

// tensor.cpp:45-53 with "hip" for "cuda".
Device parse_device(const std::string& s) {
    if (s == "cpu") return Device::CPU;
    if (s == "hip") {
        if (!sd::hip::available()) throw std::runtime_error("HIP requested but not available (no MI355X visible)");
        return Device::HIP;
    }
    if (s == "auto") return sd::hip::available() ? Device::HIP : Device::CPU;
    throw std::runtime_error("unknown device '" + s + "' (use cpu, hip or auto)");
}

int64_t Tensor::numel_of(const std::vector<int64_t>& s) {
    int64_t n = 1;
    for (int64_t d : s) n *= d;
    return n;
}

Tensor::Tensor(std::vector<int64_t> s) : shape(std::move(s)), data((size_t)numel_of(shape), 0.0f) {}

Tensor::Tensor(std::vector<int64_t> s, Device d) : shape(std::move(s)), device(d) {
    if (d == Device::CPU) {
        data.assign((size_t)numel_of(shape), 0.0f);
    } else {
        const size_t bytes = (size_t)numel_of(shape) * sizeof(float);
        dev = std::make_shared<DeviceBuffer>(bytes);
        if (bytes) sd::hip::zero(dev->p, bytes);
    }
}

Tensor Tensor::empty(std::vector<int64_t> s, Device d) {
    if (d == Device::CPU) return Tensor(std::move(s));
    Tensor t;
    t.shape = std::move(s);
    t.device = d;
    t.dev = std::make_shared<DeviceBuffer>((size_t)numel_of(t.shape) * sizeof(float));
    return t;
}

Tensor Tensor::empty_bf16(std::vector<int64_t> s) {
    Tensor t;
    t.shape = std::move(s);
    t.device = Device::HIP;
    t.dtype = DType::BF16;
    t.dev = std::make_shared<DeviceBuffer>((size_t)numel_of(t.shape) * sizeof(uint16_t));
    return t;
}

float* Tensor::dptr() { return is_hip() && dev ? (float*)dev->p + dev_off : nullptr; }
const float* Tensor::dptr() const { return is_hip() && dev ? (const float*)dev->p + dev_off : nullptr; }

float* Tensor::ptr() {
    if (is_hip()) throw std::runtime_error("tensor is on the GPU; host pointer requested " + shape_str());
    return data.data();
}
const float* Tensor::ptr() const {
    if (is_hip()) throw std::runtime_error("tensor is on the GPU; host pointer requested " + shape_str());
    return data.data();
}

Tensor Tensor::to(Device d) const {
    if (d == device) return *this;
    Tensor t;
    t.shape = shape;
    t.device = d;
    t.dtype = dtype;
    const size_t bytes = (size_t)numel() * (is_bf16() ? sizeof(uint16_t) : sizeof(float));
    if (d == Device::HIP) {
        t.dev = std::make_shared<DeviceBuffer>(bytes);
        if (bytes) sd::hip::upload(t.dev->p, is_bf16() ? (const void*)data16.data() : (const void*)data.data(), bytes);
    } else if (is_bf16()) {
        t.data16.resize((size_t)numel());
        if (bytes) sd::hip::download(t.data16.data(), dptr16(), bytes);
    } else {
        t.data.resize((size_t)numel());
        if (bytes) sd::hip::download(t.data.data(), dptr(), bytes);
    }
    return t;
}

const uint16_t* Tensor::dptr16() const { return is_hip() && dev ? (const uint16_t*)dev->p + dev_off : nullptr; }
uint16_t* Tensor::dptr16() { return is_hip() && dev ? (uint16_t*)dev->p + dev_off : nullptr; }

// tensor.cpp:114-121 rounding (nearest even; inf and NaN keep their top bits)
void Tensor::to_bf16() {
    if (is_bf16()) return;
    if (is_hip()) throw std::runtime_error("to_bf16: device tensor " + shape_str());
    data16.resize(data.size());
    for (size_t i = 0; i < data.size(); ++i) {
        uint32_t b;
        std::memcpy(&b, &data[i], 4);
        data16[i] = (b & 0x7F800000u) == 0x7F800000u ? (uint16_t)(b >> 16) : (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
    }
    data.clear();
    data.shrink_to_fit();
    dtype = DType::BF16;
}

Tensor& Tensor::reshape(std::vector<int64_t> s) {
    if (numel_of(s) != numel()) throw std::runtime_error("reshape: element count mismatch for " + shape_str());
    shape = std::move(s);
    return *this;
}

std::string Tensor::shape_str() const {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < shape.size(); ++i) os << (i ? ", " : "") << shape[i];
    os << "]";
    return os.str();
}

namespace {

// total / d, or 0 when d == 0: a zero-width row leaves the op nothing to do
// (the backend returns at once for an empty extent) instead of dividing by zero
int64_t count_of(int64_t total, int64_t d) { return d ? total / d : 0; }

// The CPU branch of every op is the reference's tensor.cpp; this library
// only implements the device branch.
void need_hip(const Tensor& t, const char* op) {
    if (!t.is_hip())
        throw std::runtime_error(std::string(op) +
                                 ": host tensor; backend_hip implements the HIP device path only (the CPU path is "
                                 "the reference's tensor.cpp)");
}
// tensor.cpp:97-99
void same_device(const Tensor& a, const Tensor& b, const char* op) {
    if (a.device != b.device) throw std::runtime_error(std::string(op) + ": tensors on different devices");
}
const float* opt(const Tensor* t) { return t ? t->dptr() : nullptr; }

}  // namespace

// tensor.cpp:592-600
Tensor group_norm(const Tensor& x, int groups, const Tensor& gamma, const Tensor& beta, float eps) {
    need_hip(x, "group_norm");
    same_device(x, gamma, "group_norm");
    same_device(x, beta, "group_norm");
    const int64_t N = x.dim(0), C = x.dim(1), HW = count_of(x.numel(), (N * C));
    if (C % groups != 0) throw std::runtime_error("group_norm: channels not divisible by groups");
    Tensor y = Tensor::empty(x.shape, Device::HIP);
    sd::hip::group_norm(x.dptr(), y.dptr(), N, C, HW, groups, gamma.dptr(), beta.dptr(), eps);
    return y;
}

// tensor.cpp:628-634
Tensor layer_norm(const Tensor& x, const Tensor* gamma, const Tensor* beta, float eps) {
    need_hip(x, "layer_norm");
    if (gamma) same_device(x, *gamma, "layer_norm");
    if (beta) same_device(x, *beta, "layer_norm");
    const int64_t C = x.dim(-1), rows = count_of(x.numel(), C);
    Tensor y = Tensor::empty(x.shape, Device::HIP);
    sd::hip::layer_norm(x.dptr(), y.dptr(), rows, C, opt(gamma), opt(beta), eps);
    return y;
}

// tensor.cpp:660-666
Tensor rms_norm(const Tensor& x, const Tensor* gamma, float eps) {
    need_hip(x, "rms_norm");
    if (gamma) same_device(x, *gamma, "rms_norm");
    const int64_t C = x.dim(-1), rows = count_of(x.numel(), C);
    Tensor y = Tensor::empty(x.shape, Device::HIP);
    sd::hip::rms_norm(x.dptr(), y.dptr(), rows, C, opt(gamma), eps);
    return y;
}

// tensor.cpp:681-686
void rms_norm_heads_(Tensor& x, int64_t dim, const Tensor* gamma, float eps) {
    need_hip(x, "rms_norm_heads_");
    if (gamma) same_device(x, *gamma, "rms_norm_heads_");
    sd::hip::rms_norm_heads(x.dptr(), count_of(x.numel(), dim), dim, opt(gamma), eps);
}

// tensor.cpp:698-705
void rope_(Tensor& x, int64_t dim, const Tensor& cos, const Tensor& sin, bool interleaved) {
    need_hip(x, "rope_");
    const int64_t inner = x.dim(-1), S = x.dim(-2), N = count_of(x.numel(), (S * inner));
    if (cos.dim(0) < S || cos.dim(1) != dim) throw std::runtime_error("rope_: table shape mismatch");
    same_device(x, cos, "rope_");
    same_device(x, sin, "rope_");
    sd::hip::rope(x.dptr(), N, S, inner, dim, cos.dptr(), sin.dptr(), interleaved);
}

// tensor.cpp:732-738
Tensor swiglu(const Tensor& gate, const Tensor& up) {
    if (gate.numel() != up.numel()) throw std::runtime_error("swiglu: shape mismatch");
    same_device(gate, up, "swiglu");
    need_hip(gate, "swiglu");
    Tensor y = Tensor::empty(gate.shape, Device::HIP);
    sd::hip::swiglu(gate.dptr(), up.dptr(), y.dptr(), y.numel());
    return y;
}

// tensor.cpp:813-821
Tensor geglu(const Tensor& x) {
    need_hip(x, "geglu");
    const int64_t D2 = x.dim(-1), D = D2 / 2, rows = count_of(x.numel(), D2);
    std::vector<int64_t> oshape = x.shape;
    oshape.back() = D;
    Tensor y = Tensor::empty(oshape, Device::HIP);
    sd::hip::geglu(x.dptr(), y.dptr(), rows, D);
    return y;
}

// tensor.cpp:843-868
void silu_(Tensor& x) {
    need_hip(x, "silu_");
    sd::hip::silu(x.dptr(), x.numel());
}
void tanh_(Tensor& x) {
    need_hip(x, "tanh_");
    sd::hip::tanh(x.dptr(), x.numel());
}
void gelu_(Tensor& x) {
    need_hip(x, "gelu_");
    sd::hip::gelu(x.dptr(), x.numel());
}
void quick_gelu_(Tensor& x) {
    need_hip(x, "quick_gelu_");
    sd::hip::quick_gelu(x.dptr(), x.numel());
}

// tensor.cpp:869-887
void add_(Tensor& a, const Tensor& b) {
    if (a.numel() != b.numel()) throw std::runtime_error("add_: " + a.shape_str() + " vs " + b.shape_str());
    same_device(a, b, "add_");
    need_hip(a, "add_");
    sd::hip::add(a.dptr(), b.dptr(), a.numel());
}
void scale_(Tensor& x, float s) {
    need_hip(x, "scale_");
    sd::hip::scale(x.dptr(), s, x.numel());
}
void affine_(Tensor& x, float a, float b) {
    need_hip(x, "affine_");
    sd::hip::affine(x.dptr(), a, b, x.numel());
}

void modulation_rows_(Tensor& x) {
    need_hip(x, "modulation_rows_");
    if (x.ndim() != 2 || x.dim(0) % 2) throw std::runtime_error("modulation_rows_: x must be [2P, D], got " + x.shape_str());
    sd::hip::modulation_rows(x.dptr(), x.dim(0) / 2, x.dim(1));
}

// tensor.cpp:889-893
void mul_rows_(Tensor& x, const Tensor& v) {
    const int64_t dim = x.dim(-1), rows = count_of(x.numel(), dim);
    if (v.numel() != dim) throw std::runtime_error("mul_rows_: vector size mismatch");
    same_device(x, v, "mul_rows_");
    need_hip(x, "mul_rows_");
    sd::hip::mul_rows(x.dptr(), v.dptr(), rows, dim);
}

// tensor.cpp:903-908
void add_rows_scaled_(Tensor& x, const Tensor& y, const Tensor& g) {
    const int64_t dim = x.dim(-1), rows = count_of(x.numel(), dim);
    if (y.numel() != x.numel() || g.numel() != dim) throw std::runtime_error("add_rows_scaled_: shape mismatch");
    same_device(x, y, "add_rows_scaled_");
    same_device(x, g, "add_rows_scaled_");
    need_hip(x, "add_rows_scaled_");
    sd::hip::add_rows_scaled(x.dptr(), y.dptr(), g.dptr(), rows, dim);
}

// tensor.cpp:919-923
void add_channel_bias_(Tensor& x, const Tensor& b) {
    const int64_t N = x.dim(0), C = x.dim(1), HW = count_of(x.numel(), (N * C));
    if (b.numel() != N * C) throw std::runtime_error("add_channel_bias_: expected [N, C] bias");
    same_device(x, b, "add_channel_bias_");
    need_hip(x, "add_channel_bias_");
    sd::hip::add_channel_bias(x.dptr(), b.dptr(), N, C, HW);
}

// ---- layout ----------------------------------------------------------------

// tensor.cpp:931-949
Tensor patchify2d(const Tensor& x, int p) {
    need_hip(x, "patchify2d");
    const int64_t C = x.dim(1), H = x.dim(2), W = x.dim(3), Ht = H / p, Wt = W / p;
    if (x.dim(0) != 1 || H % p || W % p) throw std::runtime_error("patchify2d: bad shape " + x.shape_str());
    Tensor y = Tensor::empty({Ht * Wt, (int64_t)p * p * C}, Device::HIP);
    sd::hip::patchify(x.dptr(), y.dptr(), C, H, W, p);
    return y;
}

// tensor.cpp:951-968. The device path needs whole patches: the reference's
// kernel (backend_cuda.cu:438-445) reads past the tokens otherwise.
Tensor unpatchify2d(const Tensor& tokens, int64_t C, int64_t H, int64_t W, int p) {
    need_hip(tokens, "unpatchify2d");
    const int64_t Ht = H / p, Wt = W / p;
    if (tokens.numel() < Ht * Wt * p * p * C) throw std::runtime_error("unpatchify2d: too few tokens");
    if (H % p || W % p) throw std::runtime_error("unpatchify2d: H and W must be multiples of the patch size");
    Tensor y = Tensor::empty({1, C, H, W}, Device::HIP);
    sd::hip::unpatchify(tokens.dptr(), y.dptr(), C, H, W, p);
    return y;
}

// tensor.cpp:970-980
Tensor slice_rows(const Tensor& x, int64_t from, int64_t to) {
    need_hip(x, "slice_rows");
    const int64_t D = x.dim(-1), rows = count_of(x.numel(), D);
    if (from < 0 || to > rows || from > to) throw std::runtime_error("slice_rows: range out of bounds");
    Tensor y = Tensor::empty({to - from, D}, Device::HIP);
    const size_t bytes = (size_t)((to - from) * D) * sizeof(float);
    if (bytes) sd::hip::copy(y.dptr(), x.dptr() + from * D, bytes);
    return y;
}

Tensor rows_view(const Tensor& x, int64_t from, int64_t to) {
    need_hip(x, "rows_view");
    if (x.is_bf16()) throw std::runtime_error("rows_view: F32 tensors only");
    const int64_t D = x.dim(-1), rows = count_of(x.numel(), D);
    if (from < 0 || to > rows || from > to) throw std::runtime_error("rows_view: range out of bounds");
    Tensor v;
    v.shape = {to - from, D};
    v.device = Device::HIP;
    v.dev = x.dev;
    v.dev_off = x.dev_off + from * D;
    return v;
}

// tensor.cpp:982-1004
Tensor upsample_nearest2x(const Tensor& x) {
    need_hip(x, "upsample_nearest2x");
    const int64_t N = x.dim(0), C = x.dim(1), H = x.dim(2), W = x.dim(3);
    Tensor y = Tensor::empty({N, C, 2 * H, 2 * W}, Device::HIP);
    sd::hip::upsample_nearest2x(x.dptr(), y.dptr(), N * C, H, W);
    return y;
}

// tensor.cpp:1006-1023
Tensor concat_channels(const Tensor& a, const Tensor& b) {
    const int64_t N = a.dim(0), Ca = a.dim(1), Cb = b.dim(1), H = a.dim(2), W = a.dim(3);
    if (b.dim(0) != N || b.dim(2) != H || b.dim(3) != W)
        throw std::runtime_error("concat_channels: " + a.shape_str() + " vs " + b.shape_str());
    same_device(a, b, "concat_channels");
    need_hip(a, "concat_channels");
    Tensor y = Tensor::empty({N, Ca + Cb, H, W}, Device::HIP);
    sd::hip::concat_channels(a.dptr(), b.dptr(), y.dptr(), N, Ca, Cb, H * W);
    return y;
}

// tensor.cpp:1025-1039: y takes a's shape with the batches added, then a's
// and b's elements are copied in order. Like the reference, a b with other
// trailing dimensions is copied flat and any tail it leaves stays zero
// (test_ops.cpp:467 relies on that); a b that would overrun y is an error.
Tensor concat_batch(const Tensor& a, const Tensor& b) {
    same_device(a, b, "concat_batch");
    need_hip(a, "concat_batch");
    std::vector<int64_t> s = a.shape;
    s[0] += b.dim(0);
    const int64_t n = Tensor::numel_of(s);
    if (a.numel() + b.numel() > n) throw std::runtime_error("concat_batch: " + a.shape_str() + " vs " + b.shape_str());
    Tensor y = a.numel() + b.numel() == n ? Tensor::empty(s, Device::HIP) : Tensor(s, Device::HIP);
    if (a.numel()) sd::hip::copy(y.dptr(), a.dptr(), a.numel() * sizeof(float));
    if (b.numel()) sd::hip::copy(y.dptr() + a.numel(), b.dptr(), b.numel() * sizeof(float));
    return y;
}

// tensor.cpp:1041-1056
Tensor nchw_to_nlc(const Tensor& x) {
    need_hip(x, "nchw_to_nlc");
    const int64_t N = x.dim(0), C = x.dim(1), HW = x.dim(2) * x.dim(3);
    Tensor y = Tensor::empty({N, HW, C}, Device::HIP);
    sd::hip::nchw_to_nlc(x.dptr(), y.dptr(), N, C, HW);
    return y;
}

// tensor.cpp:1058-1074
Tensor nlc_to_nchw(const Tensor& x, int64_t H, int64_t W) {
    need_hip(x, "nlc_to_nchw");
    const int64_t N = x.dim(0), HW = x.dim(1), C = x.dim(2);
    if (HW != H * W) throw std::runtime_error("nlc_to_nchw: bad spatial size");
    Tensor y = Tensor::empty({N, C, H, W}, Device::HIP);
    sd::hip::nlc_to_nchw(x.dptr(), y.dptr(), N, C, HW);
    return y;
}

// tensor.cpp:1076-1086
Tensor slice_batch(const Tensor& x, int64_t b) {
    need_hip(x, "slice_batch");
    if (b < 0 || b >= x.dim(0)) throw std::runtime_error("slice_batch: index out of range");
    std::vector<int64_t> s = x.shape;
    s[0] = 1;
    Tensor y = Tensor::empty(s, Device::HIP);
    const int64_t per = count_of(x.numel(), x.dim(0));
    if (per) sd::hip::copy(y.dptr(), x.dptr() + b * per, per * sizeof(float));
    return y;
}

// tensor.cpp:1088-1099
Tensor repeat_batch(const Tensor& x, int64_t times) {
    need_hip(x, "repeat_batch");
    std::vector<int64_t> s = x.shape;
    s[0] = x.dim(0) * times;
    Tensor y = Tensor::empty(s, Device::HIP);
    for (int64_t t = 0; t < times; ++t)
        if (x.numel()) sd::hip::copy(y.dptr() + t * x.numel(), x.dptr(), x.numel() * sizeof(float));
    return y;
}

// ---- linear ------------------------------------------------------------------

// tensor.cpp:481-494, device branch: BF16 weights on the MFMA GEMM, F32 weights on the fp32 GEMM
Tensor linear(const Tensor& x, const Tensor& W, const Tensor* b) {
    const int64_t in = x.dim(-1), out = W.dim(0);
    if (W.dim(1) != in) throw std::runtime_error("linear: input dim " + x.shape_str() + " vs weight " + W.shape_str());
    std::vector<int64_t> oshape = x.shape;
    oshape.back() = out;
    const int64_t rows = Tensor::numel_of(std::vector<int64_t>(x.shape.begin(), x.shape.end() - 1));
    same_device(x, W, "linear");
    need_hip(x, "linear");
    if (b) same_device(x, *b, "linear");
    Tensor y = Tensor::empty(oshape, Device::HIP);
    if (x.is_bf16()) {
        if (!W.is_bf16()) throw std::runtime_error("linear: a BF16 input needs BF16 weights " + W.shape_str());
        sd::hip::gemm_nt_bf16_packed(rows, out, in, x.dptr16(), in, W.dptr16(), in, y.dptr(), out, opt(b), false);
    } else if (W.is_bf16()) {
        sd::hip::gemm_nt_bf16(rows, out, in, x.dptr(), in, W.dptr16(), in, y.dptr(), out, opt(b), false);
    } else {
        sd::hip::gemm_nt_f32(rows, out, in, x.dptr(), in, W.dptr(), in, y.dptr(), out, opt(b), false);
    }
    return y;
}

Tensor linear_swiglu(const Tensor& x, const Tensor& w1, const Tensor& w3) {
    const int64_t in = x.dim(-1), hidden = w1.dim(0);
    if (w1.dim(1) != in || w3.dim(0) != hidden || w3.dim(1) != in)
        throw std::runtime_error("linear_swiglu: " + x.shape_str() + " vs " + w1.shape_str() + " / " + w3.shape_str());
    same_device(x, w1, "linear_swiglu");
    same_device(x, w3, "linear_swiglu");
    need_hip(x, "linear_swiglu");
    if (!w1.is_bf16() || !w3.is_bf16()) throw std::runtime_error("linear_swiglu: weights must be BF16");
    std::vector<int64_t> oshape = x.shape;
    oshape.back() = hidden;
    Tensor y = Tensor::empty(oshape, Device::HIP);
    sd::hip::linear_swiglu(x.dptr(), w1.dptr16(), w3.dptr16(), y.dptr(),
                           Tensor::numel_of(std::vector<int64_t>(x.shape.begin(), x.shape.end() - 1)), in, hidden);
    return y;
}

// tensor.cpp:529-541: the reference's shape checks and messages, device branch
Tensor conv2d(const Tensor& x, const Tensor& W, const Tensor* b, int stride, int pad) {
    const int64_t N = x.dim(0), Cin = x.dim(1), H = x.dim(2), Wd = x.dim(3);
    const int64_t Cout = W.dim(0), kh = W.dim(2), kw = W.dim(3);
    if (W.dim(1) != Cin) throw std::runtime_error("conv2d: input " + x.shape_str() + " vs weight " + W.shape_str());
    const int64_t Ho = (H + 2 * pad - kh) / stride + 1, Wo = (Wd + 2 * pad - kw) / stride + 1;
    same_device(x, W, "conv2d");
    need_hip(x, "conv2d");
    if (W.is_bf16()) throw std::runtime_error("conv2d: bf16 conv weights are not supported");
    if (b) same_device(x, *b, "conv2d");
    Tensor out = Tensor::empty({N, Cout, Ho, Wo}, Device::HIP);
    sd::hip::conv2d(x.dptr(), N, Cin, H, Wd, W.dptr(), Cout, kh, kw, opt(b), stride, pad, out.dptr(), Ho, Wo);
    return out;
}

// tensor.cpp:776-790: the reference's shape checks and messages, device branch
namespace {
Tensor attention_impl(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal, int kv_heads,
                      bool bf16, bool fp16_products = false) {
    if (kv_heads <= 0) kv_heads = heads;
    const int64_t N = q.dim(0), Sq = q.dim(1), inner = q.dim(2), Skv = k.dim(1), kv_inner = k.dim(2);
    if (inner % heads != 0 || heads % kv_heads != 0) throw std::runtime_error("attention: heads mismatch");
    const int64_t d = inner / heads;
    if (k.dim(0) != N || v.dim(0) != N || v.dim(1) != Skv || kv_inner != kv_heads * d || v.dim(2) != kv_inner)
        throw std::runtime_error("attention: shape mismatch q" + q.shape_str() + " k" + k.shape_str());
    same_device(q, k, "attention");
    same_device(q, v, "attention");
    need_hip(q, "attention");
    if (bf16) {
        Tensor out = Tensor::empty_bf16({N, Sq, inner});
        if (fp16_products)
            sd::hip::attention_fp16(q.dptr(), k.dptr(), v.dptr(), out.dptr16(), true, N, Sq, Skv, heads, kv_heads, d,
                                    causal);
        else
            sd::hip::attention_bf16(q.dptr(), k.dptr(), v.dptr(), out.dptr16(), N, Sq, Skv, heads, kv_heads, d, causal);
        return out;
    }
    Tensor out = Tensor::empty({N, Sq, inner}, Device::HIP);
    if (fp16_products)
        sd::hip::attention_fp16(q.dptr(), k.dptr(), v.dptr(), out.dptr(), false, N, Sq, Skv, heads, kv_heads, d, causal);
    else
        sd::hip::attention(q.dptr(), k.dptr(), v.dptr(), out.dptr(), N, Sq, Skv, heads, kv_heads, d, causal);
    return out;
}
}  // namespace

Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal, int kv_heads) {
    return attention_impl(q, k, v, heads, causal, kv_heads, false);
}

Tensor attention_bf16(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal, int kv_heads) {
    return attention_impl(q, k, v, heads, causal, kv_heads, true);
}

Tensor attention_fp16(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal, int kv_heads,
                      bool out_bf16) {
    return attention_impl(q, k, v, heads, causal, kv_heads, out_bf16, true);
}

// ---- the Z-Image block's fused ops ----
Tensor rms_norm_modulate_bf16(const Tensor& x, const Tensor* gamma, const Tensor* scale, float eps) {
    need_hip(x, "rms_norm_modulate_bf16");
    if (gamma) same_device(x, *gamma, "rms_norm_modulate_bf16");
    if (scale) same_device(x, *scale, "rms_norm_modulate_bf16");
    const int64_t C = x.dim(-1), rows = count_of(x.numel(), C);
    if ((gamma && gamma->numel() != C) || (scale && scale->numel() != C))
        throw std::runtime_error("rms_norm_modulate_bf16: vector length vs " + x.shape_str());
    Tensor y = Tensor::empty_bf16(x.shape);
    sd::hip::rms_norm_modulate_bf16(x.dptr(), y.dptr16(), rows, C, opt(gamma), opt(scale), eps);
    return y;
}

void rms_norm_gated_add_(Tensor& x, const Tensor& a, const Tensor* gamma, const Tensor* gate, float eps) {
    need_hip(x, "rms_norm_gated_add_");
    same_device(x, a, "rms_norm_gated_add_");
    if (x.numel() != a.numel() || x.dim(-1) != a.dim(-1))
        throw std::runtime_error("rms_norm_gated_add_: " + x.shape_str() + " vs " + a.shape_str());
    const int64_t C = x.dim(-1), rows = count_of(x.numel(), C);
    if ((gamma && gamma->numel() != C) || (gate && gate->numel() != C))
        throw std::runtime_error("rms_norm_gated_add_: vector length vs " + x.shape_str());
    sd::hip::rms_norm_gated_add(x.dptr(), a.dptr(), rows, C, opt(gamma), opt(gate), eps);
}

Tensor rms_norm_gated_add_modulate_bf16_(Tensor& x, const Tensor& a, const Tensor* gamma_out, const Tensor* gate,
                                         const Tensor* gamma_in, const Tensor* scale, float eps) {
    const char* op = "rms_norm_gated_add_modulate_bf16_";
    need_hip(x, op);
    same_device(x, a, op);
    if (x.numel() != a.numel() || x.dim(-1) != a.dim(-1))
        throw std::runtime_error(std::string(op) + ": " + x.shape_str() + " vs " + a.shape_str());
    const int64_t C = x.dim(-1), rows = count_of(x.numel(), C);
    for (const Tensor* v : {gamma_out, gate, gamma_in, scale}) {
        if (!v) continue;
        same_device(x, *v, op);
        if (v->numel() != C) throw std::runtime_error(std::string(op) + ": vector length vs " + x.shape_str());
    }
    Tensor y = Tensor::empty_bf16(x.shape);
    sd::hip::rms_norm_gated_add_modulate_bf16(x.dptr(), a.dptr(), y.dptr16(), rows, C, opt(gamma_out), opt(gate),
                                              opt(gamma_in), opt(scale), eps, eps);
    return y;
}

Tensor swiglu_bf16(const Tensor& gate, const Tensor& up) {
    if (gate.numel() != up.numel()) throw std::runtime_error("swiglu: " + gate.shape_str() + " vs " + up.shape_str());
    same_device(gate, up, "swiglu");
    need_hip(gate, "swiglu_bf16");
    Tensor y = Tensor::empty_bf16(gate.shape);
    sd::hip::swiglu_bf16(gate.dptr(), up.dptr(), y.dptr16(), gate.numel());
    return y;
}

// tensor.cpp:752 (device pointer)
void softmax_rows_(float* x, int64_t rows, int64_t cols, float scale, bool causal) {
    sd::hip::softmax_rows(x, rows, cols, scale, causal);
}
void softmax_rows_(Tensor& x, float scale, bool causal) {
    need_hip(x, "softmax_rows_");
    const int64_t cols = x.dim(-1);
    sd::hip::softmax_rows(x.dptr(), count_of(x.numel(), cols), cols, scale, causal);
}

// ---- fused ----
Tensor add_rms_norm_(Tensor& x, const Tensor& r, const Tensor* gamma, float eps) {
    if (x.numel() != r.numel()) throw std::runtime_error("add_: " + x.shape_str() + " vs " + r.shape_str());
    same_device(x, r, "add_rms_norm_");
    need_hip(x, "add_rms_norm_");
    const int64_t C = x.dim(-1), rows = count_of(x.numel(), C);
    Tensor y = Tensor::empty(x.shape, Device::HIP);
    sd::hip::add_rms_norm(x.dptr(), r.dptr(), y.dptr(), rows, C, opt(gamma), eps);
    return y;
}

Tensor group_norm_silu(const Tensor& x, int groups, const Tensor& gamma, const Tensor& beta, float eps) {
    need_hip(x, "group_norm_silu");
    same_device(x, gamma, "group_norm_silu");
    same_device(x, beta, "group_norm_silu");
    const int64_t N = x.dim(0), C = x.dim(1), HW = count_of(x.numel(), (N * C));
    if (C % groups != 0) throw std::runtime_error("group_norm: channels not divisible by groups");
    Tensor y = Tensor::empty(x.shape, Device::HIP);
    sd::hip::group_norm_silu(x.dptr(), y.dptr(), N, C, HW, groups, gamma.dptr(), beta.dptr(), eps);
    return y;
}

void ln_modulate_gate_(const Tensor& x, Tensor& res, const Tensor& scale, const Tensor* shift, const Tensor& gate,
                       float eps, Tensor* y_out) {
    need_hip(x, "ln_modulate_gate_");
    same_device(x, res, "ln_modulate_gate_");
    const int64_t C = x.dim(-1), rows = count_of(x.numel(), C);
    if (res.numel() != x.numel() || scale.numel() != C || gate.numel() != C || (shift && shift->numel() != C))
        throw std::runtime_error("ln_modulate_gate_: shape mismatch");
    if (y_out && (y_out->numel() != x.numel() || !y_out->is_hip()))
        throw std::runtime_error("ln_modulate_gate_: y_out must be a device tensor shaped like x");
    sd::hip::ln_modulate_gate(x.dptr(), res.dptr(), scale.dptr(), opt(shift), gate.dptr(),
                              y_out ? y_out->dptr() : nullptr, rows, C, eps);
}

void rope_qk_(Tensor& q, Tensor& k, int64_t dim, const Tensor& cos, const Tensor& sin, bool interleaved) {
    need_hip(q, "rope_qk_");
    same_device(q, k, "rope_qk_");
    const int64_t S = q.dim(-2), N = count_of(q.numel(), (S * q.dim(-1)));
    if (k.dim(-2) != S || count_of(k.numel(), (S * k.dim(-1))) != N)
        throw std::runtime_error("rope_qk_: q/k token mismatch");
    if (cos.dim(0) < S || cos.dim(1) != dim) throw std::runtime_error("rope_: table shape mismatch");
    sd::hip::rope_qk(q.dptr(), q.dim(-1), k.dptr(), k.dim(-1), N, S, dim, cos.dptr(), sin.dptr(), interleaved);
}

// zimage.cpp:117-120 / qwen3.cpp:59-62 in one launch
Tensor qknorm_rope_attention_(Tensor& q, const Tensor& k, const Tensor& v, int heads, int64_t dim,
                              const Tensor* gamma_q, const Tensor* gamma_k, float eps, const Tensor& cos,
                              const Tensor& sin, bool out_bf16, bool fp16_products) {
    const char* op = "qknorm_rope_attention_";
    need_hip(q, op);
    same_device(q, k, op);
    same_device(q, v, op);
    for (const Tensor* t : {gamma_q, gamma_k}) {
        if (!t) continue;
        same_device(q, *t, op);
        if (t->numel() != dim) throw std::runtime_error("rms_norm_heads_: weight size mismatch");
    }
    const int64_t N = q.dim(0), S = q.dim(1), inner = q.dim(2);
    if (inner != heads * dim || k.shape != q.shape || v.shape != q.shape)
        throw std::runtime_error("attention: shape mismatch q" + q.shape_str() + " k" + k.shape_str());
    if (cos.dim(0) < S || cos.dim(1) != dim || sin.shape != cos.shape)
        throw std::runtime_error("rope_: table shape mismatch");
    Tensor out = out_bf16 ? Tensor::empty_bf16({N, S, inner}) : Tensor::empty({N, S, inner}, Device::HIP);
    sd::hip::qknorm_rope_attention(q.dptr(), k.dptr(), v.dptr(), out_bf16 ? (void*)out.dptr16() : (void*)out.dptr(),
                                   out_bf16, N, S, heads, dim, opt(gamma_q), opt(gamma_k), eps, cos.dptr(),
                                   sin.dptr(), fp16_products);
    return out;
}

void qknorm_rope_(Tensor& q, Tensor& k, int64_t dim, const Tensor* gamma_q, const Tensor* gamma_k, float eps,
                  const Tensor& cos, const Tensor& sin, bool interleaved) {
    need_hip(q, "qknorm_rope_");
    same_device(q, k, "qknorm_rope_");
    if (gamma_q) same_device(q, *gamma_q, "qknorm_rope_");
    if (gamma_k) same_device(q, *gamma_k, "qknorm_rope_");
    const int64_t S = q.dim(-2), N = count_of(q.numel(), (S * q.dim(-1)));
    if (k.dim(-2) != S || count_of(k.numel(), (S * k.dim(-1))) != N)
        throw std::runtime_error("qknorm_rope_: q/k token mismatch");
    if (cos.dim(0) < S || cos.dim(1) != dim) throw std::runtime_error("rope_: table shape mismatch");
    sd::hip::qknorm_rope(q.dptr(), q.dim(-1), k.dptr(), k.dim(-1), N, S, dim, opt(gamma_q), opt(gamma_k), eps,
                         cos.dptr(), sin.dptr(), interleaved);
}

}  // namespace sdh

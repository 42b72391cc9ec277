// sanitize_host.cpp - the host side of the library under AddressSanitizer and
// UndefinedBehaviorSanitizer, on the CPU (built and run by
// tests/test_sanitize.py with g++, against the no-GPU stub backend).
//
//   sanitize_host weights <file> ...  load each .safetensors file; one line
//                                     per file: "rejected <message>" for a
//                                     header or layout error, "device <message>"
//                                     when parsing finished and the upload
//                                     reached the (absent) device
//   sanitize_host shim                 the C-ABI status -> exception shim and
//                                     the host API's argument checks
//   sanitize_host oracle               every oracle routine on small odd shapes
//
// Exit status 0 unless a check fails; the sanitizers abort on any finding.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "sd_hip.hpp"
#include "tensor_hip.h"
#include "weights_hip.h"

extern "C" {
#include "sd_oracle.h"
}

namespace {

int failures = 0;

void expect(bool ok, const std::string& what) {
    if (!ok) {
        std::printf("FAIL %s\n", what.c_str());
        ++failures;
    }
}

// f must throw std::runtime_error
void expect_throw(const std::function<void()>& f, const std::string& what) {
    try {
        f();
    } catch (const std::runtime_error&) {
        return;
    } catch (const std::exception& e) {
        expect(false, what + ": threw a non-runtime_error: " + e.what());
        return;
    }
    expect(false, what + ": did not throw");
}

int weights(int argc, char** argv) {
    for (int i = 2; i < argc; ++i) {
        sdh::Weights w;
        try {
            w.load_safetensors(argv[i], i % 2 == 0, 4);
            std::printf("loaded\n");
        } catch (const std::runtime_error& e) {
            const std::string m = e.what();
            const bool header = m.rfind("safetensors", 0) == 0 || m.rfind("cannot open", 0) == 0;
            std::printf("%s %s\n", header ? "rejected" : "device", m.c_str());
        } catch (const std::exception& e) {
            std::printf("FAIL %s: non-runtime_error %s\n", argv[i], e.what());
            ++failures;
        }
    }
    return failures ? 1 : 0;
}

int shim() {
    expect(!sd::hip::available(), "the stub reports no device");
    float h[4] = {1, 2, 3, 4};
    expect_throw([&] { sd::hip::rms_norm(h, h, 1, 4, nullptr, 1e-6f); }, "shim: stub status becomes an exception");
    expect_throw([&] { (void)sd::hip::malloc(64); }, "shim: malloc on the stub");
    expect_throw([] { (void)sdh::parse_device("hip"); }, "parse_device(hip) without a device");
    expect_throw([] { (void)sdh::parse_device("gpu"); }, "parse_device of an unknown name");
    expect(sdh::parse_device("auto") == sdh::Device::CPU, "parse_device(auto) falls back to the CPU");
    sdh::Tensor x({2, 8}), g({8}), wrong({7});
    expect_throw([&] { (void)sdh::rms_norm(x, &g, 1e-6f); }, "a host tensor is refused by a device op");
    expect_throw([&] { sdh::mul_rows_(x, wrong); }, "a vector of the wrong length is refused");
    expect_throw([&] { (void)x.to(sdh::Device::HIP); }, "an upload without a device");
    expect_throw([&] { (void)sdh::Tensor::empty({4}, sdh::Device::HIP); }, "a device tensor without a device");
    sdh::Tensor r({3, 5});
    r.reshape({5, 3});
    expect(r.numel() == 15 && r.dim(-1) == 3, "reshape keeps the element count");
    expect_throw([&] { r.reshape({4, 4}); }, "reshape to another element count");
    return failures ? 1 : 0;
}

std::vector<float> randn(int64_t n, uint64_t seed, double mean = 0.0, double std = 1.0) {
    std::vector<float> v((size_t)std::max<int64_t>(n, 1));
    orc_fill_normal(v.data(), n, seed, mean, std);
    return v;
}

bool finite(const std::vector<float>& v, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        if (!std::isfinite(v[(size_t)i])) return false;
    return true;
}

int oracle() {
    orc_set_threads(3);
    for (int64_t rows : {1, 3, 7}) {
        for (int64_t C : {1, 5, 130}) {
            const int64_t n = rows * C;
            auto x = randn(n, 1), y = randn(n, 2), g = randn(C, 3, 1.0, 0.1), b = randn(C, 4, 0.0, 0.1);
            std::vector<float> o((size_t)n);
            orc_rms_norm(x.data(), o.data(), rows, C, g.data(), 1e-6f);
            orc_layer_norm(x.data(), o.data(), rows, C, g.data(), b.data(), 1e-6f);
            orc_layer_norm(x.data(), o.data(), rows, C, nullptr, nullptr, 1e-6f);
            auto s = x;
            orc_add_rms_norm(s.data(), y.data(), o.data(), rows, C, g.data(), 1e-6f);
            auto res = y;
            orc_ln_modulate_gate(x.data(), res.data(), g.data(), b.data(), g.data(), o.data(), rows, C, 1e-6f);
            orc_softmax_rows(o.data(), rows, C, 0.5f, 1);
            orc_softmax_rows_period(o.data(), rows, C, 0.5f, 1, rows > 1 ? rows - 1 : 1);
            orc_mul_rows(o.data(), g.data(), rows, C);
            orc_add_rows_scaled(o.data(), y.data(), g.data(), rows, C);
            orc_swiglu(x.data(), y.data(), o.data(), n);
            orc_silu(o.data(), n);
            orc_tanh(o.data(), n);
            orc_gelu(o.data(), n);
            orc_quick_gelu(o.data(), n);
            orc_add(o.data(), x.data(), n);
            orc_scale(o.data(), 0.5f, n);
            orc_affine(o.data(), 1.0f, 1.0f, n);
            expect(finite(o, n), "oracle row ops finite");
            if (C % 2 == 0) {
                std::vector<float> gg((size_t)(rows * C / 2));
                orc_geglu(x.data(), gg.data(), rows, C / 2);
            }
        }
    }
    for (int groups : {1, 2, 4}) {
        const int64_t N = 2, C = 8, HW = 9, n = N * C * HW;
        auto x = randn(n, 5, 0.0, 2.0), g = randn(C, 6, 1.0, 0.1), b = randn(C, 7, 0.0, 0.1);
        std::vector<float> o((size_t)n);
        orc_group_norm(x.data(), o.data(), N, C, HW, groups, g.data(), b.data(), 1e-6f);
        orc_group_norm_silu(x.data(), o.data(), N, C, HW, groups, g.data(), b.data(), 1e-6f);
        orc_add_channel_bias(o.data(), b.data(), 1, C, N * HW);
        expect(finite(o, n), "oracle group norm finite");
    }
    {
        const int64_t N = 1, S = 6, dim = 8, heads = 3, inner = heads * dim;
        std::vector<float> cs((size_t)(S * dim)), sn((size_t)(S * dim));
        orc_rope_tables_half(S, dim, 10000.0, cs.data(), sn.data());
        const int32_t axes[3] = {2, 2, 4};
        std::vector<int32_t> pos((size_t)(S * 3));
        for (int64_t s = 0; s < S; ++s) pos[(size_t)(3 * s + 1)] = (int32_t)(s / 3), pos[(size_t)(3 * s + 2)] = (int32_t)(s % 3);
        orc_rope_tables_3axis(pos.data(), S, axes, dim, 256.0, cs.data(), sn.data());
        auto q = randn(N * S * inner, 8), k = randn(N * S * inner, 9), gq = randn(dim, 10, 1.0, 0.1);
        orc_rope(q.data(), N, S, inner, dim, cs.data(), sn.data(), 1);
        orc_rope(q.data(), N, S, inner, dim, cs.data(), sn.data(), 0);
        orc_rms_norm_heads(k.data(), N * S * heads, dim, gq.data(), 1e-6f);
        orc_qknorm_rope(q.data(), inner, k.data(), inner, N, S, dim, gq.data(), gq.data(), 1e-6f, cs.data(), sn.data(), 1);
        expect(finite(q, N * S * inner) && finite(k, N * S * inner), "oracle rotary finite");
    }
    {
        const int64_t C = 3, H = 4, W = 6;
        auto x = randn(C * H * W, 11);
        std::vector<float> up((size_t)(C * 4 * H * W)), t((size_t)(C * H * W)), back((size_t)(C * H * W));
        orc_upsample_nearest2x(x.data(), up.data(), C, H, W);
        orc_nchw_to_nlc(x.data(), t.data(), 1, C, H * W);
        orc_nlc_to_nchw(t.data(), back.data(), 1, C, H * W);
        expect(std::memcmp(x.data(), back.data(), x.size() * 4) == 0, "oracle layout round trip");
        orc_patchify(x.data(), t.data(), C, H, W, 2);
        orc_unpatchify(t.data(), back.data(), C, H, W, 2);
        expect(std::memcmp(x.data(), back.data(), x.size() * 4) == 0, "oracle patchify round trip");
        std::vector<float> cat((size_t)(2 * C * H * W));
        orc_concat_channels(x.data(), x.data(), cat.data(), 1, C, C, H * W);
    }
    return failures ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: sanitize_host weights <files> | shim | oracle\n");
        return 2;
    }
    const std::string mode = argv[1];
    int rc = 2;
    if (mode == "weights") rc = weights(argc, argv);
    else if (mode == "shim") rc = shim();
    else if (mode == "oracle") rc = oracle();
    if (rc == 0) std::printf("ok\n");
    return rc;
}

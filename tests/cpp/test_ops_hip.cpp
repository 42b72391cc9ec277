// test_ops_hip.cpp - the reference's GPU-vs-CPU op test (tests/test_ops.cpp:
// 356-477, "test_cuda") restated for backend_hip: every op runs through the
// tensor.h-style host API (sdh::Tensor, device branch) and through the CPU
// oracle on the same inputs; max|diff| must stay within the reference test's
// tolerance for that op. The fused ops are checked against their reference
// compositions, at the reference's tiny shapes and at the Z-Image config
// shapes. Exit status is non-zero if any check fails; without a GPU the
// device section is skipped, as the reference's test does (test_ops.cpp:357-360).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "sd_oracle.h"
#include "sd_hip.hpp"
#include "tensor_hip.h"

using sdh::Device;
using sdh::Tensor;

static int failures = 0;
static uint64_t g_seed = 1234;

static void check(const char* name, double err, double tol) {
    const bool ok = err <= tol;
    std::printf("%-34s max|err| = %.3e  %s\n", name, err, ok ? "ok" : "FAIL");
    if (!ok) ++failures;
}

static Tensor randn_t(std::vector<int64_t> shape, float mean = 0.f, float std = 1.f) {
    Tensor t(std::move(shape));
    orc_fill_normal(t.data.data(), t.numel(), g_seed++, mean, std);
    return t;
}

static double max_diff(const Tensor& cpu, const Tensor& dev) {
    Tensor b = dev.to(Device::CPU);
    if (cpu.numel() != b.numel()) return 1e30;
    double e = 0;
    for (int64_t i = 0; i < cpu.numel(); ++i) e = std::max(e, (double)std::fabs(cpu.data[i] - b.data[i]));
    return e;
}

// max |a-b| / max(|a|, 1): the relative bound used for reductions
static double rel_diff(const Tensor& cpu, const Tensor& dev) {
    Tensor b = dev.to(Device::CPU);
    if (cpu.numel() != b.numel()) return 1e30;
    double e = 0;
    for (int64_t i = 0; i < cpu.numel(); ++i)
        e = std::max(e, std::fabs((double)cpu.data[i] - b.data[i]) / std::max(1.0, (double)std::fabs(cpu.data[i])));
    return e;
}

static void hip_check_op(const char* name, const Tensor& cpu, const Tensor& gpu, double tol) {
    char label[80];
    std::snprintf(label, sizeof label, "hip %s", name);
    check(label, max_diff(cpu, gpu), tol);
}

static bool throws(const std::function<void()>& f) {
    try {
        f();
    } catch (const std::exception&) {
        return true;
    }
    return false;
}

// test_ops.cpp:84-114: attention restated per head in double, softmax(q k^T / sqrt(d)) v
static Tensor attention_double(const Tensor& q, const Tensor& k, const Tensor& v, int heads, bool causal,
                               int kv_heads) {
    if (kv_heads <= 0) kv_heads = heads;
    const int64_t N = q.dim(0), Sq = q.dim(1), inner = q.dim(2), Skv = k.dim(1), d = inner / heads;
    const int64_t kv_inner = kv_heads * d, group = heads / kv_heads;
    const double scale = 1.0 / std::sqrt((double)(float)d);
    Tensor o({N, Sq, inner});
    std::vector<double> sc((size_t)Skv);
    for (int64_t n = 0; n < N; ++n)
        for (int h = 0; h < heads; ++h) {
            const float* qb = q.data.data() + n * Sq * inner + h * d;
            const float* kb = k.data.data() + n * Skv * kv_inner + (h / group) * d;
            const float* vb = v.data.data() + n * Skv * kv_inner + (h / group) * d;
            for (int64_t i = 0; i < Sq; ++i) {
                double m = -1e300;
                for (int64_t j = 0; j < Skv; ++j) {
                    double s = 0;
                    for (int64_t t = 0; t < d; ++t) s += (double)qb[i * inner + t] * kb[j * kv_inner + t];
                    sc[j] = (causal && j > i) ? -1e300 : s * scale;
                    m = std::max(m, sc[j]);
                }
                double sum = 0;
                for (int64_t j = 0; j < Skv; ++j) {
                    sc[j] = (causal && j > i) ? 0.0 : std::exp(sc[j] - m);
                    sum += sc[j];
                }
                for (int64_t t = 0; t < d; ++t) {
                    double acc = 0;
                    for (int64_t j = 0; j < Skv; ++j) acc += sc[j] / sum * vb[j * kv_inner + t];
                    o.data[(n * Sq + i) * inner + h * d + t] = (float)acc;
                }
            }
        }
    return o;
}

static void test_hip() {
    const Device G = Device::HIP;
    // attention: MHA, causal, GQA, 100 tokens, 8/2 causal batch 2 (test_ops.cpp:439-451), 1e-4
    {
        Tensor q = randn_t({2, 9, 24}), k = randn_t({2, 9, 24}), v = randn_t({2, 9, 24});
        hip_check_op("attention h3", attention_double(q, k, v, 3, false, 0),
                     sdh::attention(q.to(G), k.to(G), v.to(G), 3), 1e-4);
        hip_check_op("attention h3 causal", attention_double(q, k, v, 3, true, 0),
                     sdh::attention(q.to(G), k.to(G), v.to(G), 3, true), 1e-4);
        Tensor kk = randn_t({2, 9, 8}), vv = randn_t({2, 9, 8});
        hip_check_op("attention gqa", attention_double(q, kk, vv, 3, false, 1),
                     sdh::attention(q.to(G), kk.to(G), vv.to(G), 3, false, 1), 1e-4);
        Tensor qb = randn_t({1, 100, 64}), kb = randn_t({1, 100, 64}), vb = randn_t({1, 100, 64});
        hip_check_op("attention 100 tokens", attention_double(qb, kb, vb, 2, false, 0),
                     sdh::attention(qb.to(G), kb.to(G), vb.to(G), 2), 1e-4);
        Tensor q8 = randn_t({2, 37, 8 * 16}), k2 = randn_t({2, 37, 2 * 16}), v2 = randn_t({2, 37, 2 * 16});
        hip_check_op("attention gqa 8/2 causal", attention_double(q8, k2, v2, 8, true, 2),
                     sdh::attention(q8.to(G), k2.to(G), v2.to(G), 8, true, 2), 1e-4);
        int bad = 0;
        bad += !throws([&] { sdh::attention(q.to(G), kk.to(G), vv.to(G), 3, false, 2); });  // tensor.cpp:779
        bad += !throws([&] { sdh::attention(q.to(G), qb.to(G), qb.to(G), 3); });            // tensor.cpp:781-782
        check("attention shape errors throw", (double)bad, 0.0);
    }
    // round trip (test_ops.cpp:365-368)
    {
        Tensor x = randn_t({3, 70});
        hip_check_op("to(hip).to(cpu)", x, x.to(G), 0.0);
    }
    // norms (test_ops.cpp:390-402): tolerance 1e-4
    {
        Tensor x = randn_t({2, 64, 5, 7}), g = randn_t({64}), b = randn_t({64});
        Tensor y({2, 64, 5, 7});
        orc_group_norm(x.data.data(), y.data.data(), 2, 64, 35, 32, g.data.data(), b.data.data(), 1e-6f);
        hip_check_op("group_norm", y, sdh::group_norm(x.to(G), 32, g.to(G), b.to(G), 1e-6f), 1e-4);
        Tensor z = randn_t({3, 7, 64});
        Tensor ln({3, 7, 64}), ln0({3, 7, 64}), rn({3, 7, 64});
        orc_layer_norm(z.data.data(), ln.data.data(), 21, 64, g.data.data(), b.data.data(), 1e-5f);
        orc_layer_norm(z.data.data(), ln0.data.data(), 21, 64, nullptr, nullptr, 1e-5f);
        orc_rms_norm(z.data.data(), rn.data.data(), 21, 64, g.data.data(), 1e-6f);
        Tensor gG = g.to(G), bG = b.to(G);
        hip_check_op("layer_norm", ln, sdh::layer_norm(z.to(G), gG, bG, 1e-5f), 1e-4);
        hip_check_op("layer_norm no affine", ln0, sdh::layer_norm(z.to(G), nullptr, nullptr, 1e-5f), 1e-4);
        hip_check_op("rms_norm", rn, sdh::rms_norm(z.to(G), &gG, 1e-6f), 1e-4);
        Tensor gd = randn_t({8}), zh = z;
        orc_rms_norm_heads(zh.data.data(), 21 * 8, 8, gd.data.data(), 1e-6f);
        Tensor zg = z.to(G), gdg = gd.to(G);
        sdh::rms_norm_heads_(zg, 8, &gdg, 1e-6f);
        hip_check_op("rms_norm_heads_", zh, zg, 1e-4);
    }
    // rope both conventions, swiglu, geglu, elementwise (test_ops.cpp:404-438)
    {
        const int S = 5, H = 3, D = 8;
        Tensor x = randn_t({1, S, H * D}), cs({S, D}), sn({S, D});
        for (int s = 0; s < S; ++s)
            for (int i = 0; i < D; ++i) {
                cs.data[s * D + i] = std::cos(0.1f * s * (i % (D / 2) + 1));
                sn.data[s * D + i] = std::sin(0.1f * s * (i % (D / 2) + 1));
            }
        for (bool inter : {false, true}) {
            Tensor a = x, b = x.to(G);
            orc_rope(a.data.data(), 1, S, H * D, D, cs.data.data(), sn.data.data(), inter);
            sdh::rope_(b, D, cs.to(G), sn.to(G), inter);
            hip_check_op(inter ? "rope interleaved" : "rope rotate_half", a, b, 1e-5);
        }
        Tensor u = randn_t({1, S, H * D}), sw({1, S, H * D});
        orc_swiglu(x.data.data(), u.data.data(), sw.data.data(), S * H * D);
        hip_check_op("swiglu", sw, sdh::swiglu(x.to(G), u.to(G)), 1e-5);
        Tensor gg = randn_t({6, 40}), ge({6, 20});
        orc_geglu(gg.data.data(), ge.data.data(), 6, 20);
        hip_check_op("geglu", ge, sdh::geglu(gg.to(G)), 1e-5);
        const char* names[] = {"silu_", "gelu_", "quick_gelu_", "tanh_"};
        for (int k = 0; k < 4; ++k) {
            Tensor a = randn_t({1000}), b = a.to(G);
            if (k == 0) { orc_silu(a.data.data(), 1000); sdh::silu_(b); }
            if (k == 1) { orc_gelu(a.data.data(), 1000); sdh::gelu_(b); }
            if (k == 2) { orc_quick_gelu(a.data.data(), 1000); sdh::quick_gelu_(b); }
            if (k == 3) { orc_tanh(a.data.data(), 1000); sdh::tanh_(b); }
            hip_check_op(names[k], a, b, 1e-5);
        }
        Tensor a = randn_t({1000}), b = randn_t({1000}), ag = a.to(G);
        orc_add(a.data.data(), b.data.data(), 1000);
        sdh::add_(ag, b.to(G));
        hip_check_op("add_", a, ag, 1e-6);
        orc_scale(a.data.data(), 0.37f, 1000);
        sdh::scale_(ag, 0.37f);
        hip_check_op("scale_", a, ag, 1e-6);
        orc_affine(a.data.data(), 1.5f, -0.25f, 1000);
        sdh::affine_(ag, 1.5f, -0.25f);
        hip_check_op("affine_", a, ag, 1e-5);
    }
    // softmax (the op inside attention, test_ops.cpp:439-451 shapes)
    {
        Tensor s = randn_t({2 * 3 * 9, 9}, 0.f, 3.f), sg = s.to(G);
        orc_softmax_rows(s.data.data(), 54, 9, 0.35f, 1);
        sdh::softmax_rows_(sg.dptr(), 54, 9, 0.35f, true);
        check("hip softmax_rows_ causal (rel)", rel_diff(s, sg), 1e-4);
        Tensor l = randn_t({100, 100}, 0.f, 3.f), lg = l.to(G);
        orc_softmax_rows(l.data.data(), 100, 100, 0.125f, 0);
        sdh::softmax_rows_(lg, 0.125f, false);
        check("hip softmax_rows_ 100 (rel)", rel_diff(l, lg), 1e-4);
    }
    // row helpers (test_ops.cpp:453-463)
    {
        Tensor x = randn_t({4, 6}), v = randn_t({6}), y = randn_t({4, 6});
        Tensor xg = x.to(G);
        orc_mul_rows(x.data.data(), v.data.data(), 4, 6);
        sdh::mul_rows_(xg, v.to(G));
        hip_check_op("mul_rows_", x, xg, 1e-6);
        orc_add_rows_scaled(x.data.data(), y.data.data(), v.data.data(), 4, 6);
        sdh::add_rows_scaled_(xg, y.to(G), v.to(G));
        hip_check_op("add_rows_scaled_", x, xg, 1e-6);
        Tensor img = randn_t({2, 3, 4, 5}), bias = randn_t({2, 3}), imgg = img.to(G);
        orc_add_channel_bias(img.data.data(), bias.data.data(), 2, 3, 20);
        sdh::add_channel_bias_(imgg, bias.to(G));
        hip_check_op("add_channel_bias_", img, imgg, 1e-6);
    }
    // shape ops (test_ops.cpp:464-476): exact copies, tolerance 0
    {
        Tensor img = randn_t({2, 3, 4, 5}), img2 = randn_t({2, 2, 4, 5}), x = randn_t({4, 6});
        Tensor ig = img.to(G), ig2 = img2.to(G);
        Tensor up({2, 3, 8, 10});
        orc_upsample_nearest2x(img.data.data(), up.data.data(), 6, 4, 5);
        hip_check_op("upsample_nearest2x", up, sdh::upsample_nearest2x(ig), 0.0);
        Tensor cc({2, 5, 4, 5});
        orc_concat_channels(img.data.data(), img2.data.data(), cc.data.data(), 2, 3, 2, 20);
        hip_check_op("concat_channels", cc, sdh::concat_channels(ig, ig2), 0.0);
        Tensor cb({4, 3, 4, 5});  // a's shape with the batches added; b's 80 floats leave a zero tail
        std::copy(img.data.begin(), img.data.end(), cb.data.begin());
        std::copy(img2.data.begin(), img2.data.end(), cb.data.begin() + img.numel());
        hip_check_op("concat_batch", cb, sdh::concat_batch(ig, ig2), 0.0);
        Tensor nlc({2, 20, 3}), back({2, 3, 4, 5});
        orc_nchw_to_nlc(img.data.data(), nlc.data.data(), 2, 3, 20);
        hip_check_op("nchw_to_nlc", nlc, sdh::nchw_to_nlc(ig), 0.0);
        orc_nlc_to_nchw(nlc.data.data(), back.data.data(), 2, 3, 20);
        hip_check_op("nlc_to_nchw", back, sdh::nlc_to_nchw(sdh::nchw_to_nlc(ig), 4, 5), 0.0);
        Tensor sb({1, 3, 4, 5});
        std::copy(img.data.begin() + 60, img.data.begin() + 120, sb.data.begin());
        hip_check_op("slice_batch", sb, sdh::slice_batch(ig, 1), 0.0);
        Tensor rb({6, 3, 4, 5});
        for (int t = 0; t < 3; ++t) std::copy(img.data.begin(), img.data.end(), rb.data.begin() + t * 120);
        hip_check_op("repeat_batch", rb, sdh::repeat_batch(ig, 3), 0.0);
        Tensor sr({2, 6});
        std::copy(x.data.begin() + 6, x.data.begin() + 18, sr.data.begin());
        hip_check_op("slice_rows", sr, sdh::slice_rows(x.to(G), 1, 3), 0.0);
        Tensor lat = randn_t({1, 16, 6, 8});
        Tensor tok({12, 64}), un({1, 16, 6, 8});
        orc_patchify(lat.data.data(), tok.data.data(), 16, 6, 8, 2);
        hip_check_op("patchify2d", tok, sdh::patchify2d(lat.to(G), 2), 0.0);
        orc_unpatchify(tok.data.data(), un.data.data(), 16, 6, 8, 2);
        hip_check_op("unpatchify2d", un, sdh::unpatchify2d(tok.to(G), 16, 6, 8, 2), 0.0);
        // the Z-Image 1024^2 latent and the VAE attention layout, at full size
        Tensor zl = randn_t({1, 16, 128, 128});
        Tensor ztok({4096, 64});
        orc_patchify(zl.data.data(), ztok.data.data(), 16, 128, 128, 2);
        hip_check_op("patchify2d Z-Image latent", ztok, sdh::patchify2d(zl.to(G), 2), 0.0);
        Tensor va = randn_t({1, 512, 128, 128});
        Tensor vnlc({1, 16384, 512});
        orc_nchw_to_nlc(va.data.data(), vnlc.data.data(), 1, 512, 16384);
        hip_check_op("nchw_to_nlc VAE attention", vnlc, sdh::nchw_to_nlc(va.to(G)), 0.0);
    }
    // fused ops vs their reference compositions, tiny and Z-Image shapes
    for (int64_t rows : {7, 4096}) {
        const int64_t C = rows == 7 ? 64 : 3840;
        Tensor x = randn_t({rows, C}), r = randn_t({rows, C}), w = randn_t({C}, 1.f, 0.1f);
        Tensor s = x, y({rows, C});
        orc_add_rms_norm(s.data.data(), r.data.data(), y.data.data(), rows, C, w.data.data(), 1e-6f);
        Tensor xg = x.to(G), wg = w.to(G);
        Tensor yg = sdh::add_rms_norm_(xg, r.to(G), &wg, 1e-6f);
        char nm[64];
        std::snprintf(nm, sizeof nm, "add_rms_norm_ sum [%lld,%lld]", (long long)rows, (long long)C);
        hip_check_op(nm, s, xg, 1e-5);
        std::snprintf(nm, sizeof nm, "hip add_rms_norm_ [%lld,%lld] (rel)", (long long)rows, (long long)C);
        check(nm, rel_diff(y, yg), 1e-4);

        Tensor sc = randn_t({C}, 0.f, 0.2f), sh = randn_t({C}, 0.f, 0.2f), gt = randn_t({C}, 0.f, 0.2f);
        Tensor res = r, ymod({rows, C});
        orc_ln_modulate_gate(x.data.data(), res.data.data(), sc.data.data(), sh.data.data(), gt.data.data(),
                             ymod.data.data(), rows, C, 1e-6f);
        Tensor resg = r.to(G), ymg = Tensor::empty({rows, C}, G), shg = sh.to(G);
        sdh::ln_modulate_gate_(x.to(G), resg, sc.to(G), &shg, gt.to(G), 1e-6f, &ymg);
        std::snprintf(nm, sizeof nm, "hip ln_modulate_gate_ res [%lld] (rel)", (long long)rows);
        check(nm, rel_diff(res, resg), 1e-4);
        std::snprintf(nm, sizeof nm, "hip ln_modulate_gate_ y [%lld] (rel)", (long long)rows);
        check(nm, rel_diff(ymod, ymg), 1e-4);
    }
    for (auto shp : {std::vector<int64_t>{2, 64, 5, 7}, std::vector<int64_t>{1, 512, 128, 128}}) {
        Tensor x = randn_t(shp, 0.f, 2.f), g = randn_t({shp[1]}, 1.f, 0.1f), b = randn_t({shp[1]}, 0.f, 0.1f);
        Tensor y(shp);
        const int64_t HW = x.numel() / (shp[0] * shp[1]);
        orc_group_norm_silu(x.data.data(), y.data.data(), shp[0], shp[1], HW, 32, g.data.data(), b.data.data(), 1e-6f);
        char nm[64];
        std::snprintf(nm, sizeof nm, "hip group_norm_silu %s (rel)", x.shape_str().c_str());
        check(nm, rel_diff(y, sdh::group_norm_silu(x.to(G), 32, g.to(G), b.to(G), 1e-6f)), 1e-4);
    }
    {
        const int64_t S = 64, dim = 128, inner = 30 * 128;
        std::vector<int32_t> pos;
        for (int h = 0; h < 8; ++h)
            for (int w = 0; w < 8; ++w) pos.insert(pos.end(), {0, h, w});
        const int32_t axes[3] = {32, 48, 48};
        Tensor cs({S, dim}), sn({S, dim});
        orc_rope_tables_3axis(pos.data(), S, axes, dim, 256.0, cs.data.data(), sn.data.data());
        Tensor q = randn_t({1, S, inner}), k = randn_t({1, S, inner});
        Tensor qg = q.to(G), kg = k.to(G);
        orc_rope(q.data.data(), 1, S, inner, dim, cs.data.data(), sn.data.data(), 1);
        orc_rope(k.data.data(), 1, S, inner, dim, cs.data.data(), sn.data.data(), 1);
        sdh::rope_qk_(qg, kg, dim, cs.to(G), sn.to(G), true);
        hip_check_op("rope_qk_ q (Z-Image tables)", q, qg, 1e-5);
        hip_check_op("rope_qk_ k (Z-Image tables)", k, kg, 1e-5);
        // QK-norm + RoPE fused (zimage.cpp:117-120) vs the oracle's op sequence
        Tensor q2 = randn_t({1, S, inner}), k2 = randn_t({1, S, inner});
        Tensor gq = randn_t({dim}, 1.f, 0.1f), gk = randn_t({dim}, 1.f, 0.1f);
        Tensor q2g = q2.to(G), k2g = k2.to(G), gqg = gq.to(G), gkg = gk.to(G);
        orc_qknorm_rope(q2.data.data(), inner, k2.data.data(), inner, 1, S, dim, gq.data.data(), gk.data.data(), 1e-5f,
                        cs.data.data(), sn.data.data(), 1);
        sdh::qknorm_rope_(q2g, k2g, dim, &gqg, &gkg, 1e-5f, cs.to(G), sn.to(G), true);
        check("hip qknorm_rope_ q (rel)", rel_diff(q2, q2g), 1e-4);
        check("hip qknorm_rope_ k (rel)", rel_diff(k2, k2g), 1e-4);
    }
    // error behaviour: the reference's shape/device checks throw
    {
        Tensor a = Tensor({4}).to(G), b = Tensor({5}).to(G), v = Tensor({3}).to(G), host({4});
        int bad = 0;
        bad += !throws([&] { sdh::add_(a, b); });                                // tensor.cpp:870
        bad += !throws([&] { sdh::swiglu(a, b); });                              // tensor.cpp:733
        bad += !throws([&] { sdh::mul_rows_(a, v); });                           // tensor.cpp:891
        bad += !throws([&] { sdh::add_(a, host); });                             // tensor.cpp:98
        bad += !throws([&] { sdh::silu_(host); });                               // host tensor: no CPU path here
        Tensor x6 = Tensor({1, 6, 2, 2}).to(G), g6 = Tensor({6}).to(G);
        bad += !throws([&] { sdh::group_norm(x6, 4, g6, g6, 1e-6f); });        // tensor.cpp:594
        Tensor odd = Tensor({1, 2, 5, 6}).to(G);
        bad += !throws([&] { sdh::patchify2d(odd, 2); });                      // tensor.cpp:933
        bad += !throws([&] { sdh::slice_rows(a, 2, 5); });                     // tensor.cpp:972
        bad += !throws([&] { sdh::nlc_to_nchw(Tensor({1, 6, 2}).to(G), 4, 2); });  // tensor.cpp:1060
        check("shape/device errors throw", (double)bad, 0.0);
    }
}

int main() {
    if (!sd::hip::available()) {
        std::printf("hip: not available, GPU comparisons skipped\n");
        std::printf("\nall ok\n");
        return 0;
    }
    std::printf("hip: %s\n", sd::hip::device_name());
    try {
        test_hip();
    } catch (const std::exception& e) {
        std::printf("unexpected exception: %s\n", e.what());
        ++failures;
    }
    std::printf(failures ? "\n%d FAILED\n" : "\nall ok\n", failures);
    return failures ? 1 : 0;
}

// The C++ drop-in (brosoundml::detail, kokoro_decoder_backward.h) exercised
// the way the reference's own test drives it (tests/test_kokoro_decoder_
// backward.cpp): N = 1, (C, 1) gamma / beta tensors, its miniature shapes,
// seeds and finite-difference tolerances, on HIP tensors. Three kinds of
// check per atom:
//   1. the reference's finite differences (per element for the AdaIN affine
//      and the spectral head, directional for the instance-norm stacks);
//   2. the same atom of the CPU oracle (oracle/kdec_oracle.hpp) on the same
//      inputs: forward rel-L2 <= 1e-5, grads <= 1e-4;
//   3. the inference twins (kokoro_infer.cpp) against the training forward,
//      and the producer step's frame-count error;
//   4. the closed-form special cases of closed_forms.hpp (the same runner as
//      the oracle's CPU check) through the HIP assemblies.
// Built by __graft_entry__.build() into tests/cpp/build/test_dropin and run by
// tests/test_gpu_dropin_cpp.py on a GPU. Prints one line per failure and
// exits non-zero if any check fails.
#include "kokoro_decoder_backward.h"

#include "brosoundml/decoder_lora.h"
#include "brosoundml/kokoro.h"
#include "closed_forms.hpp"
#include "kdec.h"
#include "kdec_oracle.hpp"

#include <array>
#include <cmath>
#include <cstdio>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

using brotensor::Device;
using brotensor::Tensor;
namespace bs = brosoundml;
namespace bd = brosoundml::detail;
using HVec = std::vector<float>;

static int g_failures = 0, g_checks = 0;

static void expect_near(double a, double b, double abs_eps, double rel_eps, const std::string& what) {
    ++g_checks;
    const double d = std::fabs(a - b), m = std::fmax(std::fabs(a), std::fabs(b));
    if (d <= abs_eps || d <= rel_eps * m) return;
    std::printf("  FAIL %s: %.8g vs %.8g (|d|=%.3g)\n", what.c_str(), a, b, d);
    ++g_failures;
}

static void expect_rel(const HVec& got, const HVec& ref, double tol, const std::string& what) {
    ++g_checks;
    if (got.size() != ref.size()) {
        std::printf("  FAIL %s: size %zu vs %zu\n", what.c_str(), got.size(), ref.size());
        ++g_failures;
        return;
    }
    double num = 0, den = 0;
    for (std::size_t i = 0; i < got.size(); ++i) {
        const double d = static_cast<double>(got[i]) - ref[i];
        num += d * d;
        den += static_cast<double>(ref[i]) * ref[i];
    }
    const double e = std::sqrt(num / std::fmax(den, 1e-60));
    if (e > tol) {
        std::printf("  FAIL %s: rel-L2 %.3e > %.0e\n", what.c_str(), e, tol);
        ++g_failures;
    }
}

static void expect_throw(const std::function<void()>& f, const std::string& needle, const std::string& what) {
    ++g_checks;
    try {
        f();
    } catch (const std::exception& e) {
        if (std::string(e.what()).find(needle) != std::string::npos) return;
        std::printf("  FAIL %s: message '%s' lacks '%s'\n", what.c_str(), e.what(), needle.c_str());
        ++g_failures;
        return;
    }
    std::printf("  FAIL %s: no error\n", what.c_str());
    ++g_failures;
}

// host data, as the reference's make_random draws it
static HVec rnd(int n, std::mt19937& rng, float scale) {
    std::uniform_real_distribution<float> u(-scale, scale);
    HVec v(static_cast<std::size_t>(n));
    for (auto& x : v) x = u(rng);
    return v;
}
static Tensor dev(const HVec& v, int r, int c) { return Tensor::from_host_on(Device::HIP, v.data(), r, c); }
static HVec host(const Tensor& t) { return t.to_host_vector(); }
static kdo::Vec ovec(const HVec& v) { return kdo::Vec(v.begin(), v.end()); }
static HVec hvec(const kdo::Vec& v) { return HVec(v.begin(), v.end()); }

// one conv on both sides (no bias, as the reference's make_conv)
struct ConvPair {
    bs::Conv1d g;
    kdo::Conv1d o;
};
static ConvPair make_conv(int in, int out, int k, int stride, int pad, std::mt19937& rng, int dil = 1) {
    const HVec w = rnd(out * in * k, rng, 0.3f);
    ConvPair c;
    c.g.in_channels = c.o.in_channels = in;
    c.g.out_channels = c.o.out_channels = out;
    c.g.kernel_size = c.o.kernel_size = k;
    c.g.stride = c.o.stride = stride;
    c.g.padding = c.o.padding = pad;
    c.g.dilation = c.o.dilation = dil;
    c.g.W = dev(w, out, in * k);
    c.o.W = ovec(w);
    return c;
}

static double mse(const HVec& y, const HVec& t) {
    double s = 0;
    for (std::size_t i = 0; i < y.size(); ++i) {
        const double d = static_cast<double>(y[i]) - t[i];
        s += 0.5 * d * d;
    }
    return s;
}
static HVec diff(const HVec& a, const HVec& b) {
    HVec d(a.size());
    for (std::size_t i = 0; i < a.size(); ++i) d[i] = a[i] - b[i];
    return d;
}

// central differences of the loss against the analytic grad of the host
// values behind tensor P (re-uploaded for every evaluation)
static void fd_per_element(HVec& P, Tensor& Pt, int r, int c, const HVec& an, const std::function<double()>& loss,
                           double abs_tol, double rel_tol, const std::string& name) {
    const float h = 1e-3f;
    for (std::size_t i = 0; i < P.size(); ++i) {
        const float s = P[i];
        P[i] = s + h;
        Pt = dev(P, r, c);
        const double lp = loss();
        P[i] = s - h;
        Pt = dev(P, r, c);
        const double lm = loss();
        P[i] = s;
        Pt = dev(P, r, c);
        expect_near(an[i], (lp - lm) / (2.0 * h), abs_tol, rel_tol, name + "[" + std::to_string(i) + "]");
    }
}
static void fd_directional(HVec& P, Tensor& Pt, int r, int c, const HVec& an, const std::function<double()>& loss,
                           std::mt19937& rng, const std::string& name, double abs_tol = 4e-3, double rel_tol = 8e-3) {
    std::uniform_real_distribution<float> u(-1.0f, 1.0f);
    const HVec saved = P;
    HVec v(P.size());
    double g_an = 0;
    for (std::size_t i = 0; i < P.size(); ++i) {
        v[i] = u(rng);
        g_an += static_cast<double>(an[i]) * v[i];
    }
    const float h = 1e-3f;
    for (std::size_t i = 0; i < P.size(); ++i) P[i] = saved[i] + h * v[i];
    Pt = dev(P, r, c);
    const double lp = loss();
    for (std::size_t i = 0; i < P.size(); ++i) P[i] = saved[i] - h * v[i];
    Pt = dev(P, r, c);
    const double lm = loss();
    P = saved;
    Pt = dev(P, r, c);
    expect_near(g_an, (lp - lm) / (2.0 * h), abs_tol, rel_tol, name);
}

// ─── AdaIN affine ───
static void test_adain_affine() {
    std::mt19937 rng(0xADA1u);
    const int C = 8, L = 16;
    const float eps = 1e-5f;
    HVec x = rnd(C * L, rng, 0.8f), g = rnd(C, rng, 0.5f), b = rnd(C, rng, 0.4f);
    const HVec target = rnd(C * L, rng, 0.5f);
    Tensor xt = dev(x, 1, C * L), gt = dev(g, C, 1), bt_ = dev(b, C, 1), y, xs;
    auto fwd = [&] { bd::adain_affine_forward(xt, gt, bt_, C, L, eps, y, xs); };
    fwd();
    const HVec hy = host(y), dY = diff(hy, target);
    Tensor dX, dG, dB;
    bd::adain_affine_backward(xt, xs, gt, dev(dY, 1, C * L), C, L, eps, dX, dG, dB);
    const HVec hdX = host(dX), hdG = host(dG), hdB = host(dB);
    auto loss = [&] { fwd(); return mse(host(y), target); };
    fd_per_element(x, xt, 1, C * L, hdX, loss, 3e-3, 6e-3, "adain.dX");
    fd_per_element(g, gt, C, 1, hdG, loss, 3e-3, 6e-3, "adain.dGamma");
    fd_per_element(b, bt_, C, 1, hdB, loss, 3e-3, 6e-3, "adain.dBeta");
    // the oracle's atom
    kdo::Vec oy, oxs, odX, odG, odB;
    kdo::adain_affine_forward(ovec(x), ovec(g), ovec(b), C, L, eps, oy, oxs);
    expect_rel(hy, hvec(oy), 1e-5, "adain.y vs oracle");
    kdo::adain_affine_backward(ovec(x), oxs, ovec(g), ovec(dY), C, L, eps, odX, odG, odB);
    expect_rel(hdX, hvec(odX), 1e-4, "adain.dX vs oracle");
    expect_rel(hdG, hvec(odG), 1e-4, "adain.dGamma vs oracle");
    expect_rel(hdB, hvec(odB), 1e-4, "adain.dBeta vs oracle");
}

// ─── AdainResBlk1d ───
struct ResblkPair {
    bs::AdainResBlk1dWeights g;
    kdo::AdainResBlk1dWeights o;
};
static void fill_fc(ResblkPair& p, int which, int C, std::mt19937& rng) {
    bs::AdaIN1dWeights& a = which ? p.g.norm2 : p.g.norm1;
    kdo::AdaIN1dWeights& b = which ? p.o.norm2 : p.o.norm1;
    const HVec W = rnd(2 * C * 128, rng, 0.1f), bb = rnd(2 * C, rng, 0.1f);
    a.channels = b.channels = C;
    a.style_dim = b.style_dim = 128;
    a.fc.in_features = 128;
    a.fc.out_features = 2 * C;
    a.fc.W = dev(W, 2 * C, 128);
    a.fc.b = dev(bb, 2 * C, 1);
    b.fcW = ovec(W);
    b.fcb = ovec(bb);
}
static ResblkPair make_resblk(int C_in, int C_out, bool upsample, bool learned_sc, std::mt19937& rng, bool fc) {
    ResblkPair p;
    p.g.channels_in = p.o.channels_in = C_in;
    p.g.channels_out = p.o.channels_out = C_out;
    p.g.upsample = p.o.upsample = upsample;
    p.g.learned_sc = p.o.learned_sc = learned_sc;
    ConvPair c1 = make_conv(C_in, C_out, 3, 1, 1, rng), c2 = make_conv(C_out, C_out, 3, 1, 1, rng);
    p.g.conv1 = c1.g;
    p.o.conv1 = c1.o;
    p.g.conv2 = c2.g;
    p.o.conv2 = c2.o;
    if (learned_sc) {
        ConvPair s = make_conv(C_in, C_out, 1, 1, 0, rng);
        p.g.conv1x1 = s.g;
        p.o.conv1x1 = s.o;
    }
    if (upsample) {
        const HVec pw = rnd(C_in * 3, rng, 0.3f), pb(static_cast<std::size_t>(C_in), 0.0f);
        p.g.pool_W = dev(pw, C_in, 3);
        p.g.pool_b = dev(pb, C_in, 1);
        p.o.pool_W = ovec(pw);
        p.o.pool_b = ovec(pb);
    }
    if (fc) {
        fill_fc(p, 0, C_in, rng);
        fill_fc(p, 1, C_out, rng);
    }
    return p;
}

static void test_adain_resblk(bool upsample, bool learned_sc, int C_in, int C_out, int L_in, std::uint32_t seed,
                              const std::string& label) {
    std::mt19937 rng(seed);
    const float eps = 1e-5f;
    const int L_out = upsample ? 2 * L_in : L_in;
    ResblkPair w = make_resblk(C_in, C_out, upsample, learned_sc, rng, false);
    HVec x = rnd(C_in * L_in, rng, 0.7f), g1 = rnd(C_in, rng, 0.4f), b1 = rnd(C_in, rng, 0.3f);
    HVec g2 = rnd(C_out, rng, 0.4f), b2 = rnd(C_out, rng, 0.3f);
    const HVec target = rnd(C_out * L_out, rng, 0.5f);
    Tensor xt = dev(x, 1, C_in * L_in), g1t = dev(g1, C_in, 1), b1t = dev(b1, C_in, 1), g2t = dev(g2, C_out, 1),
           b2t = dev(b2, C_out, 1), y;
    bd::AdainResBlkCache cache;
    int Lo = 0;
    auto fwd = [&] { bd::adain_resblk_1d_forward_train(w.g, xt, L_in, g1t, b1t, g2t, b2t, eps, Lo, y, cache); };
    fwd();
    const HVec hy = host(y), dY = diff(hy, target);
    // with the weight grads (the extension) for the oracle comparison
    Tensor dW1 = Tensor::zeros_on(Device::HIP, C_out, C_in * 3), dW2 = Tensor::zeros_on(Device::HIP, C_out, C_out * 3);
    bd::WeightGrads wg;
    wg.add(w.g.conv1.W, dW1);
    wg.add(w.g.conv2.W, dW2);
    Tensor dX, dG1, dB1, dG2, dB2;
    bd::adain_resblk_1d_backward(w.g, cache, g1t, g2t, dev(dY, 1, C_out * L_out), eps, dX, dG1, dB1, dG2, dB2, &wg);
    const HVec hdX = host(dX), hdG1 = host(dG1), hdB1 = host(dB1), hdG2 = host(dG2), hdB2 = host(dB2);
    auto loss = [&] { fwd(); return mse(host(y), target); };
    fd_directional(x, xt, 1, C_in * L_in, hdX, loss, rng, label + ".dX");
    fd_directional(g1, g1t, C_in, 1, hdG1, loss, rng, label + ".dGamma1");
    fd_directional(b1, b1t, C_in, 1, hdB1, loss, rng, label + ".dBeta1");
    fd_directional(g2, g2t, C_out, 1, hdG2, loss, rng, label + ".dGamma2");
    fd_directional(b2, b2t, C_out, 1, hdB2, loss, rng, label + ".dBeta2");
    // the oracle's atom on the same inputs
    kdo::AdainResBlkCache oc;
    kdo::Vec oy, odX, odG1, odB1, odG2, odB2;
    int oLo = 0;
    kdo::adain_resblk_1d_forward_train(w.o, ovec(x), L_in, ovec(g1), ovec(b1), ovec(g2), ovec(b2), eps, oLo, oy, oc);
    expect_rel(hy, hvec(oy), 1e-5, label + ".y vs oracle");
    kdo::Ext ext;
    ext.wgrad = true;
    kdo::adain_resblk_1d_backward(w.o, oc, ovec(g1), ovec(g2), ovec(dY), eps, odX, odG1, odB1, odG2, odB2, &ext);
    expect_rel(hdX, hvec(odX), 1e-4, label + ".dX vs oracle");
    expect_rel(hdG1, hvec(odG1), 1e-4, label + ".dGamma1 vs oracle");
    expect_rel(hdB1, hvec(odB1), 1e-4, label + ".dBeta1 vs oracle");
    expect_rel(hdG2, hvec(odG2), 1e-4, label + ".dGamma2 vs oracle");
    expect_rel(hdB2, hvec(odB2), 1e-4, label + ".dBeta2 vs oracle");
    expect_rel(host(dW1), hvec(w.o.conv1.dW), 1e-4, label + ".dW conv1 vs oracle");
    expect_rel(host(dW2), hvec(w.o.conv2.dW), 1e-4, label + ".dW conv2 vs oracle");
}

// ─── AdaINResBlock1 ───
struct Rb1Pair {
    bs::AdaINResBlock1Weights g;
    kdo::AdaINResBlock1Weights o;
};
static Rb1Pair make_resblock1(int C, std::mt19937& rng, bool fc, float alpha_lo = 0.5f) {
    const int k = 3, dils[3] = {1, 2, 3};
    Rb1Pair p;
    p.g.channels = p.o.channels = C;
    p.g.kernel_size = p.o.kernel_size = k;
    p.g.dilations = {1, 2, 3};
    p.o.dilations = {1, 2, 3};
    std::uniform_real_distribution<float> ua(alpha_lo, 1.5f);
    for (int i = 0; i < 3; ++i) {
        ConvPair c1 = make_conv(C, C, k, 1, dils[i] * (k - 1) / 2, rng, dils[i]);
        ConvPair c2 = make_conv(C, C, k, 1, (k - 1) / 2, rng);
        p.g.convs1[i] = c1.g;
        p.o.convs1[i] = c1.o;
        p.g.convs2[i] = c2.g;
        p.o.convs2[i] = c2.o;
        HVec a1(static_cast<std::size_t>(C)), a2(static_cast<std::size_t>(C));
        for (auto& v : a1) v = ua(rng);
        for (auto& v : a2) v = ua(rng);
        p.g.alpha1[i] = dev(a1, C, 1);
        p.g.alpha2[i] = dev(a2, C, 1);
        p.o.alpha1[i] = ovec(a1);
        p.o.alpha2[i] = ovec(a2);
        p.g.adain1[i].eps = p.g.adain2[i].eps = 1e-5f;
        p.o.adain1[i].eps = p.o.adain2[i].eps = 1e-5f;
        if (fc) {
            for (int which = 0; which < 2; ++which) {
                bs::AdaIN1dWeights& a = which ? p.g.adain2[i] : p.g.adain1[i];
                kdo::AdaIN1dWeights& b = which ? p.o.adain2[i] : p.o.adain1[i];
                const HVec W = rnd(2 * C * 128, rng, 0.1f), bb = rnd(2 * C, rng, 0.1f);
                a.channels = b.channels = C;
                a.style_dim = b.style_dim = 128;
                a.fc.in_features = 128;
                a.fc.out_features = 2 * C;
                a.fc.W = dev(W, 2 * C, 128);
                a.fc.b = dev(bb, 2 * C, 1);
                b.fcW = ovec(W);
                b.fcb = ovec(bb);
            }
        }
    }
    return p;
}

static void test_adain_resblock1() {
    std::mt19937 rng(0x5A4Eu);
    const int C = 8, L = 16;
    Rb1Pair w = make_resblock1(C, rng, false);
    std::array<HVec, 3> g1, b1, g2, b2;
    std::array<Tensor, 3> g1t, b1t, g2t, b2t;
    std::array<kdo::Vec, 3> og1, ob1, og2, ob2;
    for (int i = 0; i < 3; ++i) {
        g1[i] = rnd(C, rng, 0.4f);
        b1[i] = rnd(C, rng, 0.3f);
        g2[i] = rnd(C, rng, 0.4f);
        b2[i] = rnd(C, rng, 0.3f);
        g1t[i] = dev(g1[i], C, 1);
        b1t[i] = dev(b1[i], C, 1);
        g2t[i] = dev(g2[i], C, 1);
        b2t[i] = dev(b2[i], C, 1);
        og1[i] = ovec(g1[i]);
        ob1[i] = ovec(b1[i]);
        og2[i] = ovec(g2[i]);
        ob2[i] = ovec(b2[i]);
    }
    HVec x = rnd(C * L, rng, 0.6f);
    const HVec target = rnd(C * L, rng, 0.5f);
    Tensor xt = dev(x, 1, C * L), y;
    bd::AdainResBlock1Cache cache;
    auto fwd = [&] { bd::adain_resblock1_forward_train(w.g, xt, C, L, g1t, b1t, g2t, b2t, y, cache); };
    fwd();
    const HVec hy = host(y), dY = diff(hy, target);
    Tensor dX;
    std::array<Tensor, 3> dG1, dB1, dG2, dB2;
    bd::adain_resblock1_backward(w.g, cache, g1t, g2t, dev(dY, 1, C * L), dX, dG1, dB1, dG2, dB2);
    const HVec hdX = host(dX);
    auto loss = [&] { fwd(); return mse(host(y), target); };
    fd_directional(x, xt, 1, C * L, hdX, loss, rng, "resblock1.dX");
    for (int i = 0; i < 3; ++i) {
        const std::string s = std::to_string(i);
        fd_directional(g1[i], g1t[i], C, 1, host(dG1[i]), loss, rng, "resblock1.dG1." + s);
        fd_directional(b1[i], b1t[i], C, 1, host(dB1[i]), loss, rng, "resblock1.dB1." + s);
        fd_directional(g2[i], g2t[i], C, 1, host(dG2[i]), loss, rng, "resblock1.dG2." + s);
        fd_directional(b2[i], b2t[i], C, 1, host(dB2[i]), loss, rng, "resblock1.dB2." + s);
    }
    kdo::AdainResBlock1Cache oc;
    kdo::Vec oy, odX;
    std::array<kdo::Vec, 3> odG1, odB1, odG2, odB2;
    kdo::adain_resblock1_forward_train(w.o, ovec(x), C, L, og1, ob1, og2, ob2, oy, oc);
    expect_rel(hy, hvec(oy), 1e-5, "resblock1.y vs oracle");
    kdo::adain_resblock1_backward(w.o, oc, og1, og2, ovec(dY), odX, odG1, odB1, odG2, odB2, nullptr);
    expect_rel(hdX, hvec(odX), 1e-4, "resblock1.dX vs oracle");
    for (int i = 0; i < 3; ++i) {
        const std::string s = std::to_string(i);
        expect_rel(host(dG1[i]), hvec(odG1[i]), 1e-4, "resblock1.dG1." + s + " vs oracle");
        expect_rel(host(dB2[i]), hvec(odB2[i]), 1e-4, "resblock1.dB2." + s + " vs oracle");
    }
}

// ─── spectral head ───
static void test_spectral_head() {
    std::mt19937 rng(0x57EDu);
    const int C = 4, L = 8, n_fft = 16, hop = 4, win = 16, C_post = n_fft + 2, sig = (L - 1) * hop;
    ConvPair cp = make_conv(C, C_post, 7, 1, 3, rng);
    {
        HVec w = host(cp.g.W);
        for (auto& v : w) v *= 0.3f;  // modest exp() magnitude, as the reference
        cp.g.W = dev(w, C_post, C * 7);
        cp.o.W = ovec(w);
    }
    HVec window(static_cast<std::size_t>(win));
    for (int n = 0; n < win; ++n) window[n] = static_cast<float>(0.5 - 0.5 * std::cos(2.0 * M_PI * n / win));
    const Tensor wt = dev(window, 1, win);
    HVec x = rnd(C * L, rng, 0.4f);
    const HVec target = rnd(sig, rng, 0.4f);
    Tensor xt = dev(x, 1, C * L), audio;
    bd::SpectralHeadCache cache;
    auto fwd = [&] { bd::spectral_head_forward_train(cp.g, xt, C, L, wt, n_fft, hop, win, audio, cache); };
    fwd();
    const HVec ha = host(audio), dA = diff(ha, target);
    Tensor dX;
    bd::spectral_head_backward(cp.g, cache, wt, n_fft, hop, win, dev(dA, 1, sig), dX);
    const HVec hdX = host(dX);
    auto loss = [&] { fwd(); return mse(host(audio), target); };
    fd_per_element(x, xt, 1, C * L, hdX, loss, 2e-3, 6e-3, "spectral.dX");
    kdo::SpectralHeadCache oc;
    kdo::Vec oa, odX;
    kdo::spectral_head_forward_train(cp.o, ovec(x), C, L, ovec(window), n_fft, hop, win, oa, oc);
    expect_rel(ha, hvec(oa), 1e-5, "spectral.audio vs oracle");
    kdo::spectral_head_backward(cp.o, oc, ovec(window), n_fft, hop, win, ovec(dA), odX, nullptr);
    expect_rel(hdX, hvec(odX), 1e-4, "spectral.dX vs oracle");
}

// ─── DecoderBackbone (encode + cat'd decode blocks) ───
static void test_decoder_backbone() {
    std::mt19937 rng(0xB0BAu);
    const float eps = 1e-5f;
    const int T = 8, C_asr = 6, Ca = 4, Cenc = 10, Cdec = 8, Cgen = 5;
    bs::DecoderBackbone bb;
    kdo::DecoderBackbone ob;
    ConvPair f0 = make_conv(1, 1, 3, 2, 1, rng), nc = make_conv(1, 1, 3, 2, 1, rng),
             ar = make_conv(C_asr, Ca, 1, 1, 0, rng);
    bb.F0_conv = f0.g;
    ob.F0_conv = f0.o;
    bb.N_conv = nc.g;
    ob.N_conv = nc.o;
    bb.asr_res = ar.g;
    ob.asr_res = ar.o;
    std::vector<ResblkPair> blocks;
    blocks.push_back(make_resblk(C_asr + 2, Cenc, false, true, rng, true));
    blocks.push_back(make_resblk(Cenc + Ca + 2, Cenc, false, true, rng, true));
    blocks.push_back(make_resblk(Cenc + Ca + 2, Cdec, true, true, rng, true));
    blocks.push_back(make_resblk(Cdec, Cgen, false, true, rng, true));
    bb.encode = blocks[0].g;
    ob.encode = blocks[0].o;
    for (int i = 1; i < 4; ++i) {
        bb.decode.push_back(blocks[i].g);
        ob.decode.push_back(blocks[i].o);
    }
    const int cin[4] = {C_asr + 2, Cenc + Ca + 2, Cenc + Ca + 2, Cdec}, cout[4] = {Cenc, Cenc, Cdec, Cgen};
    std::vector<std::array<HVec, 4>> aff(4);
    std::vector<bd::BlockAffines> at(4);
    std::vector<kdo::BlockAffines> oa(4);
    for (int k = 0; k < 4; ++k) {
        aff[k] = {rnd(cin[k], rng, 0.4f), rnd(cin[k], rng, 0.3f), rnd(cout[k], rng, 0.4f), rnd(cout[k], rng, 0.3f)};
        at[k].g1 = dev(aff[k][0], cin[k], 1);
        at[k].b1 = dev(aff[k][1], cin[k], 1);
        at[k].g2 = dev(aff[k][2], cout[k], 1);
        at[k].b2 = dev(aff[k][3], cout[k], 1);
        oa[k] = {ovec(aff[k][0]), ovec(aff[k][1]), ovec(aff[k][2]), ovec(aff[k][3])};
    }
    const HVec asr = rnd(C_asr * T, rng, 0.7f), F0 = rnd(2 * T, rng, 0.5f), N = rnd(2 * T, rng, 0.5f);
    const int L_gen = 2 * T;
    const HVec target = rnd(Cgen * L_gen, rng, 0.5f);
    const Tensor asr_t = dev(asr, 1, C_asr * T), F0_t = dev(F0, 1, 2 * T), N_t = dev(N, 1, 2 * T);
    bd::BackboneCache cache;
    Tensor gen_in;
    auto fwd = [&] { bd::decoder_backbone_forward_train(bb, asr_t, F0_t, N_t, T, at, eps, gen_in, cache); };
    fwd();
    const HVec hg = host(gen_in), dG = diff(hg, target);
    std::vector<bd::BlockAffines> dAff;
    bd::decoder_backbone_backward(bb, cache, at, dev(dG, 1, Cgen * L_gen), eps, dAff);
    std::vector<std::array<HVec, 4>> hd(4);
    for (int k = 0; k < 4; ++k)
        hd[k] = {host(dAff[k].g1), host(dAff[k].b1), host(dAff[k].g2), host(dAff[k].b2)};
    auto loss = [&] { fwd(); return mse(host(gen_in), target); };
    const char* names[4] = {"encode", "decode0", "decode1", "decode2"};
    for (int k = 0; k < 4; ++k) {
        const std::string p = std::string("backbone.") + names[k];
        fd_directional(aff[k][0], at[k].g1, cin[k], 1, hd[k][0], loss, rng, p + ".dG1");
        fd_directional(aff[k][1], at[k].b1, cin[k], 1, hd[k][1], loss, rng, p + ".dB1");
        fd_directional(aff[k][2], at[k].g2, cout[k], 1, hd[k][2], loss, rng, p + ".dG2");
        fd_directional(aff[k][3], at[k].b2, cout[k], 1, hd[k][3], loss, rng, p + ".dB2");
    }
    kdo::BackboneCache oc;
    kdo::Vec ogen;
    kdo::decoder_backbone_forward_train(ob, ovec(asr), ovec(F0), ovec(N), T, oa, eps, ogen, oc);
    expect_rel(hg, hvec(ogen), 1e-5, "backbone.gen_in vs oracle");
    std::vector<kdo::BlockAffines> odA;
    kdo::decoder_backbone_backward(ob, oc, oa, ovec(dG), eps, odA, nullptr);
    for (int k = 0; k < 4; ++k) {
        const std::string p = std::string("backbone.") + names[k];
        expect_rel(hd[k][0], hvec(odA[k].g1), 1e-4, p + ".dG1 vs oracle");
        expect_rel(hd[k][3], hvec(odA[k].b2), 1e-4, p + ".dB2 vs oracle");
    }
    // the inference twin on the same weights: gamma, beta = fc(style)
    const HVec style = rnd(2 * 128, rng, 0.5f);
    const Tensor ref_s = dev(style, 1, 256);
    Tensor gi_twin;
    bb.forward(asr_t, F0_t, N_t, ref_s, T, gi_twin);
    // the training forward with the same projected affines
    std::vector<bd::BlockAffines> pa(4);
    for (int k = 0; k < 4; ++k) {
        const bs::AdainResBlk1dWeights& w = k == 0 ? bb.encode : bb.decode[k - 1];
        for (int which = 0; which < 2; ++which) {
            const bs::AdaIN1dWeights& a = which ? w.norm2 : w.norm1;
            const HVec W = host(a.fc.W), bv = host(a.fc.b);
            const int C = a.channels;
            HVec gb(2 * C);
            for (int r = 0; r < 2 * C; ++r) {
                double s = bv[r];
                for (int j = 0; j < 128; ++j) s += static_cast<double>(W[r * 128 + j]) * style[j];
                gb[r] = static_cast<float>(s);
            }
            const Tensor gt = dev(HVec(gb.begin(), gb.begin() + C), C, 1);
            const Tensor bt_ = dev(HVec(gb.begin() + C, gb.end()), C, 1);
            (which ? pa[k].g2 : pa[k].g1) = gt;
            (which ? pa[k].b2 : pa[k].b1) = bt_;
        }
    }
    bd::BackboneCache c2;
    Tensor gi_train;
    bd::decoder_backbone_forward_train(bb, asr_t, F0_t, N_t, T, pa, eps, gi_train, c2);
    expect_rel(host(gi_twin), host(gi_train), 1e-5, "DecoderBackbone::forward vs the training forward");
}

// ─── Generator (two stages, noise branch, reflect pad, spectral head) ───
struct GenPair {
    bs::Generator g;
    kdo::Generator o;
};
static GenPair build_generator(std::mt19937& rng, int noise0_in_stride) {
    GenPair p;
    p.g.num_upsamples = p.o.num_upsamples = 2;
    p.g.num_kernels = p.o.num_kernels = 2;
    p.g.n_fft = p.o.n_fft = 8;
    p.g.hop_size = p.o.hop_size = 4;
    p.g.win_size = p.o.win_size = 8;
    const int Cin[2] = {8, 4}, Cout[2] = {4, 2};
    for (int i = 0; i < 2; ++i) {
        for (auto* v : {&p.g.ups_C_in, &p.o.ups_C_in}) v->push_back(Cin[i]);
        for (auto* v : {&p.g.ups_C_out, &p.o.ups_C_out}) v->push_back(Cout[i]);
        for (auto* v : {&p.g.ups_k, &p.o.ups_k}) v->push_back(4);
        for (auto* v : {&p.g.ups_stride, &p.o.ups_stride}) v->push_back(2);
        for (auto* v : {&p.g.ups_pad, &p.o.ups_pad}) v->push_back(1);
        const HVec W = rnd(Cin[i] * Cout[i] * 4, rng, 0.3f), b(static_cast<std::size_t>(Cout[i]), 0.0f);
        p.g.ups_W.push_back(dev(W, Cin[i], Cout[i] * 4));
        p.g.ups_b.push_back(dev(b, Cout[i], 1));
        p.o.ups_W.push_back(ovec(W));
        p.o.ups_b.push_back(ovec(b));
    }
    ConvPair n0 = make_conv(1, 4, 4, noise0_in_stride, 1, rng), n1 = make_conv(1, 2, 3, 1, 1, rng);
    p.g.noise_convs = {n0.g, n1.g};
    p.o.noise_convs = {n0.o, n1.o};
    for (int C : {4, 2}) {
        Rb1Pair r = make_resblock1(C, rng, true);
        p.g.noise_res.push_back(r.g);
        p.o.noise_res.push_back(r.o);
    }
    for (int C : {4, 4, 2, 2}) {
        Rb1Pair r = make_resblock1(C, rng, true);
        p.g.resblocks.push_back(r.g);
        p.o.resblocks.push_back(r.o);
    }
    ConvPair cp = make_conv(2, 10, 7, 1, 3, rng);
    HVec w = host(cp.g.W);
    for (auto& v : w) v *= 0.3f;
    cp.g.W = dev(w, 10, 14);
    cp.o.W = ovec(w);
    p.g.conv_post = cp.g;
    p.o.conv_post = cp.o;
    return p;
}

static void test_generator() {
    std::mt19937 rng(0x6E1Eu);
    GenPair gen = build_generator(rng, 2);
    std::vector<std::array<std::array<HVec, 3>, 4>> raw;  // per block: g1, b1, g2, b2
    auto mkraff = [&](int C, bd::ResBlock1Affines& a, kdo::ResBlock1Affines& o) {
        std::array<std::array<HVec, 3>, 4> r;
        for (int i = 0; i < 3; ++i) {
            r[0][i] = rnd(C, rng, 0.4f);
            r[1][i] = rnd(C, rng, 0.3f);
            r[2][i] = rnd(C, rng, 0.4f);
            r[3][i] = rnd(C, rng, 0.3f);
            a.g1[i] = dev(r[0][i], C, 1);
            a.b1[i] = dev(r[1][i], C, 1);
            a.g2[i] = dev(r[2][i], C, 1);
            a.b2[i] = dev(r[3][i], C, 1);
            o.g1[i] = ovec(r[0][i]);
            o.b1[i] = ovec(r[1][i]);
            o.g2[i] = ovec(r[2][i]);
            o.b2[i] = ovec(r[3][i]);
        }
        raw.push_back(r);
    };
    std::vector<bd::ResBlock1Affines> naff(2), raff(4);
    std::vector<kdo::ResBlock1Affines> onaff(2), oraff(4);
    mkraff(4, naff[0], onaff[0]);
    mkraff(2, naff[1], onaff[1]);
    const int rc[4] = {4, 4, 2, 2};
    for (int i = 0; i < 4; ++i) mkraff(rc[i], raff[i], oraff[i]);
    const int L_in = 4, frames = 17, sig = (17 - 1) * 4;
    const HVec gin = rnd(8 * L_in, rng, 0.5f), har = rnd(frames, rng, 0.4f), target = rnd(sig, rng, 0.4f);
    const Tensor gin_t = dev(gin, 1, 8 * L_in), har_t = dev(har, 1, frames);
    bd::GeneratorCache cache;
    Tensor audio;
    auto fwd = [&] { bd::generator_forward_train(gen.g, gin_t, L_in, har_t, frames, naff, raff, audio, cache); };
    fwd();
    const HVec ha = host(audio), dA = diff(ha, target);
    std::vector<bd::ResBlock1Affines> dn, dr;
    Tensor dGenIn;
    bd::generator_backward(gen.g, cache, naff, raff, dev(dA, 1, sig), dGenIn, dn, dr);
    auto loss = [&] { fwd(); return mse(host(audio), target); };
    auto check_block = [&](int bi, bd::ResBlock1Affines& a, bd::ResBlock1Affines& d, const std::string& p) {
        for (int i = 0; i < 3; ++i) {
            const std::string s = std::to_string(i);
            const int C = a.g1[i].rows;
            fd_directional(raw[bi][0][i], a.g1[i], C, 1, host(d.g1[i]), loss, rng, p + ".g1." + s);
            fd_directional(raw[bi][1][i], a.b1[i], C, 1, host(d.b1[i]), loss, rng, p + ".b1." + s);
            fd_directional(raw[bi][2][i], a.g2[i], C, 1, host(d.g2[i]), loss, rng, p + ".g2." + s);
            fd_directional(raw[bi][3][i], a.b2[i], C, 1, host(d.b2[i]), loss, rng, p + ".b2." + s);
        }
    };
    for (int i = 0; i < 2; ++i) check_block(i, naff[i], dn[i], "gen.noise" + std::to_string(i));
    for (int i = 0; i < 4; ++i) check_block(2 + i, raff[i], dr[i], "gen.res" + std::to_string(i));
    // the oracle's generator (affine values as the FD left them)
    for (int b = 0; b < 6; ++b) {
        kdo::ResBlock1Affines& o = b < 2 ? onaff[b] : oraff[b - 2];
        for (int i = 0; i < 3; ++i) {
            o.g1[i] = ovec(raw[b][0][i]);
            o.b1[i] = ovec(raw[b][1][i]);
            o.g2[i] = ovec(raw[b][2][i]);
            o.b2[i] = ovec(raw[b][3][i]);
        }
    }
    fwd();
    kdo::GeneratorCache oc;
    kdo::Vec oa, odg;
    kdo::generator_forward_train(gen.o, ovec(gin), L_in, ovec(har), frames, onaff, oraff, oa, oc);
    expect_rel(host(audio), hvec(oa), 1e-5, "generator.audio vs oracle");
    std::vector<kdo::ResBlock1Affines> odn, odr;
    kdo::generator_backward(gen.o, oc, onaff, oraff, ovec(diff(host(audio), target)), odg, odn, odr, nullptr);
    std::vector<bd::ResBlock1Affines> dn2, dr2;
    Tensor dGenIn2;
    bd::generator_backward(gen.g, cache, naff, raff, dev(diff(host(audio), target), 1, sig), dGenIn2, dn2, dr2);
    expect_rel(host(dGenIn2), hvec(odg), 1e-4, "generator.dGenIn vs oracle");
    for (int i = 0; i < 4; ++i) expect_rel(host(dr2[i].g2[1]), hvec(odr[i].g2[1]), 1e-4, "generator.res dG2 vs oracle");
}

// ─── inference twins of the blocks ───
static void test_inference_twins() {
    std::mt19937 rng(0x7113u);
    const HVec style = rnd(128, rng, 0.5f);
    const Tensor st = dev(style, 1, 128);
    auto project = [&](const bs::AdaIN1dWeights& a, Tensor& g, Tensor& b) {
        const HVec W = host(a.fc.W), bv = host(a.fc.b);
        const int C = a.channels;
        HVec gb(2 * C);
        for (int r = 0; r < 2 * C; ++r) {
            double s = bv[r];
            for (int j = 0; j < 128; ++j) s += static_cast<double>(W[r * 128 + j]) * style[j];
            gb[r] = static_cast<float>(s);
        }
        g = dev(HVec(gb.begin(), gb.begin() + C), C, 1);
        b = dev(HVec(gb.begin() + C, gb.end()), C, 1);
    };
    // AdainResBlk1d with upsampling and a learned shortcut
    ResblkPair w = make_resblk(8, 6, true, true, rng, true);
    const int L = 12;
    const Tensor x = dev(rnd(8 * L, rng, 0.7f), 1, 8 * L);
    Tensor y_twin, y_train, g1, b1, g2, b2, x_seq;
    int Lo = 0;
    bs::adain_resblk_1d_forward(w.g, x, L, st, Lo, y_twin);
    project(w.g.norm1, g1, b1);
    project(w.g.norm2, g2, b2);
    bd::AdainResBlkCache c;
    bd::adain_resblk_1d_forward_train(w.g, x, L, g1, b1, g2, b2, 1e-5f, Lo, y_train, c);
    expect_rel(host(y_twin), host(y_train), 1e-5, "adain_resblk_1d_forward vs the training forward");
    // AdaINResBlock1
    Rb1Pair r = make_resblock1(6, rng, true);
    const int L2 = 20;
    Tensor xr = dev(rnd(6 * L2, rng, 0.6f), 1, 6 * L2), x_train = xr;
    std::array<Tensor, 3> rg1, rb1, rg2, rb2;
    for (int i = 0; i < 3; ++i) {
        project(r.g.adain1[i], rg1[i], rb1[i]);
        project(r.g.adain2[i], rg2[i], rb2[i]);
    }
    bd::AdainResBlock1Cache rc;
    Tensor out_train;
    bd::adain_resblock1_forward_train(r.g, x_train, 6, L2, rg1, rb1, rg2, rb2, out_train, rc);
    bs::adain_resblock1_forward(r.g, xr, 6, L2, st);
    expect_rel(host(xr), host(out_train), 1e-5, "adain_resblock1_forward vs the training forward");
    // ada_in_1d_styled
    Tensor yi, ya;
    bs::ada_in_1d_styled(w.g.norm1, 1, 8, L, x, st, yi);
    bd::adain_affine_forward(x, g1, b1, 8, L, 1e-5f, ya, x_seq);
    expect_rel(host(yi), host(ya), 1e-5, "ada_in_1d_styled vs adain_affine_forward");
}

// ─── the producer step's frame-count check ───
static void test_prep_frames_mismatch() {
    std::mt19937 rng(0x9E9u);
    GenPair gen = build_generator(rng, 2);  // upsample rates 2 x 2
    bs::DecoderBackbone bb;
    bb.asr_res = make_conv(6, 4, 1, 1, 0, rng).g;
    bs::HarmonicSource hs;
    hs.n_fft = hs.win_size = 8;
    hs.hop_size = 4;
    hs.l_linear.in_features = 9;
    hs.l_linear.out_features = 1;
    hs.l_linear.W = dev(rnd(9, rng, 0.3f), 1, 9);
    hs.l_linear.b = dev(rnd(1, rng, 0.1f), 1, 1);
    const int L = 5;
    const std::vector<int32_t> dur = {1, 2, 0, 3, 1};
    const Tensor t_en = dev(rnd(6 * L, rng, 1.0f), 1, 6 * L);
    HVec f0(14, 150.0f), nn(14, 0.1f);
    const Tensor F0 = dev(f0, 1, 14), Nn = dev(nn, 1, 14), ref_s = dev(rnd(256, rng, 0.3f), 1, 256);
    hs.upsample_scale = 2 * 2 * 4;  // consistent: prod(rates) * hop
    bs::KokoroDecodePrep p = bs::prepare_decode_context(bb, gen.g, hs, t_en, L, dur, F0, Nn, ref_s);
    expect_near(p.total, 7, 0, 0, "prep.total");
    expect_near(p.frames, 2 * 7 * 4 + 1, 0, 0, "prep.frames");
    const bs::DecoderLoraContext ctx = p.context();
    expect_near(ctx.total, 7, 0, 0, "prep.context().total");
    expect_near(ctx.asr == &p.asr && ctx.har == &p.har, 1, 0, 0, "prep.context() views");
    hs.upsample_scale = 3 * 4;  // a harmonic source whose frames disagree with the generator
    expect_throw([&] { bs::prepare_decode_context(bb, gen.g, hs, t_en, L, dur, F0, Nn, ref_s); },
                 "har_frames mismatch: hsource=", "prep har_frames mismatch");
    hs.upsample_scale = 16;
    const std::vector<int32_t> zero(5, 0);
    expect_throw([&] { bs::prepare_decode_context(bb, gen.g, hs, t_en, L, zero, F0, Nn, ref_s); },
                 "Kokoro::prepare_decode_context: predicted total frame count is 0", "prep total 0");
    const std::vector<float> bad(13, 100.0f);
    expect_throw([&] { bs::prepare_decode_context(bb, gen.g, hs, t_en, L, dur, F0, Nn, ref_s, &bad); },
                 "F0 override size must be 2*total (14)", "prep override size");
}

// ─── the closed-form cases through the HIP drop-in ───
namespace {
bs::Conv1d hconv(const cf::ConvSpec& c) {
    bs::Conv1d g;
    g.in_channels = c.in, g.out_channels = c.out, g.kernel_size = c.k;
    g.stride = c.s, g.padding = c.p, g.dilation = c.d;
    g.W = dev(c.W, c.out, c.in * c.k);
    if (!c.b.empty()) g.b = dev(c.b, c.out, 1);
    return g;
}
bs::AdainResBlk1dWeights hresblk(const cf::ResblkSpec& s) {
    bs::AdainResBlk1dWeights w;
    w.channels_in = s.Ci, w.channels_out = s.Co, w.upsample = s.upsample, w.learned_sc = s.learned_sc;
    w.norm1.channels = s.Ci, w.norm2.channels = s.Co;
    w.conv1 = hconv(s.conv1), w.conv2 = hconv(s.conv2);
    if (s.learned_sc) w.conv1x1 = hconv(s.conv1x1);
    if (s.upsample) w.pool_W = dev(s.pool_W, s.Ci, 3), w.pool_b = dev(s.pool_b, s.Ci, 1);
    return w;
}
bs::AdaINResBlock1Weights hrb1(const cf::Rb1Spec& s) {
    bs::AdaINResBlock1Weights w;
    w.channels = s.C, w.kernel_size = s.k;
    w.dilations = {s.dil[0], s.dil[1], s.dil[2]};
    for (int j = 0; j < 3; ++j) {
        w.convs1[j] = hconv(s.convs1[j]), w.convs2[j] = hconv(s.convs2[j]);
        w.alpha1[j] = dev(s.alpha1[j], s.C, 1), w.alpha2[j] = dev(s.alpha2[j], s.C, 1);
        w.adain1[j].channels = w.adain2[j].channels = s.C;
    }
    return w;
}
bd::ResBlock1Affines haff(const cf::Rb1Spec& s) {
    bd::ResBlock1Affines a;
    for (int j = 0; j < 3; ++j) {
        a.g1[j] = dev(s.g1[j], s.C, 1), a.b1[j] = dev(s.b1[j], s.C, 1);
        a.g2[j] = dev(s.g2[j], s.C, 1), a.b2[j] = dev(s.b2[j], s.C, 1);
    }
    return a;
}

struct HipBackend {
    const float eps = 1e-5f;
    cf::ResblkOut resblk(const cf::ResblkSpec& s) {
        const bs::AdainResBlk1dWeights w = hresblk(s);
        const Tensor g1 = dev(s.g1, s.Ci, 1), b1 = dev(s.b1, s.Ci, 1), g2 = dev(s.g2, s.Co, 1), b2 = dev(s.b2, s.Co, 1);
        bd::AdainResBlkCache c;
        Tensor y, dX, dG1, dB1, dG2, dB2;
        int Lo = 0;
        bd::adain_resblk_1d_forward_train(w, dev(s.x, 1, s.Ci * s.L), s.L, g1, b1, g2, b2, eps, Lo, y, c);
        bd::adain_resblk_1d_backward(w, c, g1, g2, dev(s.dY, 1, s.Co * s.L_out()), eps, dX, dG1, dB1, dG2, dB2);
        return {host(y), host(dX), host(dG1), host(dB1), host(dG2), host(dB2)};
    }
    cf::Rb1Out resblock1(const cf::Rb1Spec& s) {
        const bs::AdaINResBlock1Weights w = hrb1(s);
        const bd::ResBlock1Affines a = haff(s);
        bd::AdainResBlock1Cache c;
        Tensor y, dX;
        std::array<Tensor, 3> dG1, dB1, dG2, dB2;
        bd::adain_resblock1_forward_train(w, dev(s.x, 1, s.C * s.L), s.C, s.L, a.g1, a.b1, a.g2, a.b2, y, c);
        bd::adain_resblock1_backward(w, c, a.g1, a.g2, dev(s.dY, 1, s.C * s.L), dX, dG1, dB1, dG2, dB2);
        return {host(y), host(dX)};
    }
    void generator(const cf::GenSpec& g, HVec& stage1_in, HVec& head_in) {
        bs::Generator gen;
        gen.n_fft = g.n_fft, gen.hop_size = g.hop, gen.win_size = g.win;
        gen.num_upsamples = g.U, gen.num_kernels = g.K;
        for (int i = 0; i < g.U; ++i) {
            gen.ups_W.push_back(dev(g.ups_W[i], g.C_in[i], g.C_out[i] * g.k[i]));
            gen.ups_b.push_back(dev(g.ups_b[i], g.C_out[i], 1));
            gen.noise_convs.push_back(hconv(g.noise_convs[i]));
            gen.noise_res.push_back(hrb1(g.noise_res[i]));
        }
        gen.ups_C_in = g.C_in, gen.ups_C_out = g.C_out, gen.ups_k = g.k, gen.ups_stride = g.s, gen.ups_pad = g.p;
        std::vector<bd::ResBlock1Affines> naff, raff;
        for (const auto& r : g.noise_res) naff.push_back(haff(r));
        for (const auto& r : g.resblocks) {
            gen.resblocks.push_back(hrb1(r));
            raff.push_back(haff(r));
        }
        gen.conv_post = hconv(g.conv_post);
        bd::GeneratorCache c;
        Tensor audio;
        bd::generator_forward_train(gen, dev(g.gen_in, 1, g.C0 * g.L0), g.L0, dev(g.har, 1, (g.n_fft + 2) * g.frames),
                                    g.frames, naff, raff, audio, c);
        stage1_in = host(c.stages[1].x_in);
        head_in = host(c.head.x_pre);
    }
    HVec head(const cf::HeadSpec& h, const HVec& x, const HVec& W) {
        cf::ConvSpec cs = h.conv_post;
        cs.W = W;
        HVec window(static_cast<std::size_t>(h.win));
        for (int n = 0; n < h.win; ++n) window[n] = static_cast<float>(0.5 - 0.5 * std::cos(2.0 * M_PI * n / h.win));
        bd::SpectralHeadCache c;
        Tensor audio;
        bd::spectral_head_forward_train(hconv(cs), dev(x, 1, h.C * h.L), h.C, h.L, dev(window, 1, h.win), h.n_fft,
                                        h.hop, h.win, audio, c);
        return host(audio);
    }
    HVec backbone(const cf::BbSpec& b) {
        bs::DecoderBackbone bb;
        bb.F0_conv = hconv(b.F0_conv), bb.N_conv = hconv(b.N_conv), bb.asr_res = hconv(b.asr_res);
        bb.encode = hresblk(b.encode);
        std::vector<bd::BlockAffines> aff;
        auto push = [&](const cf::ResblkSpec& r) {
            bd::BlockAffines a;
            a.g1 = dev(r.g1, r.Ci, 1), a.b1 = dev(r.b1, r.Ci, 1), a.g2 = dev(r.g2, r.Co, 1), a.b2 = dev(r.b2, r.Co, 1);
            aff.push_back(a);
        };
        push(b.encode);
        for (const auto& d : b.decode) {
            bb.decode.push_back(hresblk(d));
            push(d);
        }
        bd::BackboneCache c;
        Tensor gen_in;
        bd::decoder_backbone_forward_train(bb, dev(b.asr, 1, b.A * b.T), dev(b.F0, 1, 2 * b.T), dev(b.N, 1, 2 * b.T),
                                           b.T, aff, eps, gen_in, c);
        return host(gen_in);
    }
    HVec pad(const HVec& x, int C, int L) {
        kdec_ctx* ctx = nullptr;
        if (kdec_ctx_create(0, &ctx) != KDEC_OK) throw std::runtime_error("kdec_ctx_create");
        const Tensor xt = dev(x, 1, C * L);
        Tensor yt = Tensor::zeros_on(Device::HIP, 1, C * (L + 1));
        const int rc = kdec_pad_reflect_left1_fwd(ctx, static_cast<const float*>(xt.data), C * L,
                                                  static_cast<float*>(yt.data), C * (L + 1), 1, C, L);
        kdec_synchronize(ctx);
        kdec_ctx_destroy(ctx);
        if (rc != KDEC_OK) throw std::runtime_error("kdec_pad_reflect_left1_fwd");
        return host(yt);
    }
};

void test_closed_forms() {
    HipBackend be;
    cf::Report r;
    cf::run_closed_forms(be, r);
    g_checks += r.checks;
    g_failures += r.failures;
}
}  // namespace

int main() {
    brotensor::init(0);
    struct Case {
        const char* name;
        std::function<void()> run;
    } cases[] = {
        {"adain_affine", test_adain_affine},
        {"resblk_plain", [] { test_adain_resblk(false, false, 8, 8, 16, 0xD001u, "resblk_plain"); }},
        {"resblk_up", [] { test_adain_resblk(true, true, 8, 6, 12, 0xD002u, "resblk_up"); }},
        {"adain_resblock1", test_adain_resblock1},
        {"spectral_head", test_spectral_head},
        {"decoder_backbone", test_decoder_backbone},
        {"generator", test_generator},
        {"inference_twins", test_inference_twins},
        {"prep", test_prep_frames_mismatch},
        {"closed_forms", test_closed_forms},
    };
    for (auto& c : cases) {
        const int before = g_failures;
        try {
            c.run();
        } catch (const std::exception& e) {
            std::printf("  FAIL %s: threw %s\n", c.name, e.what());
            ++g_failures;
        }
        std::printf("%-18s %s\n", c.name, g_failures == before ? "ok" : "FAILED");
        std::fflush(stdout);
    }
    std::printf("test_dropin: %d checks, %d failure(s)\n", g_checks, g_failures);
    return g_failures ? 1 : 0;
}

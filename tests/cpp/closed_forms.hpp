// Closed-form special cases of the decoder's assemblies (the composition of
// kokoro_decoder_backward.cpp:152-207, 287-323, 482-537, 592-667 and the
// generator of kokoro_modules.cpp:1400-1552). Each construction makes the
// output known in closed form and fails for one plausible slip:
//
//  resblk_shortcut   residual convs zero, conv1x1 = [I | 0]: y = sc(x)/sqrt(2),
//                    sc = identity or nearest-2x (the /sqrt(2), the shortcut's
//                    upsampling, its channel selection), dX = sc^T(dY)/sqrt(2)
//  resblk_slope      gamma = -1 makes each AdaIN output its beta; identity
//                    centre taps: y = (leaky(beta2, 0.2) + x)/sqrt(2), and
//                    dBeta2 = leaky'(beta2) * sum(dY)/sqrt(2) (the 0.2 slope,
//                    forward and backward)
//  resblock1_skip    convs2 = 0: AdaINResBlock1 is x + sum_j bias2_j, and the
//                    identity backward (the x = xt + x skip, every sub-block's
//                    residual, not just the last)
//  generator_stages  identity resblocks and noise_res (convs2 = 0): stage i
//                    ends at ups_i(leaky(x, 0.1)) [+ reflect pad] +
//                    noise_conv_i(har) + noise_res biases (the 1/K mean, not
//                    the K-fold sum; the 0.1 slope; the noise branch add; the
//                    pad on the last stage only)
//  head_slope        for all-negative x, head(x; W) = head(-x; -0.01 W): the
//                    spectral head's 0.01 slope without a closed-form iSTFT
//  backbone_cat      zero residual convs, shortcut 1x1 convs picking labelled
//                    constant channels: the cat orders [asr, F0, N] and
//                    [x, asr_res, F0, N], and no cat after the upsampling block
//  pad_side          an asymmetric ramp through ReflectionPad1d((1, 0))
//
// The expected values come from these formulas and from naive double
// precision convolutions below, never from either implementation. The
// runner is shared by the oracle's CPU check (test_closed_form.cpp) and the
// HIP drop-in's (test_dropin.cpp); a backend supplies the atoms.
#pragma once

#include <cmath>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

namespace cf {

using HVec = std::vector<float>;

struct ConvSpec {
    int in = 0, out = 0, k = 1, s = 1, p = 0, d = 1;
    HVec W, b;  // W (out, in*k); b (out) or empty
};
struct ResblkSpec {
    int Ci = 0, Co = 0, L = 0;
    bool upsample = false, learned_sc = false;
    ConvSpec conv1, conv2, conv1x1;
    HVec pool_W, pool_b;  // (Ci, 3), (Ci) when upsample
    HVec x, g1, b1, g2, b2, dY;
    int L_out() const { return upsample ? 2 * L : L; }
};
struct ResblkOut {
    HVec y, dX, dG1, dB1, dG2, dB2;
};
struct Rb1Spec {
    int C = 0, k = 3, L = 0;
    int dil[3] = {1, 3, 5};
    ConvSpec convs1[3], convs2[3];
    HVec alpha1[3], alpha2[3], g1[3], b1[3], g2[3], b2[3];
    HVec x, dY;
};
struct Rb1Out {
    HVec y, dX;
};
struct GenSpec {
    int n_fft = 4, hop = 1, win = 4, U = 2, K = 3;
    int C0 = 4, L0 = 3, frames = 0;
    std::vector<int> C_in, C_out, k, s, p;
    std::vector<HVec> ups_W, ups_b;  // (C_in, C_out*k), (C_out)
    std::vector<ConvSpec> noise_convs;
    std::vector<Rb1Spec> noise_res, resblocks;  // weights and affines; x / dY unused
    ConvSpec conv_post;
    HVec gen_in, har;
};
struct HeadSpec {
    int C = 3, L = 10, n_fft = 4, hop = 1, win = 4;
    ConvSpec conv_post;
};
struct BbSpec {
    int A = 3, T = 4;
    ConvSpec F0_conv, N_conv, asr_res;
    ResblkSpec encode;  // weights only (x / dY unused); affines g1..b2 used
    std::vector<ResblkSpec> decode;
    HVec asr, F0, N;
};

// ─── host reference arithmetic (double) ───
inline HVec conv1d_ref(const HVec& x, const ConvSpec& c, int L) {
    const int Lo = (L + 2 * c.p - c.d * (c.k - 1) - 1) / c.s + 1;
    HVec y(static_cast<std::size_t>(c.out) * Lo);
    for (int o = 0; o < c.out; ++o)
        for (int j = 0; j < Lo; ++j) {
            double a = c.b.empty() ? 0.0 : c.b[o];
            for (int i = 0; i < c.in; ++i)
                for (int t = 0; t < c.k; ++t) {
                    const int q = j * c.s + t * c.d - c.p;
                    if (q >= 0 && q < L) a += static_cast<double>(c.W[(o * c.in + i) * c.k + t]) * x[i * L + q];
                }
            y[o * Lo + j] = static_cast<float>(a);
        }
    return y;
}
// W (Ci, Co*k): y[o, j] += x[i, q] W[i, o*k + t] at j = q*s - p + t
inline HVec convt1d_ref(const HVec& x, const HVec& W, const HVec& b, int Ci, int Co, int k, int s, int p, int L) {
    const int Lo = (L - 1) * s - 2 * p + k;
    std::vector<double> y(static_cast<std::size_t>(Co) * Lo, 0.0);
    for (int o = 0; o < Co; ++o)
        for (int j = 0; j < Lo; ++j) y[o * Lo + j] = b.empty() ? 0.0 : b[o];
    for (int i = 0; i < Ci; ++i)
        for (int q = 0; q < L; ++q)
            for (int o = 0; o < Co; ++o)
                for (int t = 0; t < k; ++t) {
                    const int j = q * s - p + t;
                    if (j >= 0 && j < Lo) y[o * Lo + j] += static_cast<double>(x[i * L + q]) * W[(i * Co + o) * k + t];
                }
    return HVec(y.begin(), y.end());
}
inline HVec leaky_ref(const HVec& x, double slope) {
    HVec y(x.size());
    for (std::size_t i = 0; i < x.size(); ++i) y[i] = x[i] > 0.0f ? x[i] : static_cast<float>(slope * x[i]);
    return y;
}
inline HVec pad_left1_ref(const HVec& x, int C, int L) {
    HVec y(static_cast<std::size_t>(C) * (L + 1));
    for (int c = 0; c < C; ++c) {
        y[c * (L + 1)] = x[c * L + 1];
        for (int i = 0; i < L; ++i) y[c * (L + 1) + 1 + i] = x[c * L + i];
    }
    return y;
}

// ─── the constructions ───
inline HVec rnd(int n, std::mt19937& rng, float lo, float hi) {
    std::uniform_real_distribution<float> u(lo, hi);
    HVec v(static_cast<std::size_t>(n));
    for (auto& x : v) x = u(rng);
    return v;
}
inline HVec zeros(int n) { return HVec(static_cast<std::size_t>(n), 0.0f); }
inline ConvSpec conv(int in, int out, int k, int s, int p, int d, HVec W, HVec b = {}) {
    ConvSpec c;
    c.in = in, c.out = out, c.k = k, c.s = s, c.p = p, c.d = d;
    c.W = std::move(W);
    c.b = std::move(b);
    return c;
}
// conv weights whose output channel o copies input channel sel[o] (k = 1)
inline HVec select_1x1(int in, const std::vector<int>& sel) {
    HVec W(static_cast<std::size_t>(sel.size()) * in, 0.0f);
    for (std::size_t o = 0; o < sel.size(); ++o) W[o * in + sel[o]] = 1.0f;
    return W;
}
// k = 3 weights passing channel c through the centre tap
inline HVec centre_identity(int C) {
    HVec W(static_cast<std::size_t>(C) * C * 3, 0.0f);
    for (int c = 0; c < C; ++c) W[(c * C + c) * 3 + 1] = 1.0f;
    return W;
}

inline ResblkSpec resblk_shortcut(bool upsample, std::mt19937& rng) {
    ResblkSpec r;
    r.Ci = 6, r.Co = 4, r.L = 9, r.upsample = upsample, r.learned_sc = true;
    r.conv1 = conv(6, 4, 3, 1, 1, 1, zeros(4 * 6 * 3));
    r.conv2 = conv(4, 4, 3, 1, 1, 1, zeros(4 * 4 * 3));
    r.conv1x1 = conv(6, 4, 1, 1, 0, 1, select_1x1(6, {0, 1, 2, 3}));
    if (upsample) {
        r.pool_W = rnd(6 * 3, rng, -0.5f, 0.5f);
        r.pool_b = zeros(6);
    }
    r.x = rnd(6 * 9, rng, -1.0f, 1.0f);
    r.g1 = rnd(6, rng, -0.4f, 0.4f), r.b1 = rnd(6, rng, -0.3f, 0.3f);
    r.g2 = rnd(4, rng, -0.4f, 0.4f), r.b2 = rnd(4, rng, -0.3f, 0.3f);
    r.dY = rnd(4 * r.L_out(), rng, -1.0f, 1.0f);
    return r;
}
inline ResblkSpec resblk_slope(std::mt19937& rng) {
    ResblkSpec r;
    r.Ci = r.Co = 4, r.L = 9;
    r.conv1 = conv(4, 4, 3, 1, 1, 1, centre_identity(4));
    r.conv2 = conv(4, 4, 3, 1, 1, 1, centre_identity(4));
    r.x = rnd(4 * 9, rng, -1.0f, 1.0f);
    r.g1 = HVec(4, -1.0f), r.b1 = {0.5f, -0.6f, 0.3f, -0.1f};
    r.g2 = HVec(4, -1.0f), r.b2 = {-0.7f, 0.4f, -0.2f, 0.9f};
    r.dY = rnd(4 * 9, rng, -1.0f, 1.0f);
    return r;
}
inline Rb1Spec resblock1_skip(int C, int L, bool bias2, std::mt19937& rng) {
    Rb1Spec r;
    r.C = C, r.L = L;
    for (int j = 0; j < 3; ++j) {
        r.convs1[j] = conv(C, C, 3, 1, r.dil[j], r.dil[j], rnd(C * C * 3, rng, -0.4f, 0.4f), rnd(C, rng, -0.2f, 0.2f));
        r.convs2[j] = conv(C, C, 3, 1, 1, 1, zeros(C * C * 3), bias2 ? rnd(C, rng, -0.5f, 0.5f) : HVec{});
        r.alpha1[j] = rnd(C, rng, 0.5f, 2.0f), r.alpha2[j] = rnd(C, rng, 0.5f, 2.0f);
        r.g1[j] = rnd(C, rng, -0.4f, 0.4f), r.b1[j] = rnd(C, rng, -0.3f, 0.3f);
        r.g2[j] = rnd(C, rng, -0.4f, 0.4f), r.b2[j] = rnd(C, rng, -0.3f, 0.3f);
    }
    r.x = rnd(C * L, rng, -1.0f, 1.0f);
    r.dY = rnd(C * L, rng, -1.0f, 1.0f);
    return r;
}
inline GenSpec generator_stages(std::mt19937& rng) {
    GenSpec g;
    g.C_in = {4, 2}, g.C_out = {2, 2}, g.k = {4, 4}, g.s = {2, 2}, g.p = {1, 1};
    const int L1 = 2 * g.L0, L2 = 2 * L1;
    g.frames = L2 + 1;
    const int H = g.n_fft + 2;
    for (int i = 0; i < g.U; ++i) {
        g.ups_W.push_back(rnd(g.C_in[i] * g.C_out[i] * g.k[i], rng, -0.5f, 0.5f));
        g.ups_b.push_back(rnd(g.C_out[i], rng, -0.2f, 0.2f));
    }
    // stage 0 sees har at half rate, stage 1 at its rate (Kokoro's noise_convs geometry)
    g.noise_convs.push_back(conv(H, 2, 4, 2, 1, 1, rnd(2 * H * 4, rng, -0.4f, 0.4f), rnd(2, rng, -0.2f, 0.2f)));
    g.noise_convs.push_back(conv(H, 2, 1, 1, 0, 1, rnd(2 * H, rng, -0.4f, 0.4f), rnd(2, rng, -0.2f, 0.2f)));
    for (int i = 0; i < g.U; ++i) {
        g.noise_res.push_back(resblock1_skip(g.C_out[i], 1, true, rng));
        for (int j = 0; j < g.K; ++j) g.resblocks.push_back(resblock1_skip(g.C_out[i], 1, false, rng));
    }
    g.conv_post = conv(2, H, 7, 1, 3, 1, rnd(H * 2 * 7, rng, -0.3f, 0.3f), rnd(H, rng, -0.1f, 0.1f));
    g.gen_in = rnd(g.C0 * g.L0, rng, -1.0f, 1.0f);
    g.har = rnd(H * g.frames, rng, -1.0f, 1.0f);
    return g;
}
inline HeadSpec head_slope(std::mt19937& rng) {
    HeadSpec h;
    const int H = h.n_fft + 2;
    h.conv_post = conv(h.C, H, 7, 1, 3, 1, rnd(H * h.C * 7, rng, -0.3f, 0.3f), rnd(H, rng, -0.1f, 0.1f));
    return h;
}
inline BbSpec backbone_cat(std::mt19937& rng) {
    BbSpec b;
    const int A = b.A, T = b.T;
    b.F0_conv = conv(1, 1, 3, 2, 1, 1, zeros(3), HVec{7.0f});
    b.N_conv = conv(1, 1, 3, 2, 1, 1, zeros(3), HVec{11.0f});
    b.asr_res = conv(A, 2, 1, 1, 0, 1, zeros(2 * A), HVec{13.0f, 17.0f});
    auto block = [&](int Ci, int Co, bool up, bool sc, const std::vector<int>& sel) {
        ResblkSpec r;
        r.Ci = Ci, r.Co = Co, r.upsample = up, r.learned_sc = sc;
        r.conv1 = conv(Ci, Co, 3, 1, 1, 1, zeros(Co * Ci * 3));
        r.conv2 = conv(Co, Co, 3, 1, 1, 1, zeros(Co * Co * 3));
        if (sc) r.conv1x1 = conv(Ci, Co, 1, 1, 0, 1, select_1x1(Ci, sel));
        if (up) r.pool_W = rnd(Ci * 3, rng, -0.5f, 0.5f), r.pool_b = zeros(Ci);
        r.g1 = rnd(Ci, rng, -0.4f, 0.4f), r.b1 = rnd(Ci, rng, -0.3f, 0.3f);
        r.g2 = rnd(Co, rng, -0.4f, 0.4f), r.b2 = rnd(Co, rng, -0.3f, 0.3f);
        return r;
    };
    // encode input [asr 0..2, F0_dn 3, N_dn 4] -> [100, 102, 7, 11]/s2
    b.encode = block(A + 2, 4, false, true, {0, 2, 3, 4});
    // decode input [x 0..3, asr_res 4..5, F0_dn 6, N_dn 7]:
    // decode0 picks encode's F0 and N channels, asr_res1 and N -> [7/s2, 11/s2, 17, 11]/s2
    b.decode.push_back(block(4 + 2 + 2, 4, false, true, {2, 3, 5, 7}));
    // decode1 (2x) picks x0, x1, asr_res0, F0 -> [3.5, 5.5, 13, 7]/s2
    b.decode.push_back(block(4 + 2 + 2, 4, true, true, {0, 1, 4, 6}));
    b.decode.push_back(block(4, 4, false, false, {}));  // after the upsampling block: no cat
    b.asr = HVec(static_cast<std::size_t>(A) * T);
    for (int c = 0; c < A; ++c)
        for (int t = 0; t < T; ++t) b.asr[c * T + t] = 100.0f + c;
    b.F0 = rnd(2 * T, rng, 80.0f, 300.0f);
    b.N = rnd(2 * T, rng, -1.0f, 1.0f);
    return b;
}

// ─── checks ───
struct Report {
    int checks = 0, failures = 0;
    void rel(const HVec& got, const HVec& want, double tol, const std::string& what) {
        ++checks;
        if (got.size() != want.size()) {
            std::printf("  FAIL %s: size %zu vs %zu\n", what.c_str(), got.size(), want.size());
            ++failures;
            return;
        }
        double num = 0, den = 0;
        for (std::size_t i = 0; i < got.size(); ++i) {
            const double d = static_cast<double>(got[i]) - want[i];
            num += d * d;
            den += static_cast<double>(want[i]) * want[i];
        }
        const double e = std::sqrt(num / std::fmax(den, 1e-60));
        if (e > tol) {
            std::printf("  FAIL %s: rel-L2 %.3e > %.0e\n", what.c_str(), e, tol);
            ++failures;
        }
    }
    void zero(const HVec& got, double tol, const std::string& what) {
        ++checks;
        double m = 0;
        for (float v : got) m = std::fmax(m, std::fabs(v));
        if (m > tol) {
            std::printf("  FAIL %s: max |v| %.3e > %.0e\n", what.c_str(), m, tol);
            ++failures;
        }
    }
};

constexpr double kTol = 2e-6;  // float evaluation of exact closed forms

template <class Backend>
void run_closed_forms(Backend& be, Report& r, unsigned seed = 0xC105Du) {
    std::mt19937 rng(seed);
    const double rs2 = 1.0 / std::sqrt(2.0);

    for (bool up : {false, true}) {
        const std::string tag = up ? "resblk_shortcut.up" : "resblk_shortcut";
        const ResblkSpec s = resblk_shortcut(up, rng);
        const ResblkOut o = be.resblk(s);
        const int Lo = s.L_out();
        HVec y(static_cast<std::size_t>(s.Co) * Lo), dx(static_cast<std::size_t>(s.Ci) * s.L, 0.0f);
        for (int c = 0; c < s.Co; ++c)
            for (int j = 0; j < Lo; ++j) y[c * Lo + j] = static_cast<float>(s.x[c * s.L + (up ? j / 2 : j)] * rs2);
        for (int c = 0; c < s.Co; ++c)
            for (int i = 0; i < s.L; ++i)
                dx[c * s.L + i] = static_cast<float>(
                    (up ? static_cast<double>(s.dY[c * Lo + 2 * i]) + s.dY[c * Lo + 2 * i + 1] : s.dY[c * Lo + i]) * rs2);
        r.rel(o.y, y, kTol, tag + ".y = sc(x)/sqrt2");
        r.rel(o.dX, dx, kTol, tag + ".dX = sc^T(dY)/sqrt2");
        r.zero(o.dG1, 1e-6, tag + ".dGamma1 = 0");
        r.zero(o.dB1, 1e-6, tag + ".dBeta1 = 0");
        r.zero(o.dG2, 1e-6, tag + ".dGamma2 = 0");
        r.zero(o.dB2, 1e-6, tag + ".dBeta2 = 0");
    }
    {
        const ResblkSpec s = resblk_slope(rng);
        const ResblkOut o = be.resblk(s);
        HVec y(s.x.size()), db2(4);
        for (int c = 0; c < 4; ++c) {
            const double lb = s.b2[c] > 0 ? s.b2[c] : 0.2 * s.b2[c];
            double sd = 0;
            for (int j = 0; j < s.L; ++j) {
                y[c * s.L + j] = static_cast<float>((lb + s.x[c * s.L + j]) * rs2);
                sd += s.dY[c * s.L + j];
            }
            db2[c] = static_cast<float>((s.b2[c] > 0 ? 1.0 : 0.2) * sd * rs2);
        }
        r.rel(o.y, y, kTol, "resblk_slope.y = (leaky(beta2, 0.2) + x)/sqrt2");
        HVec dx(s.dY.size());
        for (std::size_t i = 0; i < dx.size(); ++i) dx[i] = static_cast<float>(s.dY[i] * rs2);
        r.rel(o.dX, dx, kTol, "resblk_slope.dX = dY/sqrt2");
        r.rel(o.dB2, db2, kTol, "resblk_slope.dBeta2 = leaky'(beta2) sum(dY)/sqrt2");
        r.zero(o.dG2, 1e-6, "resblk_slope.dGamma2 = 0");
    }
    for (bool bias2 : {false, true}) {
        const std::string tag = bias2 ? "resblock1_skip.bias" : "resblock1_skip";
        const Rb1Spec s = resblock1_skip(4, 13, bias2, rng);
        const Rb1Out o = be.resblock1(s);
        HVec y = s.x;
        if (bias2)
            for (int j = 0; j < 3; ++j)
                for (int c = 0; c < s.C; ++c)
                    for (int l = 0; l < s.L; ++l) y[c * s.L + l] += s.convs2[j].b[c];
        r.rel(o.y, y, kTol, tag + ".y = x + sum_j bias2_j");
        r.rel(o.dX, s.dY, kTol, tag + ".dX = dY");
    }
    {
        const GenSpec g = generator_stages(rng);
        HVec stage1_in, head_in;
        be.generator(g, stage1_in, head_in);
        auto noise = [&](int i) {
            HVec n = conv1d_ref(g.har, g.noise_convs[i], g.frames);
            const int L = static_cast<int>(n.size()) / g.C_out[i];
            for (int j = 0; j < 3; ++j)
                for (int c = 0; c < g.C_out[i]; ++c)
                    for (int l = 0; l < L; ++l) n[c * L + l] += g.noise_res[i].convs2[j].b[c];
            return n;
        };
        HVec u0 = convt1d_ref(leaky_ref(g.gen_in, 0.1), g.ups_W[0], g.ups_b[0], g.C_in[0], g.C_out[0], g.k[0], g.s[0],
                              g.p[0], g.L0);
        const HVec n0 = noise(0);
        for (std::size_t i = 0; i < u0.size(); ++i) u0[i] += n0[i];
        const int L1 = static_cast<int>(u0.size()) / g.C_out[0];
        HVec u1 = convt1d_ref(leaky_ref(u0, 0.1), g.ups_W[1], g.ups_b[1], g.C_in[1], g.C_out[1], g.k[1], g.s[1],
                              g.p[1], L1);
        u1 = pad_left1_ref(u1, g.C_out[1], static_cast<int>(u1.size()) / g.C_out[1]);
        const HVec n1 = noise(1);
        for (std::size_t i = 0; i < u1.size(); ++i) u1[i] += n1[i];
        r.rel(stage1_in, u0, kTol, "generator.stage0 = ups(leaky(x, 0.1)) + noise, mean of identities");
        r.rel(head_in, u1, kTol, "generator.stage1 = pad(ups(leaky(x, 0.1))) + noise");
    }
    {
        const HeadSpec h = head_slope(rng);
        const HVec xn = rnd(h.C * h.L, rng, -1.5f, -0.05f);
        HVec xp(xn.size()), Wm(h.conv_post.W.size());
        for (std::size_t i = 0; i < xn.size(); ++i) xp[i] = -xn[i];
        for (std::size_t i = 0; i < Wm.size(); ++i) Wm[i] = -0.01f * h.conv_post.W[i];
        const HVec a = be.head(h, xn, h.conv_post.W), b = be.head(h, xp, Wm);
        r.rel(a, b, 1e-5, "head_slope: head(x<0; W) = head(-x; -0.01 W)");
    }
    {
        const BbSpec b = backbone_cat(rng);
        const HVec gi = be.backbone(b);
        // encode [100, 102, 7, 11]/s2; decode0 [3.5, 5.5, 17/s2, 11/s2];
        // decode1 (2x) [3.5, 5.5, 13, 7]/s2; decode2 (no cat) /s2
        const double want[4] = {3.5 / 2.0, 5.5 / 2.0, 13.0 / 2.0, 7.0 / 2.0};
        HVec w(static_cast<std::size_t>(4) * 2 * b.T);
        for (int c = 0; c < 4; ++c)
            for (int t = 0; t < 2 * b.T; ++t) w[c * 2 * b.T + t] = static_cast<float>(want[c]);
        r.rel(gi, w, kTol, "backbone_cat: gen_in = [7/4, 11/4, 13/2, 7/2]");
    }
    {
        const int C = 3, L = 7;
        HVec x(static_cast<std::size_t>(C) * L);
        for (int c = 0; c < C; ++c)
            for (int i = 0; i < L; ++i) x[c * L + i] = 10.0f * c + static_cast<float>(i * i);
        r.rel(be.pad(x, C, L), pad_left1_ref(x, C, L), 0.0, "pad_side: y[0] = x[1], then x");
    }
}

}  // namespace cf

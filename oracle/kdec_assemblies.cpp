// Assembly atoms of the decoder back half, restated op by op from
// src/kokoro_decoder_backward.cpp. TEST INFRASTRUCTURE ONLY (parity oracle).
//
// The reference semantics (conv dgrad only, snake dAlpha discarded) are the
// default; an `Ext` adds the extensions: conv/convT/pool weight and
// bias grads and snake alpha grads, accumulated into the weight structs.
#include "kdec_oracle.hpp"

#include <cmath>
#include <stdexcept>

namespace KDO_NS {

KinkMasks* g_kinks = nullptr;
int g_kink_block = -1;
int g_kink_gen = -1;

namespace {

// The mask of leaky site `site` when one is set for a tensor of n elements.
const signed char* kink_mask(int site, std::size_t n) {
    if (!g_kinks || site < 0 || site >= static_cast<int>(g_kinks->masks.size())) return nullptr;
    const auto& m = g_kinks->masks[static_cast<std::size_t>(site)];
    return m.size() == n ? m.data() : nullptr;
}
int block_site(int k) { return g_kink_block < 0 ? -1 : g_kink_block + k; }
// site of the spectral head, set by the generator around its head calls
int g_kink_head = -1;
int gen_site(int k) { return g_kink_gen < 0 ? -1 : g_kink_gen + k; }

Vec ones(int C) { return Vec(static_cast<std::size_t>(C), 1.0f); }
Vec zeros(std::size_t n) { return Vec(n, 0.0f); }

void conv_fwd(const Conv1d& c, const Vec& x, int L, Vec& y) {
    const int Lo = c.L_out(L);
    y.assign(static_cast<std::size_t>(c.out_channels) * Lo, 0.0f);
    conv1d_forward(x.data(), c.W.data(), c.b.empty() ? nullptr : c.b.data(),
                   c.in_channels, L, c.out_channels, c.kernel_size, c.stride,
                   c.padding, c.dilation, c.groups, y.data());
}

void conv_dgrad(const Conv1d& c, const Vec& dy, int L_in, Vec& dx) {
    dx.assign(static_cast<std::size_t>(c.in_channels) * L_in, 0.0f);
    conv1d_backward_input(c.W.data(), dy.data(), c.in_channels, L_in,
                          c.out_channels, c.kernel_size, c.stride, c.padding,
                          c.dilation, c.groups, dx.data());
}

void conv_wgrad(Conv1d& c, const Vec& x, int L_in, const Vec& dy) {
    if (c.dW.size() != c.W.size()) c.dW.assign(c.W.size(), 0.0f);
    if (!c.b.empty() && c.db.size() != c.b.size()) c.db.assign(c.b.size(), 0.0f);
    conv1d_backward_weight(x.data(), dy.data(), c.in_channels, L_in,
                           c.out_channels, c.kernel_size, c.stride, c.padding,
                           c.dilation, c.groups, c.dW.data(),
                           c.b.empty() ? nullptr : c.db.data());
}

void add_inplace(Vec& a, const Vec& b) {
    if (a.size() != b.size()) throw std::runtime_error("kdo::add_inplace: size");
    for (std::size_t i = 0; i < a.size(); ++i) a[i] += b[i];
}

void scale_inplace(Vec& a, float s) {
    for (auto& v : a) v *= s;
}

// Leaky ReLU at `site` (-1: none); `count` tallies the elements whose own
// sign a mask overrides (once per site and forward).
void leaky(const Vec& x, float slope, Vec& y, int site = -1, bool count = false) {
    y.resize(x.size());
    const signed char* m = kink_mask(site, x.size());
    if (!m) {
        leaky_forward(x.data(), slope, x.size(), y.data());
        return;
    }
    long flips = 0;
    for (std::size_t i = 0; i < x.size(); ++i) {
        const bool pos = m[i] != 0;
        flips += pos != (x[i] > 0.0f);
        y[i] = pos ? x[i] : slope * x[i];
    }
    if (count) g_kinks->flips[static_cast<std::size_t>(site)] += flips;
}

void leaky_bwd(const Vec& x, const Vec& dy, float slope, Vec& dx, int site = -1) {
    dx.resize(x.size());
    const signed char* m = kink_mask(site, x.size());
    if (!m) {
        leaky_backward(x.data(), dy.data(), slope, x.size(), dx.data());
        return;
    }
    for (std::size_t i = 0; i < x.size(); ++i) dx[i] = m[i] ? dy[i] : slope * dy[i];
}

// Channel concat of (C_i, L) parts (kokoro_decoder_backward.cpp:465-478).
Vec cat_channels(const std::vector<const Vec*>& parts) {
    Vec out;
    for (const Vec* p : parts) out.insert(out.end(), p->begin(), p->end());
    return out;
}

}  // namespace

// kokoro_decoder_backward.cpp:100-120: GroupNorm(G=C, unit gamma), then the
// style affine on the (L, C) sequence layout, then back to NCL.
void adain_affine_forward(const Vec& x, const Vec& gamma, const Vec& beta,
                          int C, int L, float eps, Vec& y, Vec& x_seq) {
    Vec unit = ones(C), zero = zeros(C);
    Vec xn(static_cast<std::size_t>(C) * L);
    instnorm_forward(x.data(), unit.data(), zero.data(), C, L, eps, xn.data());
    x_seq.resize(xn.size());
    for (int c = 0; c < C; ++c)
        for (int l = 0; l < L; ++l)
            x_seq[static_cast<std::size_t>(l) * C + c] = xn[static_cast<std::size_t>(c) * L + l];
    y.resize(xn.size());
    for (int l = 0; l < L; ++l)
        for (int c = 0; c < C; ++c) {
            // modulate: Y = X * (1 + gamma) + beta on the (L, C) layout
            const Real ys = x_seq[static_cast<std::size_t>(l) * C + c] * (1.0f + gamma[c]) + beta[c];
            y[static_cast<std::size_t>(c) * L + l] = ys;
        }
}

// kokoro_decoder_backward.cpp:122-150 (modulate_backward at :41-61).
void adain_affine_backward(const Vec& x, const Vec& x_seq, const Vec& gamma,
                           const Vec& dY, int C, int L, float eps, Vec& dX,
                           Vec& dGamma, Vec& dBeta) {
    Vec dXn(static_cast<std::size_t>(C) * L);
    dGamma.assign(static_cast<std::size_t>(C), 0.0f);
    dBeta.assign(static_cast<std::size_t>(C), 0.0f);
    for (int c = 0; c < C; ++c) {
        double sg = 0.0, sb = 0.0;
        for (int l = 0; l < L; ++l) {
            const Real dy = dY[static_cast<std::size_t>(c) * L + l];
            sg += static_cast<double>(dy) * x_seq[static_cast<std::size_t>(l) * C + c];
            sb += dy;
            dXn[static_cast<std::size_t>(c) * L + l] = dy * (1.0f + gamma[c]);
        }
        dGamma[c] = static_cast<Real>(sg);
        dBeta[c] = static_cast<Real>(sb);
    }
    Vec unit = ones(C);
    dX.resize(dXn.size());
    instnorm_backward(x.data(), unit.data(), dXn.data(), C, L, eps, dX.data(),
                      nullptr, nullptr);
}

// kokoro_decoder_backward.cpp:152-207
void adain_resblk_1d_forward_train(const AdainResBlk1dWeights& w, const Vec& x,
                                   int L_in, const Vec& g1, const Vec& b1,
                                   const Vec& g2, const Vec& b2, float eps,
                                   int& L_out, Vec& y, AdainResBlkCache& cache) {
    const int C_in = w.channels_in, C_out = w.channels_out;
    L_out = w.upsample ? 2 * L_in : L_in;
    cache.x = x;
    cache.L_in = L_in;
    cache.L_out = L_out;

    adain_affine_forward(x, g1, b1, C_in, L_in, eps, cache.r_pre, cache.x_seq1);
    Vec r;
    leaky(cache.r_pre, 0.2f, r, block_site(0), true);
    Vec pooled;
    if (w.upsample) {
        pooled.assign(static_cast<std::size_t>(C_in) * L_out, 0.0f);
        convt1d_forward(r.data(), w.pool_W.data(), w.pool_b.data(), C_in, L_in,
                        C_in, 3, 2, 1, 1, 1, C_in, pooled.data());
    } else {
        pooled = r;
    }
    conv_fwd(w.conv1, pooled, L_out, cache.conv1_out);
    adain_affine_forward(cache.conv1_out, g2, b2, C_out, L_out, eps,
                         cache.n2_pre, cache.x_seq2);
    Vec n2;
    leaky(cache.n2_pre, 0.2f, n2, block_site(1), true);
    Vec conv2_out;
    conv_fwd(w.conv2, n2, L_out, conv2_out);

    Vec short_x;
    if (w.upsample) {
        short_x.assign(static_cast<std::size_t>(C_in) * L_out, 0.0f);
        nearest2x_forward(x.data(), C_in, L_in, short_x.data());
    } else {
        short_x = x;
    }
    if (w.learned_sc) {
        Vec sc;
        conv_fwd(w.conv1x1, short_x, L_out, sc);
        short_x = sc;
    }
    add_inplace(conv2_out, short_x);
    scale_inplace(conv2_out, 1.0f / std::sqrt(2.0f));
    y = conv2_out;
    (void)C_out;
}

// kokoro_decoder_backward.cpp:209-285
void adain_resblk_1d_backward(AdainResBlk1dWeights& w,
                              const AdainResBlkCache& cache, const Vec& g1,
                              const Vec& g2, const Vec& dY, float eps, Vec& dX,
                              Vec& dG1, Vec& dB1, Vec& dG2, Vec& dB2,
                              const Ext* ext) {
    const int C_in = w.channels_in, C_out = w.channels_out;
    const int L_in = cache.L_in, L_out = cache.L_out;
    const bool wg = ext && ext->wgrad;

    Vec d_branch = dY;
    scale_inplace(d_branch, 1.0f / std::sqrt(2.0f));

    // conv2 (input = leaky(n2_pre))
    Vec d_n2;
    conv_dgrad(w.conv2, d_branch, L_out, d_n2);
    if (wg) {
        Vec n2;
        leaky(cache.n2_pre, 0.2f, n2, block_site(1));
        conv_wgrad(w.conv2, n2, L_out, d_branch);
    }
    Vec d_n2_pre;
    leaky_bwd(cache.n2_pre, d_n2, 0.2f, d_n2_pre, block_site(1));
    Vec d_conv1_out;
    adain_affine_backward(cache.conv1_out, cache.x_seq2, g2, d_n2_pre, C_out,
                          L_out, eps, d_conv1_out, dG2, dB2);
    // conv1 (input = pooled)
    Vec d_pooled;
    conv_dgrad(w.conv1, d_conv1_out, L_out, d_pooled);
    Vec r;
    if (wg || w.upsample) leaky(cache.r_pre, 0.2f, r, block_site(0));
    if (wg) {
        Vec pooled;
        if (w.upsample) {
            pooled.assign(static_cast<std::size_t>(C_in) * L_out, 0.0f);
            convt1d_forward(r.data(), w.pool_W.data(), w.pool_b.data(), C_in,
                            L_in, C_in, 3, 2, 1, 1, 1, C_in, pooled.data());
        } else {
            pooled = r;
        }
        conv_wgrad(w.conv1, pooled, L_out, d_conv1_out);
    }
    Vec d_r;
    if (w.upsample) {
        d_r.assign(static_cast<std::size_t>(C_in) * L_in, 0.0f);
        convt1d_backward_input(w.pool_W.data(), d_pooled.data(), C_in, L_in,
                               C_in, 3, 2, 1, 1, 1, C_in, d_r.data());
        if (wg) {
            if (w.dpool_W.size() != w.pool_W.size()) w.dpool_W.assign(w.pool_W.size(), 0.0f);
            if (w.dpool_b.size() != w.pool_b.size()) w.dpool_b.assign(w.pool_b.size(), 0.0f);
            convt1d_backward_weight(r.data(), d_pooled.data(), C_in, L_in, C_in,
                                    3, 2, 1, 1, 1, C_in, w.dpool_W.data(),
                                    w.dpool_b.data());
        }
    } else {
        d_r = d_pooled;
    }
    Vec d_r_pre;
    leaky_bwd(cache.r_pre, d_r, 0.2f, d_r_pre, block_site(0));
    Vec dX_res;
    adain_affine_backward(cache.x, cache.x_seq1, g1, d_r_pre, C_in, L_in, eps,
                          dX_res, dG1, dB1);

    // shortcut
    Vec d_short_pre;
    if (w.learned_sc) {
        conv_dgrad(w.conv1x1, d_branch, L_out, d_short_pre);
        if (wg) {
            Vec short_x;
            if (w.upsample) {
                short_x.assign(static_cast<std::size_t>(C_in) * L_out, 0.0f);
                nearest2x_forward(cache.x.data(), C_in, L_in, short_x.data());
            } else {
                short_x = cache.x;
            }
            conv_wgrad(w.conv1x1, short_x, L_out, d_branch);
        }
    } else {
        d_short_pre = d_branch;
    }
    Vec dX_short;
    if (w.upsample) {
        dX_short.assign(static_cast<std::size_t>(C_in) * L_in, 0.0f);
        nearest2x_backward(d_short_pre.data(), C_in, L_in, dX_short.data());
    } else {
        dX_short = d_short_pre;
    }
    add_inplace(dX_res, dX_short);
    dX = dX_res;
}

// kokoro_decoder_backward.cpp:287-323
void adain_resblock1_forward_train(const AdaINResBlock1Weights& w,
                                   const Vec& x_in, int C, int L,
                                   const Arr3& g1, const Arr3& b1,
                                   const Arr3& g2, const Arr3& b2, Vec& x_out,
                                   AdainResBlock1Cache& cache) {
    cache.C = C;
    cache.L = L;
    Vec x = x_in;
    for (int i = 0; i < 3; ++i) {
        cache.x_in[i] = x;
        adain_affine_forward(x, g1[i], b1[i], C, L, w.adain1[i].eps,
                             cache.s1_pre[i], cache.x_seq1[i]);
        Vec xt1(x.size());
        snake_forward(cache.s1_pre[i].data(), w.alpha1[i].data(), C, L, xt1.data());
        conv_fwd(w.convs1[i], xt1, L, cache.c1_out[i]);
        adain_affine_forward(cache.c1_out[i], g2[i], b2[i], C, L,
                             w.adain2[i].eps, cache.s2_pre[i], cache.x_seq2[i]);
        Vec xt2(x.size());
        snake_forward(cache.s2_pre[i].data(), w.alpha2[i].data(), C, L, xt2.data());
        Vec c2_out;
        conv_fwd(w.convs2[i], xt2, L, c2_out);
        add_inplace(c2_out, x);
        x = c2_out;
    }
    x_out = x;
}

// kokoro_decoder_backward.cpp:325-376
void adain_resblock1_backward(AdaINResBlock1Weights& w,
                              const AdainResBlock1Cache& cache, const Arr3& g1,
                              const Arr3& g2, const Vec& dX_out, Vec& dX_in,
                              Arr3& dG1, Arr3& dB1, Arr3& dG2, Arr3& dB2,
                              const Ext* ext) {
    const int C = cache.C, L = cache.L;
    const bool wg = ext && ext->wgrad;
    const bool da = ext && ext->dalpha;
    Vec dx = dX_out;
    for (int i = 2; i >= 0; --i) {
        const Vec& d_c2 = dx;
        const Vec d_skip = dx;

        Vec d_xt2;
        conv_dgrad(w.convs2[i], d_c2, L, d_xt2);
        if (wg) {
            Vec xt2(d_xt2.size());
            snake_forward(cache.s2_pre[i].data(), w.alpha2[i].data(), C, L, xt2.data());
            conv_wgrad(w.convs2[i], xt2, L, d_c2);
        }
        Vec d_s2_pre(d_xt2.size());
        Vec dAlpha2(static_cast<std::size_t>(C), 0.0f);
        snake_backward(cache.s2_pre[i].data(), w.alpha2[i].data(), d_xt2.data(),
                       C, L, d_s2_pre.data(), dAlpha2.data());
        if (da) {
            if (w.dalpha2[i].size() != static_cast<std::size_t>(C)) w.dalpha2[i].assign(C, 0.0f);
            for (int c = 0; c < C; ++c) w.dalpha2[i][c] += dAlpha2[c];
        }
        Vec d_c1_out;
        adain_affine_backward(cache.c1_out[i], cache.x_seq2[i], g2[i], d_s2_pre,
                              C, L, w.adain2[i].eps, d_c1_out, dG2[i], dB2[i]);

        Vec d_xt1;
        conv_dgrad(w.convs1[i], d_c1_out, L, d_xt1);
        if (wg) {
            Vec xt1(d_xt1.size());
            snake_forward(cache.s1_pre[i].data(), w.alpha1[i].data(), C, L, xt1.data());
            conv_wgrad(w.convs1[i], xt1, L, d_c1_out);
        }
        Vec d_s1_pre(d_xt1.size());
        Vec dAlpha1(static_cast<std::size_t>(C), 0.0f);
        snake_backward(cache.s1_pre[i].data(), w.alpha1[i].data(), d_xt1.data(),
                       C, L, d_s1_pre.data(), dAlpha1.data());
        if (da) {
            if (w.dalpha1[i].size() != static_cast<std::size_t>(C)) w.dalpha1[i].assign(C, 0.0f);
            for (int c = 0; c < C; ++c) w.dalpha1[i][c] += dAlpha1[c];
        }
        Vec d_x_adain1;
        adain_affine_backward(cache.x_in[i], cache.x_seq1[i], g1[i], d_s1_pre,
                              C, L, w.adain1[i].eps, d_x_adain1, dG1[i], dB1[i]);
        add_inplace(d_x_adain1, d_skip);
        dx = d_x_adain1;
    }
    dX_in = dx;
}

// kokoro_decoder_backward.cpp:378-410
void spectral_head_forward_train(const Conv1d& conv_post, const Vec& x, int C,
                                 int L, const Vec& window, int n_fft, int hop,
                                 int win, Vec& audio, SpectralHeadCache& cache) {
    cache.C = C;
    cache.L = L;
    cache.x_pre = x;
    Vec xl;
    leaky(x, 0.01f, xl, g_kink_head, true);
    conv_fwd(conv_post, xl, L, cache.post);
    const int F = n_fft / 2 + 1;
    Vec spec(static_cast<std::size_t>(L) * 2 * F);
    for (int c = 0; c < F; ++c)
        for (int l = 0; l < L; ++l) {
            const double mag = std::exp(static_cast<double>(cache.post[static_cast<std::size_t>(c) * L + l]));
            const double ang = std::sin(static_cast<double>(cache.post[static_cast<std::size_t>(F + c) * L + l]));
            // complex_from_polar on the rounded float mag / angle
            const Real magf = static_cast<Real>(mag), angf = static_cast<Real>(ang);
            spec[(static_cast<std::size_t>(l) * F + c) * 2] =
                static_cast<Real>(static_cast<double>(magf) * std::cos(static_cast<double>(angf)));
            spec[(static_cast<std::size_t>(l) * F + c) * 2 + 1] =
                static_cast<Real>(static_cast<double>(magf) * std::sin(static_cast<double>(angf)));
        }
    const int signal_len = (L - 1) * hop;
    audio.assign(static_cast<std::size_t>(signal_len), 0.0f);
    istft(spec.data(), window.data(), L, signal_len, n_fft, hop, win, audio.data());
}

// kokoro_decoder_backward.cpp:412-458
void spectral_head_backward(Conv1d& conv_post, const SpectralHeadCache& cache,
                            const Vec& window, int n_fft, int hop, int win,
                            const Vec& dAudio, Vec& dX, const Ext* ext) {
    const int C = cache.C, L = cache.L;
    const int F = n_fft / 2 + 1;
    const int signal_len = (L - 1) * hop;
    Vec dSpec(static_cast<std::size_t>(L) * 2 * F);
    istft_backward(dAudio.data(), window.data(), L, signal_len, n_fft, hop, win,
                   dSpec.data());
    const int C_post = n_fft + 2;
    Vec dpost(static_cast<std::size_t>(C_post) * L, 0.0f);
    for (int c = 0; c < F; ++c)
        for (int l = 0; l < L; ++l) {
            const double pm = cache.post[static_cast<std::size_t>(c) * L + l];
            const double pp = cache.post[static_cast<std::size_t>(F + c) * L + l];
            const double mag = static_cast<Real>(std::exp(pm));
            const double ang = static_cast<Real>(std::sin(pp));
            const double ca = std::cos(ang), sa = std::sin(ang);
            const double dRe = dSpec[(static_cast<std::size_t>(l) * F + c) * 2];
            const double dIm = dSpec[(static_cast<std::size_t>(l) * F + c) * 2 + 1];
            const double dmag = dRe * ca + dIm * sa;
            const double dang = mag * (-dRe * sa + dIm * ca);
            dpost[static_cast<std::size_t>(c) * L + l] = static_cast<Real>(dmag * mag);
            dpost[static_cast<std::size_t>(F + c) * L + l] = static_cast<Real>(dang * std::cos(pp));
        }
    Vec dXl;
    conv_dgrad(conv_post, dpost, L, dXl);
    if (ext && ext->wgrad) {
        Vec xl;
        leaky(cache.x_pre, 0.01f, xl, g_kink_head);
        conv_wgrad(conv_post, xl, L, dpost);
    }
    leaky_bwd(cache.x_pre, dXl, 0.01f, dX, g_kink_head);
    (void)C;
}

// kokoro_decoder_backward.cpp:482-537
void decoder_backbone_forward_train(const DecoderBackbone& bb, const Vec& asr,
                                    const Vec& F0_pred, const Vec& N_pred,
                                    int T, const std::vector<BlockAffines>& aff,
                                    float eps, Vec& gen_in,
                                    BackboneCache& cache) {
    const int n_dec = static_cast<int>(bb.decode.size());
    cache.T = T;
    cache.decode.assign(n_dec, AdainResBlkCache{});
    cache.res_applied.assign(n_dec, 0);
    cache.x_channels.assign(n_dec, 0);
    cache.asr = asr;
    cache.F0 = F0_pred;
    cache.N = N_pred;

    conv_fwd(bb.F0_conv, F0_pred, 2 * T, cache.F0_dn);
    conv_fwd(bb.N_conv, N_pred, 2 * T, cache.N_dn);
    conv_fwd(bb.asr_res, asr, T, cache.asr_res_out);

    Vec dec_pre = cat_channels({&asr, &cache.F0_dn, &cache.N_dn});
    int L_after = 0;
    Vec x;
    g_kink_block = g_kinks ? 0 : -1;
    adain_resblk_1d_forward_train(bb.encode, dec_pre, T, aff[0].g1, aff[0].b1,
                                  aff[0].g2, aff[0].b2, eps, L_after, x,
                                  cache.encode);
    int L_now = L_after;
    bool res = true;
    for (int i = 0; i < n_dec; ++i) {
        cache.x_channels[i] = static_cast<int>(x.size()) / L_now;
        Vec blk_in;
        if (res) {
            cache.res_applied[i] = 1;
            blk_in = cat_channels({&x, &cache.asr_res_out, &cache.F0_dn, &cache.N_dn});
        } else {
            blk_in = x;
        }
        int L_next = 0;
        Vec y;
        g_kink_block = g_kinks ? 2 * (1 + i) : -1;
        adain_resblk_1d_forward_train(bb.decode[i], blk_in, L_now, aff[1 + i].g1,
                                      aff[1 + i].b1, aff[1 + i].g2,
                                      aff[1 + i].b2, eps, L_next, y,
                                      cache.decode[i]);
        x = y;
        L_now = L_next;
        if (bb.decode[i].upsample) res = false;
    }
    g_kink_block = -1;
    gen_in = x;
}

// kokoro_decoder_backward.cpp:539-574. With ext->wgrad the grads into the
// frozen front-conv outputs (the dropped cat channels) also feed the
// F0_conv / N_conv / asr_res weight grads.
void decoder_backbone_backward(DecoderBackbone& bb, const BackboneCache& cache,
                               const std::vector<BlockAffines>& aff,
                               const Vec& dGenIn, float eps,
                               std::vector<BlockAffines>& dAff,
                               const Ext* ext) {
    const int n_dec = static_cast<int>(bb.decode.size());
    dAff.assign(static_cast<std::size_t>(n_dec) + 1, BlockAffines{});
    const bool wg = ext && ext->wgrad;
    const int T = cache.T;
    const int C_asr_res = bb.asr_res.out_channels;
    Vec d_asr_res(static_cast<std::size_t>(C_asr_res) * T, 0.0f);
    Vec d_F0dn(static_cast<std::size_t>(T), 0.0f), d_Ndn(static_cast<std::size_t>(T), 0.0f);

    Vec dX = dGenIn;
    for (int i = n_dec - 1; i >= 0; --i) {
        Vec blk_dX;
        BlockAffines& g = dAff[1 + i];
        g_kink_block = g_kinks ? 2 * (1 + i) : -1;
        adain_resblk_1d_backward(bb.decode[i], cache.decode[i], aff[1 + i].g1,
                                 aff[1 + i].g2, dX, eps, blk_dX, g.g1, g.b1,
                                 g.g2, g.b2, ext);
        if (cache.res_applied[i]) {
            const int Cx = cache.x_channels[i];
            const int L_in = cache.decode[i].L_in;
            if (wg) {
                const Real* base = blk_dX.data() + static_cast<std::size_t>(Cx) * L_in;
                for (std::size_t j = 0; j < d_asr_res.size(); ++j) d_asr_res[j] += base[j];
                base += d_asr_res.size();
                for (int j = 0; j < T; ++j) d_F0dn[j] += base[j];
                base += T;
                for (int j = 0; j < T; ++j) d_Ndn[j] += base[j];
            }
            dX.assign(blk_dX.begin(), blk_dX.begin() + static_cast<std::size_t>(Cx) * L_in);
        } else {
            dX = blk_dX;
        }
    }
    Vec enc_dX;
    BlockAffines& ge = dAff[0];
    g_kink_block = g_kinks ? 0 : -1;
    adain_resblk_1d_backward(bb.encode, cache.encode, aff[0].g1, aff[0].g2, dX,
                             eps, enc_dX, ge.g1, ge.b1, ge.g2, ge.b2, ext);
    g_kink_block = -1;
    if (wg) {
        const std::size_t n_asr = cache.asr.size();
        const Real* base = enc_dX.data() + n_asr;
        for (int j = 0; j < T; ++j) d_F0dn[j] += base[j];
        base += T;
        for (int j = 0; j < T; ++j) d_Ndn[j] += base[j];
        conv_wgrad(bb.F0_conv, cache.F0, 2 * T, d_F0dn);
        conv_wgrad(bb.N_conv, cache.N, 2 * T, d_Ndn);
        conv_wgrad(bb.asr_res, cache.asr, T, d_asr_res);
    }
}

// kokoro_decoder_backward.cpp:592-667
void generator_forward_train(const Generator& gen, const Vec& gen_in, int L_in,
                             const Vec& har, int frames,
                             const std::vector<ResBlock1Affines>& naff,
                             const std::vector<ResBlock1Affines>& raff,
                             Vec& audio, GeneratorCache& cache) {
    const int K = gen.num_kernels;
    cache.stages.assign(gen.num_upsamples, GenStageCache{});
    cache.har = har;
    cache.frames = frames;
    Vec x = gen_in;
    int L = L_in;
    for (int i = 0; i < gen.num_upsamples; ++i) {
        GenStageCache& sc = cache.stages[i];
        sc.x_in = x;
        sc.C_in = gen.ups_C_in[i];
        sc.L_in = L;
        Vec a;
        leaky(x, 0.1f, a, gen_site(i), true);

        Vec x_source;
        conv_fwd(gen.noise_convs[i], har, frames, x_source);
        const int L_src = static_cast<int>(x_source.size()) / gen.ups_C_out[i];
        sc.L_src = L_src;
        Vec src;
        adain_resblock1_forward_train(gen.noise_res[i], x_source, gen.ups_C_out[i],
                                      L_src, naff[i].g1, naff[i].b1, naff[i].g2,
                                      naff[i].b2, src, sc.noise);

        const int kL = gen.ups_k[i], s = gen.ups_stride[i], p = gen.ups_pad[i];
        int L_x = (L - 1) * s - 2 * p + (kL - 1) + 1;
        Vec u(static_cast<std::size_t>(gen.ups_C_out[i]) * L_x);
        convt1d_forward(a.data(), gen.ups_W[i].data(), gen.ups_b[i].data(),
                        gen.ups_C_in[i], L, gen.ups_C_out[i], kL, s, p, 0, 1, 1,
                        u.data());
        if (i == gen.num_upsamples - 1) {
            Vec padded(static_cast<std::size_t>(gen.ups_C_out[i]) * (L_x + 1));
            pad_reflect_left1_forward(u.data(), gen.ups_C_out[i], L_x, padded.data());
            u = padded;
            L_x += 1;
        }
        if (L_src != L_x)
            throw std::runtime_error("kdo::generator_forward_train: noise source length mismatch");
        sc.C_out = gen.ups_C_out[i];
        sc.L_out = L_x;
        add_inplace(u, src);

        sc.res.assign(K, AdainResBlock1Cache{});
        Vec xs;
        for (int j = 0; j < K; ++j) {
            const ResBlock1Affines& ra = raff[static_cast<std::size_t>(i) * K + j];
            Vec xj;
            adain_resblock1_forward_train(gen.resblocks[i * K + j], u,
                                          gen.ups_C_out[i], L_x, ra.g1, ra.b1,
                                          ra.g2, ra.b2, xj, sc.res[j]);
            if (j == 0) xs = xj;
            else add_inplace(xs, xj);
        }
        scale_inplace(xs, 1.0f / static_cast<Real>(K));
        x = xs;
        L = L_x;
    }
    cache.window = hann_periodic(gen.win_size);
    g_kink_head = gen_site(gen.num_upsamples);
    spectral_head_forward_train(gen.conv_post, x, gen.ups_C_out[gen.num_upsamples - 1],
                                L, cache.window, gen.n_fft, gen.hop_size,
                                gen.win_size, audio, cache.head);
    g_kink_head = -1;
}

// kokoro_decoder_backward.cpp:669-737. With ext->wgrad the noise branch's dX
// (dropped by the reference) feeds the noise_convs weight grads.
void generator_backward(Generator& gen, const GeneratorCache& cache,
                        const std::vector<ResBlock1Affines>& naff,
                        const std::vector<ResBlock1Affines>& raff,
                        const Vec& dAudio, Vec& dGenIn,
                        std::vector<ResBlock1Affines>& dnaff,
                        std::vector<ResBlock1Affines>& draff, const Ext* ext) {
    const int K = gen.num_kernels;
    const int U = gen.num_upsamples;
    const bool wg = ext && ext->wgrad;
    dnaff.assign(U, ResBlock1Affines{});
    draff.assign(static_cast<std::size_t>(U) * K, ResBlock1Affines{});

    Vec dX;
    g_kink_head = gen_site(U);
    spectral_head_backward(gen.conv_post, cache.head, cache.window, gen.n_fft,
                           gen.hop_size, gen.win_size, dAudio, dX, ext);
    g_kink_head = -1;
    for (int i = U - 1; i >= 0; --i) {
        const GenStageCache& sc = cache.stages[i];
        const int L = sc.L_out;
        Vec d_scaled = dX;
        scale_inplace(d_scaled, 1.0f / static_cast<Real>(K));
        Vec d_m;
        for (int j = 0; j < K; ++j) {
            ResBlock1Affines& dr = draff[static_cast<std::size_t>(i) * K + j];
            Vec dxin_j;
            adain_resblock1_backward(gen.resblocks[i * K + j], sc.res[j],
                                     raff[static_cast<std::size_t>(i) * K + j].g1,
                                     raff[static_cast<std::size_t>(i) * K + j].g2,
                                     d_scaled, dxin_j, dr.g1, dr.b1, dr.g2,
                                     dr.b2, ext);
            if (j == 0) d_m = dxin_j;
            else add_inplace(d_m, dxin_j);
        }
        {
            ResBlock1Affines& dn = dnaff[i];
            Vec dsrc_in;
            adain_resblock1_backward(gen.noise_res[i], sc.noise, naff[i].g1,
                                     naff[i].g2, d_m, dsrc_in, dn.g1, dn.b1,
                                     dn.g2, dn.b2, ext);
            if (wg) conv_wgrad(gen.noise_convs[i], cache.har, cache.frames, dsrc_in);
        }
        Vec du = d_m;
        if (i == U - 1) {
            Vec du_pre(static_cast<std::size_t>(gen.ups_C_out[i]) * (L - 1));
            pad_reflect_left1_backward(du.data(), gen.ups_C_out[i], L - 1, du_pre.data());
            du = du_pre;
        }
        Vec da(static_cast<std::size_t>(sc.C_in) * sc.L_in);
        convt1d_backward_input(gen.ups_W[i].data(), du.data(), sc.C_in, sc.L_in,
                               gen.ups_C_out[i], gen.ups_k[i], gen.ups_stride[i],
                               gen.ups_pad[i], 0, 1, 1, da.data());
        if (wg) {
            Vec a;
            leaky(sc.x_in, 0.1f, a, gen_site(i));
            if (gen.dups_W[i].size() != gen.ups_W[i].size()) gen.dups_W[i].assign(gen.ups_W[i].size(), 0.0f);
            if (gen.dups_b[i].size() != gen.ups_b[i].size()) gen.dups_b[i].assign(gen.ups_b[i].size(), 0.0f);
            convt1d_backward_weight(a.data(), du.data(), sc.C_in, sc.L_in,
                                    gen.ups_C_out[i], gen.ups_k[i],
                                    gen.ups_stride[i], gen.ups_pad[i], 0, 1, 1,
                                    gen.dups_W[i].data(), gen.dups_b[i].data());
        }
        Vec dx_in;
        leaky_bwd(sc.x_in, da, 0.1f, dx_in, gen_site(i));
        dX = dx_in;
    }
    dGenIn = dX;
}

// HarmonicSource::forward (kokoro_modules.cpp:1574-1665). The phase
// accumulator is the reference's sequential float recurrence, evaluated in
// float exactly as written there.
void harmonic_source_forward(const HarmonicSource& hs, const Vec& F0,
                             int frame_count, int& signal_len,
                             int& stft_frames, Vec& har) {
    signal_len = frame_count * hs.upsample_scale;
    const float sr_f = static_cast<float>(hs.sample_rate);
    const int dim = hs.harmonic_num + 1;
    std::vector<float> phases(static_cast<std::size_t>(dim), 0.0f);
    Vec merged(static_cast<std::size_t>(signal_len));
    constexpr float kTwoPi = 6.28318530717958647692f;
    std::vector<float> sine(static_cast<std::size_t>(dim));
    for (int t = 0; t < signal_len; ++t) {
        const int frame = t / hs.upsample_scale;
        const float f0 = (float)F0[std::min(frame, frame_count - 1)];
        const float uv = (f0 > 0.0f) ? 1.0f : 0.0f;
        for (int h = 0; h < dim; ++h) {
            volatile float omega = kTwoPi * static_cast<float>(h + 1);
            omega = omega * f0;
            omega = omega / sr_f;
            volatile float ph = phases[h] + omega;
            if (ph > kTwoPi) ph = ph - kTwoPi;
            phases[h] = ph;
            volatile float sv = std::sin(phases[h]);
            sv = sv * hs.sine_amp;
            sv = sv * uv;
            sine[h] = sv;
        }
        // l_linear (1, dim) + bias, then tanh
        double acc = hs.lb[0];
        for (int h = 0; h < dim; ++h) acc += static_cast<double>(hs.lW[h]) * sine[h];
        merged[t] = static_cast<Real>(std::tanh(static_cast<double>(static_cast<float>(acc))));
    }
    const Vec window = hann_periodic(hs.win_size);
    Vec spec;
    stft_frames = stft(merged.data(), signal_len, window.data(), hs.n_fft,
                       hs.hop_size, hs.win_size, spec);
    const int F = hs.n_fft / 2 + 1;
    har.assign(static_cast<std::size_t>(2 * F) * stft_frames, 0.0f);
    for (int f = 0; f < stft_frames; ++f)
        for (int k = 0; k < F; ++k) {
            const double re = spec[(static_cast<std::size_t>(f) * F + k) * 2];
            const double im = spec[(static_cast<std::size_t>(f) * F + k) * 2 + 1];
            har[static_cast<std::size_t>(k) * stft_frames + f] = static_cast<Real>(std::sqrt(re * re + im * im));
            har[static_cast<std::size_t>(F + k) * stft_frames + f] = static_cast<Real>(std::atan2(im, re));
        }
}

}  // namespace KDO_NS

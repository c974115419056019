// Inference forwards of the decoder back half: the reference's twins of the
// `_train` assemblies (kokoro_modules.cpp:596-620 ada_in_1d_styled, 651-706
// adain_resblk_1d_forward, 1197-1231 adain_resblock1_forward, 1087-1141
// DecoderBackbone::forward, 1400-1552 Generator::forward), which
// decode_back_half chains (kokoro.cpp:352-407).
//
// Written as their own composition over the kdec kernels, not through the
// training assemblies, so the two forwards check each other the way the
// reference's neutral-identity test does (tests/test_kokoro_decoder_backward.cpp:
// 516-530). Nothing is cached: every intermediate is released as soon as its
// consumer has been enqueued, so device memory holds about one stage's
// activations. Each AdaIN unit's (gamma, beta) = fc(style) is one projection
// launch for all N style rows (compute_style_affine, :563-572), and the AdaIN
// statistics, the (1 + gamma) affine and the activation are one fused pass.
#include "brosoundml/kokoro_modules.h"
#include "kdec.h"

#include <cmath>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace bt = brotensor;

namespace brosoundml {
namespace {

using bt::Device;
using bt::Tensor;

kdec_ctx* rt() { return bt::runtime(); }

[[noreturn]] void fail(const std::string& where, const std::string& why) {
    throw std::runtime_error("brosoundml: " + where + ": " + why);
}

void ok(int rc, const char* where) {
    if (rc != KDEC_OK) throw std::runtime_error(std::string(kdec_last_error(rt())) + " (in " + where + ")");
}

const float* cf(const Tensor& t) { return static_cast<const float*>(t.data); }
float* mf(const Tensor& t) { return static_cast<float*>(t.data); }
long ld(const Tensor& t) { return t.row_stride(); }
Tensor make(int rows, int cols) { return Tensor::empty_on(Device::HIP, rows, cols); }

void need_device(const Tensor& t, const char* where) {
    if (t.device != Device::HIP || !t.data) fail(where, "expected a HIP device tensor (this build has no CPU path)");
}

// (gamma, beta) of one AdaIN unit for N utterances: rows of C at stride bs
// (0: one row for every utterance), and the unit's instance-norm epsilon
// (AdaIN1dWeights::eps, as ada_in_1d_styled passes it to the group norm,
// kokoro_modules.cpp:618; 1e-5 when unset).
struct Affine {
    const float* gamma;
    const float* beta;
    long bs;
    float eps = 1e-5f;
    Tensor keep;  // owns the projection buffer
};

// (gamma, beta) = chunk(fc(style)) for the N style rows (style (N, >= S) at its row stride)
Affine project(const AdaIN1dWeights& w, const Tensor& style, const char* where) {
    need_device(style, where);
    need_device(w.fc.W, where);
    const int C = w.channels, S = w.fc.in_features;
    if (w.fc.W.rows != 2 * C || w.fc.W.cols != S) fail(where, "AdaIN fc must be (2C, style_dim)");
    if (style.cols < S) fail(where, "style rows shorter than style_dim");
    Affine a;
    a.keep = make(style.rows, 2 * C);
    ok(kdec_style_proj_fwd(rt(), cf(w.fc.W), w.fc.b.data ? cf(w.fc.b) : nullptr, cf(style), ld(style), mf(a.keep),
                           2 * C, style.rows, 2 * C, S),
       where);
    a.gamma = cf(a.keep);
    a.beta = cf(a.keep) + C;
    a.bs = 2 * C;
    a.eps = w.eps > 0.0f ? w.eps : 1e-5f;
    return a;
}

// y = act((1 + gamma) * instance_norm(x) + beta), statistics in the same pass
Tensor adain(const Tensor& x, int C, int L, const Affine& a, int act, float slope, const Tensor* alpha,
             const char* where) {
    const int N = x.rows;
    Tensor st = make(N * C, 2);
    Tensor y = make(N, C * L);
    ok(kdec_adain_act_fwd_stats(rt(), cf(x), ld(x), a.eps, mf(st), a.gamma, a.beta, a.bs, act, slope,
                                alpha ? cf(*alpha) : nullptr, mf(y), ld(y), nullptr, 0, N, C, L),
       where);
    return y;
}

// Y = scale * (conv(X) + b + R) + beta * Y into a caller's buffer
void conv_into(const Conv1d& c, const Tensor& X, int L, float* Y, long y_bs, const float* R = nullptr,
               long r_bs = 0, float scale = 1.0f, float beta = 0.0f) {
    if (c.groups != 1) fail("Conv1d::forward", "grouped conv1d is not on the decoder path");
    const bool bias = c.b.data && static_cast<int>(c.b.size()) == c.out_channels;
    ok(kdec_conv1d_fwd(rt(), cf(X), ld(X), cf(c.W), bias ? cf(c.b) : nullptr, Y, y_bs, X.rows, c.in_channels, L,
                       c.out_channels, c.kernel_size, c.stride, c.padding, c.dilation, R, r_bs, scale, beta),
       "Conv1d::forward");
}

Tensor conv(const Conv1d& c, const Tensor& X, int L) {
    Tensor y = make(X.rows, c.out_channels * c.out_length(L));
    conv_into(c, X, L, mf(y), ld(y));
    return y;
}

Tensor leaky(const Tensor& x, float slope) {
    Tensor y = make(x.rows, x.cols);
    ok(kdec_leaky_fwd(rt(), cf(x), ld(x), mf(y), ld(y), x.rows, x.cols, slope), "leaky_relu_forward");
    return y;
}

// channel concat of (N, C_i * L) parts
Tensor cat(const std::vector<std::pair<const Tensor*, int>>& parts, int L) {
    int Ct = 0;
    for (const auto& p : parts) Ct += p.second;
    const int N = parts.front().first->rows;
    Tensor out = make(N, Ct * L);
    long off = 0;
    for (const auto& p : parts) {
        const long n = static_cast<long>(p.second) * L;
        ok(kdec_axpby(rt(), 1.0f, cf(*p.first), ld(*p.first), 0.0f, nullptr, 0, mf(out) + off, ld(out), N, n),
           "cat_channels_ncl");
        off += n;
    }
    return out;
}

// AdainResBlk1d: (residual + shortcut) / sqrt(2) into y (N rows at y_bs)
void resblk(const AdainResBlk1dWeights& w, const Tensor& x, int L_in, const Affine& a1, const Affine& a2,
            float* y, long y_bs) {
    const char* where = "adain_resblk_1d_forward";
    const int C_in = w.channels_in, C_out = w.channels_out, N = x.rows;
    const int L_out = w.upsample ? 2 * L_in : L_in;
    Tensor r = adain(x, C_in, L_in, a1, KDEC_ACT_LEAKY, 0.2f, nullptr, where);
    if (w.upsample) {  // depthwise ConvTranspose1d k3 s2 p1 op1
        Tensor pooled = make(N, C_in * L_out);
        ok(kdec_pool_fwd(rt(), cf(r), ld(r), cf(w.pool_W), w.pool_b.data ? cf(w.pool_b) : nullptr, mf(pooled),
                         ld(pooled), N, C_in, L_in),
           where);
        r = pooled;
    }
    Tensor c1 = conv(w.conv1, r, L_out);
    r = Tensor();
    Tensor n2 = adain(c1, C_out, L_out, a2, KDEC_ACT_LEAKY, 0.2f, nullptr, where);
    c1 = Tensor();
    // shortcut: nearest 2x then the 1x1, applied here at the input rate (a 1x1
    // conv commutes with nearest upsampling)
    Tensor sc = x;
    if (w.learned_sc) sc = conv(w.conv1x1, x, L_in);
    if (w.upsample) {
        Tensor up = make(N, sc.cols * 2);
        ok(kdec_nearest2x_fwd(rt(), cf(sc), ld(sc), mf(up), ld(up), N, sc.cols / L_in, L_in), where);
        sc = up;
    }
    conv_into(w.conv2, n2, L_out, y, y_bs, cf(sc), ld(sc), 1.0f / std::sqrt(2.0f), 0.0f);
}

// AdaINResBlock1 with the last conv's output written as
// out = scale * (convs2[2](...) + x) + beta * out
void resblock1(const AdaINResBlock1Weights& w, const Tensor& x_in, int C, int L, const std::array<Affine, 3>& a1,
               const std::array<Affine, 3>& a2, float* out, long out_bs, float scale, float beta) {
    const char* where = "adain_resblock1_forward";
    Tensor x = x_in;
    for (int i = 0; i < 3; ++i) {
        Tensor xt = adain(x, C, L, a1[i], KDEC_ACT_SNAKE, 0.0f, &w.alpha1[i], where);
        Tensor c1 = conv(w.convs1[i], xt, L);
        xt = adain(c1, C, L, a2[i], KDEC_ACT_SNAKE, 0.0f, &w.alpha2[i], where);
        c1 = Tensor();
        if (i < 2) {
            Tensor xn = make(x.rows, C * L);
            conv_into(w.convs2[i], xt, L, mf(xn), ld(xn), cf(x), ld(x));
            x = xn;
        } else {
            conv_into(w.convs2[i], xt, L, out, out_bs, cf(x), ld(x), scale, beta);
        }
    }
}

std::array<Affine, 3> project3(const std::array<AdaIN1dWeights, 3>& ws, const Tensor& style, const char* where) {
    return {project(ws[0], style, where), project(ws[1], style, where), project(ws[2], style, where)};
}

}  // namespace

// ─── the reference's inference building blocks ─────────────────────────────

void ada_in_1d_styled(const AdaIN1dWeights& w, int N, int C, int L, const Tensor& x_ncl, const Tensor& style,
                      Tensor& y_ncl) {
    const char* where = "ada_in_1d_styled";
    need_device(x_ncl, where);
    if (x_ncl.rows != N || x_ncl.cols != C * L || w.channels != C) fail(where, "x must be (N, C*L) with C = channels");
    y_ncl = adain(x_ncl, C, L, project(w, style, where), KDEC_ACT_NONE, 0.0f, nullptr, where);
}

void adain_resblk_1d_forward(const AdainResBlk1dWeights& w, const Tensor& x, int L_in, const Tensor& style,
                             int& L_out, Tensor& y) {
    const char* where = "adain_resblk_1d_forward";
    need_device(x, where);
    if (x.cols != w.channels_in * L_in) fail(where, "x must be (N, channels_in*L_in)");
    L_out = w.upsample ? 2 * L_in : L_in;
    Tensor out = make(x.rows, w.channels_out * L_out);
    resblk(w, x, L_in, project(w.norm1, style, where), project(w.norm2, style, where), mf(out), ld(out));
    y = out;
}

void adain_resblock1_forward(const AdaINResBlock1Weights& w, Tensor& x, int C, int L, const Tensor& style) {
    const char* where = "adain_resblock1_forward";
    need_device(x, where);
    if (x.cols != C * L) fail(where, "x must be (N, C*L)");
    Tensor out = make(x.rows, C * L);
    resblock1(w, x, C, L, project3(w.adain1, style, where), project3(w.adain2, style, where), mf(out), ld(out), 1.0f,
              0.0f);
    x = out;
}

// ─── DecoderBackbone / Generator inference forwards ────────────────────────

void DecoderBackbone::forward(const Tensor& asr, const Tensor& F0_pred, const Tensor& N_pred, const Tensor& ref_s,
                              int T, Tensor& gen_in) const {
    const char* where = "DecoderBackbone::forward";
    for (const Tensor* t : {&asr, &F0_pred, &N_pred, &ref_s}) need_device(*t, where);
    const int N = asr.rows;
    if (asr.cols != asr_res.in_channels * T || F0_pred.cols != 2 * T || N_pred.cols != 2 * T ||
        F0_pred.rows != N || N_pred.rows != N || ref_s.rows != N)
        fail(where, "expected asr (N, asr_dim*T), F0 / N (N, 2T), ref_s N rows");
    // F0 / N curves: (N, 2T) -> stride-2 convs -> (N, T)
    const Tensor F0_dn = conv(F0_conv, F0_pred, 2 * T);
    const Tensor N_dn = conv(N_conv, N_pred, 2 * T);
    Tensor x = cat({{&asr, asr_res.in_channels}, {&F0_dn, 1}, {&N_dn, 1}}, T);
    int L = T;
    {
        Tensor y = make(N, encode.channels_out * L);
        resblk(encode, x, L, project(encode.norm1, ref_s, where), project(encode.norm2, ref_s, where), mf(y), ld(y));
        x = y;
    }
    const Tensor res_out = conv(asr_res, asr, T);
    bool res = true;
    for (const auto& blk : decode) {
        if (res) x = cat({{&x, x.cols / L}, {&res_out, asr_res.out_channels}, {&F0_dn, 1}, {&N_dn, 1}}, L);
        const int L_next = blk.upsample ? 2 * L : L;
        Tensor y = make(N, blk.channels_out * L_next);
        resblk(blk, x, L, project(blk.norm1, ref_s, where), project(blk.norm2, ref_s, where), mf(y), ld(y));
        x = y;
        L = L_next;
        if (blk.upsample) res = false;
    }
    gen_in = x;
}

void Generator::forward(const Tensor& gen_in, int L_in, const Tensor& har, int frames, const Tensor& style,
                        Tensor& audio, const std::function<bool()>& cancel) const {
    const char* where = "Generator::forward";
    need_device(gen_in, where);
    need_device(har, where);
    const int N = gen_in.rows;
    if (gen_in.cols != ups_C_in[0] * L_in) fail(where, "gen_in must be (N, init_C*L_in)");
    const int har_ch = noise_convs.empty() ? n_fft + 2 : noise_convs[0].in_channels;
    if (har.rows != N || har.cols != har_ch * frames) fail(where, "har must be (N, noise_convs in_channels * frames)");
    const int K = num_kernels;
    Tensor x = gen_in;
    int L = L_in;
    for (int i = 0; i < num_upsamples; ++i) {
        // cooperative cancellation once per upsample stage (:1418): audio stays empty
        if (cancel && cancel()) {
            audio = Tensor{};
            return;
        }
        const int C_out = ups_C_out[i];
        Tensor a = leaky(x, 0.1f);
        x = Tensor();
        // noise branch: noise_convs(har) -> noise_res
        Tensor src = conv(noise_convs[i], har, frames);
        const int L_src = src.cols / C_out;
        {
            Tensor out = make(N, C_out * L_src);
            const AdaINResBlock1Weights& nr = noise_res[i];
            resblock1(nr, src, C_out, L_src, project3(nr.adain1, style, where), project3(nr.adain2, style, where),
                      mf(out), ld(out), 1.0f, 0.0f);
            src = out;
        }
        // ups: ConvTranspose1d (+ left reflect pad by 1 on the last stage) with
        // the noise source added, in one pass (kdec_convt1d_fwd_res)
        const int kL = ups_k[i], s = ups_stride[i], p = ups_pad[i];
        const int pad_left = i == num_upsamples - 1 ? 1 : 0;
        const int L_x = (L - 1) * s - 2 * p + (kL - 1) + 1 + pad_left;
        if (L_src != L_x)
            fail(where, "noise source length " + std::to_string(L_src) + " != upsampled length " +
                            std::to_string(L_x) + " at stage " + std::to_string(i));
        Tensor u = make(N, C_out * L_x);
        ok(kdec_convt1d_fwd_res(rt(), cf(a), ld(a), cf(ups_W[i]), ups_b[i].data ? cf(ups_b[i]) : nullptr, mf(u),
                                ld(u), N, ups_C_in[i], L, C_out, kL, s, p, 0, cf(src), ld(src), pad_left),
           "conv_transpose1d_forward");
        a = Tensor();
        src = Tensor();
        // x = mean of the stage's K resblocks: each block's last conv adds its share
        Tensor xs = make(N, C_out * L_x);
        for (int j = 0; j < K; ++j) {
            const AdaINResBlock1Weights& rb = resblocks[static_cast<std::size_t>(i) * K + j];
            resblock1(rb, u, C_out, L_x, project3(rb.adain1, style, where), project3(rb.adain2, style, where),
                      mf(xs), ld(xs), 1.0f / static_cast<float>(K), j == 0 ? 0.0f : 1.0f);
        }
        x = xs;
        L = L_x;
    }
    // leaky 0.01 -> conv_post -> exp / sin polar -> iSTFT (periodic Hann, center)
    Tensor xl = leaky(x, 0.01f);
    x = Tensor();
    if (conv_post.out_channels != n_fft + 2) fail(where, "conv_post must produce n_fft + 2 channels");
    if (win_size != n_fft) fail(where, "win_size must equal n_fft");
    Tensor post = conv(conv_post, xl, L);
    xl = Tensor();
    Tensor out = make(N, (L - 1) * hop_size);
    ok(kdec_spectral_fwd(rt(), cf(post), ld(post), nullptr, mf(out), ld(out), N, L, n_fft, hop_size), "istft");
    audio = out;
}

}  // namespace brosoundml

// The closed-form special cases (closed_forms.hpp) on the CPU oracle's
// assemblies (oracle/kdec_oracle.hpp): no GPU. Built by tests/cpp/Makefile,
// run by tests/test_closed_form.py. Prints one line per failure and exits
// non-zero if any check fails.
#include "closed_forms.hpp"
#include "kdec_oracle.hpp"

#include <cstdio>

namespace {

using cf::HVec;
kdo::Vec ov(const HVec& v) { return kdo::Vec(v.begin(), v.end()); }
HVec hv(const kdo::Vec& v) { return HVec(v.begin(), v.end()); }

kdo::Conv1d oconv(const cf::ConvSpec& c) {
    kdo::Conv1d o;
    o.in_channels = c.in, o.out_channels = c.out, o.kernel_size = c.k;
    o.stride = c.s, o.padding = c.p, o.dilation = c.d;
    o.W = ov(c.W);
    o.b = ov(c.b);
    return o;
}
kdo::AdainResBlk1dWeights oresblk(const cf::ResblkSpec& s) {
    kdo::AdainResBlk1dWeights w;
    w.channels_in = s.Ci, w.channels_out = s.Co, w.upsample = s.upsample, w.learned_sc = s.learned_sc;
    w.norm1.channels = s.Ci, w.norm2.channels = s.Co;
    w.conv1 = oconv(s.conv1), w.conv2 = oconv(s.conv2);
    if (s.learned_sc) w.conv1x1 = oconv(s.conv1x1);
    w.pool_W = ov(s.pool_W), w.pool_b = ov(s.pool_b);
    return w;
}
kdo::AdaINResBlock1Weights orb1(const cf::Rb1Spec& s) {
    kdo::AdaINResBlock1Weights w;
    w.channels = s.C, w.kernel_size = s.k;
    for (int j = 0; j < 3; ++j) {
        w.dilations[j] = s.dil[j];
        w.convs1[j] = oconv(s.convs1[j]), w.convs2[j] = oconv(s.convs2[j]);
        w.alpha1[j] = ov(s.alpha1[j]), w.alpha2[j] = ov(s.alpha2[j]);
        w.adain1[j].channels = w.adain2[j].channels = s.C;
    }
    return w;
}
kdo::ResBlock1Affines oaff(const cf::Rb1Spec& s) {
    kdo::ResBlock1Affines a;
    for (int j = 0; j < 3; ++j) a.g1[j] = ov(s.g1[j]), a.b1[j] = ov(s.b1[j]), a.g2[j] = ov(s.g2[j]), a.b2[j] = ov(s.b2[j]);
    return a;
}

struct OracleBackend {
    const float eps = 1e-5f;
    cf::ResblkOut resblk(const cf::ResblkSpec& s) {
        kdo::AdainResBlk1dWeights w = oresblk(s);
        kdo::AdainResBlkCache c;
        kdo::Vec y, dX, dG1, dB1, dG2, dB2;
        int Lo = 0;
        kdo::adain_resblk_1d_forward_train(w, ov(s.x), s.L, ov(s.g1), ov(s.b1), ov(s.g2), ov(s.b2), eps, Lo, y, c);
        kdo::adain_resblk_1d_backward(w, c, ov(s.g1), ov(s.g2), ov(s.dY), eps, dX, dG1, dB1, dG2, dB2, nullptr);
        return {hv(y), hv(dX), hv(dG1), hv(dB1), hv(dG2), hv(dB2)};
    }
    cf::Rb1Out resblock1(const cf::Rb1Spec& s) {
        kdo::AdaINResBlock1Weights w = orb1(s);
        const kdo::ResBlock1Affines a = oaff(s);
        kdo::AdainResBlock1Cache c;
        kdo::Vec y, dX;
        kdo::Arr3 dG1, dB1, dG2, dB2;
        kdo::adain_resblock1_forward_train(w, ov(s.x), s.C, s.L, a.g1, a.b1, a.g2, a.b2, y, c);
        kdo::adain_resblock1_backward(w, c, a.g1, a.g2, ov(s.dY), dX, dG1, dB1, dG2, dB2, nullptr);
        return {hv(y), hv(dX)};
    }
    void generator(const cf::GenSpec& g, HVec& stage1_in, HVec& head_in) {
        kdo::Generator gen;
        gen.n_fft = g.n_fft, gen.hop_size = g.hop, gen.win_size = g.win;
        gen.num_upsamples = g.U, gen.num_kernels = g.K;
        for (int i = 0; i < g.U; ++i) {
            gen.ups_W.push_back(ov(g.ups_W[i]));
            gen.ups_b.push_back(ov(g.ups_b[i]));
            gen.noise_convs.push_back(oconv(g.noise_convs[i]));
            gen.noise_res.push_back(orb1(g.noise_res[i]));
        }
        gen.ups_C_in = g.C_in, gen.ups_C_out = g.C_out, gen.ups_k = g.k, gen.ups_stride = g.s, gen.ups_pad = g.p;
        std::vector<kdo::ResBlock1Affines> naff, raff;
        for (const auto& r : g.noise_res) naff.push_back(oaff(r));
        for (const auto& r : g.resblocks) {
            gen.resblocks.push_back(orb1(r));
            raff.push_back(oaff(r));
        }
        gen.conv_post = oconv(g.conv_post);
        kdo::GeneratorCache c;
        kdo::Vec audio;
        kdo::generator_forward_train(gen, ov(g.gen_in), g.L0, ov(g.har), g.frames, naff, raff, audio, c);
        stage1_in = hv(c.stages[1].x_in);
        head_in = hv(c.head.x_pre);
    }
    HVec head(const cf::HeadSpec& h, const HVec& x, const HVec& W) {
        cf::ConvSpec cs = h.conv_post;
        cs.W = W;
        const kdo::Conv1d cp = oconv(cs);
        kdo::SpectralHeadCache c;
        kdo::Vec audio;
        kdo::spectral_head_forward_train(cp, ov(x), h.C, h.L, kdo::hann_periodic(h.win), h.n_fft, h.hop, h.win, audio,
                                         c);
        return hv(audio);
    }
    HVec backbone(const cf::BbSpec& b) {
        kdo::DecoderBackbone bb;
        bb.F0_conv = oconv(b.F0_conv), bb.N_conv = oconv(b.N_conv), bb.asr_res = oconv(b.asr_res);
        bb.encode = oresblk(b.encode);
        std::vector<kdo::BlockAffines> aff;
        aff.push_back({ov(b.encode.g1), ov(b.encode.b1), ov(b.encode.g2), ov(b.encode.b2)});
        for (const auto& d : b.decode) {
            bb.decode.push_back(oresblk(d));
            aff.push_back({ov(d.g1), ov(d.b1), ov(d.g2), ov(d.b2)});
        }
        kdo::BackboneCache c;
        kdo::Vec gen_in;
        kdo::decoder_backbone_forward_train(bb, ov(b.asr), ov(b.F0), ov(b.N), b.T, aff, eps, gen_in, c);
        return hv(gen_in);
    }
    HVec pad(const HVec& x, int C, int L) {
        kdo::Vec y(static_cast<std::size_t>(C) * (L + 1));
        kdo::pad_reflect_left1_forward(ov(x).data(), C, L, y.data());
        return hv(y);
    }
};

}  // namespace

int main() {
    OracleBackend be;
    cf::Report r;
    try {
        cf::run_closed_forms(be, r);
    } catch (const std::exception& e) {
        std::printf("  FAIL exception: %s\n", e.what());
        ++r.failures;
    }
    std::printf("test_closed_form (oracle): %d checks, %d failure(s)\n", r.checks, r.failures);
    return r.failures ? 1 : 0;
}

// Whole-decoder oracle with named parameters. TEST INFRASTRUCTURE ONLY.
//
// Mirrors the structure the reference builds in DecoderBackbone::load_from
// (kokoro_modules.cpp:1021-1063), load_adain_resblk (:747-767),
// load_adain_resblock1 (:1147-1195), Generator::load_from (:1237-1347) and
// HarmonicSource::load_from (:1556-1572); parameter names are the upstream
// state-dict keys those loaders read. The style projection
// (gamma, beta) = chunk(fc.W s + fc.b) follows compute_style_affine
// (kokoro_modules.cpp:563-572); its adjoint (the d(style) extension) follows
// the lora_backward contract with the LoRA term absent
// (decoder_lora.cpp:198-207).
#include "kdec_oracle.hpp"

#include <cmath>
#include <stdexcept>

namespace KDO_NS {

namespace {

void make_conv(Conv1d& c, int cin, int cout, int k, int s, int p, int d,
               bool bias) {
    c.in_channels = cin;
    c.out_channels = cout;
    c.kernel_size = k;
    c.stride = s;
    c.padding = p;
    c.dilation = d;
    c.groups = 1;
    c.W.assign(static_cast<std::size_t>(cout) * cin * k, 0.0f);
    c.dW.assign(c.W.size(), 0.0f);
    if (bias) {
        c.b.assign(static_cast<std::size_t>(cout), 0.0f);
        c.db.assign(c.b.size(), 0.0f);
    } else {
        c.b.clear();
        c.db.clear();
    }
}

void make_adain(AdaIN1dWeights& a, int C, int S) {
    a.channels = C;
    a.style_dim = S;
    a.eps = 1e-5f;
    a.fcW.assign(static_cast<std::size_t>(2 * C) * S, 0.0f);
    a.fcb.assign(static_cast<std::size_t>(2 * C), 0.0f);
    a.dfcW.assign(a.fcW.size(), 0.0f);
    a.dfcb.assign(a.fcb.size(), 0.0f);
}

// (gamma, beta) = chunk(W s + b)
void style_affine(const AdaIN1dWeights& a, const Vec& s, Vec& g, Vec& b) {
    const int C = a.channels, S = a.style_dim;
    g.assign(static_cast<std::size_t>(C), 0.0f);
    b.assign(static_cast<std::size_t>(C), 0.0f);
    for (int r = 0; r < 2 * C; ++r) {
        double acc = a.fcb[r];
        for (int j = 0; j < S; ++j) acc += static_cast<double>(a.fcW[static_cast<std::size_t>(r) * S + j]) * s[j];
        if (r < C) g[r] = static_cast<Real>(acc);
        else b[r - C] = static_cast<Real>(acc);
    }
}

// Adjoint of style_affine: accumulates dW, db and (optionally) d(style).
void style_affine_backward(AdaIN1dWeights& a, const Vec& s, const Vec& dg,
                           const Vec& db, double* dstyle, bool wgrad) {
    const int C = a.channels, S = a.style_dim;
    for (int r = 0; r < 2 * C; ++r) {
        const double dy = r < C ? dg[r] : db[r - C];
        if (wgrad) {
            for (int j = 0; j < S; ++j)
                a.dfcW[static_cast<std::size_t>(r) * S + j] =
                    static_cast<Real>(a.dfcW[static_cast<std::size_t>(r) * S + j] + dy * s[j]);
            a.dfcb[r] = static_cast<Real>(a.dfcb[r] + dy);
        }
        if (dstyle)
            for (int j = 0; j < S; ++j)
                dstyle[j] += static_cast<double>(a.fcW[static_cast<std::size_t>(r) * S + j]) * dy;
    }
}

}  // namespace

Model::Model(const Config& c) : cfg(c) { build(); }

void Model::register_param(const std::string& name, Vec* v, Vec* g, int rows,
                           int cols) {
    if (params.count(name)) throw std::runtime_error("kdo::Model: duplicate param " + name);
    if (static_cast<std::size_t>(rows) * cols != v->size())
        throw std::runtime_error("kdo::Model: shape mismatch for " + name);
    if (g->size() != v->size()) g->assign(v->size(), 0.0f);
    params[name] = ParamRef{v, g, rows, cols};
    order.push_back(name);
}

void Model::build() {
    const Config& c = cfg;
    const int S = c.style_dim;
    const std::string P = "decoder.module.";

    auto reg_conv = [&](const std::string& pfx, Conv1d& cv) {
        register_param(pfx + ".weight", &cv.W, &cv.dW, cv.out_channels,
                       cv.in_channels * cv.kernel_size);
        if (!cv.b.empty())
            register_param(pfx + ".bias", &cv.b, &cv.db, cv.out_channels, 1);
    };
    auto reg_adain = [&](const std::string& pfx, AdaIN1dWeights& a) {
        register_param(pfx + ".fc.weight", &a.fcW, &a.dfcW, 2 * a.channels, S);
        register_param(pfx + ".fc.bias", &a.fcb, &a.dfcb, 2 * a.channels, 1);
    };

    // ─── backbone ───
    make_conv(bb.F0_conv, 1, 1, 3, 2, 1, 1, true);
    make_conv(bb.N_conv, 1, 1, 3, 2, 1, 1, true);
    make_conv(bb.asr_res, c.asr_dim, c.asr_res_dim, 1, 1, 0, 1, true);
    reg_conv(P + "F0_conv", bb.F0_conv);
    reg_conv(P + "N_conv", bb.N_conv);
    reg_conv(P + "asr_res.0", bb.asr_res);

    auto make_resblk = [&](AdainResBlk1dWeights& w, int din, int dout, bool up,
                           const std::string& pfx) {
        w.channels_in = din;
        w.channels_out = dout;
        w.upsample = up;
        w.learned_sc = din != dout;
        make_adain(w.norm1, din, S);
        make_adain(w.norm2, dout, S);
        make_conv(w.conv1, din, dout, 3, 1, 1, 1, true);
        make_conv(w.conv2, dout, dout, 3, 1, 1, 1, true);
        reg_adain(pfx + ".norm1", w.norm1);
        reg_adain(pfx + ".norm2", w.norm2);
        reg_conv(pfx + ".conv1", w.conv1);
        reg_conv(pfx + ".conv2", w.conv2);
        if (w.learned_sc) {
            make_conv(w.conv1x1, din, dout, 1, 1, 0, 1, false);
            reg_conv(pfx + ".conv1x1", w.conv1x1);
        }
        if (up) {
            w.pool_W.assign(static_cast<std::size_t>(din) * 3, 0.0f);
            w.pool_b.assign(static_cast<std::size_t>(din), 0.0f);
            register_param(pfx + ".pool.weight", &w.pool_W, &w.dpool_W, din, 3);
            register_param(pfx + ".pool.bias", &w.pool_b, &w.dpool_b, din, 1);
        }
    };
    make_resblk(bb.encode, c.asr_dim + 2, c.enc_dim, false, P + "encode");
    bb.decode.assign(c.n_decode, AdainResBlk1dWeights{});
    int prev = c.enc_dim;
    bool res = true;
    for (int i = 0; i < c.n_decode; ++i) {
        const bool up = (i == c.dec_up_at);
        const int din = res ? prev + c.asr_res_dim + 2 : prev;
        make_resblk(bb.decode[i], din, c.dec_out[i], up,
                    P + "decode." + std::to_string(i));
        prev = c.dec_out[i];
        if (up) res = false;
    }

    // ─── generator ───
    const int init_C = c.dec_out[c.n_decode - 1];
    const std::string G = P + "generator.";
    gen.n_fft = c.n_fft;
    gen.hop_size = c.hop;
    gen.win_size = c.n_fft;
    gen.num_upsamples = c.n_ups;
    gen.num_kernels = c.n_kernels;
    gen.ups_W.assign(c.n_ups, Vec{});
    gen.ups_b.assign(c.n_ups, Vec{});
    gen.dups_W.assign(c.n_ups, Vec{});
    gen.dups_b.assign(c.n_ups, Vec{});
    gen.ups_C_in.assign(c.n_ups, 0);
    gen.ups_C_out.assign(c.n_ups, 0);
    gen.ups_k.assign(c.n_ups, 0);
    gen.ups_stride.assign(c.n_ups, 0);
    gen.ups_pad.assign(c.n_ups, 0);
    for (int i = 0; i < c.n_ups; ++i) {
        const int ci = init_C >> i, co = init_C >> (i + 1);
        gen.ups_C_in[i] = ci;
        gen.ups_C_out[i] = co;
        gen.ups_k[i] = c.ups_kernels[i];
        gen.ups_stride[i] = c.ups_rates[i];
        gen.ups_pad[i] = (c.ups_kernels[i] - c.ups_rates[i]) / 2;
        gen.ups_W[i].assign(static_cast<std::size_t>(ci) * co * c.ups_kernels[i], 0.0f);
        gen.ups_b[i].assign(static_cast<std::size_t>(co), 0.0f);
        register_param(G + "ups." + std::to_string(i) + ".weight", &gen.ups_W[i],
                       &gen.dups_W[i], ci, co * c.ups_kernels[i]);
        register_param(G + "ups." + std::to_string(i) + ".bias", &gen.ups_b[i],
                       &gen.dups_b[i], co, 1);
    }
    gen.noise_convs.assign(c.n_ups, Conv1d{});
    for (int i = 0; i < c.n_ups; ++i) {
        const int co = init_C >> (i + 1);
        if (i + 1 < c.n_ups) {
            int sf = 1;
            for (int j = i + 1; j < c.n_ups; ++j) sf *= c.ups_rates[j];
            make_conv(gen.noise_convs[i], c.n_fft + 2, co, 2 * sf, sf, (sf + 1) / 2, 1, true);
        } else {
            make_conv(gen.noise_convs[i], c.n_fft + 2, co, 1, 1, 0, 1, true);
        }
        reg_conv(G + "noise_convs." + std::to_string(i), gen.noise_convs[i]);
    }
    auto make_rb1 = [&](AdaINResBlock1Weights& w, int C, int k,
                        const int* dil, const std::string& pfx) {
        w.channels = C;
        w.kernel_size = k;
        for (int j = 0; j < 3; ++j) {
            w.dilations[j] = dil[j];
            make_conv(w.convs1[j], C, C, k, 1, (k * dil[j] - dil[j]) / 2, dil[j], true);
            make_conv(w.convs2[j], C, C, k, 1, (k - 1) / 2, 1, true);
            make_adain(w.adain1[j], C, S);
            make_adain(w.adain2[j], C, S);
            w.alpha1[j].assign(static_cast<std::size_t>(C), 1.0f);
            w.alpha2[j].assign(static_cast<std::size_t>(C), 1.0f);
            w.dalpha1[j].assign(static_cast<std::size_t>(C), 0.0f);
            w.dalpha2[j].assign(static_cast<std::size_t>(C), 0.0f);
            const std::string js = std::to_string(j);
            reg_conv(pfx + ".convs1." + js, w.convs1[j]);
            reg_conv(pfx + ".convs2." + js, w.convs2[j]);
            reg_adain(pfx + ".adain1." + js, w.adain1[j]);
            reg_adain(pfx + ".adain2." + js, w.adain2[j]);
            register_param(pfx + ".alpha1." + js, &w.alpha1[j], &w.dalpha1[j], C, 1);
            register_param(pfx + ".alpha2." + js, &w.alpha2[j], &w.dalpha2[j], C, 1);
        }
    };
    const int dil135[3] = {1, 3, 5};
    gen.noise_res.assign(c.n_ups, AdaINResBlock1Weights{});
    for (int i = 0; i < c.n_ups; ++i) {
        const int k = (i + 1 < c.n_ups) ? 7 : 11;
        make_rb1(gen.noise_res[i], init_C >> (i + 1), k, dil135,
                 G + "noise_res." + std::to_string(i));
    }
    gen.resblocks.assign(static_cast<std::size_t>(c.n_ups) * c.n_kernels, AdaINResBlock1Weights{});
    for (int i = 0; i < c.n_ups; ++i)
        for (int j = 0; j < c.n_kernels; ++j) {
            const int idx = i * c.n_kernels + j;
            make_rb1(gen.resblocks[idx], init_C >> (i + 1), c.rb_kernels[j],
                     c.rb_dil[j], G + "resblocks." + std::to_string(idx));
        }
    make_conv(gen.conv_post, init_C >> c.n_ups, c.n_fft + 2, c.conv_post_k, 1,
              (c.conv_post_k - 1) / 2, 1, true);
    reg_conv(G + "conv_post", gen.conv_post);

    // ─── harmonic source ───
    hs.sample_rate = c.sample_rate;
    hs.harmonic_num = c.harmonic_num;
    hs.n_fft = c.n_fft;
    hs.hop_size = c.hop;
    hs.win_size = c.n_fft;
    int upr = 1;
    for (int i = 0; i < c.n_ups; ++i) upr *= c.ups_rates[i];
    hs.upsample_scale = upr * c.hop;
    hs.lW.assign(static_cast<std::size_t>(c.harmonic_num + 1), 0.0f);
    hs.lb.assign(1, 0.0f);
    register_param(G + "m_source.l_linear.weight", &hs.lW, &hs.dlW, 1, c.harmonic_num + 1);
    register_param(G + "m_source.l_linear.bias", &hs.lb, &hs.dlb, 1, 1);

    // ─── AdaIN units (canonical order: backbone, noise_res, resblocks) ───
    bbaff.assign(1 + c.n_decode, BlockAffines{});
    dbbaff.assign(1 + c.n_decode, BlockAffines{});
    naff.assign(c.n_ups, ResBlock1Affines{});
    dnaff.assign(c.n_ups, ResBlock1Affines{});
    raff.assign(static_cast<std::size_t>(c.n_ups) * c.n_kernels, ResBlock1Affines{});
    draff.assign(raff.size(), ResBlock1Affines{});
    auto add_unit = [&](const std::string& nm, AdaIN1dWeights* w, Vec* g, Vec* b,
                        Vec* dg, Vec* db) {
        AffineUnit u;
        u.name = nm;
        u.w = w;
        u.gamma = g;
        u.beta = b;
        u.dgamma = dg;
        u.dbeta = db;
        units.push_back(std::move(u));
    };
    add_unit(P + "encode.norm1", &bb.encode.norm1, &bbaff[0].g1, &bbaff[0].b1, &dbbaff[0].g1, &dbbaff[0].b1);
    add_unit(P + "encode.norm2", &bb.encode.norm2, &bbaff[0].g2, &bbaff[0].b2, &dbbaff[0].g2, &dbbaff[0].b2);
    for (int i = 0; i < c.n_decode; ++i) {
        const std::string q = P + "decode." + std::to_string(i);
        add_unit(q + ".norm1", &bb.decode[i].norm1, &bbaff[1 + i].g1, &bbaff[1 + i].b1, &dbbaff[1 + i].g1, &dbbaff[1 + i].b1);
        add_unit(q + ".norm2", &bb.decode[i].norm2, &bbaff[1 + i].g2, &bbaff[1 + i].b2, &dbbaff[1 + i].g2, &dbbaff[1 + i].b2);
    }
    auto add_rb1_units = [&](const std::string& q, AdaINResBlock1Weights& w,
                             ResBlock1Affines& a, ResBlock1Affines& d) {
        for (int j = 0; j < 3; ++j)
            add_unit(q + ".adain1." + std::to_string(j), &w.adain1[j], &a.g1[j], &a.b1[j], &d.g1[j], &d.b1[j]);
        for (int j = 0; j < 3; ++j)
            add_unit(q + ".adain2." + std::to_string(j), &w.adain2[j], &a.g2[j], &a.b2[j], &d.g2[j], &d.b2[j]);
    };
    for (int i = 0; i < c.n_ups; ++i)
        add_rb1_units(G + "noise_res." + std::to_string(i), gen.noise_res[i], naff[i], dnaff[i]);
    for (std::size_t i = 0; i < gen.resblocks.size(); ++i)
        add_rb1_units(G + "resblocks." + std::to_string(i), gen.resblocks[i], raff[i], draff[i]);
}

void Model::zero_grad() {
    for (auto& kv : params) std::fill(kv.second.grad->begin(), kv.second.grad->end(), 0.0f);
    for (auto& u : units) {
        std::fill(u.dA.begin(), u.dA.end(), 0.0f);
        std::fill(u.dB.begin(), u.dB.end(), 0.0f);
    }
    std::fill(dgate.begin(), dgate.end(), 0.0f);
}

// Adapters start at A = 0, B = 0 (the base decoder) with a zero gate.
void Model::lora_enable(int rank, float scale) {
    if (rank <= 0) throw std::runtime_error("kdo::Model::lora_enable: rank must be positive");
    lora_rank = rank;
    lora_scale = scale;
    const std::size_t S = static_cast<std::size_t>(cfg.style_dim);
    for (auto& u : units) {
        const std::size_t rows = 2 * static_cast<std::size_t>(u.w->channels);
        u.A.assign(rank * S, 0.0f);
        u.B.assign(rows * rank, 0.0f);
        u.dA.assign(u.A.size(), 0.0f);
        u.dB.assign(u.B.size(), 0.0f);
        u.h.assign(static_cast<std::size_t>(rank), 0.0f);
    }
    gate.assign(static_cast<std::size_t>(rank), 0.0f);
    dgate.assign(static_cast<std::size_t>(rank), 0.0f);
}

namespace {
// Installs a model's leaky-site masks for the duration of a pass.
struct KinkScope {
    explicit KinkScope(Model& m) {
        if (m.kinks.masks.empty()) return;
        g_kinks = &m.kinks;
        g_kink_gen = 2 * (1 + m.cfg.n_decode);
    }
    ~KinkScope() {
        g_kinks = nullptr;
        g_kink_gen = -1;
    }
};
}  // namespace

void Model::forward(const Vec& asr, const Vec& F0, const Vec& N,
                    const Vec& style_in, int T_in, const Vec* har_in) {
    KinkScope ks(*this);
    kinks.flips.assign(kinks.masks.size(), 0);
    T = T_in;
    style = style_in;
    for (auto& u : units) {
        if (lora_rank > 0) {
            // adapter_fwd (decoder_lora.cpp:184-194): (gamma, beta) = chunk(lora_forward(...))
            const int C = u.w->channels;
            Vec y(static_cast<std::size_t>(2 * C));
            lora_forward(u.w->fcW.data(), u.w->fcb.data(), u.A.data(), u.B.data(), gate.data(), lora_scale,
                         style.data(), 2 * C, lora_rank, cfg.style_dim, y.data(), u.h.data());
            u.gamma->assign(y.begin(), y.begin() + C);
            u.beta->assign(y.begin() + C, y.end());
        } else {
            style_affine(*u.w, style, *u.gamma, *u.beta);
        }
    }
    // Harmonic source from F0 (decode_back_half, kokoro.cpp:369-383).
    int sig = 0;
    harmonic_source_forward(hs, F0, 2 * T, sig, frames, har);
    if (har_in) {
        if (har_in->size() != har.size())
            throw std::runtime_error("kdo::Model::forward: har size mismatch");
        har = *har_in;
    }
    decoder_backbone_forward_train(bb, asr, F0, N, T, bbaff, 1e-5f, gen_in, bbc);
    const int L_gen = static_cast<int>(gen_in.size()) / cfg.dec_out[cfg.n_decode - 1];
    generator_forward_train(gen, gen_in, L_gen, har, frames, naff, raff, audio, genc);
}

void Model::backward(const Vec& dAudio, const Ext& ext, bool want_dstyle) {
    KinkScope ks(*this);
    Vec dGenIn;
    std::vector<ResBlock1Affines> dn, dr;
    generator_backward(gen, genc, naff, raff, dAudio, dGenIn, dn, dr, &ext);
    for (std::size_t i = 0; i < dn.size(); ++i) dnaff[i] = dn[i];
    for (std::size_t i = 0; i < dr.size(); ++i) draff[i] = dr[i];
    std::vector<BlockAffines> db;
    decoder_backbone_backward(bb, bbc, bbaff, dGenIn, 1e-5f, db, &ext);
    for (std::size_t i = 0; i < db.size(); ++i) dbbaff[i] = db[i];
    std::vector<double> ds(static_cast<std::size_t>(cfg.style_dim), 0.0);
    if (lora_rank > 0) {
        // adapter_bwd (decoder_lora.cpp:198-207) per unit, the gate grad
        // accumulated over all units, plus d(style) and the frozen fc grads
        Vec dsv(static_cast<std::size_t>(cfg.style_dim), 0.0f);
        for (auto& u : units) {
            const int C = u.w->channels;
            Vec dy(u.dgamma->begin(), u.dgamma->end());
            dy.insert(dy.end(), u.dbeta->begin(), u.dbeta->end());
            lora_backward(u.w->fcW.data(), u.A.data(), u.B.data(), gate.data(), lora_scale, style.data(),
                          u.h.data(), dy.data(), 2 * C, lora_rank, cfg.style_dim,
                          want_dstyle ? dsv.data() : nullptr, ext.wgrad ? u.w->dfcW.data() : nullptr,
                          ext.wgrad ? u.w->dfcb.data() : nullptr, u.dA.data(), u.dB.data(), dgate.data());
        }
        for (std::size_t j = 0; j < ds.size(); ++j) ds[j] = dsv[j];
    } else {
        for (auto& u : units)
            style_affine_backward(*u.w, style, *u.dgamma, *u.dbeta,
                                  want_dstyle ? ds.data() : nullptr, ext.wgrad);
    }
    dstyle.assign(ds.size(), 0.0f);
    for (std::size_t j = 0; j < ds.size(); ++j) dstyle[j] = static_cast<Real>(ds[j]);
}

}  // namespace KDO_NS

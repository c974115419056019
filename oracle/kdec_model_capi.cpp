// ctypes-facing C ABI over the oracle's whole-decoder model. TEST
// INFRASTRUCTURE ONLY. Compiled twice: as ko_model_* over the float oracle and,
// with -DKDO_REAL=double -DKDO_NS=kdo64 -DKO_PREFIX=ko64_, as ko64_model_*
// over the FP64 shadow. Inputs and outputs cross the ABI as float.
#include "kdec_oracle.hpp"

#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>

#ifndef KO_PREFIX
#define KO_PREFIX ko_
#endif
#define KO_CAT2(a, b) a##b
#define KO_CAT(a, b) KO_CAT2(a, b)
#define KO_FN(name) KO_CAT(KO_PREFIX, name)

using namespace KDO_NS;

namespace {
thread_local std::string g_err;

template <class F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

Vec vec(const float* p, std::size_t n) { return Vec(p, p + n); }
// The oracle's own input at leaky site `site` after a forward.
const Vec& leaky_site_input(Model& m, int site) {
    const int nb = 1 + m.cfg.n_decode;
    if (site >= 0 && site < 2 * nb) {
        const AdainResBlkCache& c = site / 2 == 0 ? m.bbc.encode : m.bbc.decode[static_cast<std::size_t>(site / 2 - 1)];
        return site % 2 ? c.n2_pre : c.r_pre;
    }
    if (site >= 2 * nb && site < 2 * nb + m.cfg.n_ups) return m.genc.stages[static_cast<std::size_t>(site - 2 * nb)].x_in;
    if (site == 2 * nb + m.cfg.n_ups) return m.genc.head.x_pre;
    throw std::runtime_error("ko_model_leaky_input: site out of range");
}
void out(float* dst, const Vec& v) {
    for (std::size_t i = 0; i < v.size(); ++i) dst[i] = static_cast<float>(v[i]);
}
}  // namespace

extern "C" {

const char* KO_FN(model_last_error)() { return g_err.c_str(); }

// ─── model ───
// cfg: flat ints in this order:
//   asr_dim, asr_res_dim, style_dim, enc_dim, n_decode, dec_out[8], dec_up_at,
//   n_ups, ups_rates[4], ups_kernels[4], n_kernels, rb_kernels[4],
//   rb_dil[4][3], n_fft, hop, conv_post_k, sample_rate, harmonic_num
void* KO_FN(model_create)(const int* v, int n) {
    try {
        Config c;
        int i = 0;
        auto nx = [&]() {
            if (i >= n) throw std::runtime_error("ko_model_create: short config");
            return v[i++];
        };
        c.asr_dim = nx(); c.asr_res_dim = nx(); c.style_dim = nx(); c.enc_dim = nx();
        c.n_decode = nx();
        for (int j = 0; j < 8; ++j) c.dec_out[j] = nx();
        c.dec_up_at = nx();
        c.n_ups = nx();
        for (int j = 0; j < 4; ++j) c.ups_rates[j] = nx();
        for (int j = 0; j < 4; ++j) c.ups_kernels[j] = nx();
        c.n_kernels = nx();
        for (int j = 0; j < 4; ++j) c.rb_kernels[j] = nx();
        for (int j = 0; j < 4; ++j)
            for (int q = 0; q < 3; ++q) c.rb_dil[j][q] = nx();
        c.n_fft = nx(); c.hop = nx(); c.conv_post_k = nx();
        c.sample_rate = nx(); c.harmonic_num = nx();
        return new Model(c);
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}
void KO_FN(model_destroy)(void* m) { delete static_cast<Model*>(m); }
int KO_FN(model_param_count)(void* m) { return static_cast<int>(static_cast<Model*>(m)->order.size()); }
const char* KO_FN(model_param_name)(void* m, int i) { return static_cast<Model*>(m)->order.at(i).c_str(); }
int KO_FN(model_param_shape)(void* m, const char* name, int* rows, int* cols) {
    return guard([&] {
        const ParamRef& p = static_cast<Model*>(m)->params.at(name);
        *rows = p.rows;
        *cols = p.cols;
    });
}
int KO_FN(model_set_param)(void* m, const char* name, const float* data, long n) {
    return guard([&] {
        ParamRef& p = static_cast<Model*>(m)->params.at(name);
        if (static_cast<std::size_t>(n) != p.value->size()) throw std::runtime_error(std::string("size mismatch: ") + name);
        for (long i = 0; i < n; ++i) (*p.value)[i] = static_cast<Real>(data[i]);
    });
}
// Double-precision setter: lets finite-difference checks on the FP64 shadow
// perturb parameters below float resolution.
int KO_FN(model_set_param_f64)(void* m, const char* name, const double* data, long n) {
    return guard([&] {
        ParamRef& p = static_cast<Model*>(m)->params.at(name);
        if (static_cast<std::size_t>(n) != p.value->size()) throw std::runtime_error(std::string("size mismatch: ") + name);
        for (long i = 0; i < n; ++i) (*p.value)[i] = static_cast<Real>(data[i]);
    });
}
int KO_FN(model_get_grad)(void* m, const char* name, float* dst, long n) {
    return guard([&] {
        ParamRef& p = static_cast<Model*>(m)->params.at(name);
        if (static_cast<std::size_t>(n) != p.grad->size()) throw std::runtime_error(std::string("size mismatch: ") + name);
        out(dst, *p.grad);
    });
}
int KO_FN(model_unit_count)(void* m) { return static_cast<int>(static_cast<Model*>(m)->units.size()); }
const char* KO_FN(model_unit_name)(void* m, int i) { return static_cast<Model*>(m)->units.at(i).name.c_str(); }
int KO_FN(model_unit_channels)(void* m, int i) { return static_cast<Model*>(m)->units.at(i).w->channels; }
int KO_FN(model_get_affine)(void* m, int i, float* gamma, float* beta, float* dgamma, float* dbeta) {
    return guard([&] {
        const AffineUnit& u = static_cast<Model*>(m)->units.at(i);
        const std::size_t C = static_cast<std::size_t>(u.w->channels);
        (void)C;
        if (gamma) out(gamma, *u.gamma);
        if (beta) out(beta, *u.beta);
        if (dgamma) out(dgamma, *u.dgamma);
        if (dbeta) out(dbeta, *u.dbeta);
    });
}
// ─── LoRA adapters (decoder_lora.h:63-77) ───
int KO_FN(model_lora_enable)(void* m, int rank, float scale) {
    return guard([&] { static_cast<Model*>(m)->lora_enable(rank, scale); });
}
// unit i's A (rank*style_dim) and B (2C*rank) as doubles (stored at the
// oracle's precision, so the FP64 shadow takes finite-difference steps);
// either may be NULL
int KO_FN(model_lora_set)(void* mp, int i, const double* A, const double* B) {
    return guard([&] {
        AffineUnit& u = static_cast<Model*>(mp)->units.at(i);
        if (A) u.A.assign(A, A + u.A.size());
        if (B) u.B.assign(B, B + u.B.size());
    });
}
int KO_FN(model_lora_get_grad)(void* mp, int i, float* dA, float* dB) {
    return guard([&] {
        const AffineUnit& u = static_cast<Model*>(mp)->units.at(i);
        if (dA) out(dA, u.dA);
        if (dB) out(dB, u.dB);
    });
}
int KO_FN(model_lora_gate)(void* mp, const double* g) {
    return guard([&] {
        Model& m = *static_cast<Model*>(mp);
        m.gate.assign(g, g + m.gate.size());
    });
}
int KO_FN(model_lora_get_dgate)(void* mp, float* dG) {
    return guard([&] { out(dG, static_cast<Model*>(mp)->dgate); });
}

int KO_FN(model_zero_grad)(void* m) { return guard([&] { static_cast<Model*>(m)->zero_grad(); }); }
// asr (asr_dim*T), F0/N (2T), style (style_dim); har_in optional (frames*(n_fft+2)).
int KO_FN(model_forward)(void* mp, const float* asr, const float* F0, const float* N,
                     const float* style, int T, const float* har_in) {
    return guard([&] {
        Model& m = *static_cast<Model*>(mp);
        const Vec a = vec(asr, static_cast<std::size_t>(m.cfg.asr_dim) * T);
        const Vec f = vec(F0, static_cast<std::size_t>(2 * T));
        const Vec nn = vec(N, static_cast<std::size_t>(2 * T));
        const Vec s = vec(style, static_cast<std::size_t>(m.cfg.style_dim));
        if (har_in) {
            int upr = 1;
            for (int i = 0; i < m.cfg.n_ups; ++i) upr *= m.cfg.ups_rates[i];
            const std::size_t frames = static_cast<std::size_t>(2 * T) * upr + 1;
            const Vec h = vec(har_in, frames * (m.cfg.n_fft + 2));
            m.forward(a, f, nn, s, T, &h);
        } else {
            m.forward(a, f, nn, s, T, nullptr);
        }
    });
}
// As model_forward, with the style vector in double precision.
int KO_FN(model_forward_style_f64)(void* mp, const float* asr, const float* F0,
                                   const float* N, const double* style, int T,
                                   const float* har_in) {
    return guard([&] {
        Model& m = *static_cast<Model*>(mp);
        Vec s(static_cast<std::size_t>(m.cfg.style_dim));
        for (std::size_t j = 0; j < s.size(); ++j) s[j] = static_cast<Real>(style[j]);
        int upr = 1;
        for (int i = 0; i < m.cfg.n_ups; ++i) upr *= m.cfg.ups_rates[i];
        const std::size_t frames = static_cast<std::size_t>(2 * T) * upr + 1;
        const Vec h = har_in ? vec(har_in, frames * (m.cfg.n_fft + 2)) : Vec{};
        m.forward(vec(asr, static_cast<std::size_t>(m.cfg.asr_dim) * T),
                  vec(F0, static_cast<std::size_t>(2 * T)),
                  vec(N, static_cast<std::size_t>(2 * T)), s, T,
                  har_in ? &h : nullptr);
    });
}
// Audio in double precision (length model_audio_len).
int KO_FN(model_get_audio_f64)(void* m, double* dst) {
    const Vec& a = static_cast<Model*>(m)->audio;
    for (std::size_t i = 0; i < a.size(); ++i) dst[i] = static_cast<double>(a[i]);
    return 0;
}
long KO_FN(model_audio_len)(void* m) { return static_cast<long>(static_cast<Model*>(m)->audio.size()); }
// Leaky-site masks (KinkMasks): site count; set site `site` from the signs
// of `pre` (n values; the site's input as another implementation computed
// it); clear all; elements whose own sign the last forward overrode at
// `site` (-1: all sites).
int KO_FN(model_kink_site_count)(void* m) { return static_cast<Model*>(m)->kink_site_count(); }
int KO_FN(model_set_kink)(void* mp, int site, const float* pre, long n) {
    return guard([&] {
        Model& m = *static_cast<Model*>(mp);
        if (site < 0 || site >= m.kink_site_count()) throw std::runtime_error("ko_model_set_kink: site out of range");
        m.kinks.masks.resize(static_cast<std::size_t>(m.kink_site_count()));
        auto& mk = m.kinks.masks[static_cast<std::size_t>(site)];
        mk.resize(static_cast<std::size_t>(n));
        for (long i = 0; i < n; ++i) mk[static_cast<std::size_t>(i)] = pre[i] > 0.0f ? 1 : 0;
    });
}
int KO_FN(model_clear_kinks)(void* m) {
    static_cast<Model*>(m)->kinks = KinkMasks{};
    return 0;
}
long KO_FN(model_kink_flips)(void* mp, int site) {
    const Model& m = *static_cast<Model*>(mp);
    long total = 0;
    for (std::size_t s = 0; s < m.kinks.flips.size(); ++s)
        if (site < 0 || static_cast<int>(s) == site) total += m.kinks.flips[s];
    return total;
}


long KO_FN(model_leaky_size)(void* mp, int site) {
    try {
        return static_cast<long>(leaky_site_input(*static_cast<Model*>(mp), site).size());
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// The oracle's own input at leaky site `site` after a forward (n values).
int KO_FN(model_leaky_input)(void* mp, int site, float* dst, long n) {
    return guard([&] {
        Model& m = *static_cast<Model*>(mp);
        const Vec* v = &leaky_site_input(m, site);
        if (static_cast<long>(v->size()) != n)
            throw std::runtime_error("ko_model_leaky_input: site holds " + std::to_string(v->size()) + " values");
        out(dst, *v);
    });
}

long KO_FN(model_har_len)(void* m) { return static_cast<long>(static_cast<Model*>(m)->har.size()); }
long KO_FN(model_gen_in_len)(void* m) { return static_cast<long>(static_cast<Model*>(m)->gen_in.size()); }
int KO_FN(model_get_audio)(void* m, float* dst) {
    const Vec& a = static_cast<Model*>(m)->audio;
    out(dst, a);
    return 0;
}
int KO_FN(model_get_har)(void* m, float* dst) {
    const Vec& a = static_cast<Model*>(m)->har;
    out(dst, a);
    return 0;
}
int KO_FN(model_get_gen_in)(void* m, float* dst) {
    const Vec& a = static_cast<Model*>(m)->gen_in;
    out(dst, a);
    return 0;
}
int KO_FN(model_backward)(void* mp, const float* dAudio, int wgrad, int dalpha,
                      float* dstyle) {
    return guard([&] {
        Model& m = *static_cast<Model*>(mp);
        Ext ext;
        ext.wgrad = wgrad != 0;
        ext.dalpha = dalpha != 0;
        m.backward(vec(dAudio, m.audio.size()), ext, dstyle != nullptr);
        if (dstyle) out(dstyle, m.dstyle);
    });
}

}  // extern "C"

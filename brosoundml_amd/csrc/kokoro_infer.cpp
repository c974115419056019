// Inference forwards of the decoder back half over the gfx950 atoms: the
// reference's DecoderBackbone::forward (kokoro_modules.cpp:1087-1141) and
// Generator::forward (1400-1552), which Kokoro's decode_back_half chains
// (kokoro.cpp:352-407). Every AdaIN unit's (gamma, beta) = fc(style)
// (compute_style_affine, kokoro_modules.cpp:563-572) comes from one
// style-projection launch per unit into a packed buffer the atoms read as
// views; the `_train` assemblies then run with caches that drop each block's
// tensors as soon as it is done, so nothing is kept for a backward.
#include "brosoundml/kokoro_modules.h"
#include "kdec.h"
#include "kokoro_decoder_backward.h"

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace bt = brotensor;
namespace bd = brosoundml::detail;

namespace brosoundml {
namespace {

using bt::Device;
using bt::Tensor;

[[noreturn]] void fail(const std::string& where, const std::string& why) {
    throw std::runtime_error("brosoundml: " + where + ": " + why);
}

// (gamma, beta) of a list of AdaIN units for N style rows, packed (N, sum 2C)
struct Affines {
    Tensor buf;
    std::vector<std::pair<Tensor, Tensor>> gb;
};

Affines project(const std::vector<const AdaIN1dWeights*>& units, const Tensor& ref_s, const char* where) {
    if (ref_s.device != Device::HIP) fail(where, "style must be on the HIP device");
    int R = 0;
    for (const auto* u : units) R += 2 * u->channels;
    const int N = ref_s.rows;
    const int S = units.empty() ? 0 : units[0]->fc.in_features;
    if (ref_s.cols < S) fail(where, "style rows shorter than style_dim");
    Affines a;
    a.buf = Tensor::empty_on(Device::HIP, N, R);
    int off = 0;
    for (const auto* u : units) {
        const int C = u->channels;
        if (u->fc.W.rows != 2 * C || u->fc.W.cols != S || u->fc.W.device != Device::HIP)
            fail(where, "AdaIN fc must be (2C, style_dim) on the HIP device");
        if (kdec_style_proj_fwd(bt::runtime(), u->fc.W.f32(), u->fc.b.data ? u->fc.b.f32() : nullptr, ref_s.f32(),
                                ref_s.row_stride(), a.buf.f32() + off, R, N, 2 * C, S) != KDEC_OK)
            fail(where, kdec_last_error(bt::runtime()));
        Tensor g = Tensor::view(Device::HIP, a.buf.f32() + off, N, C, bt::Dtype::FP32, R);
        Tensor b = Tensor::view(Device::HIP, a.buf.f32() + off + C, N, C, bt::Dtype::FP32, R);
        g.storage = b.storage = a.buf.storage;
        a.gb.emplace_back(g, b);
        off += 2 * C;
    }
    return a;
}

}  // namespace

void DecoderBackbone::forward(const Tensor& asr, const Tensor& F0_pred, const Tensor& N_pred, const Tensor& ref_s,
                              int T, Tensor& gen_in) const {
    std::vector<const AdaIN1dWeights*> units;
    units.push_back(&encode.norm1);
    units.push_back(&encode.norm2);
    for (const auto& d : decode) {
        units.push_back(&d.norm1);
        units.push_back(&d.norm2);
    }
    Affines a = project(units, ref_s, "DecoderBackbone::forward");
    std::vector<bd::BlockAffines> aff(1 + decode.size());
    for (std::size_t i = 0; i < aff.size(); ++i) {
        aff[i].g1 = a.gb[2 * i].first;
        aff[i].b1 = a.gb[2 * i].second;
        aff[i].g2 = a.gb[2 * i + 1].first;
        aff[i].b2 = a.gb[2 * i + 1].second;
    }
    bd::BackboneCache cache;
    cache.keep = false;
    bd::decoder_backbone_forward_train(*this, asr, F0_pred, N_pred, T, aff, 1e-5f, gen_in, cache);
}

void Generator::forward(const Tensor& gen_in, int L_in, const Tensor& har, int frames, const Tensor& style,
                        Tensor& audio, const std::function<bool()>& cancel) const {
    if (cancel && cancel()) {
        audio = Tensor{};
        return;
    }
    std::vector<const AdaIN1dWeights*> units;
    auto rb = [&](const AdaINResBlock1Weights& w) {
        for (int j = 0; j < 3; ++j) units.push_back(&w.adain1[j]);
        for (int j = 0; j < 3; ++j) units.push_back(&w.adain2[j]);
    };
    for (const auto& w : noise_res) rb(w);
    for (const auto& w : resblocks) rb(w);
    Affines a = project(units, style, "Generator::forward");
    auto fill = [&](std::size_t base, bd::ResBlock1Affines& r) {
        for (int j = 0; j < 3; ++j) {
            r.g1[j] = a.gb[base + j].first;
            r.b1[j] = a.gb[base + j].second;
            r.g2[j] = a.gb[base + 3 + j].first;
            r.b2[j] = a.gb[base + 3 + j].second;
        }
    };
    std::vector<bd::ResBlock1Affines> na(noise_res.size()), ra(resblocks.size());
    for (std::size_t i = 0; i < na.size(); ++i) fill(6 * i, na[i]);
    for (std::size_t i = 0; i < ra.size(); ++i) fill(6 * (na.size() + i), ra[i]);
    if (cancel && cancel()) {
        audio = Tensor{};
        return;
    }
    bd::GeneratorCache cache;
    cache.keep = false;
    bd::generator_forward_train(*this, gen_in, L_in, har, frames, na, ra, audio, cache);
}

}  // namespace brosoundml

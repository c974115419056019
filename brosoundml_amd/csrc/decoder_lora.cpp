// DecoderLora over the gfx950 drop-in atoms: the forward / backward sequence
// of decoder_lora.cpp:211-296 (gate, adapter projections, cached backbone
// and generator `_train` passes, their backwards, the adapters' adjoint and
// the gate's), Adam (:298-314) and the ELRA1 checkpoint (:316-396).
//
// All units' adapters live in stacked device buffers, so the 58 adapter
// projections are one kdec_lora_proj_fwd launch and their adjoints one
// kdec_lora_proj_bwd launch (the reference runs 58 small lora_forward /
// lora_backward calls plus copies); the affine (gamma, beta) of every unit
// are views of one buffer that the atoms read, and their grads land in place
// in another.
#include "brosoundml/decoder_lora.h"

#include "brosoundml/kokoro_modules.h"
#include "kdec.h"
#include "kokoro_decoder_backward.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <utility>

namespace bt = brotensor;
namespace bd = brosoundml::detail;

namespace brosoundml {
namespace {

using bt::Device;
using bt::Tensor;

[[noreturn]] void fail(const std::string& where, const std::string& why) {
    throw std::runtime_error("brosoundml: " + where + ": " + why);
}

void check(int rc, const char* where) {
    if (rc != KDEC_OK) fail(where, kdec_last_error(bt::runtime()));
}

hipStream_t stream() { return static_cast<hipStream_t>(kdec_get_stream(bt::runtime())); }

void d2d(void* dst, const void* src, std::size_t bytes, const char* where) {
    if (bytes && hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream()) != hipSuccess)
        fail(where, "device copy failed");
}

void h2d(void* dst, const void* src, std::size_t bytes, const char* where) {
    if (bytes && hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()) != hipSuccess)
        fail(where, "upload failed");
    if (hipStreamSynchronize(stream()) != hipSuccess) fail(where, "upload failed");
}

void zero(Tensor& t, const char* where) { check(kdec_fill(bt::runtime(), t.f32(), static_cast<long>(t.size()), 0.0f), where); }

// SplitMix64 and a Glorot-uniform fill in +-sqrt(6 / (rows + cols)).
struct SplitMix {
    std::uint64_t s;
    std::uint64_t next() {
        std::uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return static_cast<double>(next() >> 11) * (1.0 / 9007199254740992.0); }
};

void glorot(float* dst, int rows, int cols, SplitMix& r) {
    const double a = std::sqrt(6.0 / (rows + cols));
    for (long i = 0; i < static_cast<long>(rows) * cols; ++i) dst[i] = static_cast<float>((2.0 * r.uniform() - 1.0) * a);
}

Tensor rows_of(const Tensor& t, int r0, int nr) {
    Tensor v = Tensor::view(Device::HIP, t.f32() + static_cast<long>(r0) * t.cols, nr, t.cols);
    v.storage = t.storage;
    return v;
}

// (N, C) view of columns [c0, c0 + C) of a (N, ld) buffer
Tensor cols_of(const Tensor& t, int c0, int C) {
    Tensor v = Tensor::view(Device::HIP, t.f32() + c0, t.rows, C, bt::Dtype::FP32, t.cols);
    v.storage = t.storage;
    return v;
}

void need_hip(Device dev, const char* where) {
    if (dev != Device::HIP) fail(where, "the gfx950 build runs on the HIP device only");
}

int cond_rows(const Tensor& v, int in_dim, const char* where) {
    if (v.device != Device::HIP) fail(where, "condition must be on the HIP device");
    if (!v.contiguous() || v.size() == 0 || v.size() % in_dim) fail(where, "condition must hold N x in_dim values");
    return static_cast<int>(v.size() / in_dim);
}

// ELRA1 tensors: int32 rows, int32 cols, rows*cols floats (little-endian)
void write_tensor(std::FILE* f, int rows, int cols, const float* h) {
    const std::int32_t r = rows, c = cols;
    std::fwrite(&r, sizeof(r), 1, f);
    std::fwrite(&c, sizeof(c), 1, f);
    std::fwrite(h, sizeof(float), static_cast<std::size_t>(rows) * cols, f);
}

std::vector<float> read_tensor(std::FILE* f, int rows, int cols, const std::string& path) {
    std::int32_t r = 0, c = 0;
    if (std::fread(&r, sizeof(r), 1, f) != 1 || std::fread(&c, sizeof(c), 1, f) != 1)
        throw std::runtime_error("DecoderLora::load: truncated tensor header");
    if (r != rows || c != cols)
        throw std::runtime_error("DecoderLora::load: architecture mismatch in " + path);
    std::vector<float> h(static_cast<std::size_t>(r) * c);
    if (std::fread(h.data(), sizeof(float), h.size(), f) != h.size())
        throw std::runtime_error("DecoderLora::load: truncated tensor data");
    return h;
}

constexpr char kMagic[8] = {'E', 'L', 'R', 'A', '1', 0, 0, 0};
constexpr int kGateHidden = 16;

}  // namespace

// ─── ConditioningGate ───────────────────────────────────────────────────────

ConditioningGate ConditioningGate::make(int gate_dim, int hidden, Device dev, std::uint64_t seed) {
    need_hip(dev, "ConditioningGate::make");
    if (gate_dim <= 0 || hidden <= 0) fail("ConditioningGate::make", "bad sizes");
    ConditioningGate g;
    g.gate_dim = gate_dim;
    g.hidden = hidden;
    g.in_dim = 3;
    SplitMix r{seed ? seed : 0x9E3779B97F4A7C15ull};
    std::vector<float> w1(static_cast<std::size_t>(hidden) * g.in_dim);
    glorot(w1.data(), hidden, g.in_dim, r);
    g.W1 = Tensor::from_host_on(Device::HIP, w1.data(), hidden, g.in_dim);
    g.W2 = Tensor::zeros_on(Device::HIP, gate_dim, hidden);
    return g;
}

void ConditioningGate::zero_grad() {
    if (dW1.size() != static_cast<std::size_t>(hidden) * in_dim) dW1 = Tensor::empty_on(Device::HIP, hidden, in_dim);
    if (dW2.size() != static_cast<std::size_t>(gate_dim) * hidden) dW2 = Tensor::empty_on(Device::HIP, gate_dim, hidden);
    zero(dW1, "ConditioningGate::zero_grad");
    zero(dW2, "ConditioningGate::zero_grad");
}

void ConditioningGate::forward(const Tensor& v, Tensor& g) {
    const int N = cond_rows(v, in_dim, "ConditioningGate::forward");
    act_ = Tensor::empty_on(Device::HIP, N, hidden);
    g = N == 1 ? Tensor::empty_on(Device::HIP, gate_dim, 1) : Tensor::empty_on(Device::HIP, N, gate_dim);
    check(kdec_lora_gate_fwd(bt::runtime(), W1.f32(), W2.f32(), v.f32(), in_dim, N, in_dim, hidden, gate_dim,
                             act_.f32(), g.f32(), gate_dim),
          "ConditioningGate::forward");
}

void ConditioningGate::backward(const Tensor& v, const Tensor& dG) {
    const int N = cond_rows(v, in_dim, "ConditioningGate::backward");
    if (act_.rows != N) fail("ConditioningGate::backward", "no matching forward");
    if (dG.size() != static_cast<std::size_t>(N) * gate_dim || !dG.contiguous())
        fail("ConditioningGate::backward", "dG must hold N x gate_dim values");
    if (dW1.size() == 0 || dW2.size() == 0) zero_grad();
    check(kdec_lora_gate_bwd(bt::runtime(), W2.f32(), v.f32(), in_dim, act_.f32(), dG.f32(), gate_dim, N, in_dim,
                             hidden, gate_dim, dW1.f32(), dW2.f32()),
          "ConditioningGate::backward");
}

// ─── DecoderLora ────────────────────────────────────────────────────────────

DecoderLora DecoderLora::make(const DecoderBackbone& bb, const Generator& gen, int rank, float scale, Device dev,
                              std::uint64_t seed) {
    need_hip(dev, "DecoderLora::make");
    if (rank <= 0) fail("DecoderLora::make", "rank must be positive");
    DecoderLora m;
    m.rank_ = rank;
    m.scale_ = scale;
    m.dev_ = dev;
    m.style_dim_ = bb.encode.norm1.fc.in_features;
    const int S = m.style_dim_;
    if (S <= 0) fail("DecoderLora::make", "backbone weights not set");

    // the adapters in the reference's canonical order (decoder_lora.cpp:112-135)
    std::vector<std::pair<const Linear*, int>> units;
    auto block = [&](const AdainResBlk1dWeights& b) {
        units.emplace_back(&b.norm1.fc, b.channels_in);
        units.emplace_back(&b.norm2.fc, b.channels_out);
    };
    block(bb.encode);
    for (const auto& d : bb.decode) block(d);
    auto rb1 = [&](const AdaINResBlock1Weights& w) {
        for (int j = 0; j < 3; ++j) units.emplace_back(&w.adain1[j].fc, w.channels);
        for (int j = 0; j < 3; ++j) units.emplace_back(&w.adain2[j].fc, w.channels);
    };
    for (const auto& w : gen.noise_res) rb1(w);
    for (const auto& w : gen.resblocks) rb1(w);
    const int U = static_cast<int>(units.size());
    m.unit_off_host_.assign(U + 1, 0);
    for (int u = 0; u < U; ++u) m.unit_off_host_[u + 1] = m.unit_off_host_[u] + 2 * units[u].second;
    const int R = m.rows_ = m.unit_off_host_[U];

    // frozen fc projections, stacked once
    m.W_ = Tensor::empty_on(Device::HIP, R, S);
    m.b_ = Tensor::zeros_on(Device::HIP, R, 1);
    for (int u = 0; u < U; ++u) {
        const Linear& fc = *units[u].first;
        const int rows = 2 * units[u].second;
        if (fc.W.device != Device::HIP || fc.W.rows != rows || fc.W.cols != S || !fc.W.contiguous())
            fail("DecoderLora::make", "an AdaIN fc is not (2C, style_dim) on the HIP device");
        d2d(m.W_.f32() + static_cast<long>(m.unit_off_host_[u]) * S, fc.W.data,
            static_cast<std::size_t>(rows) * S * sizeof(float), "DecoderLora::make");
        if (fc.b.size() == static_cast<std::size_t>(rows))
            d2d(m.b_.f32() + m.unit_off_host_[u], fc.b.data, rows * sizeof(float), "DecoderLora::make");
    }

    // A, B Glorot-uniform per adapter (A then B, in order)
    SplitMix r{seed ? seed : 0xD1B54A32D192ED03ull};
    std::vector<float> A(static_cast<std::size_t>(U) * rank * S), B(static_cast<std::size_t>(R) * rank);
    for (int u = 0; u < U; ++u) {
        glorot(A.data() + static_cast<std::size_t>(u) * rank * S, rank, S, r);
        glorot(B.data() + static_cast<std::size_t>(m.unit_off_host_[u]) * rank, 2 * units[u].second, rank, r);
    }
    m.A_ = Tensor::from_host_on(Device::HIP, A.data(), U * rank, S);
    m.B_ = Tensor::from_host_on(Device::HIP, B.data(), R, rank);
    m.dA_ = Tensor::zeros_on(Device::HIP, U * rank, S);
    m.dB_ = Tensor::zeros_on(Device::HIP, R, rank);
    m.mA_ = Tensor::zeros_on(Device::HIP, U * rank, S);
    m.vA_ = Tensor::zeros_on(Device::HIP, U * rank, S);
    m.mB_ = Tensor::zeros_on(Device::HIP, R, rank);
    m.vB_ = Tensor::zeros_on(Device::HIP, R, rank);
    m.unit_off_ = Tensor::empty_on(Device::HIP, U + 1, 1);
    h2d(m.unit_off_.data, m.unit_off_host_.data(), (U + 1) * sizeof(int), "DecoderLora::make");

    m.ads_.resize(U);
    for (int u = 0; u < U; ++u) {
        DecoderLoraAdapter& ad = m.ads_[u];
        ad.fc = units[u].first;
        ad.C = units[u].second;
        const int o = m.unit_off_host_[u];
        ad.A = rows_of(m.A_, u * rank, rank);
        ad.dA = rows_of(m.dA_, u * rank, rank);
        ad.mA = rows_of(m.mA_, u * rank, rank);
        ad.vA = rows_of(m.vA_, u * rank, rank);
        ad.B = rows_of(m.B_, o, 2 * ad.C);
        ad.dB = rows_of(m.dB_, o, 2 * ad.C);
        ad.mB = rows_of(m.mB_, o, 2 * ad.C);
        ad.vB = rows_of(m.vB_, o, 2 * ad.C);
    }

    m.gate_ = ConditioningGate::make(rank, kGateHidden, dev, seed ^ 0xABCDEFu);
    m.gate_.zero_grad();
    m.gW1_m_ = Tensor::zeros_on(Device::HIP, m.gate_.hidden, m.gate_.in_dim);
    m.gW1_v_ = Tensor::zeros_on(Device::HIP, m.gate_.hidden, m.gate_.in_dim);
    m.gW2_m_ = Tensor::zeros_on(Device::HIP, m.gate_.gate_dim, m.gate_.hidden);
    m.gW2_v_ = Tensor::zeros_on(Device::HIP, m.gate_.gate_dim, m.gate_.hidden);
    return m;
}

DecoderLora::~DecoderLora() {
    delete static_cast<bd::BackboneCache*>(bb_cache_);
    delete static_cast<bd::GeneratorCache*>(gen_cache_);
}

DecoderLora::DecoderLora(DecoderLora&& o) noexcept { *this = std::move(o); }

DecoderLora& DecoderLora::operator=(DecoderLora&& o) noexcept {
    if (this != &o) {
        delete static_cast<bd::BackboneCache*>(bb_cache_);
        delete static_cast<bd::GeneratorCache*>(gen_cache_);
        rank_ = o.rank_;
        scale_ = o.scale_;
        style_dim_ = o.style_dim_;
        rows_ = o.rows_;
        dev_ = o.dev_;
        step_ = o.step_;
        gate_ = std::move(o.gate_);
        ads_ = std::move(o.ads_);
        W_ = std::move(o.W_); b_ = std::move(o.b_);
        A_ = std::move(o.A_); B_ = std::move(o.B_); dA_ = std::move(o.dA_); dB_ = std::move(o.dB_);
        mA_ = std::move(o.mA_); vA_ = std::move(o.vA_); mB_ = std::move(o.mB_); vB_ = std::move(o.vB_);
        unit_off_ = std::move(o.unit_off_);
        unit_off_host_ = std::move(o.unit_off_host_);
        gW1_m_ = std::move(o.gW1_m_); gW1_v_ = std::move(o.gW1_v_);
        gW2_m_ = std::move(o.gW2_m_); gW2_v_ = std::move(o.gW2_v_);
        g_ = std::move(o.g_); H_ = std::move(o.H_); gb_ = std::move(o.gb_); dgb_ = std::move(o.dgb_);
        dG_ = std::move(o.dG_); gen_in_ = std::move(o.gen_in_);
        N_ = o.N_;
        style_ = o.style_;
        style_bs_ = o.style_bs_;
        style_keep_ = std::move(o.style_keep_);
        bb_cache_ = o.bb_cache_;
        gen_cache_ = o.gen_cache_;
        har_ready_ = o.har_ready_;
        o.bb_cache_ = nullptr;
        o.gen_cache_ = nullptr;
        o.har_ready_ = nullptr;
    }
    return *this;
}

std::vector<DecoderLoraAdapter*> DecoderLora::adapters() {
    std::vector<DecoderLoraAdapter*> v;
    for (auto& ad : ads_) v.push_back(&ad);
    return v;
}

const Tensor& DecoderLora::stacked(int which) const {
    switch (which) {
        case 0: return A_;
        case 1: return B_;
        case 2: return dA_;
        case 3: return dB_;
        default: fail("DecoderLora::stacked", "which must be 0..3");
    }
}

namespace {

// (gamma, beta) views of every unit into a packed (N, rows) buffer, in the
// atoms' affine structures
void affine_views(const DecoderBackbone& bb, const Generator& gen, const Tensor& buf, const std::vector<int>& off,
                  std::vector<bd::BlockAffines>& bba, std::vector<bd::ResBlock1Affines>& na,
                  std::vector<bd::ResBlock1Affines>& ra) {
    std::size_t u = 0;
    auto pair = [&](Tensor& g, Tensor& b) {
        const int C = (off[u + 1] - off[u]) / 2;
        g = cols_of(buf, off[u], C);
        b = cols_of(buf, off[u] + C, C);
        ++u;
    };
    bba.assign(1 + bb.decode.size(), bd::BlockAffines{});
    for (auto& a : bba) {
        pair(a.g1, a.b1);
        pair(a.g2, a.b2);
    }
    auto rb = [&](bd::ResBlock1Affines& a) {
        for (int j = 0; j < 3; ++j) pair(a.g1[j], a.b1[j]);
        for (int j = 0; j < 3; ++j) pair(a.g2[j], a.b2[j]);
    };
    na.assign(gen.noise_res.size(), bd::ResBlock1Affines{});
    ra.assign(gen.resblocks.size(), bd::ResBlock1Affines{});
    for (auto& a : na) rb(a);
    for (auto& a : ra) rb(a);
}

}  // namespace

void DecoderLora::forward(const DecoderBackbone& bb, const Generator& gen, const DecoderLoraContext& ctx,
                          const Tensor& cond, Tensor& audio) {
    if (!ctx.asr || !ctx.F0_pred || !ctx.N_pred || !ctx.ref_s || !ctx.har)
        fail("DecoderLora::forward", "incomplete context");
    if (A_.size() == 0) fail("DecoderLora::forward", "not built (DecoderLora::make)");
    const int N = ctx.asr->rows;
    const int S = style_dim_;
    const int U = static_cast<int>(ads_.size());
    const Tensor& rs = *ctx.ref_s;
    if (rs.device != Device::HIP || rs.rows != N || rs.cols < S)
        fail("DecoderLora::forward", "ref_s must be (N, >= style_dim) on the HIP device");
    if (cond_rows(cond, gate_.in_dim, "DecoderLora::forward") != N)
        fail("DecoderLora::forward", "one condition vector per utterance");
    // style = the first style_dim columns of ref_s, kept for the backward
    style_keep_ = Tensor::empty_on(Device::HIP, N, S);
    check(kdec_axpby(bt::runtime(), 1.0f, rs.f32(), rs.row_stride(), 0.0f, nullptr, 0, style_keep_.f32(), S, N, S),
          "DecoderLora::forward");
    N_ = N;
    gate_.forward(cond, g_);
    H_ = Tensor::empty_on(Device::HIP, N, U * rank_);
    gb_ = Tensor::empty_on(Device::HIP, N, rows_);
    check(kdec_lora_proj_fwd(bt::runtime(), W_.f32(), b_.f32(), A_.f32(), B_.f32(), g_.f32(), rank_, scale_,
                             static_cast<const int*>(unit_off_.data), U, rank_, style_keep_.f32(), S, H_.f32(),
                             gb_.f32(), rows_, N, rows_, S),
          "DecoderLora::forward");
    for (int u = 0; u < U; ++u) {
        Tensor h = Tensor::view(Device::HIP, H_.f32() + u * rank_, N, rank_, bt::Dtype::FP32, U * rank_);
        h.storage = H_.storage;
        ads_[u].h = h;
    }
    std::vector<bd::BlockAffines> bba;
    std::vector<bd::ResBlock1Affines> na, ra;
    affine_views(bb, gen, gb_, unit_off_host_, bba, na, ra);
    if (!bb_cache_) bb_cache_ = new bd::BackboneCache();
    if (!gen_cache_) gen_cache_ = new bd::GeneratorCache();
    bd::decoder_backbone_forward_train(bb, *ctx.asr, *ctx.F0_pred, *ctx.N_pred, ctx.total, bba, 1e-5f, gen_in_,
                                       *static_cast<bd::BackboneCache*>(bb_cache_));
    auto& gc = *static_cast<bd::GeneratorCache*>(gen_cache_);
    gc.har_ready = har_ready_;  // the generator waits for it before reading har
    har_ready_ = nullptr;
    bd::generator_forward_train(gen, gen_in_, 2 * ctx.total, *ctx.har, ctx.frames, na, ra, audio, gc);
    if (gc.har_ready) {  // not consumed (no upsample stage read har): join here
        if (hipStreamWaitEvent(stream(), static_cast<hipEvent_t>(gc.har_ready), 0) != hipSuccess)
            fail("DecoderLora::forward", "waiting for the harmonic source");
        gc.har_ready = nullptr;
    }
}

void DecoderLora::backward(const DecoderBackbone& bb, const Generator& gen, const Tensor& cond, const Tensor& dAudio) {
    if (!bb_cache_ || !gen_cache_ || N_ == 0) fail("DecoderLora::backward", "no forward to differentiate");
    if (cond_rows(cond, gate_.in_dim, "DecoderLora::backward") != N_)
        fail("DecoderLora::backward", "the condition must match the forward");
    const int U = static_cast<int>(ads_.size());
    std::vector<bd::BlockAffines> bba, dbba;
    std::vector<bd::ResBlock1Affines> na, ra, dna, dra;
    affine_views(bb, gen, gb_, unit_off_host_, bba, na, ra);
    dgb_ = Tensor::zeros_on(Device::HIP, N_, rows_);
    affine_views(bb, gen, dgb_, unit_off_host_, dbba, dna, dra);
    Tensor dGenIn;
    bd::generator_backward(gen, *static_cast<bd::GeneratorCache*>(gen_cache_), na, ra, dAudio, dGenIn, dna, dra);
    bd::decoder_backbone_backward(bb, *static_cast<bd::BackboneCache*>(bb_cache_), bba, dGenIn, 1e-5f, dbba);
    // every adapter's gate grad sums into one (N, rank) vector
    dG_ = Tensor::zeros_on(Device::HIP, N_, rank_);
    check(kdec_lora_proj_bwd(bt::runtime(), W_.f32(), A_.f32(), B_.f32(), g_.f32(), rank_, scale_,
                             static_cast<const int*>(unit_off_.data), U, rank_, style_keep_.f32(), style_dim_,
                             H_.f32(), dgb_.f32(), rows_, nullptr, 0, 0.0f, nullptr, nullptr, dA_.f32(), dB_.f32(),
                             dG_.f32(), N_, rows_, style_dim_),
          "DecoderLora::backward");
    gate_.backward(cond, dG_);
}

const bd::BackboneCache* DecoderLora::backbone_cache() const {
    return static_cast<const bd::BackboneCache*>(bb_cache_);
}

const bd::GeneratorCache* DecoderLora::generator_cache() const {
    return static_cast<const bd::GeneratorCache*>(gen_cache_);
}

void DecoderLora::backbone_affines(const DecoderBackbone& bb, const Generator& gen,
                                   std::vector<bd::BlockAffines>& out) const {
    std::vector<bd::ResBlock1Affines> na, ra;
    affine_views(bb, gen, gb_, unit_off_host_, out, na, ra);
}

void DecoderLora::zero_grad() {
    zero(dA_, "DecoderLora::zero_grad");
    zero(dB_, "DecoderLora::zero_grad");
    gate_.zero_grad();
}

void DecoderLora::adam_step(float lr, float beta1, float beta2, float eps) {
    ++step_;
    kdec_ctx* rt = bt::runtime();
    auto one = [&](Tensor& p, const Tensor& g, Tensor& m, Tensor& v) {
        check(kdec_adam_step(rt, p.f32(), g.f32(), m.f32(), v.f32(), static_cast<long>(p.size()), lr, beta1, beta2,
                             eps, step_),
              "DecoderLora::adam_step");
    };
    one(A_, dA_, mA_, vA_);
    one(B_, dB_, mB_, vB_);
    one(gate_.W1, gate_.dW1, gW1_m_, gW1_v_);
    one(gate_.W2, gate_.dW2, gW2_m_, gW2_v_);
}

void DecoderLora::save(const std::string& path) const {
    const std::vector<float> A = A_.to_host_vector(), B = B_.to_host_vector();
    const std::vector<float> W1 = gate_.W1.to_host_vector(), W2 = gate_.W2.to_host_vector();
    std::FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error("DecoderLora::save: cannot open " + path);
    std::fwrite(kMagic, 1, 8, f);
    const std::int32_t rank = rank_, sd = style_dim_, gh = gate_.hidden;
    std::fwrite(&rank, sizeof(rank), 1, f);
    std::fwrite(&sd, sizeof(sd), 1, f);
    std::fwrite(&scale_, sizeof(scale_), 1, f);
    std::fwrite(&gh, sizeof(gh), 1, f);
    write_tensor(f, gate_.hidden, gate_.in_dim, W1.data());
    write_tensor(f, gate_.gate_dim, gate_.hidden, W2.data());
    for (std::size_t u = 0; u < ads_.size(); ++u) {
        const std::int32_t C = ads_[u].C;
        std::fwrite(&C, sizeof(C), 1, f);
        write_tensor(f, rank_, style_dim_, A.data() + u * rank_ * style_dim_);
        write_tensor(f, 2 * C, rank_, B.data() + static_cast<std::size_t>(unit_off_host_[u]) * rank_);
    }
    const bool ok = std::ferror(f) == 0;
    std::fclose(f);
    if (!ok) throw std::runtime_error("DecoderLora::save: write failed for " + path);
}

void DecoderLora::load(const std::string& path) {
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::runtime_error("DecoderLora::load: cannot open " + path);
    struct Closer {
        std::FILE* f;
        ~Closer() { std::fclose(f); }
    } closer{f};
    char magic[8];
    if (std::fread(magic, 1, 8, f) != 8 || std::memcmp(magic, kMagic, 8) != 0)
        throw std::runtime_error("DecoderLora::load: bad magic in " + path);
    std::int32_t rank = 0, sd = 0, gh = 0;
    float scale = 0.0f;
    if (std::fread(&rank, sizeof(rank), 1, f) != 1 || std::fread(&sd, sizeof(sd), 1, f) != 1 ||
        std::fread(&scale, sizeof(scale), 1, f) != 1 || std::fread(&gh, sizeof(gh), 1, f) != 1)
        throw std::runtime_error("DecoderLora::load: truncated header in " + path);
    if (rank != rank_ || sd != style_dim_ || gh != gate_.hidden)
        throw std::runtime_error("DecoderLora::load: architecture mismatch");
    const std::vector<float> W1 = read_tensor(f, gate_.hidden, gate_.in_dim, path);
    const std::vector<float> W2 = read_tensor(f, gate_.gate_dim, gate_.hidden, path);
    std::vector<float> A(A_.size()), B(B_.size());
    for (std::size_t u = 0; u < ads_.size(); ++u) {
        std::int32_t C = 0;
        if (std::fread(&C, sizeof(C), 1, f) != 1) throw std::runtime_error("DecoderLora::load: truncated adapter");
        if (C != ads_[u].C) throw std::runtime_error("DecoderLora::load: architecture mismatch in " + path);
        const std::vector<float> a = read_tensor(f, rank_, style_dim_, path);
        const std::vector<float> b = read_tensor(f, 2 * C, rank_, path);
        std::memcpy(A.data() + u * rank_ * style_dim_, a.data(), a.size() * sizeof(float));
        std::memcpy(B.data() + static_cast<std::size_t>(unit_off_host_[u]) * rank_, b.data(), b.size() * sizeof(float));
    }
    scale_ = scale;
    h2d(gate_.W1.data, W1.data(), W1.size() * sizeof(float), "DecoderLora::load");
    h2d(gate_.W2.data, W2.data(), W2.size() * sizeof(float), "DecoderLora::load");
    h2d(A_.data, A.data(), A.size() * sizeof(float), "DecoderLora::load");
    h2d(B_.data, B.data(), B.size() * sizeof(float), "DecoderLora::load");
}

}  // namespace brosoundml

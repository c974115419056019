// The producer step of Kokoro::prepare_decode_context (kokoro.cpp:622-732)
// from the predictor's outputs, and its C ABI (kdec_model_decode_prep): the
// per-phoneme repeat of the text features runs on the device
// (kdec_length_regulate) instead of the reference's host loop, the
// overrides are uploaded once, and the harmonic source is the model's own.
#include "brosoundml/kokoro.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <stdexcept>
#include <string>

#include "kdec.h"
#include "kdec_model.h"

namespace bt = brotensor;

namespace brosoundml {
namespace {

[[noreturn]] void fail(const std::string& why) {
    throw std::runtime_error("brosoundml: Kokoro::prepare_decode_context: " + why);
}

}  // namespace

void KokoroTrace::add(std::string name, int h, int w, const bt::Tensor& t) {
    Stage st;
    st.name = std::move(name);
    st.data = t.to_host_vector();
    const long n = static_cast<long>(st.data.size());
    if (h > 0 && w > 0 && static_cast<long>(h) * w == n) {
        st.h = h;
        st.w = w;
    } else {
        st.h = 1;
        st.w = static_cast<int>(n);
    }
    stages.push_back(std::move(st));
}

void KokoroTrace::add_ints(std::string name, const std::vector<int32_t>& v) {
    Stage st;
    st.name = std::move(name);
    st.h = 1;
    st.w = static_cast<int>(v.size());
    st.data.assign(v.begin(), v.end());
    stages.push_back(std::move(st));
}

void debug_stats(const char* tag, const bt::Tensor& t) {
    static const bool on = [] {
        const char* v = std::getenv("BROSOUNDML_DEBUG_STAGES");
        return v && v[0] && v[0] != '0';
    }();
    if (!on) return;
    if (!t.data || t.size() == 0) {
        std::fprintf(stderr, "[stage] %-24s empty\n", tag);
        return;
    }
    const std::vector<float> d = t.to_host_vector();
    long bad = 0, n = 0;
    float mn = 0.0f, mx = 0.0f;
    double sum = 0.0, sumsq = 0.0;
    for (float v : d) {
        if (!std::isfinite(v)) {
            ++bad;
            continue;
        }
        if (n == 0 || v < mn) mn = v;
        if (n == 0 || v > mx) mx = v;
        sum += v;
        sumsq += static_cast<double>(v) * v;
        ++n;
    }
    const double mean = n ? sum / n : 0.0;
    const double var = n ? sumsq / n - mean * mean : 0.0;
    std::fprintf(stderr,
                 "[stage] %-24s rows=%d cols=%d  min=%+.4f  max=%+.4f  mean=%+.4f  std=%.4f  nonfinite=%ld\n", tag,
                 t.rows, t.cols, mn, mx, mean, var > 0 ? std::sqrt(var) : 0.0, bad);
}

DecoderLoraContext KokoroDecodePrep::context() const {
    DecoderLoraContext c;
    c.asr = &asr;
    c.F0_pred = &F0_pred;
    c.N_pred = &N_pred;
    c.ref_s = &ref_s;
    c.har = &har;
    c.total = total;
    c.frames = frames;
    return c;
}

KokoroDecodePrep prepare_decode_context(const DecoderBackbone& backbone, const Generator& generator,
                                        const HarmonicSource& hsource, const bt::Tensor& t_en, int L,
                                        const std::vector<int32_t>& pred_dur, const bt::Tensor& F0_pred,
                                        const bt::Tensor& N_pred, const bt::Tensor& ref_s,
                                        const std::vector<float>* F0_override, const std::vector<float>* N_override) {
    if (L <= 0 || static_cast<int>(pred_dur.size()) != L) fail("one duration per phoneme expected");
    const int C = backbone.asr_res.in_channels;
    if (t_en.device != bt::Device::HIP || !t_en.data || t_en.rows != 1 || t_en.cols != C * L)
        fail("t_en must be a (1, hidden*L) HIP tensor");
    if (ref_s.device != bt::Device::HIP || !ref_s.data || ref_s.rows != 1)
        fail("ref_s must be a (1, 2*style_dim) HIP tensor");
    for (int32_t d : pred_dur)
        if (d < 0) fail("negative predicted duration");
    const long total_l = std::accumulate(pred_dur.begin(), pred_dur.end(), 0L);
    if (total_l <= 0) fail("predicted total frame count is 0");
    if (total_l > (1 << 24)) fail("predicted total frame count is too large");
    const int total = static_cast<int>(total_l);
    kdec_ctx* ctx = bt::runtime();
    hipStream_t stream = static_cast<hipStream_t>(kdec_get_stream(ctx));

    KokoroDecodePrep prep;
    prep.total = total;
    prep.ref_s = ref_s;
    prep.backbone = &backbone;
    prep.generator = &generator;
    // length regulation: asr[c, t] = t_en[c, l] over phoneme l's run of frames
    bt::Tensor dur = bt::Tensor::empty_on(bt::Device::HIP, 1, L);
    if (hipMemcpyAsync(dur.data, pred_dur.data(), static_cast<size_t>(L) * sizeof(int32_t), hipMemcpyHostToDevice,
                       stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        fail("duration upload failed");
    prep.asr = bt::Tensor::empty_on(bt::Device::HIP, 1, C * total);
    if (kdec_length_regulate(ctx, static_cast<const float*>(t_en.data), t_en.row_stride(),
                             static_cast<const int*>(dur.data), L, 1, C, L, static_cast<float*>(prep.asr.data),
                             prep.asr.row_stride(), total, nullptr) != KDEC_OK)
        fail(kdec_last_error(ctx));
    // F0 / N: predicted, or the caller's prosody (each 2*total values)
    auto grid = [&](const std::vector<float>* ov, const bt::Tensor& pred, const char* which) {
        if (!ov) {
            if (pred.device != bt::Device::HIP || !pred.data || pred.rows != 1 || pred.cols != 2 * total)
                fail(std::string(which) + " prediction must be a (1, 2*total) HIP tensor");
            return pred;
        }
        if (static_cast<long>(ov->size()) != 2L * total)
            fail(std::string(which) + " override size must be 2*total (" + std::to_string(2 * total) + ")");
        return bt::Tensor::from_host_on(bt::Device::HIP, ov->data(), 1, 2 * total);
    };
    prep.F0_pred = grid(F0_override, F0_pred, "F0");
    prep.N_pred = grid(N_override, N_pred, "N");
    // harmonic source; frames = L_gen * prod(upsample rates) + 1 (:711-724)
    long upsample_prod = 1;
    for (int r : generator.ups_stride) upsample_prod *= r;
    const long har_frames = 2L * total * upsample_prod + 1;
    int sig_len = 0, hframes = 0;
    hsource.forward(prep.F0_pred, 2 * total, sig_len, hframes, prep.har);
    if (hframes != har_frames)
        fail("har_frames mismatch: hsource=" + std::to_string(hframes) + " vs expected=" + std::to_string(har_frames));
    prep.frames = hframes;
    return prep;
}

}  // namespace brosoundml

// The decoder-facing part of the reference's Kokoro pipeline
// (include/brosoundml/kokoro.h:133-147, src/kokoro.cpp:604-732): the
// KokoroDecodePrep bundle the decoder LoRA trains over, and the producer step
// that fills it from the predictor's outputs. The text front end, plBERT and
// the duration / F0 / N predictor networks that run before it are not part of
// this library; their outputs are this step's inputs.
#pragma once

#include <brosoundml/decoder_lora.h>
#include <brosoundml/kokoro_modules.h>
#include <brotensor/tensor.h>

#include <cstdint>
#include <string>
#include <vector>

namespace brosoundml {

// The device-resident pre-decoder intermediates of one utterance, with
// borrowed references to the frozen backbone and generator (kokoro.h:133-147).
struct KokoroDecodePrep {
    brotensor::Tensor ref_s;    // (1, 2*style_dim): style = first style_dim
    brotensor::Tensor asr;      // (1, hidden*total)
    brotensor::Tensor F0_pred;  // (1, 2*total)
    brotensor::Tensor N_pred;   // (1, 2*total)
    brotensor::Tensor har;      // (1, (n_fft+2)*frames)
    int total = 0;              // asr frame count T
    int frames = 0;             // harmonic-source frame count
    const DecoderBackbone* backbone = nullptr;
    const Generator* generator = nullptr;

    // A borrowing view over the owned tensors, valid while this prep lives
    // (kokoro.cpp:604-614).
    DecoderLoraContext context() const;
};

// Per-stage capture of the decoder pipeline's intermediates, the
// reference's KokoroTrace (include/brosoundml/kokoro.h:149-185): each stage is
// a host copy, row-major (h x w) FP32. decode_back_half records "gen_in"
// (hidden x 2T), "har" ((n_fft + 2) x frames) and "audio" (1 x samples), in
// that order; a batch of N > 1 utterances records each stage per utterance
// as "<name>.<n>". A capture copies to host (a stream synchronisation), so it
// happens only when a trace is passed.
struct KokoroTrace {
    struct Stage {
        std::string name;
        int h = 0;
        int w = 0;
        std::vector<float> data;  // h*w, row-major (row r = channel r)
    };
    std::vector<Stage> stages;

    // Copy a tensor to host and record it as an (h x w) stage; a tensor of
    // another element count is recorded as one (1 x size) row.
    void add(std::string name, int h, int w, const brotensor::Tensor& t);
    // Record an integer vector (e.g. pred_dur) as a (1 x n) stage.
    void add_ints(std::string name, const std::vector<int32_t>& v);
};

// The reference's BROSOUNDML_DEBUG_STAGES diagnostics (kokoro.cpp:46-90):
// when that environment variable is set (and not "0"), prints
//   [stage] <tag> rows=.. cols=..  min=..  max=..  mean=..  std=..  nonfinite=..
// for `t` to stderr (a host copy of the tensor); the count of NaN / Inf
// elements is an addition (min / max / mean / std are over the finite ones).
// No effect otherwise.
void debug_stats(const char* tag, const brotensor::Tensor& t);

// The producer step of Kokoro::prepare_decode_context after the predictor
// (kokoro.cpp:667-732): length regulation of the text-encoder output t_en
// (1, hidden*L) by the predicted per-phoneme durations (L of them) into asr,
// the F0 / N grids (the predicted ones, each (1, 2*total), or the caller's
// overrides of 2*total values), and the harmonic source over F0 with its
// frame-count check. Errors, as the reference's: a total of 0 frames, an
// override of the wrong size, a harmonic source whose frame count differs
// from 2*total * prod(upsample rates) + 1; and negative durations (which the
// reference's host loop cannot size).
KokoroDecodePrep prepare_decode_context(const DecoderBackbone& backbone, const Generator& generator,
                                        const HarmonicSource& hsource, const brotensor::Tensor& t_en, int L,
                                        const std::vector<int32_t>& pred_dur, const brotensor::Tensor& F0_pred,
                                        const brotensor::Tensor& N_pred, const brotensor::Tensor& ref_s,
                                        const std::vector<float>* F0_override = nullptr,
                                        const std::vector<float>* N_override = nullptr);

}  // namespace brosoundml

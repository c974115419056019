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

// DecoderLora on gfx950: the trainable LoRA over the Kokoro decoder's AdaIN
// style -> (gamma, beta) projections, with the reference's public surface
// (include/brosoundml/decoder_lora.h:19-181): ConditioningGate,
// DecoderLoraAdapter, DecoderLoraContext and DecoderLora (make, forward,
// backward, zero_grad, adam_step, save, load, adapters).
//
// The model is device resident: every adapter's A, B, grads and Adam moments
// are row blocks of one stacked buffer per kind (A (units*rank, S), B
// (sum 2C, rank)); DecoderLoraAdapter's tensors are views of them, so the
// adapter projections of all 58 units run as one launch each way
// (kdec_lora_proj_fwd / _bwd) and Adam as one launch per buffer. The frozen
// fc weights are stacked once by make(). Tensors may hold N >= 1 utterances
// as rows (the reference's N = 1 is the special case); the condition is then
// (N, in_dim), one gate per utterance.
#pragma once

#include <brotensor/tensor.h>

#include <array>
#include <cstdint>
#include <string>
#include <vector>

namespace brosoundml {

struct Linear;
struct DecoderBackbone;
struct Generator;
namespace detail {
struct BackboneCache;
struct GeneratorCache;
struct BlockAffines;
}  // namespace detail

// g(v) = W2 tanh(W1 v), no biases, so g(0) = 0 exactly; W2 starts at zero.
//   v (in_dim, 1) or (N, in_dim); W1 (hidden, in_dim); W2 (gate_dim, hidden)
//   g (gate_dim, 1) for one utterance, else (N, gate_dim).
struct ConditioningGate {
    brotensor::Tensor W1, W2;    // weights
    brotensor::Tensor dW1, dW2;  // accumulated grads
    int in_dim = 3;
    int hidden = 0;
    int gate_dim = 0;

    brotensor::Tensor pre1_;  // not kept: the backward needs tanh' = 1 - act^2 only
    brotensor::Tensor act_;   // tanh(W1 v) of the last forward, (N, hidden)

    // W1 Glorot-uniform from `seed` (SplitMix64), W2 zero.
    static ConditioningGate make(int gate_dim, int hidden, brotensor::Device dev, std::uint64_t seed);
    void zero_grad();
    void forward(const brotensor::Tensor& v, brotensor::Tensor& g);
    void backward(const brotensor::Tensor& v, const brotensor::Tensor& dG);
};

// One adapter on one AdaIN fc: (gamma, beta) = fc(s) + scale * B (g * (A s)).
struct DecoderLoraAdapter {
    const Linear* fc = nullptr;        // frozen base projection (out = 2C)
    int C = 0;                         // affine half-dim
    brotensor::Tensor A, B;            // (rank, style_dim), (2C, rank): views
    brotensor::Tensor mA, vA, mB, vB;  // Adam moments (views)
    brotensor::Tensor dA, dB;          // grad accumulators (views)
    brotensor::Tensor h, hg;           // h = A s of the last forward, (N, rank) at the
                                       // stacked stride; hg is not kept (the adjoint
                                       // forms g * h itself)
};

// Frozen intermediates of one batch of clips; pointers borrowed per call.
struct DecoderLoraContext {
    const brotensor::Tensor* asr = nullptr;      // (N, hidden*T)
    const brotensor::Tensor* F0_pred = nullptr;  // (N, 2T)
    const brotensor::Tensor* N_pred = nullptr;   // (N, 2T)
    const brotensor::Tensor* ref_s = nullptr;    // (N, 2*style_dim): style = first style_dim
    const brotensor::Tensor* har = nullptr;      // (N, har_ch*frames)
    int total = 0;                               // T
    int frames = 0;                              // har frames
};

class DecoderLora {
public:
    // Adapters over every AdaIN fc of `bb` and `gen` (backbone blocks' norm1,
    // norm2; each AdaINResBlock1's adain1[0..2], adain2[0..2]; noise_res then
    // resblocks), rank = gate width, gate hidden 16. A and B Glorot-uniform
    // from `seed`, gate W2 zero: the base decoder exactly at init and at
    // cond = 0 always. `dev` must be the HIP device.
    static DecoderLora make(const DecoderBackbone& bb, const Generator& gen, int rank, float scale,
                            brotensor::Device dev, std::uint64_t seed);

    DecoderLora() = default;
    ~DecoderLora();
    DecoderLora(DecoderLora&&) noexcept;
    DecoderLora& operator=(DecoderLora&&) noexcept;
    DecoderLora(const DecoderLora&) = delete;
    DecoderLora& operator=(const DecoderLora&) = delete;

    void forward(const DecoderBackbone& bb, const Generator& gen, const DecoderLoraContext& ctx,
                 const brotensor::Tensor& cond, brotensor::Tensor& audio);
    // Accumulates every adapter's dA, dB and the gate's dW1, dW2 from dAudio
    // (of the last forward; `cond` as in that forward).
    void backward(const DecoderBackbone& bb, const Generator& gen, const brotensor::Tensor& cond,
                  const brotensor::Tensor& dAudio);

    void zero_grad();
    void adam_step(float lr, float beta1 = 0.9f, float beta2 = 0.999f, float eps = 1e-8f);

    // The reference's ELRA1 checkpoint (decoder_lora.cpp:316-396): magic
    // "ELRA1\0\0\0", int32 rank, int32 style_dim, float scale, int32 gate
    // hidden, gate W1 and W2, then per adapter int32 C, A, B; a tensor is
    // int32 rows, int32 cols, rows*cols floats, all little-endian.
    void save(const std::string& path) const;
    void load(const std::string& path);

    int rank() const { return rank_; }
    float scale() const { return scale_; }
    int step() const { return step_; }
    ConditioningGate& gate() { return gate_; }
    const ConditioningGate& gate() const { return gate_; }
    std::vector<DecoderLoraAdapter*> adapters();

    // Stacked device buffers (for bindings and tests): 0 A, 1 B, 2 dA, 3 dB.
    const brotensor::Tensor& stacked(int which) const;
    // Extension (the reference computes har before the call): a hipEvent_t
    // recorded after the work that writes the context's har on another
    // stream; the next forward makes the generator's noise branches wait for
    // it instead of assuming har is complete. Used once, then cleared.
    void set_har_ready(void* hip_event) { har_ready_ = hip_event; }
    // Unit i's first row in B / the affine buffers.
    const std::vector<int>& unit_offsets() const { return unit_off_host_; }
    // Extension (inspection): the last forward's backbone and generator
    // caches (null before the first forward) and the backbone blocks'
    // adapted AdaIN affines, as views of the forward's (gamma, beta) buffer.
    const detail::BackboneCache* backbone_cache() const;
    const detail::GeneratorCache* generator_cache() const;
    void backbone_affines(const DecoderBackbone& bb, const Generator& gen,
                          std::vector<detail::BlockAffines>& out) const;

private:
    int rank_ = 0;
    float scale_ = 1.0f;
    int style_dim_ = 0;
    int rows_ = 0;  // sum over units of 2C
    brotensor::Device dev_ = brotensor::Device::HIP;
    int step_ = 0;
    ConditioningGate gate_;
    std::vector<DecoderLoraAdapter> ads_;  // canonical order

    brotensor::Tensor W_, b_;            // stacked frozen fc (rows, S), (rows, 1)
    brotensor::Tensor A_, B_, dA_, dB_;  // stacked adapters
    brotensor::Tensor mA_, vA_, mB_, vB_;
    brotensor::Tensor unit_off_;         // units + 1 int32 (device)
    std::vector<int> unit_off_host_;
    brotensor::Tensor gW1_m_, gW1_v_, gW2_m_, gW2_v_;

    // per-forward state read by the backward
    brotensor::Tensor g_, H_, gb_, dgb_, dG_, gen_in_;
    int N_ = 0;
    const float* style_ = nullptr;
    long style_bs_ = 0;
    brotensor::Tensor style_keep_;
    void* bb_cache_ = nullptr;   // detail::BackboneCache
    void* gen_cache_ = nullptr;  // detail::GeneratorCache
    void* har_ready_ = nullptr;  // see set_har_ready
};

}  // namespace brosoundml

#pragma once

// Drop-in for the reference's src/kokoro_decoder_backward.h: the same entry
// points, argument meaning and cache / affine structs in namespace
// brosoundml::detail, implemented on gfx950 through the kdec C ABI.
//
// What is the same: every signature of kokoro_decoder_backward.h:37-293;
// outputs are overwritten (or move-assigned) and caches are filled by the
// forward and read by the matching backward; errors throw
// std::runtime_error("brosoundml: <where>: <reason>").
//
// What is extended (source-compatible with the reference's call sites):
//  - Batch: tensors may hold N > 1 utterances as N rows of C*L (the
//    reference hard-codes N = 1, kokoro_decoder_backward.h:15-17). gamma/beta
//    are (C,1) (shared) or N rows of C (per utterance); their grads follow
//    the same shape (a shared affine receives the batch sum).
//  - Every backward takes an optional trailing `const WeightGrads*`. With it
//    the frozen-weight grads the reference never computes are accumulated:
//    conv / conv-transpose / pool weights and biases and the Snake alphas
//    (whose grad the reference computes and discards, :351-353, :364-366).
//  - Cache contents: x_seq1 / x_seq2 hold the per-(n,c) instance-norm
//    statistics (mean, rstd) instead of the normalised (L, C) sequence, and
//    the pre-activation tensors (r_pre, n2_pre, s1_pre, s2_pre) are left
//    empty: the fused backward kernels recompute them from the cached input,
//    the statistics and the affine, which the extra beta fields keep. Only
//    the matching backward reads a cache, so callers see no difference.
//
// Device: inputs must be HIP tensors (brotensor::Device::HIP); there is no
// CPU path, and a CPU tensor is rejected with an error.

#include <brotensor/tensor.h>

#include <brosoundml/kokoro_modules.h>

#include <array>
#include <unordered_map>
#include <vector>

namespace brosoundml {
namespace detail {

// ─── extension: weight grads ───────────────────────────────────────────────
struct WeightGrads {
    // weight storage (Tensor::data) -> tensor its grad accumulates into
    std::unordered_map<const void*, brotensor::Tensor*> grads;
    void add(const brotensor::Tensor& w, brotensor::Tensor& g) { grads[w.data] = &g; }
    brotensor::Tensor* find(const brotensor::Tensor& w) const {
        auto it = grads.find(w.data);
        return it == grads.end() ? nullptr : it->second;
    }
};

// ─── extension: a second stream for the conv weight grads ──────────────────
// While set, conv weight grads run on `side`'s stream, forked from the runtime
// stream after their inputs exist; join_wgrad_lane() makes the runtime stream
// wait for all of them (call it before reading or zeroing the grads).
// nullptr restores the runtime stream (after a join).
void set_wgrad_lane(kdec_ctx* side);
void join_wgrad_lane();

// ─── extension: the K resblocks of a generator stage on concurrent streams ─
// While set, generator_forward_train runs resblock j > 0 of each upsample
// stage on lane (j - 1) % 2's stream, forked from the runtime stream once the
// stage input exists and joined before the stage output is read; their
// accumulating last convs keep the order j = 0, 1, ..., so the output bits are
// those of the one-stream schedule. (nullptr, nullptr) turns it off.
void set_resblock_lanes(kdec_ctx* a, kdec_ctx* b);

// ─── AdaIN affine (instance-norm + style-conditioned scale/shift) ───────────
//   x_ncl:(N, C*L)   gamma,beta:(C,1) or (N,C)   ->   y_ncl:(N, C*L)
void adain_affine_forward(const brotensor::Tensor& x_ncl,
                          const brotensor::Tensor& gamma,
                          const brotensor::Tensor& beta,
                          int C, int L, float eps,
                          brotensor::Tensor& y_ncl,
                          brotensor::Tensor& x_seq_cache);

void adain_affine_backward(const brotensor::Tensor& x_ncl,
                           const brotensor::Tensor& x_seq_cache,
                           const brotensor::Tensor& gamma,
                           const brotensor::Tensor& dY_ncl,
                           int C, int L, float eps,
                           brotensor::Tensor& dX_ncl,
                           brotensor::Tensor& dGamma,
                           brotensor::Tensor& dBeta);

// ─── AdainResBlk1d ──────────────────────────────────────────────────────────
struct AdainResBlkCache {
    brotensor::Tensor x;          // block input (N, C_in*L_in)
    brotensor::Tensor x_seq1;     // adain1 statistics (N*C_in, 2)
    brotensor::Tensor r_pre;      // (recomputed; left empty)
    brotensor::Tensor conv1_out;  // conv1 output = adain2 input (N, C_out*L_out)
    brotensor::Tensor x_seq2;     // adain2 statistics (N*C_out, 2)
    brotensor::Tensor n2_pre;     // (recomputed; left empty)
    int L_in = 0;
    int L_out = 0;
    brotensor::Tensor beta1, beta2;  // affines kept for the recompute
};

void adain_resblk_1d_forward_train(const AdainResBlk1dWeights& w,
                                   const brotensor::Tensor& x, int L_in,
                                   const brotensor::Tensor& gamma1,
                                   const brotensor::Tensor& beta1,
                                   const brotensor::Tensor& gamma2,
                                   const brotensor::Tensor& beta2,
                                   float eps,
                                   int& L_out, brotensor::Tensor& y,
                                   AdainResBlkCache& cache);

void adain_resblk_1d_backward(const AdainResBlk1dWeights& w,
                              const AdainResBlkCache& cache,
                              const brotensor::Tensor& gamma1,
                              const brotensor::Tensor& gamma2,
                              const brotensor::Tensor& dY, float eps,
                              brotensor::Tensor& dX,
                              brotensor::Tensor& dGamma1,
                              brotensor::Tensor& dBeta1,
                              brotensor::Tensor& dGamma2,
                              brotensor::Tensor& dBeta2,
                              const WeightGrads* wgrads = nullptr);

// ─── AdaINResBlock1 (Snake) ─────────────────────────────────────────────────
struct AdainResBlock1Cache {
    std::array<brotensor::Tensor, 3> x_in;    // adain1 input per sub-block
    std::array<brotensor::Tensor, 3> x_seq1;  // adain1 statistics
    std::array<brotensor::Tensor, 3> s1_pre;  // (recomputed; left empty)
    std::array<brotensor::Tensor, 3> c1_out;  // conv1 output = adain2 input
    std::array<brotensor::Tensor, 3> x_seq2;  // adain2 statistics
    std::array<brotensor::Tensor, 3> s2_pre;  // (recomputed; left empty)
    int C = 0;
    int L = 0;
    std::array<brotensor::Tensor, 3> beta1, beta2;  // affines kept for the recompute
    // Snake outputs (the convs' inputs), kept for the weight grads so the
    // backward does not recompute them.
    std::array<brotensor::Tensor, 3> act1, act2;
};

void adain_resblock1_forward_train(const AdaINResBlock1Weights& w,
                                   const brotensor::Tensor& x_in, int C, int L,
                                   const std::array<brotensor::Tensor, 3>& g1,
                                   const std::array<brotensor::Tensor, 3>& b1,
                                   const std::array<brotensor::Tensor, 3>& g2,
                                   const std::array<brotensor::Tensor, 3>& b2,
                                   brotensor::Tensor& x_out,
                                   AdainResBlock1Cache& cache);

void adain_resblock1_backward(const AdaINResBlock1Weights& w,
                              const AdainResBlock1Cache& cache,
                              const std::array<brotensor::Tensor, 3>& g1,
                              const std::array<brotensor::Tensor, 3>& g2,
                              const brotensor::Tensor& dX_out,
                              brotensor::Tensor& dX_in,
                              std::array<brotensor::Tensor, 3>& dG1,
                              std::array<brotensor::Tensor, 3>& dB1,
                              std::array<brotensor::Tensor, 3>& dG2,
                              std::array<brotensor::Tensor, 3>& dB2,
                              const WeightGrads* wgrads = nullptr);

// ─── Spectral head (conv_post -> polar exp/sin -> iSTFT) ────────────────────
struct SpectralHeadCache {
    brotensor::Tensor x_pre;   // input to the final leaky_relu (N, C*L)
    brotensor::Tensor post;    // conv_post output (N, (n_fft+2)*L)
    int C = 0;
    int L = 0;
    // Extension: leaky_relu(x_pre, 0.01), the conv_post input, kept for the
    // conv_post weight grad (recomputed from x_pre when empty)
    brotensor::Tensor x_act;
};

// Extension: x_act, when given, is leaky_relu(x, 0.01) already formed (the
// generator's last resblock sum writes it in the same pass).
void spectral_head_forward_train(const Conv1d& conv_post,
                                 const brotensor::Tensor& x, int C, int L,
                                 const brotensor::Tensor& window,
                                 int n_fft, int hop, int win,
                                 brotensor::Tensor& audio,
                                 SpectralHeadCache& cache,
                                 const brotensor::Tensor* x_act = nullptr);

// Extension: dX comes out multiplied by dx_scale (the generator divides it by
// its K resblocks right away), the same two roundings as a separate pass.
void spectral_head_backward(const Conv1d& conv_post,
                            const SpectralHeadCache& cache,
                            const brotensor::Tensor& window,
                            int n_fft, int hop, int win,
                            const brotensor::Tensor& dAudio,
                            brotensor::Tensor& dX,
                            const WeightGrads* wgrads = nullptr,
                            float dx_scale = 1.0f);

// ─── DecoderBackbone assembly ───────────────────────────────────────────────
struct BlockAffines {
    brotensor::Tensor g1, b1;   // affine1 — channels_in
    brotensor::Tensor g2, b2;   // affine2 — channels_out
};

struct BackboneCache {
    AdainResBlkCache              encode;
    std::vector<AdainResBlkCache> decode;
    std::vector<char>            res_applied;
    std::vector<int>             x_channels;
    int T = 0;
    // kept for the front-conv weight grads (extension)
    brotensor::Tensor asr, F0, N;
    // Extension: false drops each block's cache as soon as the block is done
    // (an inference forward; the backward then cannot run on this cache).
    bool keep = true;
};

void decoder_backbone_forward_train(const DecoderBackbone& bb,
                                    const brotensor::Tensor& asr,
                                    const brotensor::Tensor& F0_pred,
                                    const brotensor::Tensor& N_pred,
                                    int T,
                                    const std::vector<BlockAffines>& affines,
                                    float eps,
                                    brotensor::Tensor& gen_in,
                                    BackboneCache& cache);

void decoder_backbone_backward(const DecoderBackbone& bb,
                               const BackboneCache& cache,
                               const std::vector<BlockAffines>& affines,
                               const brotensor::Tensor& dGenIn,
                               float eps,
                               std::vector<BlockAffines>& dAffines,
                               const WeightGrads* wgrads = nullptr);

// ─── Generator assembly ─────────────────────────────────────────────────────
struct ResBlock1Affines {
    std::array<brotensor::Tensor, 3> g1, b1;   // adain1[0..2]
    std::array<brotensor::Tensor, 3> g2, b2;   // adain2[0..2]
};

struct GenStageCache {
    brotensor::Tensor               x_in;
    // Extension: leaky_relu(x_in, 0.1), the ups input, kept for the ups
    // weight grad (recomputed from x_in when empty)
    brotensor::Tensor               a;
    AdainResBlock1Cache             noise;
    std::vector<AdainResBlock1Cache> res;
    int C_in = 0, L_in = 0;
    int C_out = 0, L_out = 0;
};

struct GeneratorCache {
    std::vector<GenStageCache> stages;
    SpectralHeadCache          head;
    brotensor::Tensor          window;
    // kept for the noise_convs weight grads (extension)
    brotensor::Tensor          har;
    int                        frames = 0;
    // Extension: false drops each block's cache as soon as the block is done.
    bool                       keep = true;
    // Extension: a hipEvent_t recorded where har is produced on another
    // stream, or null when har is ready. The forward waits on it just before
    // the first noise conv, after stage 0's upsampling, so that work overlaps
    // the producer; the forward clears it.
    void*                      har_ready = nullptr;
    // Extension: a hipEvent_t recorded on the runtime stream after the
    // generator's affine inputs are written (and after everything an earlier
    // step left on that stream). With it and har_ready set, the noise branches
    // on the resblock lanes wait for these two only, not for the runtime
    // stream's backbone work queued since; the forward clears it.
    void*                      inputs_ready = nullptr;
};

void generator_forward_train(const Generator& gen,
                             const brotensor::Tensor& gen_in, int L_in,
                             const brotensor::Tensor& har, int frames,
                             const std::vector<ResBlock1Affines>& noise_aff,
                             const std::vector<ResBlock1Affines>& res_aff,
                             brotensor::Tensor& audio,
                             GeneratorCache& cache);

void generator_backward(const Generator& gen,
                        const GeneratorCache& cache,
                        const std::vector<ResBlock1Affines>& noise_aff,
                        const std::vector<ResBlock1Affines>& res_aff,
                        const brotensor::Tensor& dAudio,
                        brotensor::Tensor& dGenIn,
                        std::vector<ResBlock1Affines>& dNoise_aff,
                        std::vector<ResBlock1Affines>& dRes_aff,
                        const WeightGrads* wgrads = nullptr);

}  // namespace detail
}  // namespace brosoundml

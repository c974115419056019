// Decoder-back-half module structs with the reference's fields
// (include/brosoundml/kokoro_modules.h:127-132, 144-158, 228-244, 259-269,
// 283-300, 312-340), with the inference forwards of DecoderBackbone and
// Generator and the inference building blocks they are made of. The structs are filled by the caller (tests, the whole-decoder
// model, whose kdec_model_load_safetensors reads the upstream keys).
#pragma once

#include <brosoundml/modules.h>
#include <brotensor/tensor.h>

#include <array>
#include <functional>
#include <vector>

namespace brosoundml {

struct AdaIN1dWeights {
    int channels = 0;
    int style_dim = 0;
    float eps = 1e-5f;
    Linear fc;  // (channels * 2, style_dim)
};

struct AdainResBlk1dWeights {
    int channels_in = 0;
    int channels_out = 0;
    bool upsample = false;
    bool learned_sc = false;  // dim_in != dim_out
    AdaIN1dWeights norm1;     // channels_in
    AdaIN1dWeights norm2;     // channels_out
    Conv1d conv1;             // (channels_out, channels_in, 3)
    Conv1d conv2;             // (channels_out, channels_out, 3)
    Conv1d conv1x1;           // (channels_out, channels_in, 1) when learned_sc
    brotensor::Tensor pool_W; // (channels_in, 3)  depthwise ConvTranspose1d
    brotensor::Tensor pool_b; // (channels_in, 1)
};

struct DecoderBackbone {
    Conv1d F0_conv;  // (1, 1, 3) stride 2 padding 1
    Conv1d N_conv;   // (1, 1, 3) stride 2 padding 1
    Conv1d asr_res;  // (64, 512, 1)
    AdainResBlk1dWeights encode;
    std::vector<AdainResBlk1dWeights> decode;  // the last upsamples 2x

    // Inference forward (kokoro_modules.cpp:1087-1141): style = the first
    // style_dim values of each ref_s row; asr (N, 512*T), F0_pred / N_pred
    // (N, 2T) -> gen_in (N, 512*2T). No training caches are kept.
    void forward(const brotensor::Tensor& asr, const brotensor::Tensor& F0_pred, const brotensor::Tensor& N_pred,
                 const brotensor::Tensor& ref_s, int T, brotensor::Tensor& gen_in) const;
};

struct AdaINResBlock1Weights {
    int channels = 0;
    int kernel_size = 0;
    std::vector<int> dilations;  // length 3
    std::array<Conv1d, 3> convs1;
    std::array<Conv1d, 3> convs2;
    std::array<AdaIN1dWeights, 3> adain1;
    std::array<AdaIN1dWeights, 3> adain2;
    std::array<brotensor::Tensor, 3> alpha1;  // (channels, 1)
    std::array<brotensor::Tensor, 3> alpha2;
};

struct HarmonicSource {
    int sample_rate = 24000;
    int harmonic_num = 8;
    int upsample_scale = 0;
    int n_fft = 0;
    int hop_size = 0;
    int win_size = 0;
    float sine_amp = 0.1f;
    Linear l_linear;  // (1, harmonic_num + 1)

    // F0_pred: (N, frame_count) Hz. har: (N, (n_fft+2) * stft_frames).
    void forward(const brotensor::Tensor& F0_pred, int frame_count, int& signal_len,
                 int& stft_frames, brotensor::Tensor& har) const;
};

struct Generator {
    int n_fft = 0;
    int hop_size = 0;
    int win_size = 0;
    int num_upsamples = 0;
    int num_kernels = 0;
    std::vector<brotensor::Tensor> ups_W;  // each (C_in, C_out*kL)
    std::vector<brotensor::Tensor> ups_b;  // each (C_out, 1)
    std::vector<int> ups_C_in, ups_C_out, ups_k, ups_stride, ups_pad;
    std::vector<Conv1d> noise_convs;
    std::vector<AdaINResBlock1Weights> noise_res;  // num_upsamples
    std::vector<AdaINResBlock1Weights> resblocks;  // num_upsamples * num_kernels
    Conv1d conv_post;

    // Inference forward (kokoro_modules.cpp:1400-1552): gen_in (N, C*L_in),
    // har (N, (n_fft+2)*frames), style (N, style_dim) -> audio (N, samples).
    // `cancel` returning true before a stage leaves `audio` empty.
    void forward(const brotensor::Tensor& gen_in, int L_in, const brotensor::Tensor& har, int frames,
                 const brotensor::Tensor& style, brotensor::Tensor& audio,
                 const std::function<bool()>& cancel = {}) const;
};

// The reference's inference building blocks (kokoro_modules.cpp:596-620,
// 651-706, 1197-1231), on N style rows (style (N, >= style_dim) at its row
// stride; gamma, beta = chunk(fc(style)) for every utterance):
//   ada_in_1d_styled: y = (1 + gamma) * instance_norm(x) + beta, x (N, C*L)
//   adain_resblk_1d_forward: (residual + shortcut) / sqrt(2), L_out = 2 L_in
//     for the upsampling block
//   adain_resblock1_forward: x <- the three dilated AdaIN + Snake stages
void ada_in_1d_styled(const AdaIN1dWeights& w, int N, int C, int L, const brotensor::Tensor& x_ncl,
                      const brotensor::Tensor& style, brotensor::Tensor& y_ncl);
void adain_resblk_1d_forward(const AdainResBlk1dWeights& w, const brotensor::Tensor& x, int L_in,
                             const brotensor::Tensor& style, int& L_out, brotensor::Tensor& y);
void adain_resblock1_forward(const AdaINResBlock1Weights& w, brotensor::Tensor& x, int C, int L,
                             const brotensor::Tensor& style);

}  // namespace brosoundml

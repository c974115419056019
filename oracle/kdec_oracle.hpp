// CPU FP32 restatement of the Kokoro-82M iSTFTNet decoder back half, forward
// (cached `_train` variant) and manual backward. TEST INFRASTRUCTURE ONLY:
// this is the parity oracle for the HIP path. It is never linked into the
// product library; only tests, the smoke check and the bench's CPU-baseline
// leg load it.
//
// It follows the reference op by op:
//   src/kokoro_decoder_backward.cpp (whole file) for the assemblies,
//   src/kokoro_modules.cpp:1021-1063, 1147-1195, 1237-1347, 1574-1665 for the
//     module shapes, paddings and the harmonic source,
//   src/modules.cpp:103-108 for Conv1d,
//   src/decoder_lora.cpp:184-207 for the style projection.
// The arithmetic the reference delegates to brotensor (absent, not vendored)
// is restated from the op definitions; conventions that only brotensor's
// source could fix follow PyTorch semantics (listed in oracle/README.md).
//
// Numerics: tensors are stored as float; every reduction (conv dot products,
// norm statistics, parameter-grad sums) accumulates in double and elementwise
// transcendental math is evaluated in double and rounded once, so the oracle
// sits closer to exact arithmetic than any FP32 implementation it checks.
//
// Layout: channel-major NCL with N = 1, element (c, l) at c * L + l
// (kokoro_decoder_backward.h:15-17). Weight layouts follow modules.h:14-21 and
// kokoro_modules.h: Conv1d W (C_out, (C_in/groups)*k) index [co][ci*k+t];
// ConvTranspose1d W (C_in, (C_out/groups)*k) index [ci][co*k+t].
#pragma once

#include <array>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

// The storage scalar is float; building with -DKDO_REAL=double -DKDO_NS=kdo64
// gives the FP64 shadow used to pin the float oracle and to run
// finite-difference checks below float rounding noise.
#ifndef KDO_REAL
#define KDO_REAL float
#endif
#ifndef KDO_NS
#define KDO_NS kdo
#endif

namespace KDO_NS {

using Real = KDO_REAL;
using Vec = std::vector<Real>;

// ─── brotensor op restatements (N = 1) ──────────────────────────────────────

int conv1d_out_len(int L, int k, int s, int p, int d);
int convt1d_out_len(int L, int k, int s, int p, int op, int d);

// y[co, l] = b[co] + sum_{ci in group, t} W[co, ci'*k + t] * x[ci, l*s + t*d - p]
void conv1d_forward(const Real* x, const Real* W, const Real* b, int C_in,
                    int L, int C_out, int k, int s, int p, int d, int g,
                    Real* y);
// dx = adjoint of conv1d w.r.t. x (overwrites dx, length C_in * L_in).
void conv1d_backward_input(const Real* W, const Real* dy, int C_in, int L_in,
                           int C_out, int k, int s, int p, int d, int g,
                           Real* dx);
// dW += sum_l dy[co,l] x[ci, l*s+t*d-p];  db += sum_l dy[co,l]  (db may be null)
void conv1d_backward_weight(const Real* x, const Real* dy, int C_in, int L_in,
                            int C_out, int k, int s, int p, int d, int g,
                            Real* dW, Real* db);

// y[co, j] = b[co] + sum_{ci in group, t, l : l*s + t*d - p == j} x[ci,l] W[ci, co'*k+t]
void convt1d_forward(const Real* x, const Real* W, const Real* b, int C_in,
                     int L, int C_out, int k, int s, int p, int op, int d,
                     int g, Real* y);
void convt1d_backward_input(const Real* W, const Real* dy, int C_in, int L_in,
                            int C_out, int k, int s, int p, int op, int d,
                            int g, Real* dx);
void convt1d_backward_weight(const Real* x, const Real* dy, int C_in,
                             int L_in, int C_out, int k, int s, int p, int op,
                             int d, int g, Real* dW, Real* db);

// GroupNorm with num_groups == C (instance norm), biased variance over L.
void instnorm_forward(const Real* x, const Real* gamma, const Real* beta,
                      int C, int L, float eps, Real* y);
// dgamma/dbeta overwritten.
void instnorm_backward(const Real* x, const Real* gamma, const Real* dy,
                       int C, int L, float eps, Real* dx, Real* dgamma,
                       Real* dbeta);

// y = x + sin^2(alpha_c x) / alpha_c   (kokoro_modules.h:251-258)
void snake_forward(const Real* x, const Real* alpha, int C, int L, Real* y);
// dx overwritten; dalpha accumulated when non-null.
void snake_backward(const Real* x, const Real* alpha, const Real* dy, int C,
                    int L, Real* dx, Real* dalpha);

void leaky_forward(const Real* x, float slope, std::size_t n, Real* y);
void leaky_backward(const Real* x, const Real* dy, float slope,
                    std::size_t n, Real* dx);

// Left reflect-pad by 1 (mode 1): y[0] = x[1], y[j+1] = x[j].
void pad_reflect_left1_forward(const Real* x, int C, int L, Real* y);
void pad_reflect_left1_backward(const Real* dy, int C, int L, Real* dx);

// Nearest 2x along L (kokoro_decoder_backward.cpp:63-96).
void nearest2x_forward(const Real* x, int C, int L_in, Real* y);
void nearest2x_backward(const Real* dy, int C, int L_in, Real* dx);

// Periodic Hann in float arithmetic (kokoro_decoder_backward.cpp:580-588).
Vec hann_periodic(int N);

// iSTFT, center = true, normalized = false, onesided (torch.istft semantics):
// spec is frame-major interleaved complex (frames, 2*(n_fft/2+1)).
void istft(const Real* spec, const Real* window, int frames, int signal_len,
           int n_fft, int hop, int win, Real* out);
// Exact adjoint of istft w.r.t. the interleaved (re, im) spectrum.
void istft_backward(const Real* dout, const Real* window, int frames,
                    int signal_len, int n_fft, int hop, int win, Real* dspec);
// STFT, center = true with reflect padding, onesided; returns frames.
int stft(const Real* x, int len, const Real* window, int n_fft, int hop,
         int win, Vec& spec);

// One DecoderLora adapter on one AdaIN fc for one utterance (the adapter
// contract of decoder_lora.h:63-77, adapter_fwd / adapter_bwd at
// decoder_lora.cpp:184-207 over bt::lora_forward / lora_backward):
//   h = A s (rank), hg = g * h, y = W s + b + scale * B hg (rows = 2C).
// W (rows, S), A (rank, S), B (rows, rank); h is kept for the backward.
void lora_forward(const Real* W, const Real* b, const Real* A, const Real* B,
                  const Real* g, float scale, const Real* s, int rows, int rank,
                  int S, Real* y, Real* h);
// Adjoint: dB += scale dy hg^T, dhg = scale B^T dy, dG += dhg * h,
// dA += (dhg * g) s^T, and dstyle += W^T dy + A^T (dhg * g) when requested
// (the reference passes dX = nullptr); dW / db accumulate the frozen fc's
// grads when non-null. Any output may be null.
void lora_backward(const Real* W, const Real* A, const Real* B, const Real* g,
                   float scale, const Real* s, const Real* h, const Real* dy,
                   int rows, int rank, int S, Real* dstyle, Real* dW, Real* db,
                   Real* dA, Real* dB, Real* dG);

// ─── module weight structs (mirror modules.h / kokoro_modules.h) ───────────

struct Conv1d {
    int in_channels = 0, out_channels = 0, kernel_size = 0;
    int stride = 1, padding = 0, dilation = 1, groups = 1;
    Vec W, b;    // W (out, in/groups*k); b (out) or empty
    Vec dW, db;  // grad accumulators (extension)
    int L_out(int L) const {
        return conv1d_out_len(L, kernel_size, stride, padding, dilation);
    }
};

struct AdaIN1dWeights {
    int channels = 0, style_dim = 0;
    float eps = 1e-5f;
    Vec fcW, fcb;    // (2C, style_dim), (2C)
    Vec dfcW, dfcb;  // grads (extension)
};

struct AdainResBlk1dWeights {
    int channels_in = 0, channels_out = 0;
    bool upsample = false, learned_sc = false;
    AdaIN1dWeights norm1, norm2;
    Conv1d conv1, conv2, conv1x1;
    Vec pool_W, pool_b;    // (C_in, 3), (C_in)
    Vec dpool_W, dpool_b;
};

struct AdaINResBlock1Weights {
    int channels = 0, kernel_size = 0;
    std::array<int, 3> dilations{{1, 3, 5}};
    std::array<Conv1d, 3> convs1, convs2;
    std::array<AdaIN1dWeights, 3> adain1, adain2;
    std::array<Vec, 3> alpha1, alpha2;    // (C)
    std::array<Vec, 3> dalpha1, dalpha2;  // grads
};

struct DecoderBackbone {
    Conv1d F0_conv, N_conv, asr_res;
    AdainResBlk1dWeights encode;
    std::vector<AdainResBlk1dWeights> decode;
};

struct Generator {
    int n_fft = 0, hop_size = 0, win_size = 0;
    int num_upsamples = 0, num_kernels = 0;
    std::vector<Vec> ups_W, ups_b, dups_W, dups_b;
    std::vector<int> ups_C_in, ups_C_out, ups_k, ups_stride, ups_pad;
    std::vector<Conv1d> noise_convs;
    std::vector<AdaINResBlock1Weights> noise_res, resblocks;
    Conv1d conv_post;
};

struct HarmonicSource {
    int sample_rate = 24000, harmonic_num = 8, upsample_scale = 300;
    int n_fft = 20, hop_size = 5, win_size = 20;
    float sine_amp = 0.1f;
    Vec lW, lb;    // (1, harmonic_num+1), (1)
    Vec dlW, dlb;  // always zero: the harmonic source is forward-only
};

// Which extensions the backward computes on top of the reference
// semantics (conv dgrad only, snake dalpha discarded, no d(style)).
struct Ext {
    bool wgrad = false;   // conv / convT / pool weight+bias grads
    bool dalpha = false;  // snake alpha grads
};

// Kink overrides. The leaky ReLUs are the decoder's only non-smooth points.
// Two float evaluations of the same forward can put an input that lies within
// rounding of zero on opposite sides of the kink; the slope's derivative then
// differs by (1 - slope) at that element and the difference spreads into
// every grad upstream of it (one such element among the 983 168 inputs of the
// spectral head at T = 64 moves every AdaIN affine grad by about 2e-3). With
// masks set on a Model, each leaky site takes its branch (x > 0) from the
// mask, in the forward and in the backward, so the oracle is evaluated on the
// same linear piece as the implementation the mask came from. Sites, in
// forward order: per AdaIN residual block (encode, decode.0, ...) the norm1
// output then the norm2 output (slope 0.2); per generator stage the stage
// input (0.1); the spectral head input (0.01).
struct KinkMasks {
    std::vector<std::vector<signed char>> masks;  // per site, empty = own sign
    std::vector<long> flips;                      // per site: own signs overridden
};
// Set while Model::forward / ::backward run with masks: the model's masks,
// the site of the AdaIN residual block being run (its norm1; norm2 is + 1),
// and the site of generator stage 0 (stage i at + i, the spectral head at
// + num_upsamples). -1: no override.
extern KinkMasks* g_kinks;
extern int g_kink_block;
extern int g_kink_gen;

// ─── assembly atoms (kokoro_decoder_backward.h) ─────────────────────────────

void adain_affine_forward(const Vec& x, const Vec& gamma, const Vec& beta,
                          int C, int L, float eps, Vec& y, Vec& x_seq);
void adain_affine_backward(const Vec& x, const Vec& x_seq, const Vec& gamma,
                           const Vec& dY, int C, int L, float eps, Vec& dX,
                           Vec& dGamma, Vec& dBeta);

struct AdainResBlkCache {
    Vec x, x_seq1, r_pre, conv1_out, x_seq2, n2_pre;
    int L_in = 0, L_out = 0;
};
void adain_resblk_1d_forward_train(const AdainResBlk1dWeights& w, const Vec& x,
                                   int L_in, const Vec& g1, const Vec& b1,
                                   const Vec& g2, const Vec& b2, float eps,
                                   int& L_out, Vec& y, AdainResBlkCache& cache);
// dX_full receives the grad into x (all channels). When ext->wgrad is set the
// conv / shortcut / pool weight grads accumulate into w's grad buffers.
void adain_resblk_1d_backward(AdainResBlk1dWeights& w,
                              const AdainResBlkCache& cache, const Vec& g1,
                              const Vec& g2, const Vec& dY, float eps, Vec& dX,
                              Vec& dG1, Vec& dB1, Vec& dG2, Vec& dB2,
                              const Ext* ext);

struct AdainResBlock1Cache {
    std::array<Vec, 3> x_in, x_seq1, s1_pre, c1_out, x_seq2, s2_pre;
    int C = 0, L = 0;
};
using Arr3 = std::array<Vec, 3>;
void adain_resblock1_forward_train(const AdaINResBlock1Weights& w,
                                   const Vec& x_in, int C, int L,
                                   const Arr3& g1, const Arr3& b1,
                                   const Arr3& g2, const Arr3& b2, Vec& x_out,
                                   AdainResBlock1Cache& cache);
void adain_resblock1_backward(AdaINResBlock1Weights& w,
                              const AdainResBlock1Cache& cache, const Arr3& g1,
                              const Arr3& g2, const Vec& dX_out, Vec& dX_in,
                              Arr3& dG1, Arr3& dB1, Arr3& dG2, Arr3& dB2,
                              const Ext* ext);

struct SpectralHeadCache {
    Vec x_pre, post;
    int C = 0, L = 0;
};
void spectral_head_forward_train(const Conv1d& conv_post, const Vec& x, int C,
                                 int L, const Vec& window, int n_fft, int hop,
                                 int win, Vec& audio, SpectralHeadCache& cache);
void spectral_head_backward(Conv1d& conv_post, const SpectralHeadCache& cache,
                            const Vec& window, int n_fft, int hop, int win,
                            const Vec& dAudio, Vec& dX, const Ext* ext);

struct BlockAffines {
    Vec g1, b1, g2, b2;
};
struct BackboneCache {
    AdainResBlkCache encode;
    std::vector<AdainResBlkCache> decode;
    std::vector<char> res_applied;
    std::vector<int> x_channels;
    int T = 0;
    // Kept for the extension's front-conv weight grads.
    Vec asr, F0, N, F0_dn, N_dn, asr_res_out;
};
void decoder_backbone_forward_train(const DecoderBackbone& bb, const Vec& asr,
                                    const Vec& F0_pred, const Vec& N_pred,
                                    int T, const std::vector<BlockAffines>& aff,
                                    float eps, Vec& gen_in,
                                    BackboneCache& cache);
void decoder_backbone_backward(DecoderBackbone& bb, const BackboneCache& cache,
                               const std::vector<BlockAffines>& aff,
                               const Vec& dGenIn, float eps,
                               std::vector<BlockAffines>& dAff,
                               const Ext* ext);

struct ResBlock1Affines {
    Arr3 g1, b1, g2, b2;
};
struct GenStageCache {
    Vec x_in;
    AdainResBlock1Cache noise;
    std::vector<AdainResBlock1Cache> res;
    int C_in = 0, L_in = 0, C_out = 0, L_out = 0;
    Vec x_source_in;  // noise_convs input (har) kept for the extension
    int L_src = 0;
};
struct GeneratorCache {
    std::vector<GenStageCache> stages;
    SpectralHeadCache head;
    Vec window;
    Vec har;
    int frames = 0;
};
void generator_forward_train(const Generator& gen, const Vec& gen_in, int L_in,
                             const Vec& har, int frames,
                             const std::vector<ResBlock1Affines>& naff,
                             const std::vector<ResBlock1Affines>& raff,
                             Vec& audio, GeneratorCache& cache);
void generator_backward(Generator& gen, const GeneratorCache& cache,
                        const std::vector<ResBlock1Affines>& naff,
                        const std::vector<ResBlock1Affines>& raff,
                        const Vec& dAudio, Vec& dGenIn,
                        std::vector<ResBlock1Affines>& dnaff,
                        std::vector<ResBlock1Affines>& draff, const Ext* ext);

// HarmonicSource::forward (kokoro_modules.cpp:1574-1665).
void harmonic_source_forward(const HarmonicSource& hs, const Vec& F0,
                             int frame_count, int& signal_len,
                             int& stft_frames, Vec& har);

// ─── whole decoder with named parameters ────────────────────────────────────

struct Config {
    int asr_dim = 512, asr_res_dim = 64, style_dim = 128;
    int enc_dim = 1024;      // encode output channels
    int n_decode = 4;
    int dec_out[8] = {1024, 1024, 1024, 512, 0, 0, 0, 0};
    int dec_up_at = 3;       // index of the 2x-upsampling decode block
    // Generator input channels = dec_out[n_decode - 1].
    int n_ups = 2;
    int ups_rates[4] = {10, 6, 0, 0};
    int ups_kernels[4] = {20, 12, 0, 0};
    int n_kernels = 3;
    int rb_kernels[4] = {3, 7, 11, 0};
    int rb_dil[4][3] = {{1, 3, 5}, {1, 3, 5}, {1, 3, 5}, {1, 3, 5}};
    int n_fft = 20, hop = 5;
    int conv_post_k = 7;
    int sample_rate = 24000, harmonic_num = 8;
};

struct ParamRef {
    Vec* value = nullptr;
    Vec* grad = nullptr;
    int rows = 0, cols = 0;
};

struct AffineUnit {
    std::string name;        // fc prefix, e.g. "decoder.module.encode.norm1"
    AdaIN1dWeights* w = nullptr;
    Vec* gamma = nullptr;    // forward (C)
    Vec* beta = nullptr;
    Vec* dgamma = nullptr;   // backward (C)
    Vec* dbeta = nullptr;
    // DecoderLora adapter on this unit's fc (decoder_lora.h:63-77), when the
    // model's lora_rank > 0: A (rank, style_dim), B (2C, rank), grads, and
    // the bottleneck h = A s of the last forward.
    Vec A, B, dA, dB, h;
};

struct Model {
    Config cfg;
    DecoderBackbone bb;
    Generator gen;
    HarmonicSource hs;
    std::vector<std::string> order;
    std::map<std::string, ParamRef> params;
    std::vector<AffineUnit> units;

    // Per-forward state.
    int T = 0;
    Vec style;
    std::vector<BlockAffines> bbaff, dbbaff;
    std::vector<ResBlock1Affines> naff, raff, dnaff, draff;
    BackboneCache bbc;
    GeneratorCache genc;
    Vec gen_in, har, audio, dstyle;
    int frames = 0;
    // LoRA adapters on every unit with a shared gate g (rank); off at rank 0.
    int lora_rank = 0;
    float lora_scale = 0.0f;
    Vec gate, dgate;
    void lora_enable(int rank, float scale);
    // Leaky-site masks (see KinkMasks); none by default.
    KinkMasks kinks;
    int kink_site_count() const { return 2 * (1 + cfg.n_decode) + cfg.n_ups + 1; }

    explicit Model(const Config& c);
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;
    void zero_grad();
    // style (style_dim): the style vector (ref_s[:style_dim]).
    // har_in: when non-null, used instead of the harmonic source output.
    void forward(const Vec& asr, const Vec& F0, const Vec& N, const Vec& style,
                 int T, const Vec* har_in);
    void backward(const Vec& dAudio, const Ext& ext, bool want_dstyle);

private:
    void register_param(const std::string& name, Vec* v, Vec* g, int rows,
                        int cols);
    void build();
};

}  // namespace KDO_NS

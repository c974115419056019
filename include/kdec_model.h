/*
 * kdec_model.h — C ABI over the whole decoder back half (style projection,
 * DecoderBackbone, harmonic source, Generator, spectral head) for N
 * utterances at once, built on the C++ drop-in atoms of
 * kokoro_decoder_backward.h.
 *
 * It stands in for the sequence DecoderLora::forward / ::backward runs
 * (src/decoder_lora.cpp:211-296): the per-AdaIN style projection
 * (gamma, beta) = fc(style) (kokoro_modules.cpp:563-572), plus the LoRA term
 * when adapters are enabled (kdec_model_lora_enable),
 * decoder_backbone_forward_train / generator_forward_train, then
 * generator_backward / decoder_backbone_backward and the projection's
 * adjoint. The harmonic source runs first, as in decode_back_half
 * (kokoro.cpp:369-383).
 *
 * Parameters are addressed by the upstream state-dict names the reference's
 * loaders read (kokoro_modules.cpp:1021-1063, 1147-1195, 1237-1347,
 * 1556-1572), e.g. "decoder.module.generator.resblocks.3.convs1.1.weight",
 * with the reference's layouts. All parameters live in one device buffer
 * and all grads in another.
 *
 * Activations cross this ABI as DEVICE pointers (the caller owns them and
 * keeps forward inputs alive until backward returns); parameters and grads
 * can be copied from / to host memory. Same error convention as kdec.h.
 */
#ifndef KDEC_MODEL_H
#define KDEC_MODEL_H

#include "kdec.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kdec_model kdec_model;

/* cfg: the decoder configuration as flat ints, in this order:
 *   asr_dim, asr_res_dim, style_dim, enc_dim, n_decode, dec_out[8],
 *   dec_up_at, n_ups, ups_rates[4], ups_kernels[4], n_kernels,
 *   rb_kernels[4], rb_dil[4][3], n_fft, hop, conv_post_k, sample_rate,
 *   harmonic_num
 * (Kokoro-82M: 512, 64, 128, 1024, 4, {1024,1024,1024,512}, 3, 2, {10,6},
 *  {20,12}, 3, {3,7,11}, {1,3,5}x3, 20, 5, 7, 24000, 8). Parameters start at
 * zero. The context must outlive the model. */
int kdec_model_create(kdec_ctx* ctx, const int* cfg, int n_cfg, kdec_model** out);
int kdec_model_destroy(kdec_model* m);

int kdec_model_param_count(const kdec_model* m);
const char* kdec_model_param_name(const kdec_model* m, int i);
int kdec_model_param_shape(const kdec_model* m, const char* name, int* rows, int* cols);
/* Host copies (synchronous). */
int kdec_model_set_param(kdec_model* m, const char* name, const float* host, long n);
int kdec_model_get_param(kdec_model* m, const char* name, float* host, long n);
int kdec_model_get_grad(kdec_model* m, const char* name, float* host, long n);
/* Device pointers into the parameter / grad buffers. */
float* kdec_model_param_ptr(kdec_model* m, const char* name);
float* kdec_model_grad_ptr(kdec_model* m, const char* name);
long kdec_model_param_total(const kdec_model* m);  /* total parameter count */
int kdec_model_zero_grad(kdec_model* m);
/* The context the model was created on (its stream and last error). */
kdec_ctx* kdec_model_context(const kdec_model* m);
/* Every parameter from a safetensors file under its upstream state-dict key
 * (DecoderBackbone / Generator / HarmonicSource::load_from over
 * brotensor::safetensors, kokoro_modules.cpp:99-122 `upload`, 1021-1063,
 * 1147-1195, 1237-1347, 1556-1572): F32 tensors of exactly the parameter's
 * element count, else KDEC_EINVAL with the reference's messages ("missing
 * safetensors key '...'", "... is not F32 ...", "... has n elements;
 * expected m"). A weight found only as weight_g / weight_v (the upstream
 * weight-norm form, fused offline by scripts/convert-kokoro.py:71-110) is
 * fused on load: weight[r] = g[r] v[r] / max(|v[r]|, 1e-12). */
int kdec_model_load_safetensors(kdec_model* m, const char* path);
/* Tensors in a safetensors file, or KDEC_EINVAL when it does not parse
 * (host only: needs no device). */
int kdec_safetensors_count(const char* path);

/* AdaIN units in canonical order (backbone, noise_res, resblocks). Unit i's
 * gamma for utterance n is affine[n * rows_total + offset + c], beta follows
 * at + C; the affine grads use the same layout. */
int kdec_model_unit_count(const kdec_model* m);
const char* kdec_model_unit_name(const kdec_model* m, int i);
int kdec_model_unit_channels(const kdec_model* m, int i);
int kdec_model_unit_offset(const kdec_model* m, int i);
int kdec_model_affine_rows(const kdec_model* m);
/* Host copies of the last forward's affines / last backward's affine grads
 * (N * rows_total floats each; either pointer may be NULL). */
int kdec_model_get_affines(kdec_model* m, float* gb, float* dgb);

/* Per-utterance lengths for T asr frames. */
int kdec_model_lengths(const kdec_model* m, int T, int* L_gen, int* frames, int* audio_len);

/* Forward for N utterances of T frames: asr (N, asr_dim*T), F0 / Nn (N, 2T),
 * style (N, style_dim) -> audio (N, audio_len). har_in (N, (n_fft+2)*frames)
 * replaces the harmonic source output when non-NULL. */
int kdec_model_forward(kdec_model* m, int N, int T, const float* asr, const float* F0,
                       const float* Nn, const float* style, const float* har_in, float* audio);
/* Backward of the last forward. wgrad: accumulate every conv / conv-transpose
 * / pool / style-fc weight and bias grad; dalpha: accumulate the Snake alpha
 * grads; dstyle (N, style_dim) may be NULL. The affine grads are always
 * produced (the reference semantics). */
int kdec_model_backward(kdec_model* m, const float* daudio, int wgrad, int dalpha, float* dstyle);
/* Inference forward (decode_back_half, kokoro.cpp:352-407: the
 * DecoderBackbone / HarmonicSource / Generator forwards of
 * kokoro_modules.cpp:1087-1141, 1400-1552, 1574-1665): the same arithmetic
 * as kdec_model_forward, arguments as there, without training caches (each
 * block's are dropped once it is done, so device memory stays at about one
 * stage's activations). The adapters apply when LoRA is on. A following
 * kdec_model_backward is refused until the next kdec_model_forward. */
int kdec_model_infer(kdec_model* m, int N, int T, const float* asr, const float* F0, const float* Nn,
                     const float* style, const float* har, float* audio);
/* Kokoro::Impl::decode_back_half (kokoro.cpp:352-407) over the model's
 * weights through the C++ inference forwards: DecoderBackbone::forward,
 * HarmonicSource::forward on F0, Generator::forward with the style = the
 * first style_dim values of each ref_s row (N rows at stride ref_bs);
 * audio (N, audio_len). For the base decoder (LoRA off). */
int kdec_model_decode_back_half(kdec_model* m, int N, int T, const float* asr, const float* F0, const float* Nn,
                                const float* ref_s, long ref_bs, float* audio);
/* decode_back_half with the reference's cooperative cancellation
 * (kokoro.cpp:387; Generator::forward, kokoro_modules.cpp:1418): cancel(user)
 * is polled on the host before the generator and before each upsample stage
 * (1 + n_ups polls when nothing cancels); once it returns nonzero no further
 * work is enqueued, *cancelled is set to 1 and `audio` is left unwritten
 * (the reference returns an empty buffer). cancel may be NULL. */
typedef int (*kdec_cancel_fn)(void* user);
int kdec_model_decode_back_half_cancellable(kdec_model* m, int N, int T, const float* asr, const float* F0,
                                            const float* Nn, const float* ref_s, long ref_bs, float* audio,
                                            kdec_cancel_fn cancel, void* user, int* cancelled);
/* Stage traces (the reference's KokoroTrace, kokoro.h:149-185, filled by
 * decode_back_half at kokoro.cpp:366, 389-390, 396): a trace holds named
 * host copies of the pipeline's intermediates as row-major (h x w) floats.
 * kdec_model_decode_back_half_traced is decode_back_half with cancellation
 * that also appends "gen_in" (hidden x 2T), "har" ((n_fft+2) x frames) and
 * "audio" (1 x samples) to `trace` (per utterance "<name>.<n>" when N > 1;
 * each capture synchronises the stream). trace may be NULL. With the
 * environment variable BROSOUNDML_DEBUG_STAGES set (not "0"), every
 * decode_back_half also prints those stages' min / max / mean / std and
 * non-finite count to stderr (kokoro.cpp:46-90, tags 09_gen_in, 10_har_stub,
 * 11_audio). kdec_trace_stage returns stage i's name (valid while the trace
 * lives) and shape, kdec_trace_data its h*w floats. */
typedef struct kdec_trace kdec_trace;
int kdec_trace_create(kdec_trace** out);
int kdec_trace_destroy(kdec_trace* t);
int kdec_trace_count(const kdec_trace* t);
const char* kdec_trace_stage(const kdec_trace* t, int i, int* h, int* w);
const float* kdec_trace_data(const kdec_trace* t, int i);
int kdec_model_decode_back_half_traced(kdec_model* m, int N, int T, const float* asr, const float* F0,
                                       const float* Nn, const float* ref_s, long ref_bs, float* audio,
                                       kdec_cancel_fn cancel, void* user, int* cancelled, kdec_trace* trace);
/* Stream overlap (no counterpart in the reference, whose calls are
 * synchronous): on = 1 (the default) runs the harmonic source and the conv
 * weight grads on a second stream beside the main chain, and the
 * generator's noise branches and per-stage resblocks on that stream and a
 * third one; on = 0 keeps every launch on the context's stream, in program
 * order. Results are identical either way (every reduction sums in a fixed
 * order, and the resblock outputs are summed in one order). */
int kdec_model_set_overlap(kdec_model* m, int on);
/* on = 1 (with overlap on and N >= 2): forwards run the batch as two
 * halves (rows [0, N - N/2) and the rest), each a whole backbone + generator
 * chain on its own stream, concurrently, and so do their backwards (the
 * second half's conv weight grads accumulate in a second buffer that is
 * added at the end). 0 (the default) keeps one chain for the whole batch.
 * On one MI355X at B = 8, T = 512 the halves lengthen the backward with
 * weight grads (the concurrent weight-grad GEMMs contend), and the one-chain
 * forward already runs its resblocks on three streams, so the training step
 * keeps one chain. Results agree either way to the rounding of the GEMMs' split
 * choices. No counterpart in the reference (its decoder runs one utterance
 * at a time); the per-utterance work is unchanged. */
int kdec_model_set_batch_split(kdec_model* m, int on);
/* DecoderLora's adapters on every AdaIN unit (the adapter contract of
 * decoder_lora.h:63-77; the adapter_fwd / adapter_bwd sequence of
 * decoder_lora.cpp:184-207): (gamma, beta) = fc(style) + scale * B_i (g *
 * (A_i style)) for unit i. rank > 0 allocates A (units*rank, style_dim; unit
 * i's rows i*rank..) and B (affine_rows, rank; unit i's rows at its affine
 * offset), both zero, and their grads; forwards then need a gate
 * (kdec_model_lora_gate) and every backward accumulates dA and dB. */
int kdec_model_lora_enable(kdec_model* m, int rank, float scale);
/* Device pointers: which 0 = A, 1 = B, 2 = dA, 3 = dB (kdec_model_zero_grad
 * clears dA and dB); NULL before kdec_model_lora_enable. */
float* kdec_model_lora_ptr(kdec_model* m, int which);
/* The gate for the following forwards: g (device, N x rank at batch stride
 * g_bs; g_bs = 0: one gate for every utterance). Backwards accumulate the
 * gate grad into dG (device, same layout) when it is not NULL. The caller
 * keeps both alive. */
int kdec_model_lora_gate(kdec_model* m, const float* g, long g_bs, float* dG);

/* ─── DecoderLora (decoder_lora.h:97-181, decoder_lora.cpp:108-396) ───
 * The trainable LoRA over every AdaIN unit's style projection with the
 * shared conditioning gate g(v) = W2 tanh(W1 v) (in_dim 3, hidden 16,
 * rank wide), Adam state and the ELRA1 checkpoint, over this model's frozen
 * weights: DecoderLora::make / forward / backward / zero_grad / adam_step /
 * save / load. Units are in kdec_model_unit_name order. Errors read through
 * kdec_last_error of the model's context. */
typedef struct kdec_dlora kdec_dlora;
/* A, B Glorot-uniform from `seed`, gate W2 zero (the base decoder exactly
 * at init and for cond = 0). */
int kdec_dlora_create(kdec_model* m, int rank, float scale, unsigned long long seed, kdec_dlora** out);
int kdec_dlora_destroy(kdec_dlora* d);
/* DecoderLora::forward over the model's weights: device pointers, N
 * utterances; ref_s (N rows at stride ref_bs >= style_dim, the style is the
 * first style_dim values), cond (N, 3), har (N, (n_fft+2)*frames) or NULL
 * to run the model's harmonic source on F0; audio (N, audio_len). */
int kdec_dlora_forward(kdec_dlora* d, int N, int T, const float* asr, const float* F0, const float* Nn,
                       const float* ref_s, long ref_bs, const float* har, const float* cond, float* audio);
/* DecoderLora::backward of the last forward (its cond): accumulates dA, dB,
 * the gate's dW1, dW2. */
int kdec_dlora_backward(kdec_dlora* d, const float* daudio);
int kdec_dlora_zero_grad(kdec_dlora* d);
int kdec_dlora_adam_step(kdec_dlora* d, float lr, float beta1, float beta2, float eps);
int kdec_dlora_save(kdec_dlora* d, const char* path);
int kdec_dlora_load(kdec_dlora* d, const char* path);
/* Device tensors: 0 A (units*rank, S), 1 B (affine_rows, rank), 2 dA, 3 dB,
 * 4 gate W1 (16, 3), 5 W2 (rank, 16), 6 dW1, 7 dW2; shape in rows, cols. */
float* kdec_dlora_ptr(kdec_dlora* d, int which, int* rows, int* cols);
float kdec_dlora_scale(const kdec_dlora* d);

/* The producer step of Kokoro::prepare_decode_context after the predictor
 * (kokoro.cpp:667-732; KokoroDecodePrep, kokoro.h:133-147) for one
 * utterance: t_en (device, asr_dim x L text-encoder features), pred_dur
 * (host, L per-phoneme frame counts), F0_pred / N_pred (device, 2*total
 * each; may be NULL where an override is given), F0_override / N_override
 * (host, 2*total values each, or NULL) and ref_s (device, 2*style_dim).
 * Builds asr (length regulation on the device), the F0 / N grids and the
 * harmonic source. Errors (KDEC_EINVAL, the reference's messages): total
 * frame count 0 ("predicted total frame count is 0"), an override of the
 * wrong size ("F0 override size must be 2*total (n)"), a harmonic-source
 * frame count other than 2*total * prod(upsample rates) + 1, negative
 * durations. The prep owns its tensors until kdec_prep_destroy; the model
 * must outlive it. */
typedef struct kdec_prep kdec_prep;
int kdec_model_decode_prep(kdec_model* m, const float* t_en, int L, const int* pred_dur, const float* F0_pred,
                           const float* N_pred, const float* F0_override, long F0_override_n,
                           const float* N_override, long N_override_n, const float* ref_s, kdec_prep** out);
int kdec_prep_destroy(kdec_prep* p);
int kdec_prep_total(const kdec_prep* p);
int kdec_prep_frames(const kdec_prep* p);
/* The DecoderLoraContext view (kokoro.cpp:604-614): which 0 asr (asr_dim *
 * total), 1 F0 (2*total), 2 N (2*total), 3 har ((n_fft+2) * frames), 4 ref_s. */
const float* kdec_prep_ptr(const kdec_prep* p, int which);

/* Leaky-ReLU sites of the decoder, in the order the forward visits them:
 * per AdaIN residual block (encode, decode.0, ...) the norm1 output and the
 * norm2 output (slope 0.2, kokoro_decoder_backward.cpp:172, 190), per
 * generator stage the stage input (0.1, :613), then the spectral head input
 * (0.01, :388). These are the decoder's only non-smooth points.
 * kdec_model_leaky_input copies site `site`'s input (the value whose sign
 * picks the slope, as the backward evaluates it) of the last training
 * forward to host: N rows of C*L floats, n = N*C*L. An inspection aid in the
 * spirit of the reference's KokoroTrace (kokoro.h): two float
 * implementations can disagree on the sign of an input within rounding of
 * zero, and a comparison of their grads needs to know where. */
int kdec_model_leaky_site_count(const kdec_model* m);
/* N*C*L of site `site` after the last training forward, or -1. */
long kdec_model_leaky_size(kdec_model* m, int site);
int kdec_model_leaky_input(kdec_model* m, int site, float* host, long n);
/* The same sites of the last kdec_dlora_forward (the DecoderLora's own
 * caches and adapted affines). */
long kdec_dlora_leaky_size(kdec_dlora* d, int site);
int kdec_dlora_leaky_input(kdec_dlora* d, int site, float* host, long n);

/* Device pointers to the last forward's har (N, (n_fft+2)*frames) and
 * generator input (N, init_C * L_gen). */
const float* kdec_model_har(const kdec_model* m);
const float* kdec_model_gen_in(const kdec_model* m);

#ifdef __cplusplus
}
#endif

#endif /* KDEC_MODEL_H */

/*
 * kdec.h — C ABI of the MI355X (gfx950) Kokoro-82M iSTFTNet decoder kernels.
 *
 * The reference (wlejon/brosoundml) drives the decoder back half through
 * brotensor ops from src/kokoro_decoder_backward.cpp. Each entry point below
 * replaces one such op or a fused group of them; the comment on each names
 * the reference call sites it stands in for (paths relative to the reference
 * repository). The C++ drop-in layer (kokoro_decoder_backward.h in this
 * project) calls these; so do the ctypes tests and the benchmark.
 *
 * Conventions
 *  - Every pointer argument named like a tensor is a DEVICE pointer to FP32
 *    data. Activations are batched NCL: utterance n, channel c, sample l at
 *    n * bs + c * L + l, where `bs` is the batch stride in elements (bs >= C*L;
 *    a larger stride addresses a channel slice of a wider tensor, which is how
 *    channel concatenation and slicing are expressed without copies).
 *  - Weight layouts are the reference's (include/brosoundml/modules.h:14-21,
 *    kokoro_modules.h): Conv1d W (C_out, C_in*k) index [co][ci*k+t];
 *    ConvTranspose1d W (C_in, C_out*k) index [ci][co*k+t]; depthwise pool
 *    W (C, 3); biases (C_out).
 *  - Per-utterance affines: gamma/beta hold N rows of C values at row stride
 *    `gb_bs` (0 broadcasts one row to every utterance).
 *  - Every call is asynchronous on the context's stream and returns 0 on
 *    success or a negative KDEC_E* code; kdec_last_error() gives the message.
 *    Output buffers are caller-allocated; the library allocates only its own
 *    workspace (split-K partials, packed weights, statistics).
 *  - Grad outputs documented as "accumulated" are added to (caller zeroes
 *    them); all others are overwritten.
 */
#ifndef KDEC_H
#define KDEC_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KDEC_OK 0
#define KDEC_EINVAL -1   /* bad argument / shape */
#define KDEC_EHIP -2     /* HIP runtime error */
#define KDEC_ENOMEM -3   /* device allocation failed */

typedef struct kdec_ctx kdec_ctx;

/* Activation applied after an AdaIN affine. */
#define KDEC_ACT_NONE 0
#define KDEC_ACT_LEAKY 1 /* leaky_relu(slope)             (bt::leaky_relu_*) */
#define KDEC_ACT_SNAKE 2 /* x + sin^2(alpha_c x)/alpha_c  (bt::snake_*)      */

/* ─── context ─────────────────────────────────────────────────────────── */

/* Creates a context on HIP device `device` with a default-priority stream of
 * its own. No reference counterpart (brotensor's runtime is implicit). */
int kdec_ctx_create(int device, kdec_ctx** out);
int kdec_ctx_destroy(kdec_ctx* ctx);
/* Last error message of this context ("" if none). */
const char* kdec_last_error(const kdec_ctx* ctx);
/* Runs subsequent work on `stream` (a hipStream_t; NULL = the HIP null
 * stream). Until the first call the context uses a stream of its own. */
int kdec_set_stream(kdec_ctx* ctx, void* stream);
void* kdec_get_stream(const kdec_ctx* ctx);
int kdec_synchronize(kdec_ctx* ctx);
/* Device memory from the context's stream-ordered caching allocator. */
int kdec_malloc(kdec_ctx* ctx, size_t bytes, void** out);
int kdec_free(kdec_ctx* ctx, void* ptr);
/* Per-kernel-family timing with HIP events on the context stream (0 = off). */
int kdec_profile_enable(kdec_ctx* ctx, int on);
/* Fills names / ms / launches / algorithmic FLOP / algorithmic HBM bytes
 * (any may be NULL) for up to `cap` families; returns the count. */
int kdec_profile_read(kdec_ctx* ctx, const char** names, double* ms,
                      long* launches, double* flops, double* bytes, int cap);
int kdec_profile_reset(kdec_ctx* ctx);

/* ─── convolutions (implicit GEMM on FP32 MFMA) ───────────────────────── */

/* Y = scale * (conv1d(X, W) + bias + R) + beta * Y
 * Replaces bt::conv1d via Conv1d::forward (src/modules.cpp:103-108) at
 * kokoro_decoder_backward.cpp:185,193,199,307,316,389,502-504,617, with the
 * residual add / scale that follow it (:204-205, :319, :642, :654-656) fused.
 * bias, R may be NULL. L_out = (L + 2p - d(k-1) - 1)/s + 1. groups = 1. */
int kdec_conv1d_fwd(kdec_ctx* ctx, const float* X, long x_bs, const float* W,
                    const float* bias, float* Y, long y_bs, int N, int C_in,
                    int L, int C_out, int k, int stride, int pad, int dil,
                    const float* R, long r_bs, float scale, float beta);

/* kdec_conv1d_fwd (beta = 0) that also writes the instance-norm statistics
 * of its output rows, stats[n*C_out + c] = (mean, 1/sqrt(var + eps)) as
 * kdec_instnorm_stats computes them. Where the GEMM runs the quad-packed
 * kernel, its epilogue records each tile's per-row count, mean and squared
 * deviations and a wave per row merges them (in double), so Y is not read
 * again; elsewhere it is the two calls. For the conv outputs that feed an
 * AdaIN (kokoro_decoder_backward.cpp:307-313, the ResBlock1 convs whose
 * output the next adain_affine_forward normalises, :100-120). */
int kdec_conv1d_fwd_stats(kdec_ctx* ctx, const float* X, long x_bs,
                          const float* W, const float* bias, float* Y,
                          long y_bs, int N, int C_in, int L, int C_out, int k,
                          int stride, int pad, int dil, const float* R,
                          long r_bs, float scale, float eps, float* stats);
/* 1 where kdec_conv1d_fwd_stats takes the fused path for this geometry, else
 * 0 (a caller may then prefer the one-pass kdec_adain_act_fwd_stats). */
int kdec_conv1d_fwd_stats_fused(kdec_ctx* ctx, int N, int C_in, int L,
                                int C_out, int k, int stride, int pad,
                                int dil);

/* dX = scale * conv1d_backward_input(W, dY) + beta * dX   (stride 1)
 * Replaces bt::conv1d_backward_input at kokoro_decoder_backward.cpp:230-234,
 * 244-248, 271-275, 347-350, 360-363, 453-456. L is the input length. */
int kdec_conv1d_dgrad(kdec_ctx* ctx, const float* W, const float* dY,
                      long dy_bs, float* dX, long dx_bs, int N, int C_in,
                      int L, int C_out, int k, int stride, int pad, int dil,
                      float scale, float beta);

/* The input grad of a stride-1 conv1d followed by the backward of the
 * AdaIN + activation whose output feeds that conv:
 *   dX = kdec_adain_act_bwd(X, ..., dY' = conv1d_dgrad(W, dY)) (+ R)
 * with dgamma / dbeta overwritten and dalpha accumulated, as the two calls
 * kdec_conv1d_dgrad + kdec_adain_act_bwd (same arguments). Where the GEMM
 * runs the quad-packed kernel, its epilogue applies the activation
 * derivative and forms the AdaIN's per-row partial sums, so dY' is never
 * written separately and the AdaIN pass reads it once; elsewhere it makes
 * those two calls. dX must not alias X or R.
 * Replaces bt::conv1d_backward_input followed by bt::snake_backward and
 * adain_affine_backward at kokoro_decoder_backward.cpp:347-356 and :360-369
 * (leaky: :230-241, :244-266). */
int kdec_conv1d_dgrad_adain_bwd(kdec_ctx* ctx, const float* W, const float* dY,
                                long dy_bs, int N, int C_in, int L, int C_out,
                                int k, int stride, int pad, int dil,
                                const float* X, long x_bs, const float* stats,
                                const float* gamma, const float* beta,
                                long gb_bs, int act, float slope,
                                const float* alpha, const float* R, long r_bs,
                                float* dX, long dx_bs, float* dgamma,
                                float* dbeta, long dgb_bs, float* dalpha);

/* dW (C_out, C_in*k) and db (C_out) accumulated over the batch; either may
 * be NULL.
 * Extension: the reference freezes conv weights; the signature of
 * its accumulating bt::conv1d_backward_weight/_bias is the one used in
 * src/bc_resnet.cpp:1006-1007, 1020-1025. */
int kdec_conv1d_wgrad(kdec_ctx* ctx, const float* X, long x_bs,
                      const float* dY, long dy_bs, float* dW, float* db, int N,
                      int C_in, int L, int C_out, int k, int stride, int pad,
                      int dil);

/* Y = convT(X, W) + bias (groups = 1, dilation 1, output_padding op).
 * Replaces bt::conv_transpose1d_forward at kokoro_decoder_backward.cpp:627-629
 * (ups). Polyphase implicit GEMM. */
int kdec_convt1d_fwd(kdec_ctx* ctx, const float* X, long x_bs, const float* W,
                     const float* bias, float* Y, long y_bs, int N, int C_in,
                     int L, int C_out, int k, int stride, int pad, int op);
/* The generator's last upsample stage in one pass (kokoro_decoder_backward.cpp
 * :627-642): Y = reflection_pad_left1(convT(X, W) + bias) + R, i.e. with
 * pad_left = 1 each output row is L_out + 1 long, column j + 1 holds the
 * transposed conv's column j and column 0 its column 1, and R (the noise
 * source, Y's layout and length, or NULL) is added to every column; with
 * pad_left = 0, Y = convT(X, W) + bias + R. Same polyphase GEMM as
 * kdec_convt1d_fwd, with the pad and the add in its epilogue. */
int kdec_convt1d_fwd_res(kdec_ctx* ctx, const float* X, long x_bs, const float* W, const float* bias, float* Y,
                         long y_bs, int N, int C_in, int L, int C_out, int k, int stride, int pad, int op,
                         const float* R, long r_bs, int pad_left);
/* dX = conv_transpose1d_backward_input(W, dY) (= strided conv1d of dY with W).
 * Replaces bt::conv_transpose1d_backward_input at :725-728. */
int kdec_convt1d_dgrad(kdec_ctx* ctx, const float* W, const float* dY,
                       long dy_bs, float* dX, long dx_bs, int N, int C_in,
                       int L, int C_out, int k, int stride, int pad, int op);
/* dW (C_in, C_out*k), db (C_out) accumulated. Extension of the reference. */
int kdec_convt1d_wgrad(kdec_ctx* ctx, const float* X, long x_bs,
                       const float* dY, long dy_bs, float* dW, float* db,
                       int N, int C_in, int L, int C_out, int k, int stride,
                       int pad, int op);

/* Depthwise ConvTranspose1d k3 s2 p1 op1 (the upsampling block's pool):
 * replaces bt::conv_transpose1d_forward / _backward_input with groups = C at
 * kokoro_decoder_backward.cpp:176-180, 252-256. L_out = 2L. */
int kdec_pool_fwd(kdec_ctx* ctx, const float* X, long x_bs, const float* W,
                  const float* bias, float* Y, long y_bs, int N, int C, int L);
int kdec_pool_dgrad(kdec_ctx* ctx, const float* W, const float* dY,
                    long dy_bs, float* dX, long dx_bs, int N, int C, int L);
/* dW (C,3), db (C) accumulated. Extension of the reference. */
int kdec_pool_wgrad(kdec_ctx* ctx, const float* X, long x_bs, const float* dY,
                    long dy_bs, float* dW, float* db, int N, int C, int L);

/* ─── AdaIN (instance norm + style affine) fused with its activation ───── */

/* Per-(n,c) mean and 1/sqrt(biased var + eps) over L (G = C group norm).
 * Replaces the statistics half of bt::group_norm_forward at
 * kokoro_decoder_backward.cpp:112-113. stats: N*C (mean, rstd) pairs. */
int kdec_instnorm_stats(kdec_ctx* ctx, const float* X, long x_bs, int N,
                        int C, int L, float eps, float* stats);

/* Y = act((1 + gamma) * (X - mean) * rstd + beta); Ypre (optional) gets the
 * pre-activation. Replaces adain_affine_forward (:100-120: group_norm,
 * nchw_to_sequence, modulate, sequence_to_nchw) plus the following
 * bt::leaky_relu_forward (:172, :190) or bt::snake_forward (:305-306,
 * :313-314). slope for LEAKY; alpha (C) for SNAKE. beta may be NULL (zero). */
int kdec_adain_act_fwd(kdec_ctx* ctx, const float* X, long x_bs,
                       const float* stats, const float* gamma,
                       const float* beta, long gb_bs, int act,
                       float slope, const float* alpha, float* Y, long y_bs,
                       float* Ypre, long ypre_bs, int N, int C, int L);

/* Statistics and the affine + activation in one pass: stats (N*C (mean,
 * rstd) pairs, as kdec_instnorm_stats) are written and used at once. Short
 * rows are held in registers, so x is read once (the two-call sequence reads
 * it twice); longer rows take the two passes. Replaces the
 * group_norm + modulate + activation sequence of kokoro_decoder_backward.cpp
 * :100-120 with :172/:190 (leaky) or :305-306/:313-314 (snake). */
int kdec_adain_act_fwd_stats(kdec_ctx* ctx, const float* X, long x_bs,
                             float eps, float* stats, const float* gamma,
                             const float* beta, long gb_bs, int act,
                             float slope, const float* alpha, float* Y,
                             long y_bs, float* Ypre, long ypre_bs, int N,
                             int C, int L);

/* Backward of kdec_adain_act_fwd given dY (grad at the activation output):
 *   dX = adain_backward(act_backward(dY)) + (R ? R : 0)
 *   dgamma/dbeta (N*C at gb_bs rows) overwritten; dalpha (C) accumulated
 *   over the batch when non-NULL (SNAKE only).
 * Replaces bt::leaky_relu_backward / bt::snake_backward followed by
 * adain_affine_backward (:237+240-241, :262+265-266, :352-356, :365-369);
 * R carries the residual skip added at :372. beta may be NULL for ACT_NONE
 * (adain_affine_backward takes no beta). */
int kdec_adain_act_bwd(kdec_ctx* ctx, const float* X, long x_bs,
                       const float* stats, const float* gamma,
                       const float* beta, long gb_bs, int act, float slope,
                       const float* alpha, const float* dY, long dy_bs,
                       const float* R, long r_bs, float* dX, long dx_bs,
                       float* dgamma, float* dbeta, long dgb_bs,
                       float* dalpha, int N, int C, int L);

/* kdec_adain_act_bwd without any allocation: same arguments, kernels and
 * results. No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Its scratch lives in a device array of
 * KDEC_NOALLOC_SCRATCH_BYTES per GPU: the per-row alpha-grad shares (4 B per
 * row, with dalpha when N > 1 or the rows take the chunked passes) and, for
 * rows that no one-block row kernel holds (longer than 62464, or longer than
 * 49152 when a row does not start on 16 B), the chunk partial sums and row
 * means (24 B per row and 4096-sample chunk, plus 8 B per row). The array is
 * held until the process ends; a call that needs more returns
 * KDEC_EINVAL with the sizes in kdec_last_error. It calls no hipMalloc /
 * hipFree and records no profiling events. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (any two streams or
 * contexts) race and must be serialised by the caller. */
#define KDEC_NOALLOC_SCRATCH_BYTES (4 << 20)
int kdec_adain_act_bwd_noalloc(kdec_ctx* ctx, const float* X, long x_bs,
                               const float* stats, const float* gamma,
                               const float* beta, long gb_bs, int act,
                               float slope, const float* alpha,
                               const float* dY, long dy_bs, const float* R,
                               long r_bs, float* dX, long dx_bs,
                               float* dgamma, float* dbeta, long dgb_bs,
                               float* dalpha, int N, int C, int L);

/* ─── elementwise ─────────────────────────────────────────────────────── */

/* Y[i] = value for i < n (a kernel, not hipMemset, so it can be captured). */
int kdec_fill(kdec_ctx* ctx, float* Y, long n, float value);

/* Y = leaky_relu(X, slope) over N rows of `len` (bt::leaky_relu_forward). */
int kdec_leaky_fwd(kdec_ctx* ctx, const float* X, long x_bs, float* Y,
                   long y_bs, int N, long len, float slope);
/* dX = (X > 0 ? 1 : slope) * dY (bt::leaky_relu_backward, :613/731 0.1). */
int kdec_leaky_bwd(kdec_ctx* ctx, const float* X, long x_bs, const float* dY,
                   long dy_bs, float* dX, long dx_bs, int N, long len,
                   float slope);
/* kdec_leaky_bwd followed by a scaling pass, in one: dX = scale * ((X > 0 ?
 * 1 : slope) * dY), the same two roundings. The generator's backward, whose
 * stage output grad is divided by the K resblocks right after a leaky
 * backward forms it (kokoro_decoder_backward.cpp:457 and :731, then
 * :689-690). */
int kdec_leaky_bwd_scaled(kdec_ctx* ctx, const float* X, long x_bs, const float* dY, long dy_bs, float* dX,
                          long dx_bs, int N, long len, float slope, float scale);
/* Y = a*A + b*B (B may be NULL) over N rows of `len` (bt::add_inplace /
 * bt::scale_inplace, copy_d2d for concat / slice). */
int kdec_axpby(kdec_ctx* ctx, float a, const float* A, long a_bs, float b,
               const float* B, long b_bs, float* Y, long y_bs, int N,
               long len);
/* Y = (A + B) + C over N rows of `len`, the float adds in that order (Y may
 * alias A). The generator stage's resblock sum (kokoro_decoder_backward.cpp:
 * 644-657, xs = x0; xs += x1; xs += x2) when the K = 3 resblocks run on
 * concurrent streams into separate buffers, each with the 1/K already applied
 * by its last conv: the same two roundings as the one-stream schedule, whose
 * last convs accumulate into one buffer in that order. */
int kdec_add3(kdec_ctx* ctx, const float* A, long a_bs, const float* B,
              long b_bs, const float* C, long c_bs, float* Y, long y_bs,
              int N, long len);
/* kdec_add3 that also writes Z = leaky_relu(Y, slope) (Y may alias A): the
 * generator stage's resblock sum (kokoro_decoder_backward.cpp:645-655) and
 * the activation the next stage's transposed conv (slope 0.1, :613) or
 * conv_post (0.01, :388) reads. */
int kdec_add3_leaky(kdec_ctx* ctx, const float* A, long a_bs, const float* B, long b_bs, const float* C, long c_bs,
                    float* Y, long y_bs, float* Z, long z_bs, int N, long len, float slope);
/* kdec_add3 over N x C rows of L + 1 that also writes the left reflect
 * pad's adjoint in the same pass (the generator's last stage backward,
 * :716-728): Y = (A + B) + C (as kdec_add3), and Z (rows of L) = the
 * gradient of the unpadded rows, Z[j] = Y[j + 1] + (j == 1 ? Y[0] : 0), the
 * bits kdec_pad_reflect_left1_bwd(Y) gives. Y may alias A; Z aliases
 * none of the others. */
int kdec_add3_unpad_left1(kdec_ctx* ctx, const float* A, long a_bs, const float* B, long b_bs, const float* C,
                          long c_bs, float* Y, long y_bs, float* Z, long z_bs, int N, int Cn, int L);
/* Left reflect pad by one sample, C rows of L -> L+1 (bt::pad1d_* mode 1 at
 * :633-634 / :720-721). */
int kdec_pad_reflect_left1_fwd(kdec_ctx* ctx, const float* X, long x_bs,
                               float* Y, long y_bs, int N, int C, int L);
int kdec_pad_reflect_left1_bwd(kdec_ctx* ctx, const float* dY, long dy_bs,
                               float* dX, long dx_bs, int N, int C, int L);
/* Nearest 2x along L (:63-96, the host round trip in the reference). */
int kdec_nearest2x_fwd(kdec_ctx* ctx, const float* X, long x_bs, float* Y,
                       long y_bs, int N, int C, int L);
/* dX = scale * (dY[2l] + dY[2l+1]) + beta * dX */
int kdec_nearest2x_bwd(kdec_ctx* ctx, const float* dY, long dy_bs, float* dX,
                       long dx_bs, int N, int C, int L, float scale,
                       float beta);

/* ─── spectral head, iSTFT, harmonic source, style projection ─────────── */

/* audio = istft(complex_from_polar(exp(post[:F]), sin(post[F:]))), center,
 * not normalized, periodic Hann of length n_fft, hop `hop`; post (N, 2F, L)
 * with F = n_fft/2+1; audio (N, (L-1)*hop). Replaces the host exp/sin, the
 * bt::complex_from_polar and bt::istft of kokoro_decoder_backward.cpp:391-409. */
int kdec_spectral_fwd(kdec_ctx* ctx, const float* post, long post_bs,
                      const float* window, float* audio, long audio_bs, int N,
                      int L, int n_fft, int hop);
/* dpost from daudio: bt::istft_backward and the host polar/exp/sin adjoint at
 * kokoro_decoder_backward.cpp:423-449. `window` (n_fft values, device) may be
 * NULL for the periodic Hann window in both calls. */
int kdec_spectral_bwd(kdec_ctx* ctx, const float* post, long post_bs,
                      const float* window, const float* daudio,
                      long daudio_bs, float* dpost, long dpost_bs, int N,
                      int L, int n_fft, int hop);

/* HarmonicSource::forward (kokoro_modules.cpp:1574-1665) for N utterances:
 * F0 (N, frame_count) -> har (N, n_fft+2, frame_count*upsample_scale/hop+1).
 * The phase recurrence runs sequentially per (utterance, harmonic) in float
 * exactly as the reference's host loop; sin / l_linear / tanh / STFT /
 * abs / atan2 run in parallel. lW (harmonic_num+1), lb (1) device pointers. */
int kdec_harmonic_source(kdec_ctx* ctx, const float* F0, long f0_bs,
                         float* har, long har_bs, int N, int frame_count,
                         const float* lW, const float* lb, int harmonic_num,
                         int sample_rate, int upsample_scale, int n_fft,
                         int hop);

/* Style projection for a group of AdaIN units stacked row-wise:
 * out[n, r] = W[r, :] . style[n, :] + b[r] for r < rows (W rows x S).
 * Replaces compute_style_affine (kokoro_modules.cpp:563-572) /
 * bt::lora_forward with the LoRA term absent (decoder_lora.cpp:184-194). */
int kdec_style_proj_fwd(kdec_ctx* ctx, const float* W, const float* b,
                        const float* style, long style_bs, float* out,
                        long out_bs, int N, int rows, int S);
/* dstyle[n, :] = beta*dstyle + sum_r W[r, :] dout[n, r]  (dstyle may be NULL);
 * dW += sum_n dout[n, r] style[n, :]; db += sum_n dout[n, r] (may be NULL).
 * The adjoint of bt::lora_backward with dX requested
 * (decoder_lora.cpp:198-207); the reference passes dX = nullptr. */
int kdec_style_proj_bwd(kdec_ctx* ctx, const float* W, const float* style,
                        long style_bs, const float* dout, long dout_bs,
                        float* dstyle, long dstyle_bs, float beta, float* dW,
                        float* db, int N, int rows, int S);

/* LoRA-adapted style projection (DecoderLora's adapter_fwd,
 * decoder_lora.cpp:184-194, over bt::lora_forward; the adapter contract of
 * decoder_lora.h:63-77): for `units` AdaIN units stacked row-wise, unit u
 * owning rows [unit_off[u], unit_off[u+1]) (unit_off: units+1 ints, device),
 *   H[n, u*rank + j] = A[u*rank + j, :] . style[n, :]
 *   out[n, r] = W[r, :] . style[n, :] + b[r]
 *               + scale * sum_j B[r, j] * g[n, j] * H[n, u(r)*rank + j]
 * A (units*rank, S), B (rows, rank), g the gate (N, rank) at batch stride
 * g_bs (0: one gate for every utterance). H (N, units*rank) is written for
 * the backward. */
int kdec_lora_proj_fwd(kdec_ctx* ctx, const float* W, const float* b,
                       const float* A, const float* B, const float* g,
                       long g_bs, float scale, const int* unit_off, int units,
                       int rank, const float* style, long style_bs, float* H,
                       float* out, long out_bs, int N, int rows, int S);
/* Its adjoint (adapter_bwd, decoder_lora.cpp:198-207, over bt::lora_backward)
 * plus the d(style) extension. With dHG[n, u*rank+j] = scale * sum_{r in u}
 * B[r, j] dout[n, r]:
 *   dB[r, j] += scale * sum_n dout[n, r] g[n, j] H[n, u(r)*rank + j]
 *   dG[n, j] += sum_u dHG[n, u*rank+j] H[n, u*rank+j]   (summed over n when g_bs = 0)
 *   dA[u*rank+j, :] += sum_n dHG[n, u*rank+j] g[n, j] style[n, :]
 *   dstyle[n, :] = beta*dstyle + W^T dout[n] + A^T (dHG g)[n]
 *   dW, db as kdec_style_proj_bwd.
 * Any of dstyle, dW, db, dA, dB, dG may be NULL. */
int kdec_lora_proj_bwd(kdec_ctx* ctx, const float* W, const float* A,
                       const float* B, const float* g, long g_bs, float scale,
                       const int* unit_off, int units, int rank,
                       const float* style, long style_bs, const float* H,
                       const float* dout, long dout_bs, float* dstyle,
                       long dstyle_bs, float beta, float* dW, float* db,
                       float* dA, float* dB, float* dG, int N, int rows, int S);

/* DecoderLora's conditioning gate g(v) = W2 tanh(W1 v), bias-free
 * (ConditioningGate::forward, decoder_lora.cpp:56-66): for N condition
 * vectors v (in_dim each, batch stride v_bs) writes act = tanh(W1 v)
 * (N, hidden; kept for the backward) and g (N, rank) at batch stride g_bs.
 * W1 (hidden, in_dim), W2 (rank, hidden). N * hidden <= 16384. */
int kdec_lora_gate_fwd(kdec_ctx* ctx, const float* W1, const float* W2,
                       const float* v, long v_bs, int N, int in_dim,
                       int hidden, int rank, float* act, float* g,
                       long g_bs);
/* Its adjoint (ConditioningGate::backward, decoder_lora.cpp:68-80): with the
 * forward's act and the gate grad dG (N, rank at batch stride dg_bs),
 * accumulates dW2 += dG^T act and dW1 += ((1 - act^2) * (dG W2))^T v. The
 * condition is an input, not a trainable: no dv. */
int kdec_lora_gate_bwd(kdec_ctx* ctx, const float* W2, const float* v,
                       long v_bs, const float* act, const float* dG,
                       long dg_bs, int N, int in_dim, int hidden, int rank,
                       float* dW1, float* dW2);
/* One Adam step over n parameters (bt::adam_step as DecoderLora::adam_step
 * calls it, decoder_lora.cpp:305-314): m = b1 m + (1-b1) g,
 * v = b2 v + (1-b2) g^2, p -= lr (m / (1 - b1^step)) /
 * (sqrt(v / (1 - b2^step)) + eps). step >= 1. */
int kdec_adam_step(kdec_ctx* ctx, float* p, const float* g, float* m,
                   float* v, long n, float lr, float beta1, float beta2,
                   float eps, int step);

/* Length regulation (the host loop of Kokoro::prepare_decode_context /
 * synthesize, kokoro.cpp:667-689): asr[n, c, t] = t_en[n, c, l] for the
 * phoneme l whose duration run covers frame t (runs in token order,
 * negative durations count as zero), zero for t >= the utterance's total.
 * t_en (N, C, L) at batch stride te_bs, dur (N, L) int32 (device) at dur_bs,
 * asr (N, C, T) at asr_bs; totals (N int32, device) receives each total
 * when not NULL. L <= 4096. */
int kdec_length_regulate(kdec_ctx* ctx, const float* t_en, long te_bs,
                         const int* dur, long dur_bs, int N, int C, int L,
                         float* asr, long asr_bs, int T, int* totals);

#ifdef __cplusplus
}
#endif

#endif /* KDEC_H */

// Spectral head (polar exp/sin -> iSTFT) forward and adjoint, the harmonic
// source, and the style projection (gamma, beta) = fc(style) with its adjoint.
//
// iSTFT semantics (center, not normalized, onesided; torch.istft): frame f
// contributes window * irfft(spec[f]) at offset f*hop, the overlap-add is
// divided by the summed squared window and the first n_fft/2 samples are
// dropped. irfft ignores the imaginary parts of the DC and Nyquist bins.
// The transforms are n_fft = 20 direct sums with twiddles staged in LDS:
// far too small for an FFT to pay, and direct sums keep the order fixed.
#include "kdec_buffer.hpp"
#include "kdec_internal.hpp"
#include "kdec_snake_math.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <vector>

namespace kdec {
namespace {

constexpr int MAXN = 64;  // largest n_fft supported by the LDS tables
constexpr int FT = 256;   // frames per block

__device__ inline float hann_at(int n, int N) {
    // periodic Hann in float arithmetic (kokoro_decoder_backward.cpp:580-588)
    const float kTwoPi = 6.28318530717958647692f;
    return 0.5f - 0.5f * cosf(kTwoPi * static_cast<float>(n) / static_cast<float>(N));
}

// Twiddles cos/sin(2*pi*k*n/N) for k < F, n < N (exact reduction of k*n mod N)
// and the window (periodic Hann when `window` is null).
__device__ inline void load_twiddles(float* tc, float* ts, float* win, int N, int F,
                                     const float* window) {
    for (int i = threadIdx.x; i < F * N; i += blockDim.x) {
        const int k = i / N, n = i - k * N;
        const int r = (k * n) % N;
        double sv, cv;
        sincospi(2.0 * r / N, &sv, &cv);
        tc[i] = static_cast<float>(cv);
        ts[i] = static_cast<float>(sv);
    }
    for (int n = threadIdx.x; n < N; n += blockDim.x) win[n] = window ? window[n] : hann_at(n, N);
}

// Squared-window overlap at ola position m (frames 0..frames-1, hop).
__device__ inline float env_at(const float* win, int m, int N, int hop, int frames) {
    int f_hi = m / hop;
    if (f_hi > frames - 1) f_hi = frames - 1;
    float e = 0.0f;
    for (int f = f_hi; f >= 0 && m - f * hop < N; --f) {
        const float w = win[m - f * hop];
        e += w * w;
    }
    return e;
}

// Per (n, frame): polar spectrum -> windowed irfft frame (N samples). NM >=
// N bounds the per-lane arrays; their loops unroll fully so they stay in
// registers.
template <int NM>
__global__ __launch_bounds__(FT) void spec_frames_k(const float* post, long post_bs,
                                                   const float* window, float* fbuf, int L, int N) {
    __shared__ float tc[MAXN / 2 + 1][MAXN], ts[MAXN / 2 + 1][MAXN], win[MAXN];
    const int F = N / 2 + 1;
    load_twiddles(&tc[0][0], &ts[0][0], win, N, F, window);
    __syncthreads();
    // load_twiddles wrote F*N contiguous values; index them as [k*N + n]
    const float* TC = &tc[0][0];
    const float* TS = &ts[0][0];
    const int b = blockIdx.y;
    const int f = blockIdx.x * FT + threadIdx.x;
    if (f >= L) return;
    const float* P = post + b * post_bs;
    constexpr int FM = NM / 2 + 1;
    float re[FM], im[FM];
    float re_last = 0.0f;  // re[F - 1]
#pragma clang loop unroll(full)
    for (int k = 0; k < FM; ++k) {
        re[k] = im[k] = 0.0f;
        if (k < F) {
            const float mag = expf(P[static_cast<long>(k) * L + f]);
            const float ang = sinf(P[static_cast<long>(F + k) * L + f]);
            re[k] = mag * cosf(ang);
            im[k] = mag * sinf(ang);
            if (k == F - 1) re_last = re[k];
        }
    }
    float* out = fbuf + (static_cast<long>(b) * L + f) * N;
    const float invN = 1.0f / N;
    const int kmax = (N & 1) == 0 ? F - 1 : F;
    for (int n = 0; n < N; ++n) {
        float acc = re[0];
        if ((N & 1) == 0) acc += (n & 1) ? -re_last : re_last;
#pragma clang loop unroll(full)
        for (int k = 1; k < FM; ++k)
            if (k < kmax) acc += 2.0f * (re[k] * TC[k * N + n] - im[k] * TS[k * N + n]);
        out[n] = acc * invN * win[n];
    }
}

// Per output sample: overlap-add of <= ceil(N/hop) frames over the envelope.
__global__ void spec_ola_k(const float* fbuf, const float* window, float* audio, long audio_bs, int L,
                           int N, int hop, int sig_len) {
    __shared__ float win[MAXN];
    for (int n = threadIdx.x; n < N; n += blockDim.x) win[n] = window ? window[n] : hann_at(n, N);
    __syncthreads();
    const int b = blockIdx.y;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= sig_len) return;
    const int m = j + N / 2;
    int f_hi = m / hop;
    if (f_hi > L - 1) f_hi = L - 1;
    float acc = 0.0f, e = 0.0f;
    const float* fb = fbuf + static_cast<long>(b) * L * N;
    for (int f = f_hi; f >= 0 && m - f * hop < N; --f) {
        const int i = m - f * hop;
        acc += fb[static_cast<long>(f) * N + i];
        e += win[i] * win[i];
    }
    audio[b * audio_bs + j] = acc / e;
}

// Per (n, frame): adjoint of the frame's windowed irfft and of the polar map
// (NM >= N as in spec_frames_k).
template <int NM>
__global__ __launch_bounds__(FT) void spec_bwd_k(const float* post, long post_bs, const float* window,
                                                const float* daudio, long da_bs, float* dpost,
                                                long dp_bs, int L, int N, int hop) {
    __shared__ float tc[MAXN / 2 + 1][MAXN], ts[MAXN / 2 + 1][MAXN], win[MAXN];
    const int F = N / 2 + 1;
    load_twiddles(&tc[0][0], &ts[0][0], win, N, F, window);
    __syncthreads();
    const float* TC = &tc[0][0];
    const float* TS = &ts[0][0];
    const int b = blockIdx.y;
    const int f = blockIdx.x * FT + threadIdx.x;
    if (f >= L) return;
    const int sig_len = (L - 1) * hop;
    const float* dy = daudio + b * da_bs;
    float dfr[NM];
    const float invN = 1.0f / N;
#pragma unroll
    for (int n = 0; n < NM; ++n) {
        dfr[n] = 0.0f;
        if (n < N) {
            const int m = f * hop + n;
            const int j = m - N / 2;
            float v = 0.0f;
            if (j >= 0 && j < sig_len) v = dy[j] / env_at(win, m, N, hop, L);
            dfr[n] = v * win[n] * invN;
        }
    }
    const float* P = post + b * post_bs;
    float* D = dpost + b * dp_bs;
    for (int k = 0; k < F; ++k) {
        const bool edge = (k == 0) || ((N & 1) == 0 && k == F - 1);
        const float c = edge ? 1.0f : 2.0f;
        float re = 0.0f, im = 0.0f;
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            if (n < N) {
                re += dfr[n] * TC[k * N + n];
                im -= dfr[n] * TS[k * N + n];
            }
        }
        const float dRe = c * re;
        const float dIm = edge ? 0.0f : c * im;
        const float pm = P[static_cast<long>(k) * L + f];
        const float pp = P[static_cast<long>(F + k) * L + f];
        const float mag = expf(pm);
        const float ang = sinf(pp);
        const float ca = cosf(ang), sa = sinf(ang);
        const float dmag = dRe * ca + dIm * sa;
        const float dang = mag * (-dRe * sa + dIm * ca);
        D[static_cast<long>(k) * L + f] = dmag * mag;
        D[static_cast<long>(F + k) * L + f] = dang * cosf(pp);
    }
}

// ─── n_fft = 20, hop = 5 (the Kokoro head), specialised ───
// The same arithmetic as spec_frames_k / spec_ola_k / spec_bwd_k with the
// transform size known at compile time: every loop unrolls, the real DFT is
// folded on its symmetry (n and N - n share the cosine and negate the sine,
// so a bin's sums run over N/2 - 1 pairs), a frame's sin / cos of one angle
// come from one sincosf, and each block stages what its frames share in LDS:
// the forward keeps its frames (plus the K - 1 = N/H - 1 frames before them
// that overlap its samples) and overlap-adds them there, so no frame buffer
// goes through HBM; the backward stages dY / envelope over its frames'
// sample span once, so each sample's envelope is formed once per block.

// cos / sin(2 pi r / N), r < N, formed on the host in double and rounded to
// float (the values load_twiddles forms on the device), passed by value so
// that they sit in scalar registers
template <int N>
struct Tw {
    float c[N], s[N];
    float w[N];  // the periodic Hann window over N (the backward's frame weights)
};
template <int N>
Tw<N> make_tw() {
    Tw<N> t;
    for (int r = 0; r < N; ++r) {
        t.c[r] = static_cast<float>(std::cos(2.0 * M_PI * r / N));
        t.s[r] = static_cast<float>(std::sin(2.0 * M_PI * r / N));
        t.w[r] = static_cast<float>((0.5 - 0.5 * std::cos(2.0 * M_PI * r / N)) / N);
    }
    return t;
}

// e^x as 2^(x log2 e) on the hardware exp2, with log2 e split in two floats
// (hi = 1.44269502, lo = log2 e - hi) so that the rounding of x hi is
// carried: 2^t (1 + r ln 2) with t = fl(x hi), r = (x hi - t) + x lo. Within a
// few ulp for the log-magnitudes the head sees; about half the operations of
// the library expf.
__device__ inline float kdec_exp(float x) {
    const float t = x * 1.44269502f;
    const float r = fmaf(x, 1.44269502f, -t) + x * 1.92596299e-08f;
    return __builtin_amdgcn_exp2f(t) * fmaf(r, 0.693147181f, 1.0f);
}

template <int N>
__device__ inline void load_win(float* win, const float* window) {
    if (threadIdx.x < N) win[threadIdx.x] = window ? window[threadIdx.x] : hann_at(threadIdx.x, N);
}

// Frames per forward block: the block forms FT frames, FT - KB of them its
// own and the KB before them, whose tails overlap its first samples.
template <int N, int H>
constexpr int fwd_own_frames() {
    return FT - ((N + H - 1) / H - 1);
}

template <int N, int H>
__global__ __launch_bounds__(FT) void spec_fwd_fixed_k(const float* post, long post_bs, const float* window,
                                                      float* audio, long audio_bs, int L, Tw<N> tw) {
    constexpr int F = N / 2 + 1;
    constexpr int KB = (N + H - 1) / H - 1;  // earlier frames overlapping the block's samples
    constexpr int OWN = fwd_own_frames<N, H>();
    constexpr int NP = N + 1;                // LDS frame stride (odd: no bank conflicts)
    __shared__ float win[N];
    __shared__ float fr[FT * NP];
    __shared__ float ienv[H];  // 1 / envelope at interior positions, by m mod H
    load_win<N>(win, window);
    const int b = blockIdx.y;
    const int f0 = blockIdx.x * OWN;  // first own frame
    const float* P = post + b * post_bs;
    {
        const int f = f0 - KB + static_cast<int>(threadIdx.x);
        float* out = fr + threadIdx.x * NP;
        float re[F], im[F];
        const bool in = f >= 0 && f < L;
        // every bin's two inputs loaded before the first use, from a frame
        // clamped into the signal (a load under the `in` branch would be
        // waited for at the branch's join, one round trip per bin)
        const int fc = min(max(f, 0), L - 1);
        float lm[F], lp[F];
#pragma unroll
        for (int k = 0; k < F; ++k) {
            lm[k] = P[static_cast<long>(k) * L + fc];
            lp[k] = P[static_cast<long>(F + k) * L + fc];
        }
#pragma unroll
        for (int k = 0; k < F; ++k) {
            re[k] = im[k] = 0.0f;
            if (in) {
                const float mag = kdec_exp(lm[k]);
                float spp, cpp, sa, ca;
                kdec_sincos(lp[k], spp, cpp);
                kdec_sincos_unit(spp, sa, ca);
                re[k] = mag * ca;
                im[k] = mag * sa;
            }
        }
        __syncthreads();  // win
        if (threadIdx.x < H) ienv[threadIdx.x] = 1.0f / env_at(win, N + ((threadIdx.x - N) % H + H) % H, N, H, L);
        // x[n] = (re0 + (-1)^n re_{N/2} + 2 sum_k re_k cos) - 2 sum_k im_k sin,
        // x[N - n] the same with the sine sum added; the sums folded on
        // k <-> N/2 - k (cos and sin at (N/2 - k) n are (-1)^n cos and
        // -(-1)^n sin at k n): even n sees A = 2(re_k + re_{N/2-k}) and C =
        // 2(im_k - im_{N/2-k}), odd n B = 2(re_k - re_{N/2-k}) and E =
        // 2(im_k + im_{N/2-k}); the middle bin k = N/4 has cos(pi n / 2) and
        // sin(pi n / 2) in {0, +-1}
        static_assert(N % 4 == 0, "the folded synthesis takes N a multiple of 4");
        constexpr int Q = N / 4;
        constexpr float invN = 1.0f / N;
        const float e0 = re[0] + re[F - 1], e1 = re[0] - re[F - 1];
        float A[Q], B[Q], C[Q], E[Q];  // k = 1 .. Q - 1
#pragma unroll
        for (int k = 1; k < Q; ++k) {
            A[k] = 2.0f * (re[k] + re[N / 2 - k]);
            B[k] = 2.0f * (re[k] - re[N / 2 - k]);
            C[k] = 2.0f * (im[k] - im[N / 2 - k]);
            E[k] = 2.0f * (im[k] + im[N / 2 - k]);
        }
        const float r5 = 2.0f * re[Q], i5 = 2.0f * im[Q];
#pragma unroll
        for (int n = 0; n <= N / 2; ++n) {
            float a, bb;
            if (n % 2 == 0) {
                a = (n % 4 == 0) ? e0 + r5 : e0 - r5;
                bb = 0.0f;
#pragma unroll
                for (int k = 1; k < Q; ++k) {
                    a += A[k] * tw.c[(k * n) % N];
                    bb += C[k] * tw.s[(k * n) % N];
                }
            } else {
                a = e1;
                bb = (n % 4 == 1) ? i5 : -i5;
#pragma unroll
                for (int k = 1; k < Q; ++k) {
                    a += B[k] * tw.c[(k * n) % N];
                    bb += E[k] * tw.s[(k * n) % N];
                }
            }
            if (n == 0 || n == N / 2) {  // the two points without a sine term
                out[n] = a * invN * win[n];
            } else {
                out[n] = (a - bb) * invN * win[n];
                out[N - n] = (a + bb) * invN * win[N - n];
            }
        }
    }
    __syncthreads();
    // samples j with ola position m = j + N/2 in [f0 * H, (f0 + OWN) * H)
    const int sig_len = (L - 1) * H;
    float* A = audio + b * audio_bs;
    for (int i = threadIdx.x; i < OWN * H; i += FT) {
        const int m = f0 * H + i;
        const int j = m - N / 2;
        if (j < 0 || j >= sig_len) continue;
        int f_hi = m / H;
        if (f_hi > L - 1) f_hi = L - 1;
        float acc = 0.0f, e = 0.0f;
        for (int f = f_hi; f >= 0 && m - f * H < N; --f) {
            const int n = m - f * H;
            acc += fr[(f - f0 + KB) * NP + n];
            e += win[n] * win[n];
        }
        A[j] = (m >= N && m <= (L - 1) * H) ? acc * ienv[m % H] : acc / e;
    }
}

// The backward, one block per FT frames of one utterance (frame f0 + t for
// thread t): every global load is issued at once and unconditionally (a load
// under a branch is waited for at the branch's join), then dY / envelope over
// the frames' sample span is staged in LDS and each thread forms its frame's
// grads. At most 64 VGPRs, so that every block of the decoder's head is
// resident at once.
template <int N, int H>
struct SpecBwdIn {
    static constexpr int F = N / 2 + 1;
    static constexpr int M = FT * H + N;  // ola positions the block's frames cover
    static constexpr int R = (M + FT - 1) / FT;
    float dv[R];        // dY samples this thread stages (clamped into the signal)
    float pm[F], pp[F]; // the frame's polar inputs (clamped to the last frame)
};

template <int N, int H>
__device__ inline void spec_bwd_load(SpecBwdIn<N, H>& in, const float* P0, const float* dy, int fg, int L,
                                     int sig_len) {
    using I = SpecBwdIn<N, H>;
#pragma unroll
    for (int r = 0; r < I::R; ++r) {
        const int j = fg * H + static_cast<int>(threadIdx.x) + r * FT - N / 2;
        in.dv[r] = dy[min(max(j, 0), sig_len - 1)];
    }
    const float* P = P0 + min(fg + static_cast<int>(threadIdx.x), L - 1);
#pragma unroll
    for (int k = 0; k < I::F; ++k) {
        in.pm[k] = P[static_cast<long>(k) * L];
        in.pp[k] = P[static_cast<long>(I::F + k) * L];
    }
}

template <int N, int H>
__global__ __launch_bounds__(FT) __attribute__((amdgpu_waves_per_eu(8)))
void spec_bwd_fixed_k(const float* post, long post_bs, const float* window, const float* daudio, long da_bs,
                      float* dpost, long dp_bs, int L, Tw<N> tw) {
    using I = SpecBwdIn<N, H>;
    constexpr int F = I::F, M = I::M, R = I::R;
    __shared__ float win[N];
    __shared__ float ienv[H];  // 1 / envelope at interior positions, by m mod H
    __shared__ float u[M];
    load_win<N>(win, window);
    const int b = blockIdx.y;
    const int f0 = blockIdx.x * FT;
    const int f = f0 + threadIdx.x;
    const int sig_len = (L - 1) * H;  // >= H: L >= 2
    const float* P0 = post + b * post_bs;
    const float* dy = daudio + b * da_bs;
    I cur;
    spec_bwd_load<N, H>(cur, P0, dy, f0, L, sig_len);
    __syncthreads();  // win
    // an interior position m (every frame that could cover it exists:
    // N <= m <= (L - 1) H) sees the same windows as m + H
    if (threadIdx.x < H) ienv[threadIdx.x] = 1.0f / env_at(win, N + ((threadIdx.x - N) % H + H) % H, N, H, L);
    __syncthreads();
    constexpr float invN = 1.0f / N;
    {
        // u[i] = dY[j] / envelope(m) at ola position m = f0 * H + i (j = m -
        // N/2; 0 outside the signal, where the envelope may be 0)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = static_cast<int>(threadIdx.x) + r * FT;
            if (i < M) {
                const int m = f0 * H + i;
                const int j = m - N / 2;
                float v = 0.0f;
                if (j >= 0 && j < sig_len)
                    v = (m >= N && m <= (L - 1) * H) ? cur.dv[r] * ienv[m % H] : cur.dv[r] / env_at(win, m, N, H, L);
                u[i] = v;
            }
        }
        __syncthreads();
        if (f < L) {
            float dfr[N];
#pragma unroll
            for (int n = 0; n < N; ++n) dfr[n] = u[threadIdx.x * H + n] * (window ? win[n] * invN : tw.w[n]);
            // Folded real DFT: with Q = N / 4, the pair sums sp and
            // differences dm over n <-> N - n, then over n <-> N/2 - n (cos
            // and sin at k (N/2 - n) are (-1)^k cos and -(-1)^k sin at k n):
            // even k sees A = sp[n] + sp[N/2 - n] and C = dm[n] - dm[N/2 - n],
            // odd k B = sp[n] - sp[N/2 - n] and E = dm[n] + dm[N/2 - n]; the
            // middle term n = Q has cos(pi k / 2) and sin(pi k / 2) in {0, +-1}
            static_assert(N % 4 == 0, "the folded DFT takes N a multiple of 4");
            constexpr int Q = N / 4;
            float sp[N / 2], dm[N / 2];  // n = 1 .. N/2 - 1
#pragma unroll
            for (int n = 1; n < N / 2; ++n) {
                sp[n] = dfr[n] + dfr[N - n];
                dm[n] = dfr[n] - dfr[N - n];
            }
            float A[Q], B[Q], C[Q], E[Q];  // n = 1 .. Q - 1
#pragma unroll
            for (int n = 1; n < Q; ++n) {
                A[n] = sp[n] + sp[N / 2 - n];
                B[n] = sp[n] - sp[N / 2 - n];
                C[n] = dm[n] - dm[N / 2 - n];
                E[n] = dm[n] + dm[N / 2 - n];
            }
            const float e0 = dfr[0] + dfr[N / 2], e1 = dfr[0] - dfr[N / 2];
            float* D = dpost + b * dp_bs + f;
#pragma unroll
            for (int k = 0; k < F; ++k) {
                const bool edge = k == 0 || k == F - 1;
                float re, im;
                if (k % 2 == 0) {
                    re = (k % 4 == 0) ? e0 + sp[Q] : e0 - sp[Q];
                    im = 0.0f;
#pragma unroll
                    for (int n = 1; n < Q; ++n) {
                        re += A[n] * tw.c[(k * n) % N];
                        im -= C[n] * tw.s[(k * n) % N];
                    }
                } else {
                    re = e1;
                    im = (k % 4 == 1) ? -dm[Q] : dm[Q];
#pragma unroll
                    for (int n = 1; n < Q; ++n) {
                        re += B[n] * tw.c[(k * n) % N];
                        im -= E[n] * tw.s[(k * n) % N];
                    }
                }
                const float dRe = edge ? re : 2.0f * re;
                const float dIm = edge ? 0.0f : 2.0f * im;
                const float mag = kdec_exp(cur.pm[k]);
                float spp, cpp, sa, ca;
                kdec_sincos(cur.pp[k], spp, cpp);
                kdec_sincos_unit(spp, sa, ca);
                const float dmag = dRe * ca + dIm * sa;
                const float dang = mag * (-dRe * sa + dIm * ca);
                D[static_cast<long>(k) * L] = dmag * mag;
                D[static_cast<long>(F + k) * L] = dang * cpp;
            }
        }
    }
}

// ─── harmonic source ───
// The reference's phase recurrence (kokoro_modules.cpp:1602-1617) is a
// sequential float accumulation per (utterance, harmonic) chain i = b*H + h:
// per sample ph = fl(ph + omega), then ph = fl(ph - 2pi) when ph > 2pi, with
// omega = fl(fl(fl(2pi * (h+1)) * f0) / sr) constant over a frame of `us`
// samples. Each step's rounding is reproduced exactly, in three passes:
//   1. hs_start_k runs every chain, one lane each, through all samples in
//      registers and keeps only the phase entering each frame;
//   2. hs_phase_k gives one thread each (frame, chain): it re-runs that
//      frame's steps from the stored start (the same operations, so the same
//      values) and writes every phase;
//   3. hs_merge_k forms the merged source per sample.
// Pass 1 is the serial part; it issues three VALU operations per step and
// stores nothing but the frame starts.
constexpr float kHsTwoPi = 6.28318530717958647692f;

__device__ inline float hs_omega(int h, float f0, float sr) {
#pragma clang fp contract(off)
    float omega = kHsTwoPi * static_cast<float>(h + 1);
    omega = omega * f0;
    return omega / sr;
}

// One step, branch free: y = fl(ph + omega); s = clamp((y - 2pi) * 2^21, 0,
// 1) is exactly 1 when y > fl(2pi) and 0 otherwise (fl(2pi) and every float
// y >= 4 are multiples of 2^-21, so a positive difference is at least 2^-21,
// and the fma's product and sum are exact); fma(s, -2pi, y) is then
// fl(y - 2pi) or y, the reference's wrap.
__device__ inline float hs_step(float ph, float omega) {
#pragma clang fp contract(off)
    const float y = ph + omega;
    const float s = __builtin_amdgcn_fmed3f(__builtin_fmaf(y, 0x1p21f, -kHsTwoPi * 0x1p21f), 0.0f, 1.0f);
    return __builtin_fmaf(s, -kHsTwoPi, y);
}

// Layout of the per-sample phases: four steps of a chain are contiguous,
// phase[((t/4)*NH + i)*4 + t%4], so a thread writes a chain's steps as float4
// runs and the lanes of a wave (consecutive chains) write contiguous memory.
__device__ inline long hs_index(int t, int i, int NH) {
    return (static_cast<long>(t >> 2) * NH + i) * 4 + (t & 3);
}

// Pass 1: start[fr * NH + i] = the phase of chain i entering frame fr.
constexpr int HS_UNROLL = 150;  // steps per unrolled trip (divides the 300-sample frames)
__global__ __launch_bounds__(64) void hs_start_k(const float* F0, long f0_bs, float* start, int N, int H,
                                                 int frame_count, int us, int sig_len, int nfr, float sr) {
    const int NH = N * H;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= NH) return;
    const int b = i / H, h = i - b * H;
    const float* f0r = F0 + b * f0_bs;
    float ph = 0.0f;
    float f0 = f0r[0];
    for (int fr = 0; fr < nfr; ++fr) {
        const float omega = hs_omega(h, f0, sr);
        f0 = f0r[min(fr + 1, frame_count - 1)];  // next frame's, used after this frame's chain
        start[static_cast<long>(fr) * NH + i] = ph;
        const int n = min(us, sig_len - fr * us);
        // long unrolled runs: the loop's scalar count / compare / branch
        // otherwise take issue cycles between the chain's dependent
        // operations (150 steps per trip: 3.18 -> 1.97 ms at 8 x 307200)
        int t = 0;
        for (; t + HS_UNROLL <= n; t += HS_UNROLL) {
#pragma unroll
            for (int u = 0; u < HS_UNROLL; ++u) ph = hs_step(ph, omega);
        }
        for (; t + 4 <= n; t += 4) {
            ph = hs_step(ph, omega);
            ph = hs_step(ph, omega);
            ph = hs_step(ph, omega);
            ph = hs_step(ph, omega);
        }
        for (; t < n; ++t) ph = hs_step(ph, omega);
    }
}

// Pass 2: thread g = fr * NH + i re-runs frame fr of chain i.
__global__ void hs_phase_k(const float* start, const float* F0, long f0_bs, float* phase, int N, int H,
                           int frame_count, int us, int sig_len, int nfr, float sr) {
    const int NH = N * H;
    const long g = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= static_cast<long>(nfr) * NH) return;
    const int fr = static_cast<int>(g / NH), i = static_cast<int>(g - static_cast<long>(fr) * NH);
    const int b = i / H, h = i - b * H;
    const float omega = hs_omega(h, F0[b * f0_bs + min(fr, frame_count - 1)], sr);
    float ph = start[g];
    const int t0 = fr * us;
    const int t1 = min(t0 + us, sig_len);
    int t = t0;
    for (; t < t1 && (t & 3) != 0; ++t) {
        ph = hs_step(ph, omega);
        phase[hs_index(t, i, NH)] = ph;
    }
    float4* out4 = reinterpret_cast<float4*>(phase) + static_cast<long>(t >> 2) * NH + i;
    for (; t + 4 <= t1; t += 4, out4 += NH) {
        float4 v;
        v.x = ph = hs_step(ph, omega);
        v.y = ph = hs_step(ph, omega);
        v.z = ph = hs_step(ph, omega);
        v.w = ph = hs_step(ph, omega);
        *out4 = v;
    }
    for (; t < t1; ++t) {
        ph = hs_step(ph, omega);
        phase[hs_index(t, i, NH)] = ph;
    }
}

// Pass 3: merged[b, t] = tanh(lb + sum_h lW[h] * sin(phase) * amp * uv)
__global__ void hs_merge_k(const float* phase, const float* F0, long f0_bs, const float* lW,
                           const float* lb, float* merged, int N, int H, int frame_count, int us,
                           int sig_len) {
#pragma clang fp contract(off)
    const int b = blockIdx.y;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= sig_len) return;
    const int fr = t / us;
    const float f0 = F0[b * f0_bs + (fr < frame_count ? fr : frame_count - 1)];
    const float uv = f0 > 0.0f ? 1.0f : 0.0f;
    double acc = lb[0];
    for (int h = 0; h < H; ++h) {
        const float ph = phase[hs_index(t, b * H + h, N * H)];
        float sv = static_cast<float>(sin(static_cast<double>(ph)));
        sv = sv * 0.1f;
        sv = sv * uv;
        acc += static_cast<double>(lW[h]) * sv;
    }
    merged[static_cast<long>(b) * sig_len + t] =
        static_cast<float>(tanh(static_cast<double>(static_cast<float>(acc))));
}

// STFT (center, reflect pad) -> har[b, k, f] = |X|, har[b, F+k, f] = atan2
// (NM >= N as in spec_frames_k)
template <int NM>
__global__ __launch_bounds__(FT) void hs_stft_k(const float* merged, float* har, long har_bs,
                                               int sig_len, int N, int hop, int frames) {
    __shared__ float tc[MAXN / 2 + 1][MAXN], ts[MAXN / 2 + 1][MAXN], win[MAXN];
    const int F = N / 2 + 1;
    load_twiddles(&tc[0][0], &ts[0][0], win, N, F, nullptr);
    __syncthreads();
    const float* TC = &tc[0][0];
    const float* TS = &ts[0][0];
    const int b = blockIdx.y;
    const int f = blockIdx.x * FT + threadIdx.x;
    if (f >= frames) return;
    const float* x = merged + static_cast<long>(b) * sig_len;
    const int pad = N / 2;
    float v[NM];
#pragma unroll
    for (int n = 0; n < NM; ++n) {
        v[n] = 0.0f;
        if (n < N) {
            int j = f * hop + n - pad;
            if (j < 0) j = -j;
            if (j >= sig_len) j = 2 * (sig_len - 1) - j;
            v[n] = win[n] * x[j];
        }
    }
    float* out = har + b * har_bs;
    for (int k = 0; k < F; ++k) {
        double re = 0.0, im = 0.0;
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            if (n < N) {
                re += static_cast<double>(v[n]) * TC[k * N + n];
                im -= static_cast<double>(v[n]) * TS[k * N + n];
            }
        }
        const float ref = static_cast<float>(re), imf = static_cast<float>(im);
        out[static_cast<long>(k) * frames + f] =
            static_cast<float>(sqrt(static_cast<double>(ref) * ref + static_cast<double>(imf) * imf));
        out[static_cast<long>(F + k) * frames + f] = static_cast<float>(atan2(static_cast<double>(imf),
                                                                             static_cast<double>(ref)));
    }
}

// ─── style projection ───
// out[n, r] = W[r, :] . style[n, :] + b[r]; one wave per (r, n).
__global__ void style_fwd_k(const float* W, const float* bias, const float* style, long s_bs,
                            float* out, long o_bs, int N, int rows, int S) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= rows * N) return;
    const int r = wave / N, n = wave - r * N;
    const float* w = W + static_cast<long>(r) * S;
    const float* s = style + n * s_bs;
    double acc = 0.0;
    for (int j = lane; j < S; j += 64) acc += static_cast<double>(w[j]) * s[j];
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_down(acc, o, 64);
    if (lane == 0) out[n * o_bs + r] = static_cast<float>(acc + (bias ? bias[r] : 0.0f));
}

// partial[blk, n, j] = sum_{r in block rows} W[r, j] dout[n, r]
constexpr int SR = 128;  // rows per block
__global__ void style_bwd_x_k(const float* W, const float* dout, long d_bs, float* part, int N,
                              int rows, int S) {
    const int blk = blockIdx.x;
    const int r0 = blk * SR, r1 = min(r0 + SR, rows);
    for (int nj = threadIdx.x; nj < N * S; nj += blockDim.x) {
        const int n = nj / S, j = nj - n * S;
        double acc = 0.0;
        for (int r = r0; r < r1; ++r)
            acc += static_cast<double>(W[static_cast<long>(r) * S + j]) * dout[n * d_bs + r];
        part[(static_cast<long>(blk) * N + n) * S + j] = static_cast<float>(acc);
    }
}

__global__ void style_bwd_x_reduce(const float* part, int nblk, float* dstyle, long ds_bs, float beta,
                                   int N, int S) {
    const int nj = blockIdx.x * blockDim.x + threadIdx.x;
    if (nj >= N * S) return;
    const int n = nj / S, j = nj - n * S;
    double acc = 0.0;
    for (int q = 0; q < nblk; ++q) acc += part[static_cast<long>(q) * N * S + nj];
    float* d = dstyle + n * ds_bs + j;
    *d = static_cast<float>(acc) + (beta != 0.0f ? beta * *d : 0.0f);
}

// dW[r, j] += sum_n dout[n, r] style[n, j];  db[r] += sum_n dout[n, r]
__global__ void style_bwd_w_k(const float* style, long s_bs, const float* dout, long d_bs, float* dW,
                              float* db, int N, int rows, int S) {
    const long tot = static_cast<long>(rows) * S;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < tot;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(i / S), j = static_cast<int>(i - static_cast<long>(r) * S);
        double acc = 0.0, accb = 0.0;
        for (int n = 0; n < N; ++n) {
            const double g = dout[n * d_bs + r];
            acc += g * style[n * s_bs + j];
            accb += g;
        }
        dW[i] += static_cast<float>(acc);
        if (db && j == 0) db[r] += static_cast<float>(accb);
    }
}

// The same projections reading each fc row once for all N utterances (the
// wave-per-(row, utterance) kernels above read the fc block N times).
//
// Forward: a block owns STR = 32 consecutive rows, staged in LDS as
// [STR][S + 4] with 16-byte loads, all in flight before the first store (the
// padded stride spreads the 16-byte row reads over the banks). Lane r of
// half-wave c forms row r's dot products over column group c (S / STG
// consecutive columns) for STQ utterances at a time: float sums of S / STG
// terms in column order, the row operands read 16 bytes at a time from LDS
// and the style operands, one address per half-wave, from the pass's style
// rows staged in LDS. The STG groups' sums are added in group order in
// double, with the bias. 32 rows per block rather than 64: the decoder's
// 37 396 rows then make 1169 blocks, where 585 left some CUs a third block
// to run after the others were done (5.4 -> 4.9 µs).
// d(style): thread (ph, j) = (t / S, t % S) sums, in
// float and in row order, rows ph, ph + PH, ... of the block's STB rows
// (PH = 256 / S phases) for STN utterances at a time, its column's weights
// loaded all at once and the d(out) operands read from LDS; the phases' sums
// are added in phase order in double, and the blocks' partials summed, in
// block order, by style_bwd_x_sum_k.
constexpr int STR = 32;           // forward rows per block (a half-wave's lanes)
constexpr int STG = 8;            // forward column groups (one per half-wave)
constexpr int STQ = 8;            // forward utterances per pass
constexpr int STB = 64;           // d(style) rows per block
constexpr int STN = 8;            // d(style) utterances per pass

// LDS floats of the forward kernel: slab, styles, group sums
inline size_t style_fwd_lds_floats(int S) {
    return static_cast<size_t>(STR) * (S + 4) + static_cast<size_t>(STG) * STQ * STR + static_cast<size_t>(STQ) * S;
}

__device__ inline float style_ld(__amdgpu_buffer_rsrc_t r, int byte_off, int soff = 0) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, soff, 0));
}

// Every global load below is issued unconditionally (a buffer load past the
// end of its array returns 0) and the bounds decide only how the value is
// used: a load under a branch is followed by a wait for it at the branch's
// join, which turns a run of guarded loads into one memory round trip each.

// Forward; KQ = STR * S / 1024 slab float4s per thread (S <= 128, a
// multiple of 32). A
// pass's STQ style rows are staged in LDS too and read there by broadcast
// (a wave's lanes all read one address): read by scalar loads, each
// utterance's operands were a round trip of their own.
template <int KQ>
__global__ __launch_bounds__(256) void style_fwd_rows_k(const float* __restrict__ W, const float* __restrict__ bias,
                                                        const float* __restrict__ style, long s_bs,
                                                        float* __restrict__ out, long o_bs, int N, int rows, int S) {
    extern __shared__ float sm[];
    const int SP = S + 4;
    float* wt = sm;                           // [STR][S + 4]
    float* red = wt + STR * SP;               // [STG][STQ][STR]
    float* sty = red + STG * STQ * STR;       // [STQ][S]: the pass's style rows
    const int t = threadIdx.x;
    const int r0 = blockIdx.x * STR;
    const int nr = min(STR, rows - r0);
    const int S4 = S >> 2;
    // a pass's style rows as STQ * S4 float4s, one per thread at most (a
    // slot past N repeats the last utterance; its sums are not stored)
    const bool sl = t < STQ * S4;
    const int sq = t / S4, sc4 = t - (t / S4) * S4;
    auto sty_fetch = [&](int n0) {
        return sl ? *reinterpret_cast<const float4*>(style + min(n0 + sq, N - 1) * s_bs + 4 * sc4)
                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    // the bias by a buffer load issued with the others (none: a descriptor
    // over nothing, which reads 0)
    const __amdgpu_buffer_rsrc_t br = uniform_rsrc(bias ? bias : W, bias ? rows * 4 : 0);
    const float bv = style_ld(br, min(r0 + (t & (STR - 1)), rows - 1) * 4);
    {  // the slab, STR * S4 == 256 * KQ float4s, and the first pass's style rows, all in flight
        const __amdgpu_buffer_rsrc_t wr = uniform_rsrc(W, rows * S * 4);
        const int wb = r0 * S * 4;
        float4 v[KQ];
#pragma unroll
        for (int k = 0; k < KQ; ++k)
            v[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wr, wb + (t + 256 * k) * 16, 0, 0));
        const float4 y0 = sty_fetch(0);
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
            const int i = t + 256 * k;
            const int row = i / S4, c4 = i - row * S4;
            *reinterpret_cast<float4*>(wt + row * SP + c4 * 4) = v[k];
        }
        if (sl) *reinterpret_cast<float4*>(sty + 4 * t) = y0;
    }
    __syncthreads();
    const int c = t / STR, r = t % STR;
    constexpr int cw = 4 * KQ;  // columns per half-wave: S / STG
    const float* w = wt + r * SP + c * cw;
    const float* sg = sty + c * cw;  // one address per half-wave: LDS broadcast
    for (int n0 = 0; n0 < N; n0 += STQ) {
        const int nn = min(STQ, N - n0);
        if (n0 > 0) {  // the previous pass ended at a barrier: its style rows are no longer read
            const float4 y0 = sty_fetch(n0);
            if (sl) *reinterpret_cast<float4*>(sty + 4 * t) = y0;
            __syncthreads();
        }
        float acc[STQ];
#pragma unroll
        for (int q = 0; q < STQ; ++q) acc[q] = 0.0f;
#pragma unroll
        for (int jj = 0; jj < cw; jj += 4) {
            // each step's LDS reads stay in the step, after the previous
            // step's sums (hoisted, the broadcast operands of every step
            // would take 8 * cw registers per lane)
            static_assert(STQ == 8, "one asm operand per utterance slot");
            asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]),
                         "+v"(acc[6]), "+v"(acc[7])::"memory");
            float4 y[STQ];
#pragma unroll
            for (int q = 0; q < STQ; ++q) y[q] = *reinterpret_cast<const float4*>(sg + q * S + jj);
            const float4 x = *reinterpret_cast<const float4*>(w + jj);
#pragma unroll
            for (int q = 0; q < STQ; ++q) {
                float a = acc[q];
                a = __builtin_fmaf(x.x, y[q].x, a);
                a = __builtin_fmaf(x.y, y[q].y, a);
                a = __builtin_fmaf(x.z, y[q].z, a);
                acc[q] = __builtin_fmaf(x.w, y[q].w, a);
            }
        }
#pragma unroll
        for (int q = 0; q < STQ; ++q)
            if (q < nn) red[(c * STQ + q) * STR + r] = acc[q];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < STQ * STR / 256; ++k) {
            const int i = t + 256 * k, q = i / STR, rr = i - q * STR;  // rr == t % STR
            if (q < nn && rr < nr) {
                double sum = 0.0;
#pragma unroll
                for (int cc = 0; cc < STG; ++cc) sum += static_cast<double>(red[(cc * STQ + q) * STR + rr]);
                out[(n0 + q) * o_bs + r0 + rr] = static_cast<float>(sum + bv);
            }
        }
        __syncthreads();
    }
}

// part[blk][n][j] = sum over the block's rows r of W[r, j] dout[n, r];
// PER = STB * S / 256 rows per thread (S divides 256, S >= 64)
template <int PER>
__global__ __launch_bounds__(256) void style_bwd_x_rows_k(const float* W, const float* dout, long d_bs, float* part,
                                                          int N, int rows, int S) {
    extern __shared__ float sm[];
    const int PH = 256 / S;           // row phases (PH * S == 256)
    float* dsl = sm;                  // [STB][STN] of the pass's utterances
    float* red = sm + STB * STN;      // [PH][STN][S]
    const int r0 = blockIdx.x * STB;
    const int nr = min(STB, rows - r0);
    const int j = threadIdx.x % S, ph = __builtin_amdgcn_readfirstlane(threadIdx.x / S);  // S >= 64
    const __amdgpu_buffer_rsrc_t wr = uniform_rsrc(W, rows * S * 4);
    const __amdgpu_buffer_rsrc_t dr = uniform_rsrc(dout, static_cast<int>(((N - 1) * d_bs + rows) * 4));
    // row ph + i * PH of the block is 1 KB * i past the thread's first one
    const int vo = ((r0 + ph) * S + j) * 4;
    float w[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) w[i] = style_ld(wr, vo, i * 1024);
    for (int n0 = 0; n0 < N; n0 += STN) {
        const int nn = min(STN, N - n0);
        {  // STB * STN == DK * 256 d(out) values
            constexpr int DK = STB * STN / 256;
            float dv[DK];
#pragma unroll
            for (int k = 0; k < DK; ++k) {
                const int i = threadIdx.x + 256 * k, rr = i / STN, q = i - rr * STN;
                dv[k] = style_ld(dr, static_cast<int>(((n0 + q) * d_bs + r0 + rr) * 4));
            }
#pragma unroll
            for (int k = 0; k < DK; ++k) {
                const int i = threadIdx.x + 256 * k, rr = i / STN, q = i - rr * STN;
                dsl[i] = (rr < nr && q < nn) ? dv[k] : 0.0f;
            }
        }
        __syncthreads();
        float acc[STN];
#pragma unroll
        for (int q = 0; q < STN; ++q) acc[q] = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int rr = ph + i * PH;
            const float x = rr < nr ? w[i] : 0.0f;  // another block's row, or past the end
            const float4 d0 = *reinterpret_cast<const float4*>(dsl + rr * STN);
            const float4 d1 = *reinterpret_cast<const float4*>(dsl + rr * STN + 4);
            acc[0] = __builtin_fmaf(x, d0.x, acc[0]);
            acc[1] = __builtin_fmaf(x, d0.y, acc[1]);
            acc[2] = __builtin_fmaf(x, d0.z, acc[2]);
            acc[3] = __builtin_fmaf(x, d0.w, acc[3]);
            acc[4] = __builtin_fmaf(x, d1.x, acc[4]);
            acc[5] = __builtin_fmaf(x, d1.y, acc[5]);
            acc[6] = __builtin_fmaf(x, d1.z, acc[6]);
            acc[7] = __builtin_fmaf(x, d1.w, acc[7]);
        }
#pragma unroll
        for (int q = 0; q < STN; ++q) red[(ph * STN + q) * S + j] = acc[q];
        __syncthreads();
        for (int i = threadIdx.x; i < nn * S; i += 256) {
            const int q = i / S, jj = i - q * S;
            double tsum = 0.0;
            for (int h = 0; h < PH; ++h) tsum += static_cast<double>(red[(h * STN + q) * S + jj]);
            part[(static_cast<long>(blockIdx.x) * N + n0 + q) * S + jj] = static_cast<float>(tsum);
        }
        __syncthreads();
    }
}

// dstyle[n, j] = beta * dstyle[n, j] + the sum over blocks q of
// part[q][n][j] in a fixed order: 16 outputs per block; lane group p (64 of
// them) sums the p-th sixty-fourth of the block range in order, up to 16
// partials in flight per lane, and the groups' sums are added in a fixed tree
__global__ __launch_bounds__(1024) void style_bwd_x_sum_k(const float* part, int nblk, float* dstyle, long ds_bs,
                                                          float beta, int N, int S) {
    __shared__ double red[64][16];
    const int o = threadIdx.x & 15, p = threadIdx.x >> 4;
    const int nj = blockIdx.x * 16 + o;
    const int NS = N * S;
    const int q0 = p * nblk / 64, q1 = (p + 1) * nblk / 64;
    const __amdgpu_buffer_rsrc_t pr = uniform_rsrc(part, nblk * NS * 4);
    double acc = 0.0;
    for (int qb = q0; qb < q1; qb += 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = style_ld(pr, ((qb + i) * NS + nj) * 4);
#pragma unroll
        for (int i = 0; i < 16; ++i) acc += qb + i < q1 ? static_cast<double>(v[i]) : 0.0;
    }
    red[p][o] = acc;
    __syncthreads();
    for (int h = 32; h >= 1; h >>= 1) {
        if (p < h) red[p][o] += red[p + h][o];
        __syncthreads();
    }
    if (p == 0 && nj < NS) {
        const int n = nj / S, j = nj - n * S;
        float* d = dstyle + n * ds_bs + j;
        *d = static_cast<float>(red[0][o]) + (beta != 0.0f ? beta * *d : 0.0f);
    }
}

// ─── LoRA term of the style projection ───────────────────────────────────
// Units are stacked row-wise: unit u owns rows [off[u], off[u+1]) of W, b, B
// and rows [u*rank, (u+1)*rank) of A; H[n, u*rank + j] = A[u*rank + j] . s[n].

// the unit owning row r (binary search over the units+1 offsets)
__device__ inline int unit_of(const int* off, int units, int r) {
    int lo = 0, hi = units;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= r) lo = mid;
        else hi = mid;
    }
    return lo;
}

// out[n, r] = W[r] . s[n] + b[r] + scale * sum_j B[r, j] g[n, j] H[n, u(r)*rank + j];
// one wave per (r, n)
__global__ void lora_fwd_k(const float* W, const float* bias, const float* B, const float* g, long g_bs,
                           float scale, const int* unit_off, int units, int rank, const float* style, long s_bs,
                           const float* H, float* out, long o_bs, int N, int rows, int S) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= rows * N) return;
    const int r = wave / N, n = wave - r * N;
    const float* w = W + static_cast<long>(r) * S;
    const float* s = style + n * s_bs;
    double acc = 0.0, lo = 0.0;
    for (int j = lane; j < S; j += 64) acc += static_cast<double>(w[j]) * s[j];
    const int u = unit_of(unit_off, units, r);
    const float* hr = H + (static_cast<long>(n) * units + u) * rank;
    for (int j = lane; j < rank; j += 64)
        lo += static_cast<double>(B[static_cast<long>(r) * rank + j]) * (g[n * g_bs + j] * hr[j]);
    for (int o = 32; o > 0; o >>= 1) {
        acc += __shfl_down(acc, o, 64);
        lo += __shfl_down(lo, o, 64);
    }
    if (lane == 0) out[n * o_bs + r] = static_cast<float>(acc + (bias ? bias[r] : 0.0f) + scale * lo);
}

// For c = u*rank + j: dHG = scale * sum_{r in u} B[r, j] dout[n, r];
// dH[n, c] = dHG * g[n, j] (the grad at A s), gp[n, c] = dHG * H[n, c] (the
// unit's share of the gate grad). One wave per (n, c).
__global__ void lora_dh_k(const float* B, const float* g, long g_bs, float scale, const int* unit_off, int units,
                          int rank, const float* H, const float* dout, long d_bs, float* dH, float* gp, int N) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const int UR = units * rank;
    if (wave >= N * UR) return;
    const int n = wave / UR, c = wave - n * UR;
    const int u = c / rank, j = c - u * rank;
    double acc = 0.0;
    for (int r = unit_off[u] + lane; r < unit_off[u + 1]; r += 64)
        acc += static_cast<double>(B[static_cast<long>(r) * rank + j]) * dout[n * d_bs + r];
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_down(acc, o, 64);
    if (lane == 0) {
        const double dhg = scale * acc;
        const long i = static_cast<long>(n) * UR + c;
        dH[i] = static_cast<float>(dhg * g[n * g_bs + j]);
        gp[i] = static_cast<float>(dhg * H[i]);
    }
}

// dG[n, j] += sum_u gp[n, u*rank + j] at the gate's stride; a shared gate
// (g_bs = 0) also sums over the utterances, in order.
__global__ void lora_dg_k(const float* gp, float* dG, long g_bs, int N, int units, int rank) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int NG = g_bs ? N : 1;
    if (t >= NG * rank) return;
    const int n0 = t / rank, j = t - n0 * rank;
    const int na = g_bs ? n0 : 0, nb = g_bs ? n0 + 1 : N;
    double acc = 0.0;
    for (int n = na; n < nb; ++n)
        for (int u = 0; u < units; ++u) acc += gp[(static_cast<long>(n) * units + u) * rank + j];
    dG[n0 * g_bs + j] += static_cast<float>(acc);
}

// dB[r, j] += scale * sum_n dout[n, r] g[n, j] H[n, u(r)*rank + j]
__global__ void lora_db_k(const float* g, long g_bs, float scale, const int* unit_off, int units, int rank,
                          const float* H, const float* dout, long d_bs, float* dB, int N, int rows) {
    const long tot = static_cast<long>(rows) * rank;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < tot;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(i / rank), j = static_cast<int>(i - static_cast<long>(r) * rank);
        const int u = unit_of(unit_off, units, r);
        double acc = 0.0;
        for (int n = 0; n < N; ++n)
            acc += static_cast<double>(dout[n * d_bs + r]) *
                   (g[n * g_bs + j] * H[(static_cast<long>(n) * units + u) * rank + j]);
        dB[i] += static_cast<float>(scale * acc);
    }
}

unsigned g1(long n, long per = 256, long cap = 65535) {
    long g = (n + per - 1) / per;
    if (g > cap) g = cap;
    if (g < 1) g = 1;
    return static_cast<unsigned>(g);
}

}  // namespace
}  // namespace kdec

namespace kdec {
namespace {
// Calls fn with the smallest per-lane array bound (8, 16, 32 or 64) that
// holds an n_fft-point frame.
template <typename Fn>
void with_nfft_bound(int n_fft, Fn&& fn) {
    if (n_fft <= 8)
        fn(std::integral_constant<int, 8>{});
    else if (n_fft <= 16)
        fn(std::integral_constant<int, 16>{});
    else if (n_fft <= 32)
        fn(std::integral_constant<int, 32>{});
    else
        fn(std::integral_constant<int, MAXN>{});
}
}  // namespace
}  // namespace kdec

using namespace kdec;

extern "C" {

int kdec_spectral_fwd(kdec_ctx* ctx, const float* post, long post_bs,
                      const float* window, float* audio, long audio_bs, int N,
                      int L, int n_fft, int hop) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, post && audio && N > 0 && L > 1 && n_fft >= 2 && n_fft <= MAXN && hop > 0 && hop <= n_fft,
               "kdec_spectral_fwd: bad arguments");
    const int sig = (L - 1) * hop;
    // post in, audio out
    const double bytes = 4.0 * N * (static_cast<double>(n_fft + 2) * L + sig);
    if (n_fft == 20 && hop == 5) {
        ProfScope ps(ctx, "spectral", 0, bytes);
        hipLaunchKernelGGL((spec_fwd_fixed_k<20, 5>),
                           dim3(static_cast<unsigned>(cdiv(L, fwd_own_frames<20, 5>())), N), dim3(FT), 0, ctx->stream,
                           post, post_bs, window, audio, audio_bs, L, make_tw<20>());
        return launch_check(ctx, "spec_fwd");
    }
    Workspace fb(ctx, static_cast<size_t>(N) * L * n_fft * sizeof(float));
    if (!fb.p) return KDEC_ENOMEM;
    ProfScope ps(ctx, "spectral", 0, bytes);
    with_nfft_bound(n_fft, [&](auto nm) {
        hipLaunchKernelGGL(spec_frames_k<decltype(nm)::value>, dim3(static_cast<unsigned>(cdiv(L, FT)), N),
                           dim3(FT), 0, ctx->stream, post, post_bs, window, fb.as<float>(), L, n_fft);
    });
    if (int rc = launch_check(ctx, "spec_frames")) return rc;
    hipLaunchKernelGGL(spec_ola_k, dim3(static_cast<unsigned>(cdiv(sig, 256)), N), dim3(256), 0, ctx->stream,
                       fb.as<float>(), window, audio, audio_bs, L, n_fft, hop, sig);
    return launch_check(ctx, "spec_ola");
}

int kdec_spectral_bwd(kdec_ctx* ctx, const float* post, long post_bs,
                      const float* window, const float* daudio,
                      long daudio_bs, float* dpost, long dpost_bs, int N,
                      int L, int n_fft, int hop) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, post && daudio && dpost && N > 0 && L > 1 && n_fft >= 2 && n_fft <= MAXN && hop > 0 &&
                        hop <= n_fft,
               "kdec_spectral_bwd: bad arguments");
    // post in, dAudio in, dpost out
    const double bytes = 4.0 * N * (2.0 * (n_fft + 2) * L + static_cast<double>(L - 1) * hop);
    ProfScope ps(ctx, "spectral_bwd", 0, bytes);
    if (n_fft == 20 && hop == 5) {
        hipLaunchKernelGGL((spec_bwd_fixed_k<20, 5>), dim3(static_cast<unsigned>(cdiv(L, FT)), N), dim3(FT), 0,
                           ctx->stream, post, post_bs, window, daudio, daudio_bs, dpost, dpost_bs, L, make_tw<20>());
        return launch_check(ctx, "spec_bwd");
    }
    with_nfft_bound(n_fft, [&](auto nm) {
        hipLaunchKernelGGL(spec_bwd_k<decltype(nm)::value>, dim3(static_cast<unsigned>(cdiv(L, FT)), N), dim3(FT),
                           0, ctx->stream, post, post_bs, window, daudio, daudio_bs, dpost, dpost_bs, L, n_fft, hop);
    });
    return launch_check(ctx, "spec_bwd");
}

int kdec_harmonic_source(kdec_ctx* ctx, const float* F0, long f0_bs,
                         float* har, long har_bs, int N, int frame_count,
                         const float* lW, const float* lb, int harmonic_num,
                         int sample_rate, int upsample_scale, int n_fft,
                         int hop) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, F0 && har && lW && lb && N > 0 && frame_count > 0 && harmonic_num >= 0 && sample_rate > 0 &&
                        upsample_scale > 0 && n_fft >= 2 && n_fft <= MAXN && hop > 0,
               "kdec_harmonic_source: bad arguments");
    const int H = harmonic_num + 1;
    const int sig = frame_count * upsample_scale;
    KDEC_CHECK(ctx, sig > n_fft / 2, "kdec_harmonic_source: signal shorter than the STFT pad");
    const int frames = sig / hop + 1;
    KDEC_CHECK(ctx, har_bs >= static_cast<long>(n_fft + 2) * frames, "kdec_harmonic_source: har stride too small");
    const int nfr = static_cast<int>(cdiv(sig, upsample_scale));
    Workspace st(ctx, static_cast<size_t>(nfr) * N * H * sizeof(float));
    Workspace ph(ctx, static_cast<size_t>(N) * H * ((sig + 3) / 4 * 4) * sizeof(float));
    Workspace mg(ctx, static_cast<size_t>(N) * sig * sizeof(float));
    if (!st.p || !ph.p || !mg.p) return KDEC_ENOMEM;
    ProfScope ps(ctx, "harmonic_source", 0);
    const float sr = static_cast<float>(sample_rate);
    hipLaunchKernelGGL(hs_start_k, dim3(static_cast<unsigned>(cdiv(N * H, 64))), dim3(64), 0, ctx->stream, F0,
                       f0_bs, st.as<float>(), N, H, frame_count, upsample_scale, sig, nfr, sr);
    if (int rc = launch_check(ctx, "hs_start")) return rc;
    hipLaunchKernelGGL(hs_phase_k, dim3(static_cast<unsigned>(cdiv(static_cast<long>(nfr) * N * H, 256))), dim3(256), 0,
                       ctx->stream, st.as<float>(), F0, f0_bs, ph.as<float>(), N, H, frame_count, upsample_scale, sig,
                       nfr, sr);
    if (int rc = launch_check(ctx, "hs_phase")) return rc;
    hipLaunchKernelGGL(hs_merge_k, dim3(static_cast<unsigned>(cdiv(sig, 256)), N), dim3(256), 0, ctx->stream,
                       ph.as<float>(), F0, f0_bs, lW, lb, mg.as<float>(), N, H, frame_count, upsample_scale, sig);
    if (int rc = launch_check(ctx, "hs_merge")) return rc;
    with_nfft_bound(n_fft, [&](auto nm) {
        hipLaunchKernelGGL(hs_stft_k<decltype(nm)::value>, dim3(static_cast<unsigned>(cdiv(frames, FT)), N),
                           dim3(FT), 0, ctx->stream, mg.as<float>(), har, har_bs, sig, n_fft, hop, frames);
    });
    return launch_check(ctx, "hs_stft");
}

int kdec_style_proj_fwd(kdec_ctx* ctx, const float* W, const float* b,
                        const float* style, long style_bs, float* out,
                        long out_bs, int N, int rows, int S) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W && style && out && N > 0 && rows > 0 && S > 0, "kdec_style_proj_fwd: bad arguments");
    // W once, style and out per utterance
    ProfScope ps(ctx, "style_proj", 0, 4.0 * (static_cast<double>(rows) * S + static_cast<double>(N) * (S + rows)));
    const size_t lds = style_fwd_lds_floats(S) * sizeof(float);
    if (lds <= 64 * 1024 && S <= 128 && S % (1024 / STR) == 0 && (reinterpret_cast<unsigned long long>(W) & 15) == 0 &&
        (reinterpret_cast<unsigned long long>(style) & 15) == 0 && style_bs % 4 == 0 &&
        static_cast<long>(rows) * S * 4 < (1L << 31)) {
        const void* k = nullptr;
        switch (S * STR / 1024) {  // slab float4s per thread
            case 1: k = reinterpret_cast<const void*>(&style_fwd_rows_k<1>); break;
            case 2: k = reinterpret_cast<const void*>(&style_fwd_rows_k<2>); break;
            case 3: k = reinterpret_cast<const void*>(&style_fwd_rows_k<3>); break;
            default: k = reinterpret_cast<const void*>(&style_fwd_rows_k<4>); break;
        }
        void* args[] = {&W, &b, &style, &style_bs, &out, &out_bs, &N, &rows, &S};
        if (hipLaunchKernel(k, dim3(static_cast<unsigned>(cdiv(rows, STR))), dim3(256), args, lds, ctx->stream) !=
            hipSuccess)
            return fail(ctx, KDEC_EHIP, "style_proj_fwd: launch failed");
        return launch_check(ctx, "style_proj_fwd");
    }
    const long waves = static_cast<long>(rows) * N;
    hipLaunchKernelGGL(style_fwd_k, dim3(static_cast<unsigned>(cdiv(waves * 64, 256))), dim3(256), 0,
                       ctx->stream, W, b, style, style_bs, out, out_bs, N, rows, S);
    return launch_check(ctx, "style_proj_fwd");
}

int kdec_style_proj_bwd(kdec_ctx* ctx, const float* W, const float* style,
                        long style_bs, const float* dout, long dout_bs,
                        float* dstyle, long dstyle_bs, float beta, float* dW,
                        float* db, int N, int rows, int S) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W && style && dout && N > 0 && rows > 0 && S > 0, "kdec_style_proj_bwd: bad arguments");
    ProfScope ps(ctx, "style_proj", 0,
                 4.0 * (static_cast<double>(rows) * S * ((dstyle ? 1 : 0) + (dW ? 2 : 0)) +
                        static_cast<double>(N) * (rows + S)));
    const size_t xlds = (static_cast<size_t>(STB) * STN + static_cast<size_t>(256 / std::max(S, 1)) * STN * S) *
                        sizeof(float);
    if (dstyle && S >= 64 && S <= 256 && 256 % S == 0 && xlds <= 64 * 1024 &&
        static_cast<long>(rows) * S * 4 < (1L << 31) && cdiv(rows, STB) * N * S * 4 < (1L << 31) &&
        dout_bs >= rows && (static_cast<long>(N) * dout_bs + rows) * 4 < (1L << 31)) {
        const int nblk = static_cast<int>(cdiv(rows, STB));
        Workspace part(ctx, static_cast<size_t>(nblk) * N * S * sizeof(float));
        if (!part.p) return KDEC_ENOMEM;
        float* pp = part.as<float>();
        const void* k = S == 64    ? reinterpret_cast<const void*>(&style_bwd_x_rows_k<STB * 64 / 256>)
                        : S == 128 ? reinterpret_cast<const void*>(&style_bwd_x_rows_k<STB * 128 / 256>)
                                   : reinterpret_cast<const void*>(&style_bwd_x_rows_k<STB * 256 / 256>);
        void* args[] = {&W, &dout, &dout_bs, &pp, &N, &rows, &S};
        if (hipLaunchKernel(k, dim3(static_cast<unsigned>(nblk)), dim3(256), args, xlds, ctx->stream) != hipSuccess)
            return fail(ctx, KDEC_EHIP, "style_bwd_x: launch failed");
        if (int rc = launch_check(ctx, "style_bwd_x")) return rc;
        hipLaunchKernelGGL(style_bwd_x_sum_k, dim3(static_cast<unsigned>(cdiv(static_cast<long>(N) * S, 16))),
                           dim3(1024), 0, ctx->stream, part.as<float>(), nblk, dstyle, dstyle_bs, beta, N, S);
        if (int rc = launch_check(ctx, "style_bwd_x_reduce")) return rc;
    } else if (dstyle) {
        const int nblk = static_cast<int>(cdiv(rows, SR));
        Workspace part(ctx, static_cast<size_t>(nblk) * N * S * sizeof(float));
        if (!part.p) return KDEC_ENOMEM;
        hipLaunchKernelGGL(style_bwd_x_k, dim3(nblk), dim3(256), 0, ctx->stream, W, dout, dout_bs,
                           part.as<float>(), N, rows, S);
        if (int rc = launch_check(ctx, "style_bwd_x")) return rc;
        hipLaunchKernelGGL(style_bwd_x_reduce, dim3(static_cast<unsigned>(cdiv(N * S, 256))), dim3(256), 0,
                           ctx->stream, part.as<float>(), nblk, dstyle, dstyle_bs, beta, N, S);
        if (int rc = launch_check(ctx, "style_bwd_x_reduce")) return rc;
    }
    if (dW) {
        hipLaunchKernelGGL(style_bwd_w_k, dim3(g1(static_cast<long>(rows) * S)), dim3(256), 0, ctx->stream,
                           style, style_bs, dout, dout_bs, dW, db, N, rows, S);
        if (int rc = launch_check(ctx, "style_bwd_w")) return rc;
    }
    return KDEC_OK;
}

int kdec_lora_proj_fwd(kdec_ctx* ctx, const float* W, const float* b, const float* A, const float* B,
                       const float* g, long g_bs, float scale, const int* unit_off, int units, int rank,
                       const float* style, long style_bs, float* H, float* out, long out_bs, int N, int rows,
                       int S) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W && A && B && g && unit_off && style && H && out && N > 0 && rows > 0 && S > 0 && units > 0 &&
                        rank > 0 && g_bs >= 0,
               "kdec_lora_proj_fwd: bad arguments");
    ProfScope ps(ctx, "style_proj", 0);
    const long UR = static_cast<long>(units) * rank;
    hipLaunchKernelGGL(style_fwd_k, dim3(static_cast<unsigned>(cdiv(UR * N * 64, 256))), dim3(256), 0, ctx->stream,
                       A, nullptr, style, style_bs, H, UR, N, static_cast<int>(UR), S);
    if (int rc = launch_check(ctx, "lora_h")) return rc;
    const long waves = static_cast<long>(rows) * N;
    hipLaunchKernelGGL(lora_fwd_k, dim3(static_cast<unsigned>(cdiv(waves * 64, 256))), dim3(256), 0, ctx->stream, W,
                       b, B, g, g_bs, scale, unit_off, units, rank, style, style_bs, H, out, out_bs, N, rows, S);
    return launch_check(ctx, "lora_fwd");
}

int kdec_lora_proj_bwd(kdec_ctx* ctx, const float* W, const float* A, const float* B, const float* g, long g_bs,
                       float scale, const int* unit_off, int units, int rank, const float* style, long style_bs,
                       const float* H, const float* dout, long dout_bs, float* dstyle, long dstyle_bs, float beta,
                       float* dW, float* db, float* dA, float* dB, float* dG, int N, int rows, int S) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W && A && B && g && unit_off && style && H && dout && N > 0 && rows > 0 && S > 0 && units > 0 &&
                        rank > 0 && g_bs >= 0,
               "kdec_lora_proj_bwd: bad arguments");
    // the base projection's share: dstyle = beta*dstyle + W^T dout, dW, db
    if (dstyle || dW)
        if (int rc = kdec_style_proj_bwd(ctx, W, style, style_bs, dout, dout_bs, dstyle, dstyle_bs, beta, dW, db, N,
                                         rows, S))
            return rc;
    ProfScope ps(ctx, "style_proj", 0);
    const long UR = static_cast<long>(units) * rank;
    if (dB) {
        hipLaunchKernelGGL(lora_db_k, dim3(g1(static_cast<long>(rows) * rank)), dim3(256), 0, ctx->stream, g, g_bs,
                           scale, unit_off, units, rank, H, dout, dout_bs, dB, N, rows);
        if (int rc = launch_check(ctx, "lora_db")) return rc;
    }
    if (!dA && !dG && !dstyle) return KDEC_OK;
    Workspace dH(ctx, static_cast<size_t>(N) * UR * sizeof(float));
    Workspace gp(ctx, static_cast<size_t>(N) * UR * sizeof(float));
    if (!dH.p || !gp.p) return KDEC_ENOMEM;
    hipLaunchKernelGGL(lora_dh_k, dim3(static_cast<unsigned>(cdiv(UR * N * 64, 256))), dim3(256), 0, ctx->stream, B,
                       g, g_bs, scale, unit_off, units, rank, H, dout, dout_bs, dH.as<float>(), gp.as<float>(), N);
    if (int rc = launch_check(ctx, "lora_dh")) return rc;
    if (dG) {
        const long NG = g_bs ? N : 1;
        hipLaunchKernelGGL(lora_dg_k, dim3(static_cast<unsigned>(cdiv(NG * rank, 256))), dim3(256), 0, ctx->stream,
                           gp.as<float>(), dG, g_bs, N, units, rank);
        if (int rc = launch_check(ctx, "lora_dg")) return rc;
    }
    // dA += dH^T style and dstyle += A^T dH: the style projection's adjoint over A
    if (dA || dstyle)
        return kdec_style_proj_bwd(ctx, A, style, style_bs, dH.as<float>(), UR, dstyle, dstyle_bs, 1.0f, dA, nullptr,
                                   N, static_cast<int>(UR), S);
    return KDEC_OK;
}

}  // extern "C"

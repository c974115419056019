// Spectral head (polar exp/sin -> iSTFT) forward and adjoint, the harmonic
// source, and the style projection (gamma, beta) = fc(style) with its adjoint.
//
// iSTFT semantics (center, not normalized, onesided; torch.istft): frame f
// contributes window * irfft(spec[f]) at offset f*hop, the overlap-add is
// divided by the summed squared window and the first n_fft/2 samples are
// dropped. irfft ignores the imaginary parts of the DC and Nyquist bins.
// The transforms are n_fft = 20 direct sums with twiddles staged in LDS:
// far too small for an FFT to pay, and direct sums keep the order fixed.
#include "kdec_internal.hpp"

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
    Workspace fb(ctx, static_cast<size_t>(N) * L * n_fft * sizeof(float));
    if (!fb.p) return KDEC_ENOMEM;
    ProfScope ps(ctx, "spectral", 0);
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
    ProfScope ps(ctx, "spectral", 0);
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
    ProfScope ps(ctx, "style_proj", 0);
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
    ProfScope ps(ctx, "style_proj", 0);
    if (dstyle) {
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

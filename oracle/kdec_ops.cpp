// Op-level restatements of the brotensor ops the decoder back half calls.
// TEST INFRASTRUCTURE ONLY (parity oracle); see kdec_oracle.hpp.
//
// Each op cites the reference call site that fixes its contract. Where the
// reference leaves a convention to brotensor (absent), PyTorch semantics are
// used and the test suite pins them against torch on small shapes.
#include "kdec_oracle.hpp"

#include <cmath>
#include <cstring>
#include <stdexcept>

namespace KDO_NS {

namespace {
inline long floordiv(long a, long b) {
    long q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
    return q;
}
}  // namespace

int conv1d_out_len(int L, int k, int s, int p, int d) {
    // modules.h / Appendix of the op contract: floor((L+2p-d(k-1)-1)/s)+1
    return (L + 2 * p - d * (k - 1) - 1) / s + 1;
}

int convt1d_out_len(int L, int k, int s, int p, int op, int d) {
    // kokoro_decoder_backward.cpp:630
    return (L - 1) * s - 2 * p + d * (k - 1) + op + 1;
}

// conv1d (modules.cpp:103-108 -> bt::conv1d). Cross-correlation, zero padding.
void conv1d_forward(const Real* x, const Real* W, const Real* b, int C_in,
                    int L, int C_out, int k, int s, int p, int d, int g,
                    Real* y) {
    const int Lo = conv1d_out_len(L, k, s, p, d);
    const int cig = C_in / g, cog = C_out / g;
#pragma omp parallel for schedule(dynamic)
    for (int co = 0; co < C_out; ++co) {
        std::vector<double> acc(static_cast<std::size_t>(Lo),
                                b ? static_cast<double>(b[co]) : 0.0);
        const int grp = co / cog;
        for (int cl = 0; cl < cig; ++cl) {
            const int ci = grp * cig + cl;
            const Real* xr = x + static_cast<std::size_t>(ci) * L;
            for (int t = 0; t < k; ++t) {
                const double w = W[(static_cast<std::size_t>(co) * cig + cl) * k + t];
                const long off = static_cast<long>(t) * d - p;
                // valid lo: 0 <= lo*s + off < L
                long lo0 = off >= 0 ? 0 : floordiv(-off + s - 1, s);
                long lo1 = floordiv(L - 1 - off, s);
                if (lo1 > Lo - 1) lo1 = Lo - 1;
                for (long lo = lo0; lo <= lo1; ++lo)
                    acc[lo] += w * xr[lo * s + off];
            }
        }
        for (int lo = 0; lo < Lo; ++lo)
            y[static_cast<std::size_t>(co) * Lo + lo] = static_cast<Real>(acc[lo]);
    }
}

// conv1d_backward_input (kokoro_decoder_backward.cpp:230-234): the `L`
// argument there is the input length.
void conv1d_backward_input(const Real* W, const Real* dy, int C_in, int L_in,
                           int C_out, int k, int s, int p, int d, int g,
                           Real* dx) {
    const int Lo = conv1d_out_len(L_in, k, s, p, d);
    const int cig = C_in / g, cog = C_out / g;
#pragma omp parallel for schedule(dynamic)
    for (int ci = 0; ci < C_in; ++ci) {
        std::vector<double> acc(static_cast<std::size_t>(L_in), 0.0);
        const int grp = ci / cig, cl = ci % cig;
        for (int col = 0; col < cog; ++col) {
            const int co = grp * cog + col;
            const Real* dyr = dy + static_cast<std::size_t>(co) * Lo;
            for (int t = 0; t < k; ++t) {
                const double w = W[(static_cast<std::size_t>(co) * cig + cl) * k + t];
                const long off = static_cast<long>(t) * d - p;
                long lo0 = off >= 0 ? 0 : floordiv(-off + s - 1, s);
                long lo1 = floordiv(L_in - 1 - off, s);
                if (lo1 > Lo - 1) lo1 = Lo - 1;
                for (long lo = lo0; lo <= lo1; ++lo)
                    acc[lo * s + off] += w * dyr[lo];
            }
        }
        for (int l = 0; l < L_in; ++l)
            dx[static_cast<std::size_t>(ci) * L_in + l] = static_cast<Real>(acc[l]);
    }
}

// conv1d weight/bias grad with accumulate semantics (the signature the
// reference uses elsewhere, bc_resnet.cpp:1006-1007, 1020-1025).
void conv1d_backward_weight(const Real* x, const Real* dy, int C_in, int L_in,
                            int C_out, int k, int s, int p, int d, int g,
                            Real* dW, Real* db) {
    const int Lo = conv1d_out_len(L_in, k, s, p, d);
    const int cig = C_in / g, cog = C_out / g;
#pragma omp parallel for schedule(dynamic)
    for (int co = 0; co < C_out; ++co) {
        const int grp = co / cog;
        const Real* dyr = dy + static_cast<std::size_t>(co) * Lo;
        for (int cl = 0; cl < cig; ++cl) {
            const int ci = grp * cig + cl;
            const Real* xr = x + static_cast<std::size_t>(ci) * L_in;
            for (int t = 0; t < k; ++t) {
                const long off = static_cast<long>(t) * d - p;
                long lo0 = off >= 0 ? 0 : floordiv(-off + s - 1, s);
                long lo1 = floordiv(L_in - 1 - off, s);
                if (lo1 > Lo - 1) lo1 = Lo - 1;
                double acc = 0.0;
                for (long lo = lo0; lo <= lo1; ++lo)
                    acc += static_cast<double>(dyr[lo]) * xr[lo * s + off];
                Real& dst = dW[(static_cast<std::size_t>(co) * cig + cl) * k + t];
                dst = static_cast<Real>(dst + acc);
            }
        }
        if (db) {
            double acc = 0.0;
            for (int lo = 0; lo < Lo; ++lo) acc += dyr[lo];
            db[co] = static_cast<Real>(db[co] + acc);
        }
    }
}

// conv_transpose1d_forward (kokoro_decoder_backward.cpp:176-180, 627-629).
void convt1d_forward(const Real* x, const Real* W, const Real* b, int C_in,
                     int L, int C_out, int k, int s, int p, int op, int d,
                     int g, Real* y) {
    const int Lo = convt1d_out_len(L, k, s, p, op, d);
    const int cig = C_in / g, cog = C_out / g;
#pragma omp parallel for schedule(dynamic)
    for (int co = 0; co < C_out; ++co) {
        std::vector<double> acc(static_cast<std::size_t>(Lo),
                                b ? static_cast<double>(b[co]) : 0.0);
        const int grp = co / cog, col = co % cog;
        for (int cl = 0; cl < cig; ++cl) {
            const int ci = grp * cig + cl;
            const Real* xr = x + static_cast<std::size_t>(ci) * L;
            for (int t = 0; t < k; ++t) {
                const double w = W[(static_cast<std::size_t>(ci) * cog + col) * k + t];
                const long off = static_cast<long>(t) * d - p;
                for (int l = 0; l < L; ++l) {
                    const long j = static_cast<long>(l) * s + off;
                    if (j >= 0 && j < Lo) acc[j] += w * xr[l];
                }
            }
        }
        for (int j = 0; j < Lo; ++j)
            y[static_cast<std::size_t>(co) * Lo + j] = static_cast<Real>(acc[j]);
    }
}

// conv_transpose1d_backward_input (kokoro_decoder_backward.cpp:252-256,
// 725-728): the strided correlation of dY with W.
void convt1d_backward_input(const Real* W, const Real* dy, int C_in, int L_in,
                            int C_out, int k, int s, int p, int op, int d,
                            int g, Real* dx) {
    const int Lo = convt1d_out_len(L_in, k, s, p, op, d);
    const int cig = C_in / g, cog = C_out / g;
#pragma omp parallel for schedule(dynamic)
    for (int ci = 0; ci < C_in; ++ci) {
        std::vector<double> acc(static_cast<std::size_t>(L_in), 0.0);
        const int grp = ci / cig;
        for (int col = 0; col < cog; ++col) {
            const int co = grp * cog + col;
            const Real* dyr = dy + static_cast<std::size_t>(co) * Lo;
            for (int t = 0; t < k; ++t) {
                const double w = W[(static_cast<std::size_t>(ci) * cog + col) * k + t];
                const long off = static_cast<long>(t) * d - p;
                for (int l = 0; l < L_in; ++l) {
                    const long j = static_cast<long>(l) * s + off;
                    if (j >= 0 && j < Lo) acc[l] += w * dyr[j];
                }
            }
        }
        for (int l = 0; l < L_in; ++l)
            dx[static_cast<std::size_t>(ci) * L_in + l] = static_cast<Real>(acc[l]);
    }
}

void convt1d_backward_weight(const Real* x, const Real* dy, int C_in,
                             int L_in, int C_out, int k, int s, int p, int op,
                             int d, int g, Real* dW, Real* db) {
    const int Lo = convt1d_out_len(L_in, k, s, p, op, d);
    const int cig = C_in / g, cog = C_out / g;
#pragma omp parallel for schedule(dynamic)
    for (int ci = 0; ci < C_in; ++ci) {
        const int grp = ci / cig;
        const Real* xr = x + static_cast<std::size_t>(ci) * L_in;
        for (int col = 0; col < cog; ++col) {
            const int co = grp * cog + col;
            const Real* dyr = dy + static_cast<std::size_t>(co) * Lo;
            for (int t = 0; t < k; ++t) {
                const long off = static_cast<long>(t) * d - p;
                double acc = 0.0;
                for (int l = 0; l < L_in; ++l) {
                    const long j = static_cast<long>(l) * s + off;
                    if (j >= 0 && j < Lo) acc += static_cast<double>(xr[l]) * dyr[j];
                }
                Real& dst = dW[(static_cast<std::size_t>(ci) * cog + col) * k + t];
                dst = static_cast<Real>(dst + acc);
            }
        }
    }
    if (db) {
        for (int co = 0; co < C_out; ++co) {
            double acc = 0.0;
            for (int j = 0; j < Lo; ++j) acc += dy[static_cast<std::size_t>(co) * Lo + j];
            db[co] = static_cast<Real>(db[co] + acc);
        }
    }
}

// group_norm_forward with num_groups == C (kokoro_decoder_backward.cpp:112-113).
void instnorm_forward(const Real* x, const Real* gamma, const Real* beta,
                      int C, int L, float eps, Real* y) {
#pragma omp parallel for
    for (int c = 0; c < C; ++c) {
        const Real* xr = x + static_cast<std::size_t>(c) * L;
        double m = 0.0;
        for (int l = 0; l < L; ++l) m += xr[l];
        m /= L;
        double v = 0.0;
        for (int l = 0; l < L; ++l) { const double e = xr[l] - m; v += e * e; }
        v /= L;
        const double rstd = 1.0 / std::sqrt(v + static_cast<double>(eps));
        for (int l = 0; l < L; ++l)
            y[static_cast<std::size_t>(c) * L + l] =
                static_cast<Real>(gamma[c] * (xr[l] - m) * rstd + beta[c]);
    }
}

// group_norm_backward (kokoro_decoder_backward.cpp:148-149).
void instnorm_backward(const Real* x, const Real* gamma, const Real* dy,
                       int C, int L, float eps, Real* dx, Real* dgamma,
                       Real* dbeta) {
#pragma omp parallel for
    for (int c = 0; c < C; ++c) {
        const Real* xr = x + static_cast<std::size_t>(c) * L;
        const Real* gr = dy + static_cast<std::size_t>(c) * L;
        double m = 0.0;
        for (int l = 0; l < L; ++l) m += xr[l];
        m /= L;
        double v = 0.0;
        for (int l = 0; l < L; ++l) { const double e = xr[l] - m; v += e * e; }
        v /= L;
        const double rstd = 1.0 / std::sqrt(v + static_cast<double>(eps));
        double sdy = 0.0, sdyx = 0.0;
        for (int l = 0; l < L; ++l) {
            const double xh = (xr[l] - m) * rstd;
            sdy += gr[l];
            sdyx += gr[l] * xh;
        }
        if (dgamma) dgamma[c] = static_cast<Real>(sdyx);
        if (dbeta) dbeta[c] = static_cast<Real>(sdy);
        const double gm = gamma[c];
        const double mg = gm * sdy / L, mgx = gm * sdyx / L;
        for (int l = 0; l < L; ++l) {
            const double xh = (xr[l] - m) * rstd;
            dx[static_cast<std::size_t>(c) * L + l] =
                static_cast<Real>(rstd * (gm * gr[l] - mg - xh * mgx));
        }
    }
}

void snake_forward(const Real* x, const Real* alpha, int C, int L, Real* y) {
#pragma omp parallel for
    for (int c = 0; c < C; ++c) {
        const double a = alpha[c];
        for (int l = 0; l < L; ++l) {
            const std::size_t i = static_cast<std::size_t>(c) * L + l;
            const double sn = std::sin(a * x[i]);
            y[i] = static_cast<Real>(x[i] + sn * sn / a);
        }
    }
}

void snake_backward(const Real* x, const Real* alpha, const Real* dy, int C,
                    int L, Real* dx, Real* dalpha) {
#pragma omp parallel for
    for (int c = 0; c < C; ++c) {
        const double a = alpha[c];
        double da = 0.0;
        for (int l = 0; l < L; ++l) {
            const std::size_t i = static_cast<std::size_t>(c) * L + l;
            const double xv = x[i];
            const double sn = std::sin(a * xv);
            const double s2 = std::sin(2.0 * a * xv);
            dx[i] = static_cast<Real>(dy[i] * (1.0 + s2));
            da += dy[i] * (xv * s2 / a - sn * sn / (a * a));
        }
        if (dalpha) dalpha[c] = static_cast<Real>(dalpha[c] + da);
    }
}

void leaky_forward(const Real* x, float slope, std::size_t n, Real* y) {
    for (std::size_t i = 0; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : slope * x[i];
}

void leaky_backward(const Real* x, const Real* dy, float slope,
                    std::size_t n, Real* dx) {
    for (std::size_t i = 0; i < n; ++i) dx[i] = x[i] > 0.0f ? dy[i] : slope * dy[i];
}

// pad1d mode=1 (reflect), pad_left=1, pad_right=0
// (kokoro_decoder_backward.cpp:633-634, 720-721).
void pad_reflect_left1_forward(const Real* x, int C, int L, Real* y) {
    for (int c = 0; c < C; ++c) {
        const Real* xr = x + static_cast<std::size_t>(c) * L;
        Real* yr = y + static_cast<std::size_t>(c) * (L + 1);
        yr[0] = xr[1];
        for (int j = 0; j < L; ++j) yr[j + 1] = xr[j];
    }
}

void pad_reflect_left1_backward(const Real* dy, int C, int L, Real* dx) {
    for (int c = 0; c < C; ++c) {
        const Real* dr = dy + static_cast<std::size_t>(c) * (L + 1);
        Real* xr = dx + static_cast<std::size_t>(c) * L;
        for (int j = 0; j < L; ++j) xr[j] = dr[j + 1];
        xr[1] += dr[0];
    }
}

void nearest2x_forward(const Real* x, int C, int L_in, Real* y) {
    for (int c = 0; c < C; ++c)
        for (int l = 0; l < L_in; ++l) {
            const Real v = x[static_cast<std::size_t>(c) * L_in + l];
            y[static_cast<std::size_t>(c) * 2 * L_in + 2 * l] = v;
            y[static_cast<std::size_t>(c) * 2 * L_in + 2 * l + 1] = v;
        }
}

void nearest2x_backward(const Real* dy, int C, int L_in, Real* dx) {
    for (int c = 0; c < C; ++c)
        for (int l = 0; l < L_in; ++l)
            dx[static_cast<std::size_t>(c) * L_in + l] =
                dy[static_cast<std::size_t>(c) * 2 * L_in + 2 * l] +
                dy[static_cast<std::size_t>(c) * 2 * L_in + 2 * l + 1];
}

Vec hann_periodic(int N) {
    Vec w(static_cast<std::size_t>(N));
    constexpr float kTwoPi = 6.28318530717958647692f;
    for (int n = 0; n < N; ++n)
        w[n] = 0.5f - 0.5f * std::cos(kTwoPi * static_cast<Real>(n) /
                                      static_cast<Real>(N));
    return w;
}

namespace {
// Window of length n_fft: a shorter window is centred and zero-padded
// (torch.istft / torch.stft convention for win_length < n_fft).
std::vector<double> full_window(const Real* window, int n_fft, int win) {
    std::vector<double> w(static_cast<std::size_t>(n_fft), 0.0);
    const int left = (n_fft - win) / 2;
    for (int n = 0; n < win; ++n) w[left + n] = window[n];
    return w;
}
}  // namespace

// istft (kokoro_decoder_backward.cpp:407-409): center, not normalized,
// onesided. Frame f contributes window * irfft(spec[f]) at offset f*hop; the
// overlap-add is divided by the summed squared window, the first n_fft/2
// samples are dropped, signal_len samples kept. irfft ignores the imaginary
// parts of the DC and Nyquist bins.
void istft(const Real* spec, const Real* window, int frames, int signal_len,
           int n_fft, int hop, int win, Real* out) {
    const int F = n_fft / 2 + 1;
    const std::vector<double> w = full_window(window, n_fft, win);
    const int total = n_fft + hop * (frames - 1);
    std::vector<double> ola(static_cast<std::size_t>(total), 0.0),
        env(static_cast<std::size_t>(total), 0.0);
    const double two_pi = 6.283185307179586476925286766559;
    std::vector<double> frame(static_cast<std::size_t>(n_fft));
    for (int f = 0; f < frames; ++f) {
        const Real* S = spec + static_cast<std::size_t>(f) * 2 * F;
        for (int n = 0; n < n_fft; ++n) {
            double acc = S[0];
            if (n_fft % 2 == 0) acc += ((n & 1) ? -1.0 : 1.0) * S[2 * (F - 1)];
            const int kmax = (n_fft % 2 == 0) ? F - 1 : F;
            for (int k = 1; k < kmax; ++k) {
                const double ang = two_pi * static_cast<double>((static_cast<long>(k) * n) % n_fft) / n_fft;
                acc += 2.0 * (S[2 * k] * std::cos(ang) - S[2 * k + 1] * std::sin(ang));
            }
            frame[n] = acc / n_fft;
        }
        for (int n = 0; n < n_fft; ++n) {
            ola[static_cast<std::size_t>(f) * hop + n] += frame[n] * w[n];
            env[static_cast<std::size_t>(f) * hop + n] += w[n] * w[n];
        }
    }
    const int start = n_fft / 2;
    for (int j = 0; j < signal_len; ++j) {
        const int m = start + j;
        if (m >= total || env[m] <= 1e-11)
            throw std::runtime_error("kdo::istft: window envelope vanishes");
        out[j] = static_cast<Real>(ola[m] / env[m]);
    }
}

void istft_backward(const Real* dout, const Real* window, int frames,
                    int signal_len, int n_fft, int hop, int win, Real* dspec) {
    const int F = n_fft / 2 + 1;
    const std::vector<double> w = full_window(window, n_fft, win);
    const int total = n_fft + hop * (frames - 1);
    std::vector<double> env(static_cast<std::size_t>(total), 0.0),
        dola(static_cast<std::size_t>(total), 0.0);
    for (int f = 0; f < frames; ++f)
        for (int n = 0; n < n_fft; ++n)
            env[static_cast<std::size_t>(f) * hop + n] += w[n] * w[n];
    const int start = n_fft / 2;
    for (int j = 0; j < signal_len; ++j) {
        const int m = start + j;
        dola[m] = dout[j] / env[m];
    }
    const double two_pi = 6.283185307179586476925286766559;
    for (int f = 0; f < frames; ++f) {
        Real* D = dspec + static_cast<std::size_t>(f) * 2 * F;
        std::vector<double> dfr(static_cast<std::size_t>(n_fft));
        for (int n = 0; n < n_fft; ++n)
            dfr[n] = dola[static_cast<std::size_t>(f) * hop + n] * w[n] / n_fft;
        for (int k = 0; k < F; ++k) {
            const bool edge = (k == 0) || (n_fft % 2 == 0 && k == F - 1);
            const double c = edge ? 1.0 : 2.0;
            double re = 0.0, im = 0.0;
            for (int n = 0; n < n_fft; ++n) {
                const double ang = two_pi * static_cast<double>((static_cast<long>(k) * n) % n_fft) / n_fft;
                re += dfr[n] * std::cos(ang);
                im -= dfr[n] * std::sin(ang);
            }
            D[2 * k] = static_cast<Real>(c * re);
            D[2 * k + 1] = edge ? 0.0f : static_cast<Real>(c * im);
        }
    }
}

// stft (kokoro_modules.cpp:1638-1644): center with reflect padding, onesided,
// not normalized; frames = len / hop + 1.
int stft(const Real* x, int len, const Real* window, int n_fft, int hop,
         int win, Vec& spec) {
    const int F = n_fft / 2 + 1;
    const int pad = n_fft / 2;
    if (len <= pad) throw std::runtime_error("kdo::stft: signal shorter than pad");
    const std::vector<double> w = full_window(window, n_fft, win);
    const int frames = (len + 2 * pad - n_fft) / hop + 1;
    spec.assign(static_cast<std::size_t>(frames) * 2 * F, 0.0f);
    const double two_pi = 6.283185307179586476925286766559;
    auto at = [&](long i) -> double {  // reflect-padded sample
        long j = i - pad;
        if (j < 0) j = -j;
        if (j >= len) j = 2 * (len - 1) - j;
        return x[j];
    };
#pragma omp parallel for
    for (int f = 0; f < frames; ++f) {
        for (int k = 0; k < F; ++k) {
            double re = 0.0, im = 0.0;
            for (int n = 0; n < n_fft; ++n) {
                const double v = w[n] * at(static_cast<long>(f) * hop + n);
                const double ang = two_pi * static_cast<double>((static_cast<long>(k) * n) % n_fft) / n_fft;
                re += v * std::cos(ang);
                im -= v * std::sin(ang);
            }
            spec[(static_cast<std::size_t>(f) * F + k) * 2] = static_cast<Real>(re);
            spec[(static_cast<std::size_t>(f) * F + k) * 2 + 1] = static_cast<Real>(im);
        }
    }
    return frames;
}

// decoder_lora.h:63-77, decoder_lora.cpp:184-194
void lora_forward(const Real* W, const Real* b, const Real* A, const Real* B,
                  const Real* g, float scale, const Real* s, int rows, int rank,
                  int S, Real* y, Real* h) {
    for (int j = 0; j < rank; ++j) {
        double acc = 0.0;
        for (int k = 0; k < S; ++k) acc += static_cast<double>(A[static_cast<std::size_t>(j) * S + k]) * s[k];
        h[j] = static_cast<Real>(acc);
    }
    for (int r = 0; r < rows; ++r) {
        double acc = b ? static_cast<double>(b[r]) : 0.0;
        for (int k = 0; k < S; ++k) acc += static_cast<double>(W[static_cast<std::size_t>(r) * S + k]) * s[k];
        double lo = 0.0;
        for (int j = 0; j < rank; ++j)
            lo += static_cast<double>(B[static_cast<std::size_t>(r) * rank + j]) * (static_cast<double>(g[j]) * h[j]);
        y[r] = static_cast<Real>(acc + static_cast<double>(scale) * lo);
    }
}

// decoder_lora.cpp:198-207 (lora_backward), plus d(style)
void lora_backward(const Real* W, const Real* A, const Real* B, const Real* g,
                   float scale, const Real* s, const Real* h, const Real* dy,
                   int rows, int rank, int S, Real* dstyle, Real* dW, Real* db,
                   Real* dA, Real* dB, Real* dG) {
    std::vector<double> dhg(static_cast<std::size_t>(rank), 0.0);
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < rank; ++j)
            dhg[j] += static_cast<double>(scale) * B[static_cast<std::size_t>(r) * rank + j] * dy[r];
    if (dB)
        for (int r = 0; r < rows; ++r)
            for (int j = 0; j < rank; ++j) {
                const std::size_t i = static_cast<std::size_t>(r) * rank + j;
                dB[i] = static_cast<Real>(dB[i] + static_cast<double>(scale) * dy[r] * (static_cast<double>(g[j]) * h[j]));
            }
    if (dG)
        for (int j = 0; j < rank; ++j) dG[j] = static_cast<Real>(dG[j] + dhg[j] * h[j]);
    std::vector<double> dh(static_cast<std::size_t>(rank));
    for (int j = 0; j < rank; ++j) dh[j] = dhg[j] * g[j];
    if (dA)
        for (int j = 0; j < rank; ++j)
            for (int k = 0; k < S; ++k) {
                const std::size_t i = static_cast<std::size_t>(j) * S + k;
                dA[i] = static_cast<Real>(dA[i] + dh[j] * s[k]);
            }
    if (dW || db)
        for (int r = 0; r < rows; ++r) {
            if (dW)
                for (int k = 0; k < S; ++k) {
                    const std::size_t i = static_cast<std::size_t>(r) * S + k;
                    dW[i] = static_cast<Real>(dW[i] + static_cast<double>(dy[r]) * s[k]);
                }
            if (db) db[r] = static_cast<Real>(db[r] + dy[r]);
        }
    if (dstyle)
        for (int k = 0; k < S; ++k) {
            double acc = 0.0;
            for (int r = 0; r < rows; ++r) acc += static_cast<double>(W[static_cast<std::size_t>(r) * S + k]) * dy[r];
            for (int j = 0; j < rank; ++j) acc += static_cast<double>(A[static_cast<std::size_t>(j) * S + k]) * dh[j];
            dstyle[k] = static_cast<Real>(dstyle[k] + acc);
        }
}

}  // namespace KDO_NS

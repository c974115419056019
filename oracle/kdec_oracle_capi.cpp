// ctypes-facing C ABI over the CPU oracle. TEST INFRASTRUCTURE ONLY: loaded by
// tests/, the smoke check and the bench's CPU-baseline leg. All pointers are
// host pointers; every entry returns 0 on success and a negative value on
// error (message via ko_last_error()).
#include "kdec_oracle.hpp"

#include <omp.h>

#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>

using namespace kdo;

namespace {
thread_local std::string g_err;

template <class F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

Vec vec(const float* p, std::size_t n) { return Vec(p, p + n); }
}  // namespace

extern "C" {

const char* ko_last_error() { return g_err.c_str(); }

// OpenMP threads for the oracle's parallel loops: n > 0 sets n, n <= 0 all
// the process may use; returns the number now in effect.
int ko_set_threads(int n) {
    omp_set_num_threads(n > 0 ? n : omp_get_num_procs());
    return omp_get_max_threads();
}

int ko_conv1d_out_len(int L, int k, int s, int p, int d) { return conv1d_out_len(L, k, s, p, d); }
int ko_convt1d_out_len(int L, int k, int s, int p, int op, int d) { return convt1d_out_len(L, k, s, p, op, d); }

int ko_conv1d_fwd(const float* x, const float* W, const float* b, float* y,
                  int C_in, int L, int C_out, int k, int s, int p, int d, int g) {
    return guard([&] { conv1d_forward(x, W, b, C_in, L, C_out, k, s, p, d, g, y); });
}
int ko_conv1d_dgrad(const float* W, const float* dy, float* dx, int C_in,
                    int L_in, int C_out, int k, int s, int p, int d, int g) {
    return guard([&] { conv1d_backward_input(W, dy, C_in, L_in, C_out, k, s, p, d, g, dx); });
}
int ko_conv1d_wgrad(const float* x, const float* dy, float* dW, float* db,
                    int C_in, int L_in, int C_out, int k, int s, int p, int d,
                    int g) {
    return guard([&] { conv1d_backward_weight(x, dy, C_in, L_in, C_out, k, s, p, d, g, dW, db); });
}
int ko_convt1d_fwd(const float* x, const float* W, const float* b, float* y,
                   int C_in, int L, int C_out, int k, int s, int p, int op,
                   int d, int g) {
    return guard([&] { convt1d_forward(x, W, b, C_in, L, C_out, k, s, p, op, d, g, y); });
}
int ko_convt1d_dgrad(const float* W, const float* dy, float* dx, int C_in,
                     int L_in, int C_out, int k, int s, int p, int op, int d,
                     int g) {
    return guard([&] { convt1d_backward_input(W, dy, C_in, L_in, C_out, k, s, p, op, d, g, dx); });
}
int ko_convt1d_wgrad(const float* x, const float* dy, float* dW, float* db,
                     int C_in, int L_in, int C_out, int k, int s, int p, int op,
                     int d, int g) {
    return guard([&] { convt1d_backward_weight(x, dy, C_in, L_in, C_out, k, s, p, op, d, g, dW, db); });
}
int ko_instnorm_fwd(const float* x, const float* gamma, const float* beta,
                    float* y, int C, int L, float eps) {
    return guard([&] { instnorm_forward(x, gamma, beta, C, L, eps, y); });
}
int ko_instnorm_bwd(const float* x, const float* gamma, const float* dy,
                    float* dx, float* dgamma, float* dbeta, int C, int L,
                    float eps) {
    return guard([&] { instnorm_backward(x, gamma, dy, C, L, eps, dx, dgamma, dbeta); });
}
int ko_adain_affine_fwd(const float* x, const float* gamma, const float* beta,
                        float* y, int C, int L, float eps) {
    return guard([&] {
        const std::size_t n = static_cast<std::size_t>(C) * L;
        Vec yy, xs;
        adain_affine_forward(vec(x, n), vec(gamma, C), vec(beta, C), C, L, eps, yy, xs);
        std::memcpy(y, yy.data(), n * sizeof(float));
    });
}
int ko_adain_affine_bwd(const float* x, const float* gamma, const float* dy,
                        float* dx, float* dgamma, float* dbeta, int C, int L,
                        float eps) {
    return guard([&] {
        const std::size_t n = static_cast<std::size_t>(C) * L;
        Vec yy, xs, zero(static_cast<std::size_t>(C), 0.0f);
        adain_affine_forward(vec(x, n), vec(gamma, C), zero, C, L, eps, yy, xs);
        Vec dX, dG, dB;
        adain_affine_backward(vec(x, n), xs, vec(gamma, C), vec(dy, n), C, L, eps, dX, dG, dB);
        std::memcpy(dx, dX.data(), n * sizeof(float));
        std::memcpy(dgamma, dG.data(), C * sizeof(float));
        std::memcpy(dbeta, dB.data(), C * sizeof(float));
    });
}
int ko_snake_fwd(const float* x, const float* alpha, float* y, int C, int L) {
    return guard([&] { snake_forward(x, alpha, C, L, y); });
}
int ko_snake_bwd(const float* x, const float* alpha, const float* dy, float* dx,
                 float* dalpha, int C, int L) {
    return guard([&] { snake_backward(x, alpha, dy, C, L, dx, dalpha); });
}
int ko_lora_fwd(const float* W, const float* b, const float* A, const float* B, const float* g, float scale,
                const float* s, int rows, int rank, int S, float* y, float* h) {
    return guard([&] { lora_forward(W, b, A, B, g, scale, s, rows, rank, S, y, h); });
}
int ko_lora_bwd(const float* W, const float* A, const float* B, const float* g, float scale, const float* s,
                const float* h, const float* dy, int rows, int rank, int S, float* dstyle, float* dW, float* db,
                float* dA, float* dB, float* dG) {
    return guard([&] { lora_backward(W, A, B, g, scale, s, h, dy, rows, rank, S, dstyle, dW, db, dA, dB, dG); });
}
int ko_leaky_fwd(const float* x, float slope, long n, float* y) {
    return guard([&] { leaky_forward(x, slope, static_cast<std::size_t>(n), y); });
}
int ko_leaky_bwd(const float* x, const float* dy, float slope, long n, float* dx) {
    return guard([&] { leaky_backward(x, dy, slope, static_cast<std::size_t>(n), dx); });
}
int ko_pad_reflect_left1_fwd(const float* x, int C, int L, float* y) {
    return guard([&] { pad_reflect_left1_forward(x, C, L, y); });
}
int ko_pad_reflect_left1_bwd(const float* dy, int C, int L, float* dx) {
    return guard([&] { pad_reflect_left1_backward(dy, C, L, dx); });
}
int ko_hann(float* w, int N) {
    return guard([&] { Vec h = hann_periodic(N); std::memcpy(w, h.data(), N * sizeof(float)); });
}
int ko_istft(const float* spec, const float* window, float* out, int frames,
             int signal_len, int n_fft, int hop, int win) {
    return guard([&] { istft(spec, window, frames, signal_len, n_fft, hop, win, out); });
}
int ko_istft_bwd(const float* dout, const float* window, float* dspec,
                 int frames, int signal_len, int n_fft, int hop, int win) {
    return guard([&] { istft_backward(dout, window, frames, signal_len, n_fft, hop, win, dspec); });
}
// Returns the frame count (>= 0) or -1; spec_out holds max_frames*2*(n_fft/2+1).
int ko_stft(const float* x, int len, const float* window, int n_fft, int hop,
            int win, float* spec_out, int max_frames) {
    int frames = -1;
    const int rc = guard([&] {
        Vec sp;
        frames = stft(x, len, window, n_fft, hop, win, sp);
        if (frames > max_frames) throw std::runtime_error("ko_stft: output too small");
        std::memcpy(spec_out, sp.data(), sp.size() * sizeof(float));
    });
    return rc ? rc : frames;
}
int ko_spectral_head_fwd(const float* x, int C, int L, const float* W,
                         const float* b, int k, int n_fft, int hop,
                         float* audio, float* post) {
    return guard([&] {
        Conv1d cp;
        cp.in_channels = C; cp.out_channels = n_fft + 2; cp.kernel_size = k;
        cp.padding = (k - 1) / 2;
        cp.W = vec(W, static_cast<std::size_t>(n_fft + 2) * C * k);
        cp.b = vec(b, static_cast<std::size_t>(n_fft + 2));
        SpectralHeadCache cache;
        Vec au;
        const Vec win = hann_periodic(n_fft);
        spectral_head_forward_train(cp, vec(x, static_cast<std::size_t>(C) * L), C, L, win,
                                    n_fft, hop, n_fft, au, cache);
        std::memcpy(audio, au.data(), au.size() * sizeof(float));
        if (post) std::memcpy(post, cache.post.data(), cache.post.size() * sizeof(float));
    });
}
int ko_spectral_head_bwd(const float* x, int C, int L, const float* W,
                         const float* b, int k, int n_fft, int hop,
                         const float* daudio, float* dx, float* dW, float* db) {
    return guard([&] {
        Conv1d cp;
        cp.in_channels = C; cp.out_channels = n_fft + 2; cp.kernel_size = k;
        cp.padding = (k - 1) / 2;
        cp.W = vec(W, static_cast<std::size_t>(n_fft + 2) * C * k);
        cp.b = vec(b, static_cast<std::size_t>(n_fft + 2));
        cp.dW.assign(cp.W.size(), 0.0f);
        cp.db.assign(cp.b.size(), 0.0f);
        SpectralHeadCache cache;
        Vec au;
        const Vec win = hann_periodic(n_fft);
        spectral_head_forward_train(cp, vec(x, static_cast<std::size_t>(C) * L), C, L, win,
                                    n_fft, hop, n_fft, au, cache);
        Vec dX;
        Ext ext;
        ext.wgrad = dW != nullptr;
        spectral_head_backward(cp, cache, win, n_fft, hop, n_fft,
                               vec(daudio, static_cast<std::size_t>(L - 1) * hop), dX, &ext);
        std::memcpy(dx, dX.data(), dX.size() * sizeof(float));
        if (dW) std::memcpy(dW, cp.dW.data(), cp.dW.size() * sizeof(float));
        if (db) std::memcpy(db, cp.db.data(), cp.db.size() * sizeof(float));
    });
}
// Returns stft frames (>= 0) or -1. har_out: (2*(n_fft/2+1)) * max_frames.
int ko_harmonic_source(const float* F0, int frame_count, const float* lW,
                       const float* lb, int harmonic_num, int sample_rate,
                       int upsample_scale, int n_fft, int hop, float* har_out,
                       int max_frames) {
    int frames = -1;
    const int rc = guard([&] {
        HarmonicSource hs;
        hs.harmonic_num = harmonic_num;
        hs.sample_rate = sample_rate;
        hs.upsample_scale = upsample_scale;
        hs.n_fft = n_fft;
        hs.hop_size = hop;
        hs.win_size = n_fft;
        hs.lW = vec(lW, static_cast<std::size_t>(harmonic_num + 1));
        hs.lb = vec(lb, 1);
        int sig = 0;
        Vec har;
        harmonic_source_forward(hs, vec(F0, frame_count), frame_count, sig, frames, har);
        if (frames > max_frames) throw std::runtime_error("ko_harmonic_source: output too small");
        std::memcpy(har_out, har.data(), har.size() * sizeof(float));
    });
    return rc ? rc : frames;
}

}  // extern "C"

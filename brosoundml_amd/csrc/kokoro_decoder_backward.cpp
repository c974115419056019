// brosoundml::detail atoms of the decoder back half on gfx950 — the drop-in
// for the reference's src/kokoro_decoder_backward.cpp. Same entry points and
// op order; each reference brotensor call (or fused group of them) becomes
// one kdec kernel call on the HIP runtime context's stream.
//
// Design notes (where this differs from the reference's op sequence):
//  - AdaIN + its activation run as one fused kernel each way; the (L, C)
//    transposes, the ones_col uploads and the separate modulate pass are gone.
//  - Caches keep the instance-norm statistics and recompute pre-activations
//    from (input, stats, affine) in the backward kernels.
//  - Residual adds, the 1/sqrt(2) and the 1/K resblock mean are folded into
//    conv epilogues; the 1x1 shortcut on a nearest-2x input runs at the input
//    rate (conv1x1 commutes with nearest upsampling, and every output is the
//    same dot product).
//  - nearest2x, exp/sin and the Hann window never touch the host.
#include "kokoro_decoder_backward.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <deque>
#include <string>
#include <vector>

#include "kdec.h"

namespace bt = brotensor;
using bt::Device;
using bt::Tensor;

namespace brosoundml {

namespace {

kdec_ctx* kctx() { return bt::runtime(); }

[[noreturn]] void fail(const std::string& where, const std::string& msg) {
    throw std::runtime_error("brosoundml: " + where + ": " + msg);
}

void ck(int rc, const char* where) {
    if (rc != KDEC_OK)
        throw std::runtime_error(std::string(kdec_last_error(kctx())) + " (in " + where + ")");
}

void need_hip(const Tensor& t, const char* where) {
    if (t.device != Device::HIP || !t.data)
        fail(where, "expected a HIP device tensor (this build has no CPU path)");
}

const float* cp(const Tensor& t) { return static_cast<const float*>(t.data); }
float* mp(const Tensor& t) { return static_cast<float*>(t.data); }
Tensor dev(int r, int c) { return Tensor::empty_on(Device::HIP, r, c); }
Tensor devz(int r, int c) { return Tensor::zeros_on(Device::HIP, r, c); }
long rs(const Tensor& t) { return t.row_stride(); }

// A view of channels [c0, c0+C) of an (N, Ctot*L) tensor.
Tensor chan_view(const Tensor& t, int c0, int C, int L) {
    Tensor v = Tensor::view(t.device, mp(t) + static_cast<long>(c0) * L, t.rows, C * L, t.dtype, rs(t));
    v.storage = t.storage;  // the view keeps its buffer alive
    return v;
}

const float* bias_of(const Conv1d& c) {
    return (c.b.data && static_cast<int>(c.b.size()) == c.out_channels) ? cp(c.b) : nullptr;
}

float* grad_of(const detail::WeightGrads* wg, const Tensor& w) {
    if (!wg || !w.data) return nullptr;
    Tensor* g = wg->find(w);
    return g ? mp(*g) : nullptr;
}

void check_batch(const Tensor& x, int C, int L, const char* where) {
    need_hip(x, where);
    if (x.cols != C * L)
        fail(where, "expected (N, " + std::to_string(C) + "*" + std::to_string(L) + "), got cols " +
                        std::to_string(x.cols));
}

// ─── convolutions ───
void conv_fwd(const Conv1d& c, const Tensor& X, int L, float* Y, long y_bs,
              const float* R = nullptr, long r_bs = 0, float scale = 1.0f, float beta = 0.0f) {
    if (c.groups != 1) fail("Conv1d", "grouped conv1d is not on the decoder path");
    ck(kdec_conv1d_fwd(kctx(), cp(X), rs(X), cp(c.W), bias_of(c), Y, y_bs, X.rows, c.in_channels, L,
                       c.out_channels, c.kernel_size, c.stride, c.padding, c.dilation, R, r_bs, scale,
                       beta),
       "conv1d forward");
}

Tensor conv_fwd(const Conv1d& c, const Tensor& X, int L) {
    Tensor Y = dev(X.rows, c.out_channels * c.out_length(L));
    conv_fwd(c, X, L, mp(Y), rs(Y));
    return Y;
}

// conv_fwd (beta = 0) that also returns the instance-norm statistics of its
// output rows, (N*C_out, 2) (mean, rstd) with eps, where the GEMM's epilogue
// forms them (kdec_conv1d_fwd_stats_fused); elsewhere the plain conv and an
// empty tensor, leaving the statistics to the one-pass AdaIN forward.
Tensor conv_fwd_stats(const Conv1d& c, const Tensor& X, int L, float* Y, long y_bs, const float* R, long r_bs,
                      float eps) {
    if (c.groups != 1) fail("Conv1d", "grouped conv1d is not on the decoder path");
    if (!kdec_conv1d_fwd_stats_fused(kctx(), X.rows, c.in_channels, L, c.out_channels, c.kernel_size, c.stride,
                                     c.padding, c.dilation)) {
        conv_fwd(c, X, L, Y, y_bs, R, r_bs);
        return Tensor();
    }
    Tensor st = dev(X.rows * c.out_channels, 2);
    ck(kdec_conv1d_fwd_stats(kctx(), cp(X), rs(X), cp(c.W), bias_of(c), Y, y_bs, X.rows, c.in_channels, L,
                             c.out_channels, c.kernel_size, c.stride, c.padding, c.dilation, R, r_bs, 1.0f, eps,
                             mp(st)),
       "conv1d forward");
    return st;
}

// dX = scale * dgrad(dY) + beta * dX; L = input length
void conv_dgrad(const Conv1d& c, const Tensor& dY, int L, float* dX, long dx_bs, float scale = 1.0f,
                float beta = 0.0f) {
    ck(kdec_conv1d_dgrad(kctx(), cp(c.W), cp(dY), rs(dY), dX, dx_bs, dY.rows, c.in_channels, L, c.out_channels,
                         c.kernel_size, c.stride, c.padding, c.dilation, scale, beta),
       "conv1d backward_input");
}

Tensor conv_dgrad(const Conv1d& c, const Tensor& dY, int L, float scale = 1.0f) {
    Tensor dX = dev(dY.rows, c.in_channels * L);
    conv_dgrad(c, dY, L, mp(dX), rs(dX), scale);
    return dX;
}

// Weight-grad lane: while set, conv weight grads run on a second context's
// stream, forked from the runtime stream after their inputs are produced, so
// the MFMA-bound weight grads overlap the input-grad chain. Their inputs are
// held until the lane's event for them has completed (then no later kernel
// of the runtime stream can still race with their reads), and join() makes
// the runtime stream wait for everything the lane has queued.
struct WgradLane {
    kdec_ctx* side = nullptr;
    struct Held {
        hipEvent_t ev;
        Tensor a, b;
    };
    std::deque<Held> held;
    std::vector<hipEvent_t> free_ev;

    hipEvent_t event() {
        hipEvent_t e = nullptr;
        if (!free_ev.empty()) {
            e = free_ev.back();
            free_ev.pop_back();
        } else if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            fail("wgrad lane", "hipEventCreate failed");
        }
        return e;
    }
    void release_done() {
        while (!held.empty() && hipEventQuery(held.front().ev) == hipSuccess) {
            free_ev.push_back(held.front().ev);
            held.pop_front();
        }
    }
    void fork() {
        hipEvent_t e = event();
        hipStream_t ms = static_cast<hipStream_t>(kdec_get_stream(kctx()));
        if (hipEventRecord(e, ms) != hipSuccess ||
            hipStreamWaitEvent(static_cast<hipStream_t>(kdec_get_stream(side)), e, 0) != hipSuccess)
            fail("wgrad lane", "fork failed");
        free_ev.push_back(e);  // reusable once recorded again later (record order is stream order)
    }
    void done(const Tensor& a, const Tensor& b) {
        hipEvent_t e = event();
        if (hipEventRecord(e, static_cast<hipStream_t>(kdec_get_stream(side))) != hipSuccess)
            fail("wgrad lane", "event record failed");
        held.push_back({e, a, b});
        release_done();
    }
    void join() {
        if (!side) return;
        hipEvent_t e = event();
        if (hipEventRecord(e, static_cast<hipStream_t>(kdec_get_stream(side))) != hipSuccess ||
            hipStreamWaitEvent(static_cast<hipStream_t>(kdec_get_stream(kctx())), e, 0) != hipSuccess)
            fail("wgrad lane", "join failed");
        // everything queued on the runtime stream from here on runs after the lane's work
        for (auto& h : held) free_ev.push_back(h.ev);
        held.clear();
        free_ev.push_back(e);
    }
};
WgradLane g_lane;

// Extension: the K resblocks of a generator stage read the same input u and
// only meet in the sum of their outputs, so while lanes are set they run on
// up to three streams (forked from the runtime stream once u exists; see
// ctx_for), and so do the stages' noise branches, which read only har. For
// K = 3 each resblock's last conv writes its own buffer (1/K applied) and
// kdec_add3 forms (x0 + x1) + x2 after the join, on one stream as well, so
// both schedules run the same kernels and give the same bits. Other K keep
// the accumulating convs, each waiting for the previous one's event. The
// lanes' streams overlap one branch's epilogues, statistics finalizes and
// AdaIN passes with another branch's GEMM rounds.
//
// Tensors crossing streams: u, the output and the affine views belong to the
// runtime context and are reused only after the join; the branch caches
// belong to the lane contexts, whose next allocation is ordered after the
// next fork, i.e. after every kernel the runtime stream had queued by then.
struct BranchLanes {
    kdec_ctx* lane[2] = {nullptr, nullptr};  // noise branches: stage 0 on [1], later stages on [0]
    std::vector<hipEvent_t> ev;  // [0]: fork, [1 + j]: branch j's last conv done
    std::vector<hipEvent_t> noise_ev;  // [i]: stage i's noise branch done

    bool on() const { return lane[0] != nullptr && lane[1] != nullptr; }
    static hipEvent_t grow(std::vector<hipEvent_t>& v, std::size_t i) {
        while (v.size() <= i) {
            hipEvent_t e = nullptr;
            if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
                fail("resblock lanes", "hipEventCreate failed");
            v.push_back(e);
        }
        return v[i];
    }
    hipEvent_t event(std::size_t i) { return grow(ev, i); }
    hipEvent_t noise_event(std::size_t i) { return grow(noise_ev, i); }
    kdec_ctx* noise_lane(int stage) const { return stage == 0 ? lane[1] : lane[0]; }
    // One branch per stream: 0 on the runtime stream, 1 on lane 0 (in stage
    // 0 behind the later stages' noise branches), 2 on lane 1 (behind stage
    // 0's), further ones alternating. (Putting both short branches on the
    // runtime stream instead, to keep lane 0 free for the noise work, measured
    // 0.3-0.4 ms slower per forward.)
    kdec_ctx* ctx_for(int j, kdec_ctx* main) const { return j == 0 ? main : lane[(j - 1) % 2]; }
    static void wait_on(kdec_ctx* c, hipEvent_t e) {
        if (hipStreamWaitEvent(static_cast<hipStream_t>(kdec_get_stream(c)), e, 0) != hipSuccess)
            fail("resblock lanes", "stream wait failed");
    }
    void fork(kdec_ctx* main) {
        hipEvent_t e = event(0);
        if (hipEventRecord(e, static_cast<hipStream_t>(kdec_get_stream(main))) != hipSuccess)
            fail("resblock lanes", "fork failed");
        for (kdec_ctx* c : lane) wait_on(c, e);
    }
    // the runtime stream waits for every branch's last conv
    void join(kdec_ctx* main, int K) {
        for (int j = 1; j <= K; ++j) wait_on(main, event(static_cast<std::size_t>(j)));
    }
};
BranchLanes g_branch;

// Makes `c` the runtime context for a scope (the previous one comes back on
// exit, also when the scope throws).
struct RuntimeScope {
    kdec_ctx* prev;
    explicit RuntimeScope(kdec_ctx* c) : prev(bt::runtime()) { bt::set_runtime(c); }
    ~RuntimeScope() { bt::set_runtime(prev); }
    RuntimeScope(const RuntimeScope&) = delete;
    RuntimeScope& operator=(const RuntimeScope&) = delete;
};

void conv_wgrad(const Conv1d& c, const detail::WeightGrads* wg, const Tensor& X, int L, const Tensor& dY) {
    float* dW = grad_of(wg, c.W);
    float* db = bias_of(c) ? grad_of(wg, c.b) : nullptr;
    if (!dW && !db) return;
    kdec_ctx* k = kctx();
    if (g_lane.side) {
        g_lane.fork();
        k = g_lane.side;
    }
    const int rc = kdec_conv1d_wgrad(k, cp(X), rs(X), cp(dY), rs(dY), dW, db, X.rows, c.in_channels, L,
                                     c.out_channels, c.kernel_size, c.stride, c.padding, c.dilation);
    if (rc != KDEC_OK) fail("conv1d backward_weight", kdec_last_error(k));
    if (g_lane.side) g_lane.done(X, dY);
}

// ─── AdaIN ───
struct Affine {
    const float* p;
    long bs;
};

bool is_shared(const Tensor& g, int C) {
    return static_cast<int>(g.size()) == C && (g.cols == 1 || g.rows == 1);
}

Affine affine_in(const Tensor& g, int N, int C, const char* where) {
    need_hip(g, where);
    if (is_shared(g, C)) return {cp(g), 0};
    if (g.rows == N && g.cols == C) return {cp(g), rs(g)};
    fail(where, "gamma/beta must be (C,1) or (N,C)");
}

// Destination for a (dGamma, dBeta) pair shaped like gamma. Writes in place
// into tensors that already have that shape on the device (so a caller can
// hand in views of a packed buffer); a shared affine over N > 1 utterances is
// reduced over the batch after the kernel.
struct AffineGrads {
    Tensor* dg;
    Tensor* db;
    bool reduce = false;
    Tensor tg, tb;
    int N, C;
    float* pg = nullptr;
    float* pb = nullptr;
    long bs = 0;

    AffineGrads(Tensor& dG, Tensor& dB, const Tensor& like, int N_, int C_)
        : dg(&dG), db(&dB), N(N_), C(C_) {
        const bool shared = is_shared(like, C);
        if (shared && N > 1) {
            reduce = true;
            tg = dev(N, C);
            tb = dev(N, C);
            pg = mp(tg);
            pb = mp(tb);
            bs = C;
            return;
        }
        const int r = shared ? like.rows : N, c = shared ? like.cols : C;
        auto fits = [&](const Tensor& t) {
            return t.device == Device::HIP && t.data && t.rows == r && t.cols == c;
        };
        if (!fits(dG)) dG = dev(r, c);
        if (!fits(dB) || rs(dB) != rs(dG)) dB = dev(r, c);
        if (rs(dB) != rs(dG)) dG = dev(r, c);
        pg = mp(dG);
        pb = mp(dB);
        bs = shared ? 0 : rs(dG);
    }

    void finish() {
        if (!reduce) return;
        for (int which = 0; which < 2; ++which) {
            Tensor& src = which ? tb : tg;
            Tensor& out = which ? *db : *dg;
            out = dev(C, 1);
            ck(kdec_axpby(kctx(), 1.0f, mp(src), C, 0.0f, nullptr, 0, mp(out), C, 1, C), "affine grad sum");
            for (int n = 1; n < N; ++n)
                ck(kdec_axpby(kctx(), 1.0f, mp(out), C, 1.0f, mp(src) + static_cast<long>(n) * C, C, mp(out), C,
                              1, C),
                   "affine grad sum");
        }
    }
};

Tensor in_stats(const Tensor& x, int C, int L, float eps) {
    Tensor st = dev(x.rows * C, 2);
    ck(kdec_instnorm_stats(kctx(), cp(x), rs(x), x.rows, C, L, eps, mp(st)), "instance-norm statistics");
    return st;
}

// Y = act(adain(x)) into a fresh tensor
Tensor adain_act(const Tensor& x, const Tensor& st, const Tensor& g, const Tensor& b, int C, int L, int act,
                 float slope, const Tensor* alpha, const char* where) {
    const int N = x.rows;
    const Affine ga = affine_in(g, N, C, where), ba = affine_in(b, N, C, where);
    if (ga.bs != ba.bs) fail(where, "gamma and beta must share one layout");
    Tensor y = dev(N, C * L);
    ck(kdec_adain_act_fwd(kctx(), cp(x), rs(x), cp(st), ga.p, ba.p, ga.bs, act, slope, alpha ? cp(*alpha) : nullptr,
                          mp(y), rs(y), nullptr, 0, N, C, L),
       where);
    return y;
}

// Y = act(adain(x)) with the statistics (st, (mean, rstd) per row) computed in
// the same pass over x
Tensor adain_act_stats(const Tensor& x, float eps, Tensor& st, const Tensor& g, const Tensor& b, int C, int L, int act,
                       float slope, const Tensor* alpha, const char* where) {
    const int N = x.rows;
    const Affine ga = affine_in(g, N, C, where), ba = affine_in(b, N, C, where);
    if (ga.bs != ba.bs) fail(where, "gamma and beta must share one layout");
    st = dev(N * C, 2);
    Tensor y = dev(N, C * L);
    ck(kdec_adain_act_fwd_stats(kctx(), cp(x), rs(x), eps, mp(st), ga.p, ba.p, ga.bs, act, slope,
                                alpha ? cp(*alpha) : nullptr, mp(y), rs(y), nullptr, 0, N, C, L),
       where);
    return y;
}

// dX = adain_backward(act_backward(dY)) (+ R)
Tensor adain_act_bwd(const Tensor& x, const Tensor& st, const Tensor& g, const Tensor* b, int C, int L, int act,
                     float slope, const Tensor* alpha, const Tensor& dY, const Tensor* R, Tensor& dG,
                     Tensor& dB, float* dalpha, const char* where) {
    const int N = x.rows;
    const Affine ga = affine_in(g, N, C, where);
    Affine ba{nullptr, ga.bs};
    if (b) {
        ba = affine_in(*b, N, C, where);
        if (ga.bs != ba.bs) fail(where, "gamma and beta must share one layout");
    }
    if (static_cast<long>(st.size()) != 2L * N * C) fail(where, "statistics cache does not match the input");
    Tensor dX = dev(N, C * L);
    AffineGrads out(dG, dB, g, N, C);
    ck(kdec_adain_act_bwd(kctx(), cp(x), rs(x), cp(st), ga.p, ba.p, ga.bs, act, slope,
                          alpha ? cp(*alpha) : nullptr, cp(dY), rs(dY), R ? cp(*R) : nullptr, R ? rs(*R) : 0,
                          mp(dX), rs(dX), out.pg, out.pb, out.bs, dalpha, N, C, L),
       where);
    out.finish();
    return dX;
}

// conv_dgrad of `c` followed by the adain_act_bwd of the AdaIN + activation
// that feeds it (C = c.in_channels), as one kdec call: where the input-grad
// GEMM allows, its epilogue applies the activation derivative and sums the
// AdaIN's rows, so the intermediate grad is not written separately.
Tensor conv_dgrad_adain_bwd(const Conv1d& c, const Tensor& dY, int L, const Tensor& x, const Tensor& st,
                            const Tensor& g, const Tensor* b, int act, float slope, const Tensor* alpha,
                            const Tensor* R, Tensor& dG, Tensor& dB, float* dalpha, const char* where) {
    if (c.groups != 1) fail(where, "grouped conv1d is not on the decoder path");
    const int N = x.rows, C = c.in_channels;
    const Affine ga = affine_in(g, N, C, where);
    Affine ba{nullptr, ga.bs};
    if (b) {
        ba = affine_in(*b, N, C, where);
        if (ga.bs != ba.bs) fail(where, "gamma and beta must share one layout");
    }
    if (static_cast<long>(st.size()) != 2L * N * C) fail(where, "statistics cache does not match the input");
    Tensor dX = dev(N, C * L);
    AffineGrads out(dG, dB, g, N, C);
    ck(kdec_conv1d_dgrad_adain_bwd(kctx(), cp(c.W), cp(dY), rs(dY), N, C, L, c.out_channels, c.kernel_size,
                                   c.stride, c.padding, c.dilation, cp(x), rs(x), cp(st), ga.p, ba.p, ga.bs, act,
                                   slope, alpha ? cp(*alpha) : nullptr, R ? cp(*R) : nullptr, R ? rs(*R) : 0,
                                   mp(dX), rs(dX), out.pg, out.pb, out.bs, dalpha),
       where);
    out.finish();
    return dX;
}

Tensor leaky(const Tensor& x, float slope) {
    Tensor y = dev(x.rows, x.cols);
    ck(kdec_leaky_fwd(kctx(), cp(x), rs(x), mp(y), rs(y), x.rows, x.cols, slope), "leaky_relu forward");
    return y;
}

// dx = scale * leaky_relu_backward(x, dy) (scale 1: the plain backward)
Tensor leaky_bwd(const Tensor& x, const Tensor& dy, float slope, float scale = 1.0f) {
    Tensor dx = dev(x.rows, x.cols);
    if (scale == 1.0f)
        ck(kdec_leaky_bwd(kctx(), cp(x), rs(x), cp(dy), rs(dy), mp(dx), rs(dx), x.rows, x.cols, slope),
           "leaky_relu backward");
    else
        ck(kdec_leaky_bwd_scaled(kctx(), cp(x), rs(x), cp(dy), rs(dy), mp(dx), rs(dx), x.rows, x.cols, slope, scale),
           "leaky_relu backward, scaled");
    return dx;
}

Tensor scaled(const Tensor& x, float a) {
    Tensor y = dev(x.rows, x.cols);
    ck(kdec_axpby(kctx(), a, cp(x), rs(x), 0.0f, nullptr, 0, mp(y), rs(y), x.rows, x.cols), "scale");
    return y;
}

void add_into(Tensor& y, const Tensor& x) {
    ck(kdec_axpby(kctx(), 1.0f, cp(y), rs(y), 1.0f, cp(x), rs(x), mp(y), rs(y), y.rows, y.cols), "add_inplace");
}

// copy x into channels [c0, c0 + C) of the (N, Ctot*L) tensor `dst`
void copy_channels(Tensor& dst, int c0, const Tensor& x, int C, int L) {
    Tensor v = chan_view(dst, c0, C, L);
    ck(kdec_axpby(kctx(), 1.0f, cp(x), rs(x), 0.0f, nullptr, 0, mp(v), rs(v), x.rows, static_cast<long>(C) * L),
       "cat_channels");
}

}  // namespace

// ─── nn-module forwards used by the atoms ───────────────────────────────────

void Conv1d::forward(const Tensor& X, int N, int L, Tensor& Y) const {
    check_batch(X, in_channels, L, "Conv1d::forward");
    if (X.rows != N) fail("Conv1d::forward", "batch mismatch");
    Y = conv_fwd(*this, X, L);
}

void HarmonicSource::forward(const Tensor& F0_pred, int frame_count, int& signal_len, int& stft_frames,
                             Tensor& har) const {
    need_hip(F0_pred, "HarmonicSource::forward");
    need_hip(l_linear.W, "HarmonicSource::forward");
    need_hip(l_linear.b, "HarmonicSource::forward");
    if (F0_pred.cols != frame_count) fail("HarmonicSource::forward", "F0 length mismatch");
    if (win_size != n_fft) fail("HarmonicSource::forward", "win_size must equal n_fft");
    signal_len = frame_count * upsample_scale;
    stft_frames = signal_len / hop_size + 1;
    har = dev(F0_pred.rows, (n_fft + 2) * stft_frames);
    ck(kdec_harmonic_source(kctx(), cp(F0_pred), rs(F0_pred), mp(har), rs(har), F0_pred.rows, frame_count,
                            cp(l_linear.W), cp(l_linear.b), harmonic_num, sample_rate, upsample_scale, n_fft,
                            hop_size),
       "HarmonicSource::forward");
}

namespace detail {

void set_wgrad_lane(kdec_ctx* side) {
    if (g_lane.side && g_lane.side != side) g_lane.join();
    g_lane.side = side;
}

void join_wgrad_lane() { g_lane.join(); }

void set_resblock_lanes(kdec_ctx* a, kdec_ctx* b) {
    g_branch.lane[0] = a && b ? a : nullptr;
    g_branch.lane[1] = a && b ? b : nullptr;
}

// ─── AdaIN affine ───────────────────────────────────────────────────────────

void adain_affine_forward(const Tensor& x_ncl, const Tensor& gamma, const Tensor& beta, int C, int L,
                          float eps, Tensor& y_ncl, Tensor& x_seq_cache) {
    check_batch(x_ncl, C, L, "adain_affine_forward");
    Tensor st;
    y_ncl = adain_act_stats(x_ncl, eps, st, gamma, beta, C, L, KDEC_ACT_NONE, 0.0f, nullptr, "adain_affine_forward");
    x_seq_cache = st;
}

void adain_affine_backward(const Tensor& x_ncl, const Tensor& x_seq_cache, const Tensor& gamma,
                           const Tensor& dY_ncl, int C, int L, float eps, Tensor& dX_ncl, Tensor& dGamma,
                           Tensor& dBeta) {
    check_batch(x_ncl, C, L, "adain_affine_backward");
    check_batch(dY_ncl, C, L, "adain_affine_backward");
    // The statistics are recomputed from x when the cache is not ours.
    const bool ours = x_seq_cache.device == Device::HIP &&
                      static_cast<long>(x_seq_cache.size()) == 2L * x_ncl.rows * C;
    const Tensor st = ours ? x_seq_cache : in_stats(x_ncl, C, L, eps);
    dX_ncl = adain_act_bwd(x_ncl, st, gamma, nullptr, C, L, KDEC_ACT_NONE, 0.0f, nullptr, dY_ncl, nullptr, dGamma,
                           dBeta, nullptr, "adain_affine_backward");
}

// ─── AdainResBlk1d ──────────────────────────────────────────────────────────

namespace {

Tensor pool_fwd(const AdainResBlk1dWeights& w, const Tensor& r, int L_in) {
    const int C = w.channels_in;
    need_hip(w.pool_W, "AdainResBlk1d pool");
    Tensor pooled = dev(r.rows, C * 2 * L_in);
    ck(kdec_pool_fwd(kctx(), cp(r), rs(r), cp(w.pool_W), w.pool_b.data ? cp(w.pool_b) : nullptr, mp(pooled),
                     rs(pooled), r.rows, C, L_in),
       "conv_transpose1d (pool) forward");
    return pooled;
}

}  // namespace

void adain_resblk_1d_forward_train(const AdainResBlk1dWeights& w, const Tensor& x, int L_in,
                                   const Tensor& gamma1, const Tensor& beta1, const Tensor& gamma2,
                                   const Tensor& beta2, float eps, int& L_out, Tensor& y,
                                   AdainResBlkCache& cache) {
    const char* where = "adain_resblk_1d_forward_train";
    const int C_in = w.channels_in, C_out = w.channels_out;
    check_batch(x, C_in, L_in, where);
    const int N = x.rows;
    L_out = w.upsample ? 2 * L_in : L_in;
    cache.x = x;
    cache.L_in = L_in;
    cache.L_out = L_out;
    cache.beta1 = beta1;
    cache.beta2 = beta2;
    cache.r_pre = Tensor();
    cache.n2_pre = Tensor();

    // residual: adain1 -> leaky 0.2 -> [pool] -> conv1 -> adain2 -> leaky -> conv2
    Tensor r = adain_act_stats(x, eps, cache.x_seq1, gamma1, beta1, C_in, L_in, KDEC_ACT_LEAKY, 0.2f, nullptr, where);
    Tensor pooled = w.upsample ? pool_fwd(w, r, L_in) : r;
    r = Tensor();
    cache.conv1_out = conv_fwd(w.conv1, pooled, L_out);
    pooled = Tensor();
    Tensor n2 = adain_act_stats(cache.conv1_out, eps, cache.x_seq2, gamma2, beta2, C_out, L_out, KDEC_ACT_LEAKY, 0.2f,
                                nullptr, where);

    // shortcut: [nearest2x] -> [conv1x1]  (1x1 applied before the upsample)
    Tensor sc;
    if (w.learned_sc) {
        Tensor s_small = conv_fwd(w.conv1x1, x, L_in);
        if (w.upsample) {
            sc = dev(N, C_out * L_out);
            ck(kdec_nearest2x_fwd(kctx(), cp(s_small), rs(s_small), mp(sc), rs(sc), N, C_out, L_in), where);
        } else {
            sc = s_small;
        }
    } else if (w.upsample) {
        sc = dev(N, C_in * L_out);
        ck(kdec_nearest2x_fwd(kctx(), cp(x), rs(x), mp(sc), rs(sc), N, C_in, L_in), where);
    } else {
        sc = x;
    }
    // y = (conv2(n2) + shortcut) / sqrt(2)
    y = dev(N, C_out * L_out);
    conv_fwd(w.conv2, n2, L_out, mp(y), rs(y), cp(sc), rs(sc), 1.0f / std::sqrt(2.0f), 0.0f);
}

void adain_resblk_1d_backward(const AdainResBlk1dWeights& w, const AdainResBlkCache& cache, const Tensor& gamma1,
                              const Tensor& gamma2, const Tensor& dY, float eps, Tensor& dX, Tensor& dGamma1,
                              Tensor& dBeta1, Tensor& dGamma2, Tensor& dBeta2, const WeightGrads* wg) {
    (void)eps;
    const char* where = "adain_resblk_1d_backward";
    const int C_in = w.channels_in, C_out = w.channels_out;
    const int L_in = cache.L_in, L_out = cache.L_out;
    check_batch(dY, C_out, L_out, where);
    const int N = dY.rows;
    const float inv_sqrt2 = 1.0f / std::sqrt(2.0f);
    const bool want_w = wg != nullptr;

    // conv2: d_n2 = dgrad(dY / sqrt(2))
    Tensor d_n2 = conv_dgrad(w.conv2, dY, L_out, inv_sqrt2);
    Tensor d_branch;
    if (want_w && (grad_of(wg, w.conv2.W) || grad_of(wg, w.conv2.b))) {
        d_branch = scaled(dY, inv_sqrt2);
        Tensor n2 = adain_act(cache.conv1_out, cache.x_seq2, gamma2, cache.beta2, C_out, L_out, KDEC_ACT_LEAKY,
                              0.2f, nullptr, where);
        conv_wgrad(w.conv2, wg, n2, L_out, d_branch);
    }
    // leaky + adain2
    Tensor d_conv1_out = adain_act_bwd(cache.conv1_out, cache.x_seq2, gamma2, &cache.beta2, C_out, L_out,
                                       KDEC_ACT_LEAKY, 0.2f, nullptr, d_n2, nullptr, dGamma2, dBeta2, nullptr,
                                       where);
    d_n2 = Tensor();
    // conv1
    Tensor d_pooled = conv_dgrad(w.conv1, d_conv1_out, L_out);
    if (want_w) {
        const bool need_conv1 = grad_of(wg, w.conv1.W) || grad_of(wg, w.conv1.b);
        const bool need_pool = w.upsample && (grad_of(wg, w.pool_W) || grad_of(wg, w.pool_b));
        if (need_conv1 || need_pool) {
            Tensor r = adain_act(cache.x, cache.x_seq1, gamma1, cache.beta1, C_in, L_in, KDEC_ACT_LEAKY, 0.2f,
                                 nullptr, where);
            if (need_conv1) {
                Tensor pooled = w.upsample ? pool_fwd(w, r, L_in) : r;
                conv_wgrad(w.conv1, wg, pooled, L_out, d_conv1_out);
            }
            if (need_pool) {
                float* dW = grad_of(wg, w.pool_W);
                float* db = grad_of(wg, w.pool_b);
                Tensor tmpW, tmpb;
                if (!dW) { tmpW = devz(C_in, 3); dW = mp(tmpW); }
                ck(kdec_pool_wgrad(kctx(), cp(r), rs(r), cp(d_pooled), rs(d_pooled), dW, db, N, C_in, L_in),
                   "conv_transpose1d (pool) backward_weight");
            }
        }
    }
    d_conv1_out = Tensor();
    Tensor d_r;
    if (w.upsample) {
        d_r = dev(N, C_in * L_in);
        ck(kdec_pool_dgrad(kctx(), cp(w.pool_W), cp(d_pooled), rs(d_pooled), mp(d_r), rs(d_r), N, C_in, L_in),
           "conv_transpose1d (pool) backward_input");
    } else {
        d_r = d_pooled;
    }
    d_pooled = Tensor();

    // shortcut: adjoint of conv1x1(nearest2x(x)) / sqrt(2)
    Tensor dX_short;
    if (w.learned_sc) {
        Tensor g_small;  // grad at the 1x1 output, folded to L_in
        if (w.upsample) {
            g_small = dev(N, C_out * L_in);
            ck(kdec_nearest2x_bwd(kctx(), cp(dY), rs(dY), mp(g_small), rs(g_small), N, C_out, L_in, inv_sqrt2, 0.0f),
               where);
            dX_short = conv_dgrad(w.conv1x1, g_small, L_in);
        } else {
            dX_short = conv_dgrad(w.conv1x1, dY, L_in, inv_sqrt2);
            if (want_w && grad_of(wg, w.conv1x1.W)) g_small = d_branch.data ? d_branch : scaled(dY, inv_sqrt2);
        }
        if (want_w && grad_of(wg, w.conv1x1.W)) conv_wgrad(w.conv1x1, wg, cache.x, L_in, g_small);
    } else if (w.upsample) {
        dX_short = dev(N, C_in * L_in);
        ck(kdec_nearest2x_bwd(kctx(), cp(dY), rs(dY), mp(dX_short), rs(dX_short), N, C_in, L_in, inv_sqrt2, 0.0f),
           where);
    } else {
        dX_short = scaled(dY, inv_sqrt2);
    }
    // leaky + adain1, plus the shortcut contribution
    dX = adain_act_bwd(cache.x, cache.x_seq1, gamma1, &cache.beta1, C_in, L_in, KDEC_ACT_LEAKY, 0.2f, nullptr, d_r,
                       &dX_short, dGamma1, dBeta1, nullptr, where);
}

// ─── AdaINResBlock1 ─────────────────────────────────────────────────────────

namespace {

using Arr3 = std::array<Tensor, 3>;

// Forward of one AdaINResBlock1; the last sub-block writes
// out = out_scale * (conv2 + bias + x) + out_beta * out.
// With `out_wait`, the last conv waits for that event first; with
// `out_done`, the event is recorded after it (the resblock lanes' order).
void resblock1_fwd(const AdaINResBlock1Weights& w, const Tensor& x_in, int C, int L, const Arr3& g1,
                   const Arr3& b1, const Arr3& g2, const Arr3& b2, float* out, long out_bs, float out_scale,
                   float out_beta, AdainResBlock1Cache& cache, hipEvent_t out_wait = nullptr,
                   hipEvent_t out_done = nullptr) {
    const char* where = "adain_resblock1_forward_train";
    check_batch(x_in, C, L, where);
    const int N = x_in.rows;
    cache.C = C;
    cache.L = L;
    auto eps_of = [](const AdaIN1dWeights& a) { return a.eps > 0.0f ? a.eps : 1e-5f; };
    Tensor x = x_in;
    Tensor x_st;  // statistics of x, when the conv that produced it formed them
    for (int i = 0; i < 3; ++i) {
        cache.x_in[i] = x;
        cache.beta1[i] = b1[i];
        cache.beta2[i] = b2[i];
        cache.s1_pre[i] = Tensor();
        cache.s2_pre[i] = Tensor();
        Tensor xt1;
        if (x_st.data) {
            cache.x_seq1[i] = x_st;
            xt1 = adain_act(x, x_st, g1[i], b1[i], C, L, KDEC_ACT_SNAKE, 0.0f, &w.alpha1[i], where);
        } else {
            xt1 = adain_act_stats(x, eps_of(w.adain1[i]), cache.x_seq1[i], g1[i], b1[i], C, L, KDEC_ACT_SNAKE, 0.0f,
                                  &w.alpha1[i], where);
        }
        Tensor c1 = dev(N, C * L);
        const Tensor st2 = conv_fwd_stats(w.convs1[i], xt1, L, mp(c1), rs(c1), nullptr, 0, eps_of(w.adain2[i]));
        cache.c1_out[i] = c1;
        cache.act1[i] = xt1;
        Tensor xt2;
        if (st2.data) {
            cache.x_seq2[i] = st2;
            xt2 = adain_act(c1, st2, g2[i], b2[i], C, L, KDEC_ACT_SNAKE, 0.0f, &w.alpha2[i], where);
        } else {
            xt2 = adain_act_stats(c1, eps_of(w.adain2[i]), cache.x_seq2[i], g2[i], b2[i], C, L, KDEC_ACT_SNAKE, 0.0f,
                                  &w.alpha2[i], where);
        }
        cache.act2[i] = xt2;
        if (i < 2) {
            Tensor xn = dev(N, C * L);
            x_st = conv_fwd_stats(w.convs2[i], xt2, L, mp(xn), rs(xn), cp(x), rs(x), eps_of(w.adain1[i + 1]));
            x = xn;
        } else {
            hipStream_t st = static_cast<hipStream_t>(kdec_get_stream(kctx()));
            if (out_wait && hipStreamWaitEvent(st, out_wait, 0) != hipSuccess)
                fail(where, "waiting for the previous resblock's output");
            conv_fwd(w.convs2[i], xt2, L, out, out_bs, cp(x), rs(x), out_scale, out_beta);
            if (out_done && hipEventRecord(out_done, st) != hipSuccess) fail(where, "event record failed");
        }
    }
}

Tensor resblock1_bwd(const AdaINResBlock1Weights& w, const AdainResBlock1Cache& cache, const Arr3& g1,
                     const Arr3& g2, const Tensor& dX_out, Arr3& dG1, Arr3& dB1, Arr3& dG2, Arr3& dB2,
                     const WeightGrads* wg) {
    const char* where = "adain_resblock1_backward";
    const int C = cache.C, L = cache.L;
    check_batch(dX_out, C, L, where);
    Tensor dx = dX_out;
    for (int i = 2; i >= 0; --i) {
        // convs2[i] -> snake2 -> adain2
        if (wg && (grad_of(wg, w.convs2[i].W) || grad_of(wg, w.convs2[i].b))) {
            const Tensor xt2 = cache.act2[i].data ? cache.act2[i]
                                                  : adain_act(cache.c1_out[i], cache.x_seq2[i], g2[i], cache.beta2[i],
                                                              C, L, KDEC_ACT_SNAKE, 0.0f, &w.alpha2[i], where);
            conv_wgrad(w.convs2[i], wg, xt2, L, dx);
        }
        Tensor d_c1 = conv_dgrad_adain_bwd(w.convs2[i], dx, L, cache.c1_out[i], cache.x_seq2[i], g2[i],
                                           &cache.beta2[i], KDEC_ACT_SNAKE, 0.0f, &w.alpha2[i], nullptr, dG2[i],
                                           dB2[i], grad_of(wg, w.alpha2[i]), where);
        // convs1[i] -> snake1 -> adain1 (+ the residual skip)
        if (wg && (grad_of(wg, w.convs1[i].W) || grad_of(wg, w.convs1[i].b))) {
            const Tensor xt1 = cache.act1[i].data ? cache.act1[i]
                                                  : adain_act(cache.x_in[i], cache.x_seq1[i], g1[i], cache.beta1[i],
                                                              C, L, KDEC_ACT_SNAKE, 0.0f, &w.alpha1[i], where);
            conv_wgrad(w.convs1[i], wg, xt1, L, d_c1);
        }
        dx = conv_dgrad_adain_bwd(w.convs1[i], d_c1, L, cache.x_in[i], cache.x_seq1[i], g1[i], &cache.beta1[i],
                                  KDEC_ACT_SNAKE, 0.0f, &w.alpha1[i], &dx, dG1[i], dB1[i], grad_of(wg, w.alpha1[i]),
                                  where);
        d_c1 = Tensor();
    }
    return dx;
}

}  // namespace

void adain_resblock1_forward_train(const AdaINResBlock1Weights& w, const Tensor& x_in, int C, int L,
                                   const std::array<Tensor, 3>& g1, const std::array<Tensor, 3>& b1,
                                   const std::array<Tensor, 3>& g2, const std::array<Tensor, 3>& b2,
                                   Tensor& x_out, AdainResBlock1Cache& cache) {
    check_batch(x_in, C, L, "adain_resblock1_forward_train");
    Tensor out = dev(x_in.rows, C * L);
    resblock1_fwd(w, x_in, C, L, g1, b1, g2, b2, mp(out), rs(out), 1.0f, 0.0f, cache);
    x_out = out;
}

void adain_resblock1_backward(const AdaINResBlock1Weights& w, const AdainResBlock1Cache& cache,
                              const std::array<Tensor, 3>& g1, const std::array<Tensor, 3>& g2,
                              const Tensor& dX_out, Tensor& dX_in, std::array<Tensor, 3>& dG1,
                              std::array<Tensor, 3>& dB1, std::array<Tensor, 3>& dG2, std::array<Tensor, 3>& dB2,
                              const WeightGrads* wgrads) {
    dX_in = resblock1_bwd(w, cache, g1, g2, dX_out, dG1, dB1, dG2, dB2, wgrads);
}

// ─── Spectral head ──────────────────────────────────────────────────────────

namespace {
const float* window_ptr(const Tensor& window, int n_fft, int win, const char* where) {
    if (win != n_fft) fail(where, "win_length must equal n_fft");
    if (!window.data) return nullptr;  // periodic Hann
    need_hip(window, where);
    if (static_cast<int>(window.size()) != n_fft) fail(where, "window length must equal n_fft");
    return cp(window);
}
}  // namespace

void spectral_head_forward_train(const Conv1d& conv_post, const Tensor& x, int C, int L, const Tensor& window,
                                 int n_fft, int hop, int win, Tensor& audio, SpectralHeadCache& cache,
                                 const Tensor* x_act) {
    const char* where = "spectral_head_forward_train";
    check_batch(x, C, L, where);
    if (conv_post.out_channels != n_fft + 2) fail(where, "conv_post must produce n_fft + 2 channels");
    const float* wp = window_ptr(window, n_fft, win, where);
    cache.C = C;
    cache.L = L;
    cache.x_pre = x;
    if (x_act && x_act->data) check_batch(*x_act, C, L, where);
    Tensor xl = x_act && x_act->data ? *x_act : leaky(x, 0.01f);
    cache.x_act = xl;
    cache.post = conv_fwd(conv_post, xl, L);
    audio = dev(x.rows, (L - 1) * hop);
    ck(kdec_spectral_fwd(kctx(), cp(cache.post), rs(cache.post), wp, mp(audio), rs(audio), x.rows, L, n_fft, hop),
       where);
}

void spectral_head_backward(const Conv1d& conv_post, const SpectralHeadCache& cache, const Tensor& window,
                            int n_fft, int hop, int win, const Tensor& dAudio, Tensor& dX,
                            const WeightGrads* wgrads, float dx_scale) {
    const char* where = "spectral_head_backward";
    const int C = cache.C, L = cache.L;
    check_batch(dAudio, 1, (L - 1) * hop, where);
    const float* wp = window_ptr(window, n_fft, win, where);
    const int N = dAudio.rows;
    Tensor dpost = dev(N, (n_fft + 2) * L);
    ck(kdec_spectral_bwd(kctx(), cp(cache.post), rs(cache.post), wp, cp(dAudio), rs(dAudio), mp(dpost), rs(dpost), N,
                         L, n_fft, hop),
       where);
    Tensor dXl = conv_dgrad(conv_post, dpost, L);
    if (wgrads && (grad_of(wgrads, conv_post.W) || grad_of(wgrads, conv_post.b))) {
        const Tensor xl = cache.x_act.data ? cache.x_act : leaky(cache.x_pre, 0.01f);
        conv_wgrad(conv_post, wgrads, xl, L, dpost);
    }
    dX = leaky_bwd(cache.x_pre, dXl, 0.01f, dx_scale);
    (void)C;
}

// ─── DecoderBackbone ────────────────────────────────────────────────────────

void decoder_backbone_forward_train(const DecoderBackbone& bb, const Tensor& asr, const Tensor& F0_pred,
                                    const Tensor& N_pred, int T, const std::vector<BlockAffines>& aff, float eps,
                                    Tensor& gen_in, BackboneCache& cache) {
    const char* where = "decoder_backbone_forward_train";
    const int n_dec = static_cast<int>(bb.decode.size());
    if (static_cast<int>(aff.size()) < 1 + n_dec) fail(where, "one BlockAffines per block expected");
    const int C_asr = bb.asr_res.in_channels;
    check_batch(asr, C_asr, T, where);
    check_batch(F0_pred, 1, 2 * T, where);
    check_batch(N_pred, 1, 2 * T, where);
    const int N = asr.rows;
    cache.T = T;
    cache.decode.assign(n_dec, AdainResBlkCache{});
    cache.res_applied.assign(n_dec, 0);
    cache.x_channels.assign(n_dec, 0);
    if (cache.keep) {
        cache.asr = asr;
        cache.F0 = F0_pred;
        cache.N = N_pred;
    }

    // the channels every residual decode block appends, cat[asr_res, F0_dn,
    // N_dn], written in place by their convs (one copy per block after)
    const int C_res = bb.asr_res.out_channels;
    if (bb.F0_conv.out_channels != 1 || bb.N_conv.out_channels != 1 || bb.F0_conv.out_length(2 * T) != T ||
        bb.N_conv.out_length(2 * T) != T || bb.asr_res.out_length(T) != T)
        fail(where, "F0/N downsample length mismatch");
    Tensor tail = dev(N, (C_res + 2) * T);
    conv_fwd(bb.asr_res, asr, T, mp(tail), rs(tail));
    conv_fwd(bb.F0_conv, F0_pred, 2 * T, mp(tail) + static_cast<long>(C_res) * T, rs(tail));
    conv_fwd(bb.N_conv, N_pred, 2 * T, mp(tail) + static_cast<long>(C_res + 1) * T, rs(tail));

    // encode over cat[asr, F0_dn, N_dn]
    Tensor dec_pre = dev(N, (C_asr + 2) * T);
    copy_channels(dec_pre, 0, asr, C_asr, T);
    copy_channels(dec_pre, C_asr, chan_view(tail, C_res, 2, T), 2, T);
    int L_after = 0;
    Tensor x;
    adain_resblk_1d_forward_train(bb.encode, dec_pre, T, aff[0].g1, aff[0].b1, aff[0].g2, aff[0].b2, eps, L_after,
                                  x, cache.encode);
    if (!cache.keep) cache.encode = AdainResBlkCache{};
    int L_now = L_after;
    bool res = true;
    for (int i = 0; i < n_dec; ++i) {
        const int Cx = x.cols / L_now;
        cache.x_channels[i] = Cx;
        Tensor blk_in;
        if (res) {
            cache.res_applied[i] = 1;
            if (L_now != T) fail(where, "a residual decode block after the upsampling one");
            blk_in = dev(N, (Cx + C_res + 2) * L_now);
            copy_channels(blk_in, 0, x, Cx, L_now);
            copy_channels(blk_in, Cx, tail, C_res + 2, L_now);
        } else {
            blk_in = x;
        }
        int L_next = 0;
        Tensor y;
        adain_resblk_1d_forward_train(bb.decode[i], blk_in, L_now, aff[1 + i].g1, aff[1 + i].b1, aff[1 + i].g2,
                                      aff[1 + i].b2, eps, L_next, y, cache.decode[i]);
        if (!cache.keep) cache.decode[i] = AdainResBlkCache{};
        x = y;
        L_now = L_next;
        if (bb.decode[i].upsample) res = false;
    }
    gen_in = x;
}

void decoder_backbone_backward(const DecoderBackbone& bb, const BackboneCache& cache,
                               const std::vector<BlockAffines>& aff, const Tensor& dGenIn, float eps,
                               std::vector<BlockAffines>& dAff, const WeightGrads* wg) {
    const int n_dec = static_cast<int>(bb.decode.size());
    dAff.resize(static_cast<std::size_t>(n_dec) + 1);
    const int T = cache.T;
    const int N = dGenIn.rows;
    const int C_res = bb.asr_res.out_channels;
    const bool front = wg && (grad_of(wg, bb.F0_conv.W) || grad_of(wg, bb.N_conv.W) || grad_of(wg, bb.asr_res.W) ||
                              grad_of(wg, bb.F0_conv.b) || grad_of(wg, bb.N_conv.b) || grad_of(wg, bb.asr_res.b));
    // grads of the appended channels cat[asr_res, F0_dn, N_dn], summed over
    // the residual blocks (and the encoder's F0 / N channels) in block order
    Tensor d_tail;
    if (front) d_tail = devz(N, (C_res + 2) * T);

    Tensor dX = dGenIn;
    for (int i = n_dec - 1; i >= 0; --i) {
        Tensor blk_dX;
        BlockAffines& g = dAff[1 + i];
        adain_resblk_1d_backward(bb.decode[i], cache.decode[i], aff[1 + i].g1, aff[1 + i].g2, dX, eps, blk_dX, g.g1,
                                 g.b1, g.g2, g.b2, wg);
        if (cache.res_applied[i]) {
            const int Cx = cache.x_channels[i];
            const int L_in = cache.decode[i].L_in;
            if (front) add_into(d_tail, chan_view(blk_dX, Cx, C_res + 2, L_in));
            // the leading x channels flow on; the frozen-input channels drop
            Tensor sliced = chan_view(blk_dX, 0, Cx, L_in);
            sliced.storage = blk_dX.storage;
            dX = sliced;
        } else {
            dX = blk_dX;
        }
    }
    Tensor enc_dX;
    BlockAffines& ge = dAff[0];
    adain_resblk_1d_backward(bb.encode, cache.encode, aff[0].g1, aff[0].g2, dX, eps, enc_dX, ge.g1, ge.b1, ge.g2,
                             ge.b2, wg);
    if (front) {
        const int C_asr = bb.asr_res.in_channels;
        Tensor d_fn = chan_view(d_tail, C_res, 2, T);
        add_into(d_fn, chan_view(enc_dX, C_asr, 2, T));
        conv_wgrad(bb.F0_conv, wg, cache.F0, 2 * T, chan_view(d_tail, C_res, 1, T));
        conv_wgrad(bb.N_conv, wg, cache.N, 2 * T, chan_view(d_tail, C_res + 1, 1, T));
        conv_wgrad(bb.asr_res, wg, cache.asr, T, chan_view(d_tail, 0, C_res, T));
    }
}

// ─── Generator ──────────────────────────────────────────────────────────────

void generator_forward_train(const Generator& gen, const Tensor& gen_in, int L_in, const Tensor& har, int frames,
                             const std::vector<ResBlock1Affines>& naff, const std::vector<ResBlock1Affines>& raff,
                             Tensor& audio, GeneratorCache& cache) {
    const char* where = "generator_forward_train";
    const int K = gen.num_kernels;
    const int U = gen.num_upsamples;
    if (static_cast<int>(naff.size()) < U || static_cast<int>(raff.size()) < U * K)
        fail(where, "one ResBlock1Affines per noise_res / resblock expected");
    check_batch(gen_in, gen.ups_C_in[0], L_in, where);
    check_batch(har, gen.noise_convs.empty() ? gen.n_fft + 2 : gen.noise_convs[0].in_channels, frames, where);
    const int N = gen_in.rows;
    cache.stages.resize(U);
    if (cache.keep) cache.har = har;
    cache.frames = frames;

    // With the lanes set, every stage's noise branch (noise_convs[i] ->
    // noise_res[i]) reads only har, so all of them are queued first, in stage
    // order (stage 0 on lane 1, the others on lane 0, so that stage 1's runs
    // beside stage 0's); each stage's runtime stream waits for its own.
    kdec_ctx* const main_ctx = kctx();
    const bool par = g_branch.on();
    if (!par) cache.inputs_ready = nullptr;
    std::vector<Tensor> srcs(static_cast<std::size_t>(U));
    std::vector<int> src_len(static_cast<std::size_t>(U), 0);
    if (par) {
        if (cache.har_ready && cache.inputs_ready) {
            // har and the affines are all the noise branches read besides
            // their weights: they need not wait for the backbone
            for (kdec_ctx* c : g_branch.lane) {
                BranchLanes::wait_on(c, static_cast<hipEvent_t>(cache.inputs_ready));
                BranchLanes::wait_on(c, static_cast<hipEvent_t>(cache.har_ready));
            }
        } else {
            g_branch.fork(main_ctx);  // har may have been written on the runtime stream
            if (cache.har_ready)
                for (kdec_ctx* c : g_branch.lane) BranchLanes::wait_on(c, static_cast<hipEvent_t>(cache.har_ready));
        }
        cache.har_ready = nullptr;  // the runtime stream joins through the noise events
        cache.inputs_ready = nullptr;
        for (int i = 0; i < U; ++i) {
            kdec_ctx* const nl = g_branch.noise_lane(i);
            RuntimeScope scope(nl);
            const int C_out = gen.ups_C_out[i];
            Tensor x_source = conv_fwd(gen.noise_convs[i], har, frames);
            src_len[i] = x_source.cols / C_out;
            adain_resblock1_forward_train(gen.noise_res[i], x_source, C_out, src_len[i], naff[i].g1, naff[i].b1,
                                          naff[i].g2, naff[i].b2, srcs[i], cache.stages[i].noise);
            if (!cache.keep) cache.stages[i].noise = AdainResBlock1Cache{};
            if (hipEventRecord(g_branch.noise_event(static_cast<std::size_t>(i)),
                               static_cast<hipStream_t>(kdec_get_stream(nl))) != hipSuccess)
                fail(where, "event record failed");
        }
    }

    Tensor x = gen_in;
    Tensor x_act;  // leaky_relu of x for the next layer, when already formed
    int L = L_in;
    for (int i = 0; i < U; ++i) {
        GenStageCache& sc = cache.stages[i];
        if (cache.keep) sc.x_in = x;
        sc.C_in = gen.ups_C_in[i];
        sc.L_in = L;
        const int C_out = gen.ups_C_out[i];
        // leaky_relu(x, 0.1): formed by the previous stage's resblock sum when
        // that ran as one kdec_add3_leaky pass
        Tensor a = x_act.data ? x_act : leaky(x, 0.1f);
        x_act = Tensor();
        if (cache.keep) sc.a = a;

        // ups (+ left reflect pad on the last stage) + the noise source: the
        // transposed conv adds the source in its epilogue (kdec_convt1d_fwd_res;
        // on the last stage it also writes the reflected column), so it runs
        // once the noise branch is done.
        const int kL = gen.ups_k[i], s = gen.ups_stride[i], p = gen.ups_pad[i];
        const bool last = i == U - 1;
        int L_x = (L - 1) * s - 2 * p + (kL - 1) + 1;
        const float* ub = gen.ups_b[i].data ? cp(gen.ups_b[i]) : nullptr;
        Tensor u;

        // noise branch
        Tensor src;
        int L_src = 0;
        if (par) {
            BranchLanes::wait_on(main_ctx, g_branch.noise_event(static_cast<std::size_t>(i)));
            src = srcs[i];
            srcs[i] = Tensor();
            L_src = src_len[i];
        } else {
            if (cache.har_ready) {
                if (hipStreamWaitEvent(static_cast<hipStream_t>(kdec_get_stream(kctx())),
                                       static_cast<hipEvent_t>(cache.har_ready), 0) != hipSuccess)
                    fail(where, "waiting for the harmonic source");
                cache.har_ready = nullptr;
            }
            Tensor x_source = conv_fwd(gen.noise_convs[i], har, frames);
            L_src = x_source.cols / C_out;
            adain_resblock1_forward_train(gen.noise_res[i], x_source, C_out, L_src, naff[i].g1, naff[i].b1,
                                          naff[i].g2, naff[i].b2, src, sc.noise);
            if (!cache.keep) sc.noise = AdainResBlock1Cache{};
        }
        if (last) L_x += 1;  // reflection_pad (1, 0)
        if (L_src != L_x)
            fail(where, "noise source length " + std::to_string(L_src) + " != upsampled length " +
                            std::to_string(L_x) + " at stage " + std::to_string(i));
        sc.C_out = C_out;
        sc.L_out = L_x;
        u = dev(N, C_out * L_x);
        ck(kdec_convt1d_fwd_res(kctx(), cp(a), rs(a), cp(gen.ups_W[i]), ub, mp(u), rs(u), N, sc.C_in, L, C_out, kL,
                                s, p, 0, cp(src), rs(src), last ? 1 : 0),
           last ? "conv_transpose1d forward + reflection_pad + noise source" : "conv_transpose1d forward + noise source");
        a = Tensor();
        src = Tensor();

        // x = mean_j resblocks[i*K + j](u): each block's last conv accumulates
        // (on the resblock lanes when they are set, in the same accumulation order)
        sc.res.resize(K);
        Tensor xs = dev(N, C_out * L_x);
        const bool par_rb = par && K > 1;
        const bool sep = K == 3;  // separate outputs summed by kdec_add3, on one stream too
        Tensor outs[2];
        if (sep)
            for (Tensor& o : outs) o = dev(N, C_out * L_x);
        if (par_rb) g_branch.fork(main_ctx);
        for (int j = 0; j < K; ++j) {
            const ResBlock1Affines& ra = raff[static_cast<std::size_t>(i) * K + j];
            RuntimeScope scope(par_rb ? g_branch.ctx_for(j, main_ctx) : main_ctx);
            const Tensor& dst = sep && j > 0 ? outs[j - 1] : xs;
            const bool acc = j > 0 && !sep;
            resblock1_fwd(gen.resblocks[static_cast<std::size_t>(i) * K + j], u, C_out, L_x, ra.g1, ra.b1, ra.g2,
                          ra.b2, mp(dst), rs(dst), 1.0f / static_cast<float>(K), acc ? 1.0f : 0.0f, sc.res[j],
                          par_rb && acc ? g_branch.event(static_cast<std::size_t>(j)) : nullptr,
                          par_rb ? g_branch.event(static_cast<std::size_t>(j) + 1) : nullptr);
            if (!cache.keep) sc.res[j] = AdainResBlock1Cache{};
        }
        if (par_rb) g_branch.join(main_ctx, K);
        if (sep) {
            // the sum and the activation the next layer reads (the next
            // stage's ups: slope 0.1; conv_post: 0.01), in one pass
            x_act = dev(N, C_out * L_x);
            ck(kdec_add3_leaky(main_ctx, cp(xs), rs(xs), cp(outs[0]), rs(outs[0]), cp(outs[1]), rs(outs[1]), mp(xs),
                               rs(xs), mp(x_act), rs(x_act), N, static_cast<long>(C_out) * L_x,
                               last ? 0.01f : 0.1f),
               "resblock sum");
        }
        x = xs;
        L = L_x;
    }
    // an empty window: the spectral kernels form the periodic Hann of
    // kokoro_decoder_backward.cpp:580-588 themselves (hann_at, the same float
    // formula), so no host-built window is uploaded (an upload would block
    // the host until the stream drains)
    cache.window = Tensor();
    spectral_head_forward_train(gen.conv_post, x, gen.ups_C_out[U - 1], L, cache.window, gen.n_fft, gen.hop_size,
                                gen.win_size, audio, cache.head, &x_act);
    x_act = Tensor();
    if (!cache.keep) cache.head = SpectralHeadCache{};
}

void generator_backward(const Generator& gen, const GeneratorCache& cache, const std::vector<ResBlock1Affines>& naff,
                        const std::vector<ResBlock1Affines>& raff, const Tensor& dAudio, Tensor& dGenIn,
                        std::vector<ResBlock1Affines>& dnaff, std::vector<ResBlock1Affines>& draff,
                        const WeightGrads* wg) {
    const int K = gen.num_kernels;
    const int U = gen.num_upsamples;
    dnaff.resize(U);
    draff.resize(static_cast<std::size_t>(U) * K);

    // dX: the grad into the stage output x already divided by the K
    // resblocks (mean over the resblocks) for every stage but the first
    // one's input: the leaky backwards that form it apply the 1/K
    Tensor dX;
    spectral_head_backward(gen.conv_post, cache.head, cache.window, gen.n_fft, gen.hop_size, gen.win_size, dAudio,
                           dX, wg, 1.0f / static_cast<float>(K));
    const int N = dAudio.rows;
    // With the resblock lanes set (the caller does so when no conv weight
    // grads occupy a second stream), each stage's resblock backwards run on
    // the runtime stream and both lanes, and every stage's noise branch
    // backward on lane 1 (its input grad feeds only weight grads, so the
    // runtime stream joins it once, at the end). The tensors lane work reads
    // are held until that join.
    kdec_ctx* const main_ctx = kctx();
    const bool par = g_branch.on() && K == 3;
    std::vector<Tensor> lane_inputs;
    hipEvent_t noise_last = nullptr;
    auto record_on = [](hipEvent_t e, kdec_ctx* c) {
        if (hipEventRecord(e, static_cast<hipStream_t>(kdec_get_stream(c))) != hipSuccess)
            fail("generator_backward", "event record failed");
    };
    for (int i = U - 1; i >= 0; --i) {
        const GenStageCache& sc = cache.stages[i];
        const int L = sc.L_out;
        const int C_out = sc.C_out;
        Tensor d_scaled = dX;
        dX = Tensor();
        // d_m = sum_j of the resblocks' input grads, in the order j = 0, 1, ...
        // (one pass for K = 3)
        if (par) g_branch.fork(main_ctx);
        std::vector<Tensor> dxin(static_cast<std::size_t>(K));
        for (int j = 0; j < K; ++j) {
            const std::size_t idx = static_cast<std::size_t>(i) * K + j;
            ResBlock1Affines& dr = draff[idx];
            kdec_ctx* const cj = par ? g_branch.ctx_for(j, main_ctx) : main_ctx;
            RuntimeScope scope(cj);
            dxin[static_cast<std::size_t>(j)] = resblock1_bwd(gen.resblocks[idx], sc.res[j], raff[idx].g1,
                                                              raff[idx].g2, d_scaled, dr.g1, dr.b1, dr.g2, dr.b2, wg);
            if (par && j > 0) record_on(g_branch.event(static_cast<std::size_t>(j) + 1), cj);
        }
        if (par)
            for (int j = 1; j < K; ++j) BranchLanes::wait_on(main_ctx, g_branch.event(static_cast<std::size_t>(j) + 1));
        Tensor d_m = dxin[0];
        // the last stage's input was left reflect padded by one sample: its
        // adjoint (du_pre) comes out of the pass that sums the resblock grads
        Tensor du_pre;
        if (K == 3 && i == U - 1) {
            du_pre = dev(N, C_out * (L - 1));
            ck(kdec_add3_unpad_left1(kctx(), cp(d_m), rs(d_m), cp(dxin[1]), rs(dxin[1]), cp(dxin[2]), rs(dxin[2]),
                                     mp(d_m), rs(d_m), mp(du_pre), rs(du_pre), N, C_out, L - 1),
               "resblock grad sum and pad1d backward");
        } else if (K == 3) {
            ck(kdec_add3(kctx(), cp(d_m), rs(d_m), cp(dxin[1]), rs(dxin[1]), cp(dxin[2]), rs(dxin[2]), mp(d_m), rs(d_m),
                         N, d_m.cols),
               "resblock grad sum");
        } else {
            for (int j = 1; j < K; ++j) add_into(d_m, dxin[static_cast<std::size_t>(j)]);
        }
        dxin.clear();
        d_scaled = Tensor();
        {
            ResBlock1Affines& dn = dnaff[i];
            kdec_ctx* const nl = par ? g_branch.lane[1] : main_ctx;
            if (par) {
                record_on(g_branch.noise_event(static_cast<std::size_t>(i)), main_ctx);
                BranchLanes::wait_on(nl, g_branch.noise_event(static_cast<std::size_t>(i)));
                lane_inputs.push_back(d_m);
            }
            RuntimeScope scope(nl);
            Tensor dsrc_in = resblock1_bwd(gen.noise_res[i], sc.noise, naff[i].g1, naff[i].g2, d_m, dn.g1, dn.b1,
                                           dn.g2, dn.b2, wg);
            if (wg) conv_wgrad(gen.noise_convs[i], wg, cache.har, cache.frames, dsrc_in);
            if (par) {
                noise_last = g_branch.noise_event(static_cast<std::size_t>(U + i));
                record_on(noise_last, nl);
            }
        }
        Tensor du = d_m;
        if (i == U - 1) {
            if (!du_pre.data) {
                du_pre = dev(N, C_out * (L - 1));
                ck(kdec_pad_reflect_left1_bwd(kctx(), cp(d_m), rs(d_m), mp(du_pre), rs(du_pre), N, C_out, L - 1),
                   "pad1d backward");
            }
            du = du_pre;
        }
        d_m = Tensor();
        Tensor da = dev(N, sc.C_in * sc.L_in);
        ck(kdec_convt1d_dgrad(kctx(), cp(gen.ups_W[i]), cp(du), rs(du), mp(da), rs(da), N, sc.C_in, sc.L_in, C_out,
                              gen.ups_k[i], gen.ups_stride[i], gen.ups_pad[i], 0),
           "conv_transpose1d backward_input");
        if (wg) {
            float* dW = grad_of(wg, gen.ups_W[i]);
            float* db = grad_of(wg, gen.ups_b[i]);
            if (dW || db) {
                // on the weight-grad lane when one is set (as the conv weight
                // grads), with the leaky input the forward kept (or
                // recomputed there)
                kdec_ctx* k = kctx();
                if (g_lane.side) {
                    g_lane.fork();
                    k = g_lane.side;
                }
                Tensor a = sc.a;
                if (!a.data) {
                    a = dev(N, sc.C_in * sc.L_in);
                    const int rc1 = kdec_leaky_fwd(k, cp(sc.x_in), rs(sc.x_in), mp(a), rs(a), N, a.cols, 0.1f);
                    if (rc1 != KDEC_OK) fail("generator_backward", kdec_last_error(k));
                }
                const int rc2 = kdec_convt1d_wgrad(k, cp(a), rs(a), cp(du), rs(du), dW, db, N, sc.C_in, sc.L_in, C_out,
                                                   gen.ups_k[i], gen.ups_stride[i], gen.ups_pad[i], 0);
                if (rc2 != KDEC_OK) fail("conv_transpose1d backward_weight", kdec_last_error(k));
                if (g_lane.side) g_lane.done(a, du);  // both held until the lane is past them
            }
        }
        dX = leaky_bwd(sc.x_in, da, 0.1f, i > 0 ? 1.0f / static_cast<float>(K) : 1.0f);
    }
    if (noise_last) BranchLanes::wait_on(main_ctx, noise_last);  // lane 1 is in order: its last event covers all
    lane_inputs.clear();
    dGenIn = dX;
}

}  // namespace detail
}  // namespace brosoundml

// Whole-decoder model over the C++ drop-in atoms: named parameters in one
// device buffer, the per-AdaIN style projection batched over all units, and
// the forward / backward sequence of DecoderLora (decoder_lora.cpp:211-296)
// without the LoRA term.
#include <functional>
#include <map>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "kdec.h"
#include "kdec_internal.hpp"
#include "kdec_model.h"
#include "brosoundml/decoder_lora.h"
#include "brosoundml/kokoro.h"
#include "kokoro_decoder_backward.h"

namespace bt = brotensor;
using bt::Device;
using bt::Tensor;
namespace bd = brosoundml::detail;

struct kdec_model {
    kdec_ctx* ctx = nullptr;
    // configuration
    int asr_dim = 0, asr_res_dim = 0, style_dim = 0, enc_dim = 0, n_decode = 0;
    int dec_out[8] = {}, dec_up_at = -1, n_ups = 0, ups_rates[4] = {}, ups_kernels[4] = {};
    int n_kernels = 0, rb_kernels[4] = {}, rb_dil[4][3] = {};
    int n_fft = 0, hop = 0, conv_post_k = 0, sample_rate = 0, harmonic_num = 0;

    brosoundml::DecoderBackbone bb;
    brosoundml::Generator gen;
    brosoundml::HarmonicSource hs;

    struct Param {
        Tensor* value = nullptr;  // points into a module struct
        Tensor grad;
        Tensor grad2;             // the second batch part's share (gbuf2)
        int rows = 0, cols = 0;
        long offset = 0;          // into the flat buffers
    };
    std::vector<std::string> order;
    std::map<std::string, Param> params;
    Tensor pbuf, gbuf;            // flat parameter / grad storage
    // The second batch part's conv / alpha weight grads accumulate here while
    // the two parts' backwards run concurrently; gbuf then adds it.
    Tensor gbuf2;
    long total = 0;

    struct Unit {
        std::string name;
        int C = 0;
        int offset = 0;           // row offset in the stacked fc
    };
    std::vector<Unit> units;
    int rows_total = 0;
    std::vector<brosoundml::AdaIN1dWeights*> unit_w;  // same order as units

    bd::WeightGrads wg_all, wg_conv, wg_alpha;
    bd::WeightGrads wg_all2, wg_conv2, wg_alpha2;  // into gbuf2

    // per forward
    int N = 0, T = 0;
    Tensor style_v, gb, dgb;
    // The batch runs as one or (kdec_model_set_batch_split) two parts:
    // contiguous row ranges, each a whole backbone + generator chain with its
    // own affine views and caches on its own context (part 0 on ctx, part 1
    // on ctx2, each with its allocator and stream), forwards and backwards
    // concurrent; part 1's conv weight grads accumulate into gbuf2 (on side2)
    // and are added to gbuf at the end.
    struct Part {
        int n0 = 0, n = 0;          // rows [n0, n0 + n)
        kdec_ctx* ctx = nullptr;
        std::vector<bd::BlockAffines> bbaff, dbbaff;
        std::vector<bd::ResBlock1Affines> naff, raff, dnaff, draff;
        bd::BackboneCache bbc;
        bd::GeneratorCache genc;
        Tensor gen_in;
    };
    Part part[2];
    int parts = 0;                  // of the last training forward
    bool split = false;             // kdec_model_set_batch_split
    kdec_ctx* ctx2 = nullptr;
    kdec_ctx* side2 = nullptr;      // part 1's conv weight-grad stream
    hipEvent_t ev_split = nullptr, ev_part1 = nullptr;
    Tensor har;
    mutable Tensor gen_in_all;      // both parts' generator inputs, on demand
    std::string err;

    // The harmonic source depends only on F0: it runs on a side context's
    // stream, forked after the inputs and joined before the generator, so it
    // overlaps the style projection and the backbone.
    kdec_ctx* side = nullptr;
    bool overlap = true;  // use `side` at all (kdec_model_set_overlap)
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;

    // DecoderLora adapters (off at lora_rank 0): A (units*rank, S), B
    // (rows_total, rank), their grads, the unit row offsets (units+1 int32
    // in a 4-byte-element buffer), the gate set for the forwards and the
    // bottleneck H (N, units*rank) of the last forward.
    int lora_rank = 0;
    float lora_scale = 0.0f;
    Tensor loraA, loraB, dloraA, dloraB, unit_off, lora_H;
    const float* gate = nullptr;
    long gate_bs = 0;
    float* dgate = nullptr;
};

namespace {

struct Spec {
    std::string name;
    Tensor* t;
    int rows, cols;
    int kind;  // 0 conv/convT/pool weight or bias, 1 alpha, 2 fc weight, 3 fc bias, 4 forward-only
};

void conv_geom(brosoundml::Conv1d& c, int cin, int cout, int k, int s, int p, int d) {
    c.in_channels = cin;
    c.out_channels = cout;
    c.kernel_size = k;
    c.stride = s;
    c.padding = p;
    c.dilation = d;
    c.groups = 1;
}

// Errors are reported through the context's last-error message.
int fail(kdec_model* m, int code, const std::string& msg) {
    if (m) m->err = msg;
    if (m && m->ctx) m->ctx->err = msg.rfind("brosoundml:", 0) == 0 ? msg : "brosoundml: kdec_model: " + msg;
    return code;
}

// Builds the module structs and the parameter list (names, shapes, kinds).
void build(kdec_model* m, std::vector<Spec>& specs) {
    const int S = m->style_dim;
    const std::string P = "decoder.module.";
    auto conv = [&](const std::string& pfx, brosoundml::Conv1d& c, bool bias) {
        specs.push_back({pfx + ".weight", &c.W, c.out_channels, c.in_channels * c.kernel_size, 0});
        if (bias) specs.push_back({pfx + ".bias", &c.b, c.out_channels, 1, 0});
    };
    auto adain = [&](const std::string& pfx, brosoundml::AdaIN1dWeights& a, int C) {
        a.channels = C;
        a.style_dim = S;
        a.eps = 1e-5f;
        a.fc.in_features = S;
        a.fc.out_features = 2 * C;
        m->units.push_back({pfx, C, m->rows_total});
        m->unit_w.push_back(&a);
        m->rows_total += 2 * C;
    };

    conv_geom(m->bb.F0_conv, 1, 1, 3, 2, 1, 1);
    conv_geom(m->bb.N_conv, 1, 1, 3, 2, 1, 1);
    conv_geom(m->bb.asr_res, m->asr_dim, m->asr_res_dim, 1, 1, 0, 1);
    conv(P + "F0_conv", m->bb.F0_conv, true);
    conv(P + "N_conv", m->bb.N_conv, true);
    conv(P + "asr_res.0", m->bb.asr_res, true);

    auto resblk = [&](brosoundml::AdainResBlk1dWeights& w, int din, int dout, bool up, const std::string& pfx) {
        w.channels_in = din;
        w.channels_out = dout;
        w.upsample = up;
        w.learned_sc = din != dout;
        adain(pfx + ".norm1", w.norm1, din);
        adain(pfx + ".norm2", w.norm2, dout);
        conv_geom(w.conv1, din, dout, 3, 1, 1, 1);
        conv_geom(w.conv2, dout, dout, 3, 1, 1, 1);
        conv(pfx + ".conv1", w.conv1, true);
        conv(pfx + ".conv2", w.conv2, true);
        if (w.learned_sc) {
            conv_geom(w.conv1x1, din, dout, 1, 1, 0, 1);
            conv(pfx + ".conv1x1", w.conv1x1, false);
        }
        if (up) {
            specs.push_back({pfx + ".pool.weight", &w.pool_W, din, 3, 0});
            specs.push_back({pfx + ".pool.bias", &w.pool_b, din, 1, 0});
        }
    };
    resblk(m->bb.encode, m->asr_dim + 2, m->enc_dim, false, P + "encode");
    m->bb.decode.assign(m->n_decode, brosoundml::AdainResBlk1dWeights{});
    int prev = m->enc_dim;
    bool res = true;
    for (int i = 0; i < m->n_decode; ++i) {
        const bool up = i == m->dec_up_at;
        const int din = res ? prev + m->asr_res_dim + 2 : prev;
        resblk(m->bb.decode[i], din, m->dec_out[i], up, P + "decode." + std::to_string(i));
        prev = m->dec_out[i];
        if (up) res = false;
    }

    const int init_C = m->dec_out[m->n_decode - 1];
    const std::string G = P + "generator.";
    auto& g = m->gen;
    g.n_fft = m->n_fft;
    g.hop_size = m->hop;
    g.win_size = m->n_fft;
    g.num_upsamples = m->n_ups;
    g.num_kernels = m->n_kernels;
    g.ups_W.resize(m->n_ups);
    g.ups_b.resize(m->n_ups);
    g.ups_C_in.resize(m->n_ups);
    g.ups_C_out.resize(m->n_ups);
    g.ups_k.resize(m->n_ups);
    g.ups_stride.resize(m->n_ups);
    g.ups_pad.resize(m->n_ups);
    for (int i = 0; i < m->n_ups; ++i) {
        const int ci = init_C >> i, co = init_C >> (i + 1);
        g.ups_C_in[i] = ci;
        g.ups_C_out[i] = co;
        g.ups_k[i] = m->ups_kernels[i];
        g.ups_stride[i] = m->ups_rates[i];
        g.ups_pad[i] = (m->ups_kernels[i] - m->ups_rates[i]) / 2;
        specs.push_back({G + "ups." + std::to_string(i) + ".weight", &g.ups_W[i], ci, co * m->ups_kernels[i], 0});
        specs.push_back({G + "ups." + std::to_string(i) + ".bias", &g.ups_b[i], co, 1, 0});
    }
    g.noise_convs.resize(m->n_ups);
    for (int i = 0; i < m->n_ups; ++i) {
        const int co = init_C >> (i + 1);
        if (i + 1 < m->n_ups) {
            int sf = 1;
            for (int j = i + 1; j < m->n_ups; ++j) sf *= m->ups_rates[j];
            conv_geom(g.noise_convs[i], m->n_fft + 2, co, 2 * sf, sf, (sf + 1) / 2, 1);
        } else {
            conv_geom(g.noise_convs[i], m->n_fft + 2, co, 1, 1, 0, 1);
        }
        conv(G + "noise_convs." + std::to_string(i), g.noise_convs[i], true);
    }
    auto rb1 = [&](brosoundml::AdaINResBlock1Weights& w, int C, int k, const int* dil, const std::string& pfx,
                   std::vector<Spec>& alpha_specs) {
        w.channels = C;
        w.kernel_size = k;
        w.dilations.assign(dil, dil + 3);
        for (int j = 0; j < 3; ++j) {
            const std::string js = std::to_string(j);
            conv_geom(w.convs1[j], C, C, k, 1, (k * dil[j] - dil[j]) / 2, dil[j]);
            conv_geom(w.convs2[j], C, C, k, 1, (k - 1) / 2, 1);
            conv(pfx + ".convs1." + js, w.convs1[j], true);
            conv(pfx + ".convs2." + js, w.convs2[j], true);
            alpha_specs.push_back({pfx + ".alpha1." + js, &w.alpha1[j], C, 1, 1});
            alpha_specs.push_back({pfx + ".alpha2." + js, &w.alpha2[j], C, 1, 1});
        }
        for (int j = 0; j < 3; ++j) adain(pfx + ".adain1." + std::to_string(j), w.adain1[j], C);
        for (int j = 0; j < 3; ++j) adain(pfx + ".adain2." + std::to_string(j), w.adain2[j], C);
    };
    const int dil135[3] = {1, 3, 5};
    std::vector<Spec> alphas;
    g.noise_res.resize(m->n_ups);
    for (int i = 0; i < m->n_ups; ++i)
        rb1(g.noise_res[i], init_C >> (i + 1), i + 1 < m->n_ups ? 7 : 11, dil135,
            G + "noise_res." + std::to_string(i), alphas);
    g.resblocks.resize(static_cast<std::size_t>(m->n_ups) * m->n_kernels);
    for (int i = 0; i < m->n_ups; ++i)
        for (int j = 0; j < m->n_kernels; ++j) {
            const int idx = i * m->n_kernels + j;
            rb1(g.resblocks[idx], init_C >> (i + 1), m->rb_kernels[j], m->rb_dil[j],
                G + "resblocks." + std::to_string(idx), alphas);
        }
    specs.insert(specs.end(), alphas.begin(), alphas.end());
    conv_geom(g.conv_post, init_C >> m->n_ups, m->n_fft + 2, m->conv_post_k, 1, (m->conv_post_k - 1) / 2, 1);
    conv(G + "conv_post", g.conv_post, true);

    auto& h = m->hs;
    h.sample_rate = m->sample_rate;
    h.harmonic_num = m->harmonic_num;
    h.n_fft = m->n_fft;
    h.hop_size = m->hop;
    h.win_size = m->n_fft;
    int upr = 1;
    for (int i = 0; i < m->n_ups; ++i) upr *= m->ups_rates[i];
    h.upsample_scale = upr * m->hop;
    h.l_linear.in_features = m->harmonic_num + 1;
    h.l_linear.out_features = 1;
    specs.push_back({G + "m_source.l_linear.weight", &h.l_linear.W, 1, m->harmonic_num + 1, 4});
    specs.push_back({G + "m_source.l_linear.bias", &h.l_linear.b, 1, 1, 4});

    // the style fc of every unit, stacked (weights then biases) in unit order
    for (std::size_t u = 0; u < m->units.size(); ++u) {
        auto* a = m->unit_w[u];
        specs.push_back({m->units[u].name + ".fc.weight", &a->fc.W, 2 * a->channels, S, 2});
    }
    for (std::size_t u = 0; u < m->units.size(); ++u) {
        auto* a = m->unit_w[u];
        specs.push_back({m->units[u].name + ".fc.bias", &a->fc.b, 2 * a->channels, 1, 3});
    }
}

Tensor view_of(const Tensor& buf, long off, int rows, int cols) {
    Tensor t = Tensor::view(Device::HIP, static_cast<float*>(buf.data) + off, rows, cols);
    t.storage = buf.storage;
    return t;
}

int check(kdec_model* m, int rc) {
    if (rc != KDEC_OK) m->err = kdec_last_error(m->ctx);
    return rc;
}

}  // namespace

extern "C" {

int kdec_model_create(kdec_ctx* ctx, const int* v, int n, kdec_model** out) {
    if (!ctx || !v || !out) return KDEC_EINVAL;
    *out = nullptr;
    kdec_model* m = new kdec_model();
    m->ctx = ctx;
    int i = 0;
    auto nx = [&]() { return i < n ? v[i++] : -1; };
    m->asr_dim = nx(); m->asr_res_dim = nx(); m->style_dim = nx(); m->enc_dim = nx(); m->n_decode = nx();
    for (int j = 0; j < 8; ++j) m->dec_out[j] = nx();
    m->dec_up_at = nx(); m->n_ups = nx();
    for (int j = 0; j < 4; ++j) m->ups_rates[j] = nx();
    for (int j = 0; j < 4; ++j) m->ups_kernels[j] = nx();
    m->n_kernels = nx();
    for (int j = 0; j < 4; ++j) m->rb_kernels[j] = nx();
    for (int j = 0; j < 4; ++j)
        for (int q = 0; q < 3; ++q) m->rb_dil[j][q] = nx();
    m->n_fft = nx(); m->hop = nx(); m->conv_post_k = nx(); m->sample_rate = nx(); m->harmonic_num = nx();
    if (i != n || n != 45 || m->n_decode < 1 || m->n_decode > 8 || m->n_ups < 1 || m->n_ups > 4 ||
        m->n_kernels < 1 || m->n_kernels > 4 || m->style_dim < 1 || m->n_fft < 2 || m->hop < 1) {
        delete m;
        return KDEC_EINVAL;
    }
    if (kdec_ctx_create(ctx->device, &m->side) != KDEC_OK || kdec_ctx_create(ctx->device, &m->ctx2) != KDEC_OK ||
        kdec_ctx_create(ctx->device, &m->side2) != KDEC_OK ||
        hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_join, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_split, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_part1, hipEventDisableTiming) != hipSuccess) {
        kdec_model_destroy(m);
        return kdec::fail(ctx, KDEC_EHIP, "kdec_model_create: side streams");
    }
    m->side->prof = ctx->prof;
    m->ctx2->prof = ctx->prof;
    m->side2->prof = ctx->prof;
    ctx->peers.push_back(m->side);
    ctx->peers.push_back(m->ctx2);
    ctx->peers.push_back(m->side2);
    m->part[0].ctx = ctx;
    m->part[1].ctx = m->ctx2;
    try {
        bt::set_runtime(ctx);
        std::vector<Spec> specs;
        build(m, specs);
        long total = 0;
        for (auto& s : specs) total += static_cast<long>(s.rows) * s.cols;
        m->total = total;
        m->pbuf = Tensor::zeros_on(Device::HIP, 1, static_cast<int>(total));
        m->gbuf = Tensor::zeros_on(Device::HIP, 1, static_cast<int>(total));
        m->gbuf2 = Tensor::zeros_on(Device::HIP, 1, static_cast<int>(total));
        long off = 0;
        for (auto& s : specs) {
            kdec_model::Param p;
            p.value = s.t;
            p.rows = s.rows;
            p.cols = s.cols;
            p.offset = off;
            *s.t = view_of(m->pbuf, off, s.rows, s.cols);
            p.grad = view_of(m->gbuf, off, s.rows, s.cols);
            p.grad2 = view_of(m->gbuf2, off, s.rows, s.cols);
            off += static_cast<long>(s.rows) * s.cols;
            m->order.push_back(s.name);
            auto& slot = m->params[s.name];
            slot = p;
            if (s.kind == 0) {
                m->wg_all.add(*s.t, slot.grad);
                m->wg_conv.add(*s.t, slot.grad);
                m->wg_all2.add(*s.t, slot.grad2);
                m->wg_conv2.add(*s.t, slot.grad2);
            } else if (s.kind == 1) {
                m->wg_all.add(*s.t, slot.grad);
                m->wg_alpha.add(*s.t, slot.grad);
                m->wg_all2.add(*s.t, slot.grad2);
                m->wg_alpha2.add(*s.t, slot.grad2);
            }
        }
    } catch (const std::exception& e) {
        delete m;
        return KDEC_EINVAL;
    }
    *out = m;
    return KDEC_OK;
}

int kdec_model_destroy(kdec_model* m) {
    if (!m) return KDEC_OK;
    for (kdec_ctx** sp : {&m->side, &m->ctx2, &m->side2}) {
        kdec_ctx* sc = *sp;
        if (!sc) continue;
        (void)hipStreamSynchronize(sc->stream);
        auto& pv = m->ctx->peers;
        for (auto it = pv.begin(); it != pv.end(); ++it)
            if (*it == sc) {
                pv.erase(it);
                break;
            }
        kdec_ctx_destroy(sc);  // blocks still held by the caches release it later
        *sp = nullptr;
    }
    for (hipEvent_t e : {m->ev_fork, m->ev_join, m->ev_split, m->ev_part1})
        if (e) (void)hipEventDestroy(e);
    delete m;
    return KDEC_OK;
}

int kdec_model_param_count(const kdec_model* m) { return m ? static_cast<int>(m->order.size()) : 0; }

const char* kdec_model_param_name(const kdec_model* m, int i) {
    if (!m || i < 0 || i >= static_cast<int>(m->order.size())) return nullptr;
    return m->order[i].c_str();
}

int kdec_model_param_shape(const kdec_model* m, const char* name, int* rows, int* cols) {
    if (!m || !name) return KDEC_EINVAL;
    auto it = m->params.find(name);
    if (it == m->params.end()) return KDEC_EINVAL;
    if (rows) *rows = it->second.rows;
    if (cols) *cols = it->second.cols;
    return KDEC_OK;
}

static int copy_param(kdec_model* m, const char* name, float* host, long n, bool to_dev, bool grad) {
    if (!m || !name || !host) return KDEC_EINVAL;
    auto it = m->params.find(name);
    if (it == m->params.end()) return fail(m, KDEC_EINVAL, std::string("unknown parameter ") + name);
    const auto& p = it->second;
    if (n != static_cast<long>(p.rows) * p.cols) return fail(m, KDEC_EINVAL, std::string("size mismatch ") + name);
    float* d = static_cast<float*>(grad ? m->gbuf.data : m->pbuf.data) + p.offset;
    hipStream_t s = static_cast<hipStream_t>(kdec_get_stream(m->ctx));
    hipError_t e = to_dev ? hipMemcpyAsync(d, host, n * sizeof(float), hipMemcpyHostToDevice, s)
                          : hipMemcpyAsync(host, d, n * sizeof(float), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? KDEC_OK : fail(m, KDEC_EHIP, hipGetErrorString(e));
}

int kdec_model_set_param(kdec_model* m, const char* name, const float* host, long n) {
    return copy_param(m, name, const_cast<float*>(host), n, true, false);
}
int kdec_model_get_param(kdec_model* m, const char* name, float* host, long n) {
    return copy_param(m, name, host, n, false, false);
}
int kdec_model_get_grad(kdec_model* m, const char* name, float* host, long n) {
    return copy_param(m, name, host, n, false, true);
}

float* kdec_model_param_ptr(kdec_model* m, const char* name) {
    if (!m || !name) return nullptr;
    auto it = m->params.find(name);
    return it == m->params.end() ? nullptr : static_cast<float*>(m->pbuf.data) + it->second.offset;
}

float* kdec_model_grad_ptr(kdec_model* m, const char* name) {
    if (!m || !name) return nullptr;
    auto it = m->params.find(name);
    return it == m->params.end() ? nullptr : static_cast<float*>(m->gbuf.data) + it->second.offset;
}

long kdec_model_param_total(const kdec_model* m) { return m ? m->total : 0; }

int kdec_model_zero_grad(kdec_model* m) {
    if (!m) return KDEC_EINVAL;
    if (m->lora_rank > 0) {
        if (int rc = check(m, kdec_fill(m->ctx, static_cast<float*>(m->dloraA.data),
                                        static_cast<long>(m->dloraA.rows) * m->dloraA.cols, 0.0f)))
            return rc;
        if (int rc = check(m, kdec_fill(m->ctx, static_cast<float*>(m->dloraB.data),
                                        static_cast<long>(m->dloraB.rows) * m->dloraB.cols, 0.0f)))
            return rc;
    }
    return check(m, kdec_fill(m->ctx, static_cast<float*>(m->gbuf.data), m->total, 0.0f));
}

int kdec_model_lora_enable(kdec_model* m, int rank, float scale) {
    if (!m || rank <= 0) return KDEC_EINVAL;
    try {
        bt::set_runtime(m->ctx);
        const int U = static_cast<int>(m->units.size());
        m->lora_rank = rank;
        m->lora_scale = scale;
        m->loraA = Tensor::zeros_on(Device::HIP, U * rank, m->style_dim);
        m->dloraA = Tensor::zeros_on(Device::HIP, U * rank, m->style_dim);
        m->loraB = Tensor::zeros_on(Device::HIP, m->rows_total, rank);
        m->dloraB = Tensor::zeros_on(Device::HIP, m->rows_total, rank);
        std::vector<int> off(static_cast<std::size_t>(U) + 1);
        for (int i = 0; i < U; ++i) off[i] = m->units[i].offset;
        off[U] = m->rows_total;
        m->unit_off = Tensor::empty_on(Device::HIP, 1, U + 1);
        if (hipMemcpyAsync(m->unit_off.data, off.data(), off.size() * sizeof(int), hipMemcpyHostToDevice,
                           m->ctx->stream) != hipSuccess ||
            hipStreamSynchronize(m->ctx->stream) != hipSuccess)
            return fail(m, KDEC_EHIP, "kdec_model_lora_enable: upload of the unit offsets");
    } catch (const std::exception& e) {
        return fail(m, KDEC_ENOMEM, e.what());
    }
    return KDEC_OK;
}

float* kdec_model_lora_ptr(kdec_model* m, int which) {
    if (!m || m->lora_rank <= 0) return nullptr;
    switch (which) {
        case 0: return static_cast<float*>(m->loraA.data);
        case 1: return static_cast<float*>(m->loraB.data);
        case 2: return static_cast<float*>(m->dloraA.data);
        case 3: return static_cast<float*>(m->dloraB.data);
        default: return nullptr;
    }
}

int kdec_model_lora_gate(kdec_model* m, const float* g, long g_bs, float* dG) {
    if (!m || m->lora_rank <= 0 || !g || g_bs < 0) return KDEC_EINVAL;
    m->gate = g;
    m->gate_bs = g_bs;
    m->dgate = dG;
    return KDEC_OK;
}

int kdec_model_unit_count(const kdec_model* m) { return m ? static_cast<int>(m->units.size()) : 0; }
const char* kdec_model_unit_name(const kdec_model* m, int i) {
    return (m && i >= 0 && i < static_cast<int>(m->units.size())) ? m->units[i].name.c_str() : nullptr;
}
int kdec_model_unit_channels(const kdec_model* m, int i) {
    return (m && i >= 0 && i < static_cast<int>(m->units.size())) ? m->units[i].C : -1;
}
int kdec_model_unit_offset(const kdec_model* m, int i) {
    return (m && i >= 0 && i < static_cast<int>(m->units.size())) ? m->units[i].offset : -1;
}
int kdec_model_affine_rows(const kdec_model* m) { return m ? m->rows_total : 0; }

int kdec_model_get_affines(kdec_model* m, float* gb, float* dgb) {
    if (!m || m->N == 0) return KDEC_EINVAL;
    try {
        if (gb && m->gb.data) {
            auto h = m->gb.to_host_vector();
            std::copy(h.begin(), h.end(), gb);
        }
        if (dgb && m->dgb.data) {
            auto h = m->dgb.to_host_vector();
            std::copy(h.begin(), h.end(), dgb);
        }
    } catch (const std::exception& e) {
        return fail(m, KDEC_EHIP, e.what());
    }
    return KDEC_OK;
}

int kdec_model_lengths(const kdec_model* m, int T, int* L_gen, int* frames, int* audio_len) {
    if (!m || T <= 0) return KDEC_EINVAL;
    int upr = 1;
    for (int i = 0; i < m->n_ups; ++i) upr *= m->ups_rates[i];
    const int lg = 2 * T;
    const int fr = lg * upr + 1;
    if (L_gen) *L_gen = lg;
    if (frames) *frames = fr;
    if (audio_len) *audio_len = (fr - 1) * m->hop;
    return KDEC_OK;
}

int kdec_model_forward(kdec_model* m, int N, int T, const float* asr, const float* F0, const float* Nn,
                       const float* style, const float* har_in, float* audio) {
    if (!m || N <= 0 || T <= 0 || !asr || !F0 || !Nn || !style || !audio) return KDEC_EINVAL;
    try {
        bt::set_runtime(m->ctx);
        m->N = N;
        m->T = T;
        const int S = m->style_dim;
        const int R = m->rows_total;
        auto in = [&](const float* p, int cols) {
            return Tensor::view(Device::HIP, const_cast<float*>(p), N, cols);
        };
        m->style_v = in(style, S);
        // style projection for every unit at once
        m->gb = Tensor::empty_on(Device::HIP, N, R);
        const long fc_off = m->params.at(m->units[0].name + ".fc.weight").offset;
        const long fcb_off = m->params.at(m->units[0].name + ".fc.bias").offset;
        const float* W = static_cast<const float*>(m->pbuf.data) + fc_off;
        const float* b = static_cast<const float*>(m->pbuf.data) + fcb_off;
        if (m->lora_rank > 0) {
            if (!m->gate) return fail(m, KDEC_EINVAL, "kdec_model_forward: LoRA enabled but no gate set");
            const int UR = static_cast<int>(m->units.size()) * m->lora_rank;
            m->lora_H = Tensor::empty_on(Device::HIP, N, UR);
            if (int rc = check(m, kdec_lora_proj_fwd(m->ctx, W, b, static_cast<const float*>(m->loraA.data),
                                                     static_cast<const float*>(m->loraB.data), m->gate, m->gate_bs,
                                                     m->lora_scale, static_cast<const int*>(m->unit_off.data),
                                                     static_cast<int>(m->units.size()), m->lora_rank, style, S,
                                                     static_cast<float*>(m->lora_H.data),
                                                     static_cast<float*>(m->gb.data), R, N, R, S)))
                return rc;
        } else if (int rc = check(m, kdec_style_proj_fwd(m->ctx, W, b, style, S, static_cast<float*>(m->gb.data), R,
                                                          N, R, S))) {
            return rc;
        }
        // harmonic source (side stream) -- HarmonicSource::forward's work
        const auto& hs = m->hs;
        const int sig = 2 * T * hs.upsample_scale;
        const int frames = sig / hs.hop_size + 1;
        const int har_cols = (m->n_fft + 2) * frames;
        hipStream_t ms = static_cast<hipStream_t>(kdec_get_stream(m->ctx));
        bool forked = false;
        if (har_in) {
            Tensor h = in(har_in, har_cols);
            m->har = h.clone();
        } else if (!m->overlap) {
            m->har = Tensor::empty_on(Device::HIP, N, har_cols);
            const int rc = kdec_harmonic_source(m->ctx, F0, 2 * T, static_cast<float*>(m->har.data), har_cols, N,
                                                2 * T, static_cast<const float*>(hs.l_linear.W.data),
                                                static_cast<const float*>(hs.l_linear.b.data), hs.harmonic_num,
                                                hs.sample_rate, hs.upsample_scale, hs.n_fft, hs.hop_size);
            if (rc != KDEC_OK) return rc;
        } else {
            m->har = Tensor::empty_on(Device::HIP, N, har_cols);
            if (hipEventRecord(m->ev_fork, ms) != hipSuccess ||
                hipStreamWaitEvent(m->side->stream, m->ev_fork, 0) != hipSuccess)
                return fail(m, KDEC_EHIP, "kdec_model_forward: fork");
            const int rc = kdec_harmonic_source(m->side, F0, 2 * T, static_cast<float*>(m->har.data), har_cols, N,
                                                2 * T, static_cast<const float*>(hs.l_linear.W.data),
                                                static_cast<const float*>(hs.l_linear.b.data), hs.harmonic_num,
                                                hs.sample_rate, hs.upsample_scale, hs.n_fft, hs.hop_size);
            if (rc != KDEC_OK) return fail(m, rc, std::string("harmonic source: ") + kdec_last_error(m->side));
            if (hipEventRecord(m->ev_join, m->side->stream) != hipSuccess)
                return fail(m, KDEC_EHIP, "kdec_model_forward: join");
            forked = true;
        }

        // the parts: two halves of the batch on two streams, or one
        m->parts = (m->overlap && m->split && N >= 2) ? 2 : 1;
        if (m->parts == 1) {  // an earlier forward's second-part caches go
            kdec_model::Part& p1 = m->part[1];
            const bool keep_b = p1.bbc.keep, keep_g = p1.genc.keep;
            p1.bbc = bd::BackboneCache{};
            p1.genc = bd::GeneratorCache{};
            p1.bbc.keep = keep_b;
            p1.genc.keep = keep_g;
            p1.gen_in = Tensor();
            p1.bbaff.clear();
            p1.naff.clear();
            p1.raff.clear();
        }
        m->part[0].n0 = 0;
        m->part[0].n = m->parts == 2 ? N - N / 2 : N;
        m->part[1].n0 = m->part[0].n;
        m->part[1].n = N - m->part[0].n;
        if (m->parts == 2 && (hipEventRecord(m->ev_split, ms) != hipSuccess ||
                              hipStreamWaitEvent(m->ctx2->stream, m->ev_split, 0) != hipSuccess))
            return fail(m, KDEC_EHIP, "kdec_model_forward: fork of the second part");
        const int n_dec = m->n_decode;
        int alen = 0;
        kdec_model_lengths(m, T, nullptr, nullptr, &alen);
        // one chain: the stages' resblocks run beside the runtime stream on
        // the second part's context and on the side context (whose harmonic
        // source, queued first, is done before the generator needs it). Each
        // context's stream was created on its own hardware queue; the second
        // part's weight-grad context shares the runtime stream's.
        struct ResblockLanes {
            explicit ResblockLanes(kdec_ctx* a, kdec_ctx* b) { bd::set_resblock_lanes(a, b); }
            ~ResblockLanes() { bd::set_resblock_lanes(nullptr, nullptr); }
        } resblock_lanes(m->parts == 1 && m->overlap ? m->ctx2 : nullptr,
                         m->parts == 1 && m->overlap ? m->side : nullptr);
        for (int pi = 0; pi < m->parts; ++pi) {
            kdec_model::Part& pt = m->part[pi];
            bt::set_runtime(pt.ctx);
            const int n0 = pt.n0, n = pt.n;
            auto rows = [&](const float* base, int cols, long ld) {
                return Tensor::view(Device::HIP, const_cast<float*>(base) + static_cast<long>(n0) * ld, n, cols,
                                    bt::Dtype::FP32, ld);
            };
            auto gv = [&](const Tensor& buf, int off, int C) {
                Tensor t = rows(static_cast<const float*>(buf.data) + off, C, R);
                t.storage = buf.storage;
                return t;
            };
            pt.bbaff.assign(1 + n_dec, bd::BlockAffines{});
            pt.naff.assign(m->n_ups, bd::ResBlock1Affines{});
            pt.raff.assign(static_cast<std::size_t>(m->n_ups) * m->n_kernels, bd::ResBlock1Affines{});
            std::size_t u = 0;
            auto pair = [&](Tensor& g, Tensor& bb) {
                const auto& un = m->units[u++];
                g = gv(m->gb, un.offset, un.C);
                bb = gv(m->gb, un.offset + un.C, un.C);
            };
            for (auto& a : pt.bbaff) { pair(a.g1, a.b1); pair(a.g2, a.b2); }
            auto rb = [&](bd::ResBlock1Affines& a) {
                for (int j = 0; j < 3; ++j) pair(a.g1[j], a.b1[j]);
                for (int j = 0; j < 3; ++j) pair(a.g2[j], a.b2[j]);
            };
            for (auto& a : pt.naff) rb(a);
            for (auto& a : pt.raff) rb(a);
            Tensor har_p = rows(static_cast<const float*>(m->har.data), har_cols, har_cols);
            har_p.storage = m->har.storage;
            bd::decoder_backbone_forward_train(m->bb, rows(asr, m->asr_dim * T, static_cast<long>(m->asr_dim) * T),
                                               rows(F0, 2 * T, 2 * T), rows(Nn, 2 * T, 2 * T), T, pt.bbaff, 1e-5f,
                                               pt.gen_in, pt.bbc);
            const int init_C = m->dec_out[n_dec - 1];
            const int L_gen = pt.gen_in.cols / init_C;
            Tensor out;
            // the generator waits for har itself, after stage 0's upsampling;
            // ev_fork (recorded after the style projection) covers its affines
            pt.genc.har_ready = forked ? static_cast<void*>(m->ev_join) : nullptr;
            pt.genc.inputs_ready = forked && m->parts == 1 ? static_cast<void*>(m->ev_fork) : nullptr;
            bd::generator_forward_train(m->gen, pt.gen_in, L_gen, har_p, frames, pt.naff, pt.raff, out, pt.genc);
            hipStream_t ps = static_cast<hipStream_t>(kdec_get_stream(pt.ctx));
            if (pt.genc.har_ready) {  // no noise conv consumed it: join here
                pt.genc.har_ready = nullptr;
                if (hipStreamWaitEvent(ps, m->ev_join, 0) != hipSuccess)
                    return fail(m, KDEC_EHIP, "kdec_model_forward: join");
            }
            if (out.cols != alen) return fail(m, KDEC_EINVAL, "kdec_model_forward: audio length mismatch");
            hipError_t e = hipMemcpyAsync(audio + static_cast<long>(n0) * alen, out.data,
                                          static_cast<size_t>(n) * alen * sizeof(float), hipMemcpyDeviceToDevice, ps);
            if (e != hipSuccess) return fail(m, KDEC_EHIP, hipGetErrorString(e));
        }
        bt::set_runtime(m->ctx);
        if (m->parts == 2 && (hipEventRecord(m->ev_part1, m->ctx2->stream) != hipSuccess ||
                              hipStreamWaitEvent(ms, m->ev_part1, 0) != hipSuccess))
            return fail(m, KDEC_EHIP, "kdec_model_forward: join of the second part");
    } catch (const std::exception& e) {
        return fail(m, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_model_backward(kdec_model* m, const float* daudio, int wgrad, int dalpha, float* dstyle) {
    if (!m || !daudio) return KDEC_EINVAL;
    if (m->N == 0) return fail(m, KDEC_EINVAL, "kdec_model_backward: no training forward to differentiate");
    try {
        bt::set_runtime(m->ctx);
        const int N = m->N;
        const int R = m->rows_total;
        const int S = m->style_dim;
        int alen = 0;
        kdec_model_lengths(m, m->T, nullptr, nullptr, &alen);
        const bd::WeightGrads* wg = wgrad ? (dalpha ? &m->wg_all : &m->wg_conv) : (dalpha ? &m->wg_alpha : nullptr);
        const bd::WeightGrads* wg2 =
            wgrad ? (dalpha ? &m->wg_all2 : &m->wg_conv2) : (dalpha ? &m->wg_alpha2 : nullptr);
        // affine grads land in place in the packed dgb buffer
        m->dgb = Tensor::empty_on(Device::HIP, N, R);
        hipStream_t ms = static_cast<hipStream_t>(kdec_get_stream(m->ctx));
        // Both parts' backwards run concurrently, each with its conv weight
        // grads on its own side stream; part 1's weight grads go to gbuf2
        // (cleared first), which gbuf adds once both are done.
        if (m->parts == 2 && (hipEventRecord(m->ev_split, ms) != hipSuccess ||
                              hipStreamWaitEvent(m->ctx2->stream, m->ev_split, 0) != hipSuccess))
            return fail(m, KDEC_EHIP, "kdec_model_backward: fork of the second part");
        struct LaneReset {  // the weight-grad lane never outlives this call
            ~LaneReset() {
                try {
                    bd::join_wgrad_lane();
                    bd::set_wgrad_lane(nullptr);
                } catch (...) {
                }
            }
        } lane_reset;
        // without conv weight grads the second stream would idle: the
        // generator's resblock and noise-branch backwards use it and the
        // second part's context instead (one chain only)
        const bool rb_lanes = m->parts == 1 && m->overlap && !wgrad;
        struct ResblockLanes {
            explicit ResblockLanes(kdec_ctx* a, kdec_ctx* b) { bd::set_resblock_lanes(a, b); }
            ~ResblockLanes() { bd::set_resblock_lanes(nullptr, nullptr); }
        } resblock_lanes(rb_lanes ? m->ctx2 : nullptr, rb_lanes ? m->side : nullptr);
        for (int pi = 0; pi < m->parts; ++pi) {
            kdec_model::Part& pt = m->part[pi];
            bt::set_runtime(pt.ctx);
            const bd::WeightGrads* pwg = pi == 0 ? wg : wg2;
            if (pi == 1 && pwg)
                if (int rc = check(m, kdec_fill(pt.ctx, static_cast<float*>(m->gbuf2.data), m->total, 0.0f)))
                    return rc;
            bd::set_wgrad_lane(pwg && m->overlap ? (pi == 0 ? m->side : m->side2) : nullptr);
            const int n0 = pt.n0, n = pt.n;
            auto gv = [&](int off, int C) {
                Tensor t = Tensor::view(Device::HIP, static_cast<float*>(m->dgb.data) + static_cast<long>(n0) * R + off,
                                        n, C, bt::Dtype::FP32, R);
                t.storage = m->dgb.storage;
                return t;
            };
            pt.dbbaff.assign(1 + m->n_decode, bd::BlockAffines{});
            pt.dnaff.assign(m->n_ups, bd::ResBlock1Affines{});
            pt.draff.assign(static_cast<std::size_t>(m->n_ups) * m->n_kernels, bd::ResBlock1Affines{});
            std::size_t u = 0;
            auto pair = [&](Tensor& g, Tensor& bb) {
                const auto& un = m->units[u++];
                g = gv(un.offset, un.C);
                bb = gv(un.offset + un.C, un.C);
            };
            for (auto& a : pt.dbbaff) { pair(a.g1, a.b1); pair(a.g2, a.b2); }
            auto rb = [&](bd::ResBlock1Affines& a) {
                for (int j = 0; j < 3; ++j) pair(a.g1[j], a.b1[j]);
                for (int j = 0; j < 3; ++j) pair(a.g2[j], a.b2[j]);
            };
            for (auto& a : pt.dnaff) rb(a);
            for (auto& a : pt.draff) rb(a);
            Tensor dA = Tensor::view(Device::HIP, const_cast<float*>(daudio) + static_cast<long>(n0) * alen, n, alen);
            Tensor dGenIn;
            bd::generator_backward(m->gen, pt.genc, pt.naff, pt.raff, dA, dGenIn, pt.dnaff, pt.draff, pwg);
            bd::decoder_backbone_backward(m->bb, pt.bbc, pt.bbaff, dGenIn, 1e-5f, pt.dbbaff, pwg);
            // the part's stream waits for its lane; the lane is released here,
            // before the next part sets its own
            bd::join_wgrad_lane();
            bd::set_wgrad_lane(nullptr);
        }
        bt::set_runtime(m->ctx);
        if (m->parts == 2) {
            if (hipEventRecord(m->ev_part1, m->ctx2->stream) != hipSuccess ||
                hipStreamWaitEvent(ms, m->ev_part1, 0) != hipSuccess)
                return fail(m, KDEC_EHIP, "kdec_model_backward: join of the second part");
            if (wg2)
                if (int rc = check(m, kdec_axpby(m->ctx, 1.0f, static_cast<const float*>(m->gbuf.data), m->total,
                                                 1.0f, static_cast<const float*>(m->gbuf2.data), m->total,
                                                 static_cast<float*>(m->gbuf.data), m->total, 1, m->total)))
                    return rc;
        }
        // style projection adjoint over every unit
        const long fc_off = m->params.at(m->units[0].name + ".fc.weight").offset;
        const long fcb_off = m->params.at(m->units[0].name + ".fc.bias").offset;
        const float* W = static_cast<const float*>(m->pbuf.data) + fc_off;
        float* dW = wgrad ? static_cast<float*>(m->gbuf.data) + fc_off : nullptr;
        float* db = wgrad ? static_cast<float*>(m->gbuf.data) + fcb_off : nullptr;
        if (m->lora_rank > 0) {
            // adapter_bwd on every unit: dA, dB, the gate grad, d(style), fc grads
            if (int rc = check(m, kdec_lora_proj_bwd(
                                      m->ctx, W, static_cast<const float*>(m->loraA.data),
                                      static_cast<const float*>(m->loraB.data), m->gate, m->gate_bs, m->lora_scale,
                                      static_cast<const int*>(m->unit_off.data), static_cast<int>(m->units.size()),
                                      m->lora_rank, static_cast<const float*>(m->style_v.data), S,
                                      static_cast<const float*>(m->lora_H.data),
                                      static_cast<const float*>(m->dgb.data), R, dstyle, S, 0.0f, dW, db,
                                      static_cast<float*>(m->dloraA.data), static_cast<float*>(m->dloraB.data),
                                      m->dgate, N, R, S)))
                return rc;
        } else if (dstyle || dW) {
            if (int rc = check(m, kdec_style_proj_bwd(m->ctx, W, static_cast<const float*>(m->style_v.data), S,
                                                      static_cast<const float*>(m->dgb.data), R, dstyle, S, 0.0f, dW,
                                                      db, N, R, S)))
                return rc;
        }
    } catch (const std::exception& e) {
        return fail(m, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

kdec_ctx* kdec_model_context(const kdec_model* m) { return m ? m->ctx : nullptr; }

int kdec_model_infer(kdec_model* m, int N, int T, const float* asr, const float* F0, const float* Nn,
                     const float* style, const float* har, float* audio) {
    if (!m) return KDEC_EINVAL;
    // the training forward with every block's cache dropped once the block is done
    for (auto& pt : m->part) {
        pt.bbc.keep = false;
        pt.genc.keep = false;
    }
    const int rc = kdec_model_forward(m, N, T, asr, F0, Nn, style, har, audio);
    for (auto& pt : m->part) {
        pt.bbc.keep = true;
        pt.genc.keep = true;
    }
    m->N = 0;  // nothing to differentiate
    return rc;
}

namespace {

// Kokoro::Impl::decode_back_half (kokoro.cpp:352-407): DecoderBackbone,
// HarmonicSource and Generator inference forwards; `cancel` is polled before
// the generator (:387) and by the generator before each upsample stage.
// With `trace`, the stages the reference records (kokoro.cpp:366, 389-390,
// 396) are copied to it; with BROSOUNDML_DEBUG_STAGES set, each is also
// summarised on stderr under the reference's tags (:365, 388, 395).
int decode_back_half(kdec_model* m, int N, int T, const float* asr, const float* F0, const float* Nn,
                     const float* ref_s, long ref_bs, float* audio, const std::function<bool()>& cancel,
                     int* cancelled, brosoundml::KokoroTrace* trace = nullptr) {
    const char* where = "kdec_model_decode_back_half";
    if (cancelled) *cancelled = 0;
    if (!m || N <= 0 || T <= 0 || !asr || !F0 || !Nn || !ref_s || !audio) return KDEC_EINVAL;
    if (ref_bs < m->style_dim) return fail(m, KDEC_EINVAL, std::string(where) + ": ref_s stride below style_dim");
    if (m->lora_rank > 0) return fail(m, KDEC_EINVAL, std::string(where) + ": the base decoder has no adapters");
    try {
        bt::set_runtime(m->ctx);
        auto in = [&](const float* p, int cols, long ld = 0) {
            return Tensor::view(Device::HIP, const_cast<float*>(p), N, cols, bt::Dtype::FP32, ld);
        };
        const Tensor rs = in(ref_s, m->style_dim, ref_bs);
        Tensor gen_in, har, out;
        // stage `name` of each utterance: (h x w) per utterance row
        auto record = [&](const char* tag, const char* name, const Tensor& t, int h, int w) {
            brosoundml::debug_stats(tag, t);
            if (!trace) return;
            if (N == 1) {
                trace->add(name, h, w, t);
                return;
            }
            for (int n = 0; n < N; ++n) {
                Tensor row = Tensor::view(Device::HIP, static_cast<float*>(t.data) + n * t.row_stride(), 1, t.cols);
                trace->add(std::string(name) + "." + std::to_string(n), h, w, row);
            }
        };
        m->bb.forward(in(asr, m->asr_dim * T), in(F0, 2 * T), in(Nn, 2 * T), rs, T, gen_in);
        record("09_gen_in", "gen_in", gen_in, gen_in.cols / (2 * T), 2 * T);
        int sig = 0, frames = 0;
        m->hs.forward(in(F0, 2 * T), 2 * T, sig, frames, har);
        int upr = 1;
        for (int i = 0; i < m->n_ups; ++i) upr *= m->ups_rates[i];
        if (frames != 2 * T * upr + 1)
            return fail(m, KDEC_EINVAL, "brosoundml: Kokoro::decode: har_frames mismatch: hsource=" +
                                            std::to_string(frames) + " vs expected=" +
                                            std::to_string(2 * T * upr + 1));
        record("10_har_stub", "har", har, m->n_fft + 2, frames);
        if (cancel && cancel()) {
            if (cancelled) *cancelled = 1;
            return KDEC_OK;
        }
        m->gen.forward(gen_in, 2 * T, har, frames, rs, out, cancel);
        if (!out.data) {  // cancelled between stages: the audio stays unwritten
            if (cancelled) *cancelled = 1;
            return KDEC_OK;
        }
        record("11_audio", "audio", out, 1, out.cols);
        if (hipMemcpyAsync(audio, out.data, out.size() * sizeof(float), hipMemcpyDeviceToDevice,
                           static_cast<hipStream_t>(kdec_get_stream(m->ctx))) != hipSuccess)
            return fail(m, KDEC_EHIP, std::string(where) + ": output copy");
    } catch (const std::exception& e) {
        return fail(m, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

}  // namespace

int kdec_model_decode_back_half(kdec_model* m, int N, int T, const float* asr, const float* F0, const float* Nn,
                                const float* ref_s, long ref_bs, float* audio) {
    return decode_back_half(m, N, T, asr, F0, Nn, ref_s, ref_bs, audio, {}, nullptr);
}

int kdec_model_decode_back_half_cancellable(kdec_model* m, int N, int T, const float* asr, const float* F0,
                                            const float* Nn, const float* ref_s, long ref_bs, float* audio,
                                            kdec_cancel_fn cancel, void* user, int* cancelled) {
    std::function<bool()> poll;
    if (cancel) poll = [cancel, user] { return cancel(user) != 0; };
    return decode_back_half(m, N, T, asr, F0, Nn, ref_s, ref_bs, audio, poll, cancelled);
}

// ─── stage traces ───────────────────────────────────────────────────────────

struct kdec_trace {
    brosoundml::KokoroTrace t;
};

int kdec_trace_create(kdec_trace** out) {
    if (!out) return KDEC_EINVAL;
    *out = new kdec_trace();
    return KDEC_OK;
}

int kdec_trace_destroy(kdec_trace* t) {
    delete t;
    return KDEC_OK;
}

int kdec_trace_count(const kdec_trace* t) { return t ? static_cast<int>(t->t.stages.size()) : -1; }

const char* kdec_trace_stage(const kdec_trace* t, int i, int* h, int* w) {
    if (!t || i < 0 || i >= static_cast<int>(t->t.stages.size())) return nullptr;
    const auto& st = t->t.stages[static_cast<std::size_t>(i)];
    if (h) *h = st.h;
    if (w) *w = st.w;
    return st.name.c_str();
}

const float* kdec_trace_data(const kdec_trace* t, int i) {
    if (!t || i < 0 || i >= static_cast<int>(t->t.stages.size())) return nullptr;
    return t->t.stages[static_cast<std::size_t>(i)].data.data();
}

int kdec_model_decode_back_half_traced(kdec_model* m, int N, int T, const float* asr, const float* F0,
                                       const float* Nn, const float* ref_s, long ref_bs, float* audio,
                                       kdec_cancel_fn cancel, void* user, int* cancelled, kdec_trace* trace) {
    std::function<bool()> poll;
    if (cancel) poll = [cancel, user] { return cancel(user) != 0; };
    return decode_back_half(m, N, T, asr, F0, Nn, ref_s, ref_bs, audio, poll, cancelled,
                            trace ? &trace->t : nullptr);
}

int kdec_model_set_overlap(kdec_model* m, int on) {
    if (!m) return KDEC_EINVAL;
    m->overlap = on != 0;
    return KDEC_OK;
}

int kdec_model_set_batch_split(kdec_model* m, int on) {
    if (!m) return KDEC_EINVAL;
    m->split = on != 0;
    return KDEC_OK;
}

const float* kdec_model_har(const kdec_model* m) { return m ? static_cast<const float*>(m->har.data) : nullptr; }
const float* kdec_model_gen_in(const kdec_model* m) {
    if (!m || m->parts == 0) return nullptr;
    if (m->parts == 1) return static_cast<const float*>(m->part[0].gen_in.data);
    // both parts' rows in one (N, cols) buffer, assembled on the model stream
    try {
        bt::set_runtime(m->ctx);
        const Tensor& a = m->part[0].gen_in;
        const Tensor& b = m->part[1].gen_in;
        m->gen_in_all = Tensor::empty_on(Device::HIP, m->N, a.cols);
        hipStream_t s = static_cast<hipStream_t>(kdec_get_stream(m->ctx));
        if (hipMemcpyAsync(m->gen_in_all.data, a.data, a.size() * sizeof(float), hipMemcpyDeviceToDevice, s) !=
                hipSuccess ||
            hipMemcpyAsync(static_cast<float*>(m->gen_in_all.data) + a.size(), b.data, b.size() * sizeof(float),
                           hipMemcpyDeviceToDevice, s) != hipSuccess)
            return nullptr;
        return static_cast<const float*>(m->gen_in_all.data);
    } catch (const std::exception&) {
        return nullptr;
    }
}

// ─── the producer step (KokoroDecodePrep) ───────────────────────────────────

struct kdec_prep {
    kdec_model* m = nullptr;
    brosoundml::KokoroDecodePrep p;
};

int kdec_model_decode_prep(kdec_model* m, const float* t_en, int L, const int* pred_dur, const float* F0_pred,
                           const float* N_pred, const float* F0_override, long F0_override_n,
                           const float* N_override, long N_override_n, const float* ref_s, kdec_prep** out) {
    if (!m || !out || !t_en || !pred_dur || !ref_s || L <= 0) return KDEC_EINVAL;
    *out = nullptr;
    try {
        bt::set_runtime(m->ctx);
        const std::vector<int32_t> dur(pred_dur, pred_dur + L);
        long total = 0;
        for (int d : dur) total += d;
        const int cols = total > 0 && total < (1 << 24) ? static_cast<int>(2 * total) : 0;
        auto view = [&](const float* p, int c) {
            return p ? Tensor::view(Device::HIP, const_cast<float*>(p), 1, c) : Tensor{};
        };
        std::vector<float> f0v, nv;
        if (F0_override) f0v.assign(F0_override, F0_override + F0_override_n);
        if (N_override) nv.assign(N_override, N_override + N_override_n);
        auto* pr = new kdec_prep;
        pr->m = m;
        try {
            pr->p = brosoundml::prepare_decode_context(
                m->bb, m->gen, m->hs, view(t_en, m->asr_dim * L), L, dur, view(F0_pred, cols), view(N_pred, cols),
                view(ref_s, 2 * m->style_dim), F0_override ? &f0v : nullptr, N_override ? &nv : nullptr);
        } catch (...) {
            delete pr;
            throw;
        }
        *out = pr;
    } catch (const std::exception& e) {
        return fail(m, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_prep_destroy(kdec_prep* p) {
    if (p) {
        bt::set_runtime(p->m->ctx);
        delete p;
    }
    return KDEC_OK;
}

int kdec_prep_total(const kdec_prep* p) { return p ? p->p.total : -1; }
int kdec_prep_frames(const kdec_prep* p) { return p ? p->p.frames : -1; }

const float* kdec_prep_ptr(const kdec_prep* p, int which) {
    if (!p) return nullptr;
    const brosoundml::DecoderLoraContext c = p->p.context();
    const Tensor* t = nullptr;
    switch (which) {
        case 0: t = c.asr; break;
        case 1: t = c.F0_pred; break;
        case 2: t = c.N_pred; break;
        case 3: t = c.har; break;
        case 4: t = c.ref_s; break;
        default: return nullptr;
    }
    return static_cast<const float*>(t->data);
}

// ─── leaky-ReLU sites (inspection) ──────────────────────────────────────────

int kdec_model_leaky_site_count(const kdec_model* m) {
    return m ? 2 * (1 + m->n_decode) + m->n_ups + 1 : 0;
}

namespace {

// One training forward's caches, as the leaky-site inspection reads them.
struct ChainView {
    kdec_ctx* ctx;
    int n;
    const bd::BackboneCache* bbc;
    const std::vector<bd::BlockAffines>* bbaff;
    const bd::GeneratorCache* genc;
};

long leaky_site_size(const kdec_model* m, const ChainView& cv, int site) {
    const int n_blocks = 1 + m->n_decode;
    if (site < 2 * n_blocks) {
        const int b = site / 2;
        const bd::AdainResBlkCache& c = b == 0 ? cv.bbc->encode : cv.bbc->decode[b - 1];
        const brosoundml::AdainResBlk1dWeights& w = b == 0 ? m->bb.encode : m->bb.decode[b - 1];
        return site % 2 ? static_cast<long>(cv.n) * w.channels_out * c.L_out
                        : static_cast<long>(cv.n) * w.channels_in * c.L_in;
    }
    const Tensor& t = site < 2 * n_blocks + m->n_ups ? cv.genc->stages[site - 2 * n_blocks].x_in : cv.genc->head.x_pre;
    return static_cast<long>(t.size());
}

// Site `site`'s input of the chain's forward, copied to host + at. An AdaIN
// residual block's norm output is recomputed from the cached input and
// statistics, as the backward recomputes it; the generator sites are cached.
void leaky_site_copy(const kdec_model* m, const ChainView& cv, int site, float* host) {
    const int n_blocks = 1 + m->n_decode;
    bt::set_runtime(cv.ctx);
    Tensor t;
    if (site < 2 * n_blocks) {
        const int b = site / 2;
        const bool second = site % 2;
        const bd::AdainResBlkCache& c = b == 0 ? cv.bbc->encode : cv.bbc->decode[b - 1];
        const brosoundml::AdainResBlk1dWeights& w = b == 0 ? m->bb.encode : m->bb.decode[b - 1];
        const bd::BlockAffines& a = (*cv.bbaff)[b];
        const Tensor& x = second ? c.conv1_out : c.x;
        const Tensor& st = second ? c.x_seq2 : c.x_seq1;
        const Tensor& g = second ? a.g2 : a.g1;
        const Tensor& be = second ? a.b2 : a.b1;
        const int C = second ? w.channels_out : w.channels_in;
        const int L = second ? c.L_out : c.L_in;
        if (!x.data || !st.data) throw std::runtime_error("leaky_input: no cache for this site");
        t = Tensor::empty_on(Device::HIP, cv.n, C * L);
        const long gbs = cv.n == 1 ? 0 : g.row_stride();
        if (kdec_adain_act_fwd(cv.ctx, static_cast<const float*>(x.data), x.row_stride(),
                               static_cast<const float*>(st.data), static_cast<const float*>(g.data),
                               static_cast<const float*>(be.data), gbs, KDEC_ACT_NONE, 0.0f, nullptr,
                               static_cast<float*>(t.data), t.row_stride(), nullptr, 0, cv.n, C, L) != KDEC_OK)
            throw std::runtime_error(std::string("leaky_input: ") + kdec_last_error(cv.ctx));
    } else if (site < 2 * n_blocks + m->n_ups) {
        t = cv.genc->stages[site - 2 * n_blocks].x_in;  // the stage input (leaky 0.1)
    } else {
        t = cv.genc->head.x_pre;  // the spectral head input (leaky 0.01)
    }
    if (!t.data) throw std::runtime_error("leaky_input: no cache for this site");
    const std::vector<float> h = t.to_host_vector();
    std::copy(h.begin(), h.end(), host);
}

std::vector<ChainView> model_chains(kdec_model* m) {
    std::vector<ChainView> v;
    for (int pi = 0; pi < m->parts; ++pi) {
        kdec_model::Part& pt = m->part[pi];
        v.push_back({pt.ctx, pt.n, &pt.bbc, &pt.bbaff, &pt.genc});
    }
    return v;
}

// kdec_model_leaky_input / kdec_dlora_leaky_input over the chains of one forward.
int leaky_input_of(kdec_model* m, const std::vector<ChainView>& chains, int site, float* host, long n,
                   const char* who) {
    if (site < 0 || site >= kdec_model_leaky_site_count(m))
        return fail(m, KDEC_EINVAL, std::string(who) + ": site out of range");
    long want = 0;
    for (const auto& cv : chains) want += leaky_site_size(m, cv, site);
    if (n != want)
        return fail(m, KDEC_EINVAL, std::string(who) + ": site holds " + std::to_string(want) + " values, not " +
                                        std::to_string(n));
    try {
        long at = 0;
        for (const auto& cv : chains) {
            leaky_site_copy(m, cv, site, host + at);
            at += leaky_site_size(m, cv, site);
        }
        bt::set_runtime(m->ctx);
    } catch (const std::exception& e) {
        bt::set_runtime(m->ctx);
        return fail(m, KDEC_EHIP, std::string(who) + ": " + e.what());
    }
    return KDEC_OK;
}

bool model_has_forward(const kdec_model* m) {
    return m->N != 0 && m->parts != 0 && !m->part[0].genc.stages.empty();
}

}  // namespace

long kdec_model_leaky_size(kdec_model* m, int site) {
    if (!m || !model_has_forward(m) || site < 0 || site >= kdec_model_leaky_site_count(m)) {
        if (m) fail(m, KDEC_EINVAL, "kdec_model_leaky_size: no training forward or site out of range");
        return -1;
    }
    long total = 0;
    for (const auto& cv : model_chains(m)) total += leaky_site_size(m, cv, site);
    return total;
}

int kdec_model_leaky_input(kdec_model* m, int site, float* host, long n) {
    if (!m || !host) return KDEC_EINVAL;
    if (!model_has_forward(m)) return fail(m, KDEC_EINVAL, "kdec_model_leaky_input: no training forward to inspect");
    return leaky_input_of(m, model_chains(m), site, host, n, "kdec_model_leaky_input");
}

// ─── DecoderLora over the model's weights ───────────────────────────────────

struct kdec_dlora {
    kdec_model* m = nullptr;
    brosoundml::DecoderLora lora;
    Tensor audio, cond, har;
    int N = 0, T = 0;
};

namespace {
int dlora_fail(kdec_dlora* d, int code, const std::string& msg) {
    if (d && d->m) return fail(d->m, code, msg);
    return code;
}
}  // namespace

int kdec_dlora_create(kdec_model* m, int rank, float scale, unsigned long long seed, kdec_dlora** out) {
    if (!m || !out || rank <= 0) return KDEC_EINVAL;
    try {
        bt::set_runtime(m->ctx);
        auto* d = new kdec_dlora();
        d->m = m;
        d->lora = brosoundml::DecoderLora::make(m->bb, m->gen, rank, scale, Device::HIP, seed);
        *out = d;
    } catch (const std::exception& e) {
        return fail(m, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_dlora_destroy(kdec_dlora* d) {
    if (!d) return KDEC_EINVAL;
    bt::set_runtime(d->m->ctx);
    (void)hipStreamSynchronize(static_cast<hipStream_t>(kdec_get_stream(d->m->ctx)));
    delete d;
    return KDEC_OK;
}

// The resblock lanes for a DecoderLora call (one chain; none with overlap off).
struct DlLanes {
    explicit DlLanes(kdec_model* m) {
        if (m->overlap) bd::set_resblock_lanes(m->ctx2, m->side);
    }
    ~DlLanes() { bd::set_resblock_lanes(nullptr, nullptr); }
    DlLanes(const DlLanes&) = delete;
    DlLanes& operator=(const DlLanes&) = delete;
};

int kdec_dlora_forward(kdec_dlora* d, int N, int T, const float* asr, const float* F0, const float* Nn,
                       const float* ref_s, long ref_bs, const float* har, const float* cond, float* audio) {
    if (!d || N <= 0 || T <= 0 || !asr || !F0 || !Nn || !ref_s || !cond || !audio) return KDEC_EINVAL;
    kdec_model* m = d->m;
    if (ref_bs < m->style_dim) return dlora_fail(d, KDEC_EINVAL, "kdec_dlora_forward: ref_s stride below style_dim");
    try {
        bt::set_runtime(m->ctx);
        int frames = 0, alen = 0;
        kdec_model_lengths(m, T, nullptr, &frames, &alen);
        const int har_cols = (m->n_fft + 2) * frames;
        auto in = [&](const float* p, int cols) { return Tensor::view(Device::HIP, const_cast<float*>(p), N, cols); };
        Tensor h;
        if (har) {
            h = in(har, har_cols);
        } else {  // HarmonicSource::forward on the model's l_linear
            d->har = Tensor::empty_on(Device::HIP, N, har_cols);
            const auto& hs = m->hs;
            // with overlap, on the side stream beside the backbone (as
            // kdec_model_forward runs it); the generator waits for its event
            kdec_ctx* hc = m->ctx;
            hipStream_t ms = static_cast<hipStream_t>(kdec_get_stream(m->ctx));
            if (m->overlap) {
                if (hipEventRecord(m->ev_fork, ms) != hipSuccess ||
                    hipStreamWaitEvent(m->side->stream, m->ev_fork, 0) != hipSuccess)
                    return dlora_fail(d, KDEC_EHIP, "kdec_dlora_forward: fork");
                hc = m->side;
            }
            if (int rc = kdec_harmonic_source(hc, F0, 2 * T, d->har.f32(), har_cols, N, 2 * T,
                                              static_cast<const float*>(hs.l_linear.W.data),
                                              static_cast<const float*>(hs.l_linear.b.data), hs.harmonic_num,
                                              hs.sample_rate, hs.upsample_scale, hs.n_fft, hs.hop_size))
                return dlora_fail(d, rc, std::string("harmonic source: ") + kdec_last_error(hc));
            if (m->overlap) {
                if (hipEventRecord(m->ev_join, m->side->stream) != hipSuccess)
                    return dlora_fail(d, KDEC_EHIP, "kdec_dlora_forward: join");
                d->lora.set_har_ready(m->ev_join);
            }
            h = d->har;
        }
        const Tensor asr_t = in(asr, m->asr_dim * T), F0_t = in(F0, 2 * T), N_t = in(Nn, 2 * T);
        const Tensor rs = Tensor::view(Device::HIP, const_cast<float*>(ref_s), N, m->style_dim, bt::Dtype::FP32, ref_bs);
        brosoundml::DecoderLoraContext c{&asr_t, &F0_t, &N_t, &rs, &h, T, frames};
        d->cond = Tensor::view(Device::HIP, const_cast<float*>(cond), N, d->lora.gate().in_dim);
        {
            // the generator's noise branches and resblocks on three streams,
            // as in kdec_model_forward (forked after har exists)
            DlLanes lanes(m);
            d->lora.forward(m->bb, m->gen, c, d->cond, d->audio);
        }
        d->N = N;
        d->T = T;
        if (hipMemcpyAsync(audio, d->audio.data, static_cast<size_t>(N) * alen * sizeof(float),
                           hipMemcpyDeviceToDevice, static_cast<hipStream_t>(kdec_get_stream(m->ctx))) != hipSuccess)
            return dlora_fail(d, KDEC_EHIP, "kdec_dlora_forward: output copy");
    } catch (const std::exception& e) {
        return dlora_fail(d, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_dlora_backward(kdec_dlora* d, const float* daudio) {
    if (!d || !daudio || d->N == 0) return KDEC_EINVAL;
    kdec_model* m = d->m;
    try {
        bt::set_runtime(m->ctx);
        int alen = 0;
        kdec_model_lengths(m, d->T, nullptr, nullptr, &alen);
        const Tensor dA = Tensor::view(Device::HIP, const_cast<float*>(daudio), d->N, alen);
        DlLanes lanes(m);  // the frozen decoder computes no weight grads: the side stream is free
        d->lora.backward(m->bb, m->gen, d->cond, dA);
    } catch (const std::exception& e) {
        return dlora_fail(d, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_dlora_zero_grad(kdec_dlora* d) {
    if (!d) return KDEC_EINVAL;
    try {
        bt::set_runtime(d->m->ctx);
        d->lora.zero_grad();
    } catch (const std::exception& e) {
        return dlora_fail(d, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_dlora_adam_step(kdec_dlora* d, float lr, float beta1, float beta2, float eps) {
    if (!d) return KDEC_EINVAL;
    try {
        bt::set_runtime(d->m->ctx);
        d->lora.adam_step(lr, beta1, beta2, eps);
    } catch (const std::exception& e) {
        return dlora_fail(d, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_dlora_save(kdec_dlora* d, const char* path) {
    if (!d || !path) return KDEC_EINVAL;
    try {
        bt::set_runtime(d->m->ctx);
        d->lora.save(path);
    } catch (const std::exception& e) {
        return dlora_fail(d, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

int kdec_dlora_load(kdec_dlora* d, const char* path) {
    if (!d || !path) return KDEC_EINVAL;
    try {
        bt::set_runtime(d->m->ctx);
        d->lora.load(path);
    } catch (const std::exception& e) {
        return dlora_fail(d, KDEC_EINVAL, e.what());
    }
    return KDEC_OK;
}

float* kdec_dlora_ptr(kdec_dlora* d, int which, int* rows, int* cols) {
    if (!d) return nullptr;
    const Tensor* t = nullptr;
    auto& g = d->lora.gate();
    switch (which) {
        case 0: case 1: case 2: case 3: t = &d->lora.stacked(which); break;
        case 4: t = &g.W1; break;
        case 5: t = &g.W2; break;
        case 6: t = &g.dW1; break;
        case 7: t = &g.dW2; break;
        default: return nullptr;
    }
    if (rows) *rows = t->rows;
    if (cols) *cols = t->cols;
    return t->f32();
}

float kdec_dlora_scale(const kdec_dlora* d) { return d ? d->lora.scale() : 0.0f; }

namespace {
bool dlora_chain(kdec_dlora* d, ChainView& cv, std::vector<bd::BlockAffines>& bba) {
    const bd::BackboneCache* bbc = d->lora.backbone_cache();
    const bd::GeneratorCache* genc = d->lora.generator_cache();
    if (d->N == 0 || !bbc || !genc || genc->stages.empty()) return false;
    d->lora.backbone_affines(d->m->bb, d->m->gen, bba);
    cv = {d->m->ctx, d->N, bbc, &bba, genc};
    return true;
}
}  // namespace

long kdec_dlora_leaky_size(kdec_dlora* d, int site) {
    ChainView cv{};
    std::vector<bd::BlockAffines> bba;
    if (!d || !dlora_chain(d, cv, bba) || site < 0 || site >= kdec_model_leaky_site_count(d->m)) {
        if (d) dlora_fail(d, KDEC_EINVAL, "kdec_dlora_leaky_size: no forward or site out of range");
        return -1;
    }
    return leaky_site_size(d->m, cv, site);
}

int kdec_dlora_leaky_input(kdec_dlora* d, int site, float* host, long n) {
    if (!d || !host) return KDEC_EINVAL;
    ChainView cv{};
    std::vector<bd::BlockAffines> bba;
    if (!dlora_chain(d, cv, bba)) return dlora_fail(d, KDEC_EINVAL, "kdec_dlora_leaky_input: no forward to inspect");
    return leaky_input_of(d->m, {cv}, site, host, n, "kdec_dlora_leaky_input");
}

}  // extern "C"

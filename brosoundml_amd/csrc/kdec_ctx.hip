// Context, caching allocator, error reporting and per-family timing of the
// gfx950 decoder library. No reference counterpart: brotensor's runtime keeps
// this state implicitly.
#include "kdec_internal.hpp"

#include <cstdio>

namespace kdec {

int fail(kdec_ctx* ctx, int code, const std::string& msg) {
    if (ctx) ctx->err = "brosoundml: " + msg;
    return code;
}

int hip_fail(kdec_ctx* ctx, hipError_t e, const char* where) {
    return fail(ctx, KDEC_EHIP,
                std::string(where) + ": " + hipGetErrorString(e));
}

void* ws_alloc(kdec_ctx* ctx, size_t bytes) {
    if (bytes == 0) bytes = 256;
    bytes = (bytes + 255) & ~size_t(255);
    // Reuse a pooled block of at least `bytes` but not absurdly larger.
    auto it = ctx->pool.lower_bound(bytes);
    if (it != ctx->pool.end() && it->first <= bytes * 2 + (1 << 20)) {
        void* p = it->second;
        ctx->live[p] = it->first;
        ctx->pooled_bytes -= it->first;
        ctx->pool.erase(it);
        return p;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        // Return every pooled block to the driver and try once more.
        hipStreamSynchronize(ctx->stream);
        for (auto& kv : ctx->pool) hipFree(kv.second);
        ctx->pool.clear();
        ctx->pooled_bytes = 0;
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            hip_fail(ctx, e, "hipMalloc");
            return nullptr;
        }
    }
    ctx->live[p] = bytes;
    return p;
}

void ws_free(kdec_ctx* ctx, void* p) {
    if (!p) return;
    auto it = ctx->live.find(p);
    if (it == ctx->live.end()) return;
    if (ctx->destroyed) {
        hipFree(p);
        ctx->live.erase(it);
        if (ctx->live.empty()) delete ctx;
        return;
    }
    ctx->pool.emplace(it->second, p);
    ctx->pooled_bytes += it->second;
    ctx->live.erase(it);
}

static hipEvent_t get_event(kdec_ctx* ctx) {
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    hipEventCreate(&e);
    return e;
}

ProfScope::ProfScope(kdec_ctx* c, const char* n, double f, double b)
    : ctx(c), name(n), flops(f), bytes(b) {
    if (ctx->prof) {
        start = get_event(ctx);
        hipEventRecord(start, ctx->stream);
    }
}

ProfScope::~ProfScope() {
    if (!ctx->prof || !start) return;
    hipEvent_t stop = get_event(ctx);
    hipEventRecord(stop, ctx->stream);
    auto& f = ctx->fams[name];
    f.pending.emplace_back(start, stop);
    f.launches += 1;
    f.flops += flops;
    f.bytes += bytes;
}

int launch_check(kdec_ctx* ctx, const char* where) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(ctx, e, where);
    return KDEC_OK;
}

}  // namespace kdec

using namespace kdec;

extern "C" {

int kdec_ctx_create(int device, kdec_ctx** out) {
    if (!out) return KDEC_EINVAL;
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return KDEC_EHIP;
    if (device < 0 || device >= n) return KDEC_EINVAL;
    e = hipSetDevice(device);
    if (e != hipSuccess) return KDEC_EHIP;
    kdec_ctx* c = new kdec_ctx();
    c->device = device;
    if (hipDeviceGetAttribute(&c->num_cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        c->num_cus <= 0)
        c->num_cus = 256;
    e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return KDEC_EHIP;
    }
    c->stream = c->own_stream;
    *out = c;
    return KDEC_OK;
}

int kdec_ctx_destroy(kdec_ctx* ctx) {
    if (!ctx || ctx->destroyed) return KDEC_OK;
    kdec::forget_runtime(ctx);
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->pool) hipFree(kv.second);
    ctx->pool.clear();
    for (auto& f : ctx->fams)
        for (auto& pr : f.second.pending) {
            hipEventDestroy(pr.first);
            hipEventDestroy(pr.second);
        }
    ctx->fams.clear();
    for (hipEvent_t e : ctx->event_pool) hipEventDestroy(e);
    ctx->event_pool.clear();
    if (ctx->own_stream) hipStreamDestroy(ctx->own_stream);
    ctx->own_stream = nullptr;
    ctx->stream = nullptr;
    // Blocks still owned by live tensors are freed as those tensors go; the
    // last one releases the context (see ws_free).
    if (ctx->live.empty()) delete ctx;
    else ctx->destroyed = true;
    return KDEC_OK;
}

const char* kdec_last_error(const kdec_ctx* ctx) {
    return ctx ? ctx->err.c_str() : "brosoundml: null context";
}

int kdec_set_stream(kdec_ctx* ctx, void* stream) {
    if (!ctx) return KDEC_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);  // NULL: the null stream
    if (s != ctx->stream) {
        // Pooled blocks may still be in use by work on the old stream.
        KDEC_HIP(ctx, hipStreamSynchronize(ctx->stream));
        ctx->stream = s;
    }
    return KDEC_OK;
}

void* kdec_get_stream(const kdec_ctx* ctx) { return ctx ? ctx->stream : nullptr; }

int kdec_synchronize(kdec_ctx* ctx) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return KDEC_OK;
}

int kdec_malloc(kdec_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return KDEC_EINVAL;
    *out = ws_alloc(ctx, bytes);
    return *out ? KDEC_OK : KDEC_ENOMEM;
}

int kdec_free(kdec_ctx* ctx, void* ptr) {
    if (!ctx) return KDEC_EINVAL;
    ws_free(ctx, ptr);
    return KDEC_OK;
}

int kdec_profile_enable(kdec_ctx* ctx, int on) {
    if (!ctx) return KDEC_EINVAL;
    ctx->prof = on != 0;
    for (kdec_ctx* p : ctx->peers) kdec_profile_enable(p, on);
    return KDEC_OK;
}

int kdec_profile_reset(kdec_ctx* ctx) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (auto& f : ctx->fams)
        for (auto& pr : f.second.pending) {
            ctx->event_pool.push_back(pr.first);
            ctx->event_pool.push_back(pr.second);
        }
    ctx->fams.clear();
    for (kdec_ctx* p : ctx->peers)
        if (int rc = kdec_profile_reset(p)) return rc;
    return KDEC_OK;
}

int kdec_profile_read(kdec_ctx* ctx, const char** names, double* ms,
                      long* launches, double* flops, double* bytes, int cap) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_HIP(ctx, hipStreamSynchronize(ctx->stream));
    // fold the peers' families in (their events are on their own streams)
    for (kdec_ctx* p : ctx->peers) {
        if (kdec_profile_read(p, nullptr, nullptr, nullptr, nullptr, nullptr, 0) < 0) return KDEC_EHIP;
        for (auto& kv : p->fams) {
            auto& f = ctx->fams[kv.first];
            f.ms += kv.second.ms;
            f.launches += kv.second.launches;
            f.flops += kv.second.flops;
            f.bytes += kv.second.bytes;
        }
        p->fams.clear();
    }
    int i = 0;
    for (auto& kv : ctx->fams) {
        auto& f = kv.second;
        for (auto& pr : f.pending) {
            float t = 0.0f;
            hipEventElapsedTime(&t, pr.first, pr.second);
            f.ms += t;
            ctx->event_pool.push_back(pr.first);
            ctx->event_pool.push_back(pr.second);
        }
        f.pending.clear();
        if (i < cap) {
            if (names) names[i] = kv.first.c_str();
            if (ms) ms[i] = f.ms;
            if (launches) launches[i] = f.launches;
            if (flops) flops[i] = f.flops;
            if (bytes) bytes[i] = f.bytes;
        }
        ++i;
    }
    return i;
}

}  // extern "C"

// Context, caching allocator, error reporting and per-family timing of the
// gfx950 decoder library. No reference counterpart: brotensor's runtime keeps
// this state implicitly.
#include "kdec_internal.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace kdec {

int fail(kdec_ctx* ctx, int code, const std::string& msg) {
    if (ctx) ctx->err = "brosoundml: " + msg;
    return code;
}

int hip_fail(kdec_ctx* ctx, hipError_t e, const char* where) {
    return fail(ctx, KDEC_EHIP,
                std::string(where) + ": " + hipGetErrorString(e));
}

namespace {

constexpr size_t kGuard = 64 << 10;         // bytes of each guard band
constexpr unsigned kGuardWord = 0x7FBADBADu;  // a quiet-NaN bit pattern

// Fills both guard bands of a block handed out at `user` (bytes long).
void guard_fill(kdec_ctx* ctx, const kdec_ctx::Block& b) {
    char* base = static_cast<char*>(b.base);
    hipMemsetD32Async(base, static_cast<int>(kGuardWord), kGuard / 4, ctx->stream);
    hipMemsetD32Async(base + kGuard + b.bytes, static_cast<int>(kGuardWord), kGuard / 4, ctx->stream);
}

// Checks both bands of one block (the stream must be synchronised); returns
// the number of overwritten bands and reports each.
int guard_check(kdec_ctx* ctx, void* user, const kdec_ctx::Block& b, const char* where) {
    static std::vector<unsigned> h(kGuard / 4);
    int hits = 0;
    for (int side = 0; side < 2; ++side) {
        const char* band = static_cast<const char*>(b.base) + (side ? kGuard + b.bytes : 0);
        if (hipMemcpy(h.data(), band, kGuard, hipMemcpyDeviceToHost) != hipSuccess) return hits;
        size_t first = h.size(), last = 0, n = 0;
        for (size_t i = 0; i < h.size(); ++i)
            if (h[i] != kGuardWord) {
                first = std::min(first, i);
                last = i;
                ++n;
            }
        if (!n) continue;
        ++hits;
        char msg[320];
        std::snprintf(msg, sizeof(msg),
                      "guard band %s the %zu-byte block at %p overwritten (%zu words, band words %zu..%zu), "
                      "found at %s",
                      side ? "after" : "before", b.bytes, user, n, first, last, where);
        std::fprintf(stderr, "kdec: %s\n", msg);
        ctx->err = std::string("brosoundml: ") + msg;
        // restore the band so a later check reports only new writes
        hipMemsetD32(const_cast<char*>(band), static_cast<int>(kGuardWord), kGuard / 4);
    }
    return hits;
}

}  // namespace

int guard_mode() {
    static const int mode = [] {
        const char* e = std::getenv("KDEC_GUARD");
        return e ? std::atoi(e) : 0;
    }();
    return mode;
}

int guard_check_all(kdec_ctx* ctx, const char* where) {
    if (!guard_mode()) return 0;
    hipStreamSynchronize(ctx->stream);
    int hits = 0;
    for (const auto& kv : ctx->live) hits += guard_check(ctx, kv.first, kv.second, where);
    return hits;
}

void* ws_alloc(kdec_ctx* ctx, size_t bytes) {
    if (bytes == 0) bytes = 256;
    bytes = (bytes + 255) & ~size_t(255);
    const size_t need = guard_mode() ? bytes + 2 * kGuard : bytes;
    void* base = nullptr;
    size_t size = need;
    // Reuse a pooled block of at least `need` bytes but not absurdly larger.
    auto it = ctx->pool.lower_bound(need);
    if (it != ctx->pool.end() && it->first <= need * 2 + (1 << 20)) {
        base = it->second;
        size = it->first;
        ctx->pooled_bytes -= it->first;
        ctx->pool.erase(it);
    } else {
        hipError_t e = hipMalloc(&base, need);
        if (e != hipSuccess) {
            // Return every pooled block to the driver and try once more.
            hipStreamSynchronize(ctx->stream);
            for (auto& kv : ctx->pool) hipFree(kv.second);
            ctx->pool.clear();
            ctx->pooled_bytes = 0;
            e = hipMalloc(&base, need);
            if (e != hipSuccess) {
                hip_fail(ctx, e, "hipMalloc");
                return nullptr;
            }
        }
    }
    const kdec_ctx::Block blk{base, size, bytes};
    void* user = guard_mode() ? static_cast<char*>(base) + kGuard : base;
    if (guard_mode()) guard_fill(ctx, blk);
    ctx->live[user] = blk;
    return user;
}

void ws_free(kdec_ctx* ctx, void* p) {
    if (!p) return;
    auto it = ctx->live.find(p);
    if (it == ctx->live.end()) return;
    const kdec_ctx::Block blk = it->second;
    if (guard_mode()) {
        hipStreamSynchronize(ctx->stream);
        guard_check(ctx, p, blk, "free");
    }
    ctx->live.erase(it);
    if (ctx->destroyed) {
        hipFree(blk.base);
        if (ctx->live.empty()) delete ctx;
        return;
    }
    ctx->pool.emplace(blk.size, blk.base);
    ctx->pooled_bytes += blk.size;
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
    if (ctx && ctx->prof) {
        start = get_event(ctx);
        hipEventRecord(start, ctx->stream);
    }
}

ProfScope::~ProfScope() {
    if (!ctx || !ctx->prof || !start) return;
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
    if (guard_mode() >= 2 && guard_check_all(ctx, where)) return KDEC_EHIP;
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
    // This device's copy of the no-allocation entry point's scratch; a
    // failure here only disables that entry point (it reports why).
    if (kdec::noalloc_scratch_setup(c) != KDEC_OK) c->scratch_err = c->err;
    c->err.clear();
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
    if (guard_check_all(ctx, "kdec_synchronize")) return KDEC_EHIP;
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

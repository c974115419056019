// Internal declarations shared by the HIP translation units of libkdec.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <map>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "kdec.h"

struct kdec_ctx {
    int device = 0;
    int num_cus = 0;  // compute units of the device
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err;

    // Stream-ordered caching allocator: every kernel of a context runs on one
    // stream, so a block returned to the pool can be handed out again at once;
    // stream order keeps the reuse behind the previous user's kernels.
    std::multimap<size_t, void*> pool;  // block size -> block base
    struct Block {
        void* base;    // start of the device block
        size_t size;   // bytes of the device block
        size_t bytes;  // bytes handed out (after the front guard in guard mode)
    };
    std::unordered_map<void*, Block> live;  // handed-out pointer -> its block
    size_t pooled_bytes = 0;
    // Set by kdec_ctx_destroy while blocks are still live (tensors that
    // outlive their context): the last ws_free then releases the context.
    bool destroyed = false;

    // Per-kernel-family timing (HIP events on the context stream).
    struct Family {
        double ms = 0.0;
        long launches = 0;
        double flops = 0.0;
        double bytes = 0.0;
        std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
    };
    bool prof = false;
    std::map<std::string, Family> fams;
    std::vector<hipEvent_t> event_pool;
    // Contexts whose streams run work forked from this one (a model's side
    // stream); their profiles follow this context's enable / reset / read.
    std::vector<kdec_ctx*> peers;
    // Why this device's no-allocation scratch is unavailable ("" if it is).
    std::string scratch_err;
};

namespace kdec {

// Error helpers: set the context message and return the code.
int fail(kdec_ctx* ctx, int code, const std::string& msg);
int hip_fail(kdec_ctx* ctx, hipError_t e, const char* where);

#define KDEC_HIP(ctx, expr)                                         \
    do {                                                            \
        hipError_t e_ = (expr);                                     \
        if (e_ != hipSuccess) return kdec::hip_fail(ctx, e_, #expr); \
    } while (0)

#define KDEC_CHECK(ctx, cond, msg)                                  \
    do {                                                            \
        if (!(cond)) return kdec::fail(ctx, KDEC_EINVAL, msg);      \
    } while (0)

// Workspace from the context allocator (returns nullptr and sets the error on
// failure); release with ws_free once the kernels that use it are enqueued.
void* ws_alloc(kdec_ctx* ctx, size_t bytes);
void ws_free(kdec_ctx* ctx, void* p);

// RAII workspace block.
struct Workspace {
    kdec_ctx* ctx;
    void* p = nullptr;
    Workspace(kdec_ctx* c, size_t bytes) : ctx(c) { p = ws_alloc(c, bytes); }
    ~Workspace() { if (p) ws_free(ctx, p); }
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    template <class T> T* as() const { return static_cast<T*>(p); }
};

// Profiling bracket around the launches of one kernel family (a null
// context records nothing).
struct ProfScope {
    kdec_ctx* ctx;
    const char* name;
    double flops, bytes;
    hipEvent_t start = nullptr;
    ProfScope(kdec_ctx* c, const char* n, double f, double b = 0.0);
    ~ProfScope();
};

// Looks up, once per device and with that device current, the address of
// this device's copy of the no-allocation scratch array (kdec_norm.hip).
int noalloc_scratch_setup(kdec_ctx* ctx);
// That address for ctx's device, or nullptr when the lookup failed.
void* noalloc_scratch(kdec_ctx* ctx);

// Drops `ctx` as the C++ layer's runtime context if it is the current one
// (defined with the brotensor runtime, tensor.cpp).
void forget_runtime(kdec_ctx* ctx);

// Checks the last launch; returns KDEC_OK or the HIP error code. In guard
// mode 2 it also synchronises and checks every live block's guard bands.
int launch_check(kdec_ctx* ctx, const char* where);

// Guard mode (environment KDEC_GUARD=1 or 2): every workspace block sits
// between two guard bands of a fixed word pattern; a write past either end
// of a block lands in a band and is reported (stderr and the context error)
// when the block is freed, at kdec_synchronize, and with KDEC_GUARD=2 after
// every launch, naming that launch. A debugging aid: it costs a device sync
// per check. Returns the number of overwritten bands found.
int guard_mode();
int guard_check_all(kdec_ctx* ctx, const char* where);

inline long cdiv(long a, long b) { return (a + b - 1) / b; }

// The AdaIN backward after a GEMM epilogue wrote ds = dY * act'(s) and the
// per-row partial sums part[(row*nch + slot)*3 + {sum ds, sum ds*xh, alpha
// term / a^2}] (kdec_norm.hip): dgamma / dbeta overwritten, dalpha
// accumulated, dX = rstd (1 + gamma) (ds - mean ds - xh mean(ds xh)) + R.
int adain_bwd_finish(kdec_ctx* ctx, const float* X, long x_bs, const float* stats, const float* gamma, long gb_bs,
                     int act, const double* part, int nch, const float* ds, long ds_bs, const float* R, long r_bs,
                     float* dX, long dx_bs, float* dgamma, float* dbeta, long dgb_bs, float* dalpha, int N, int C,
                     int L);

}  // namespace kdec

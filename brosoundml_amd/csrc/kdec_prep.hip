// Length regulation on gfx950: the aligned text features the decoder reads
// as `asr` (Kokoro::prepare_decode_context / synthesize, kokoro.cpp:667-689,
// a per-phoneme repeat the reference runs on the host): frame t of an
// utterance takes column l of t_en, where l is the phoneme whose duration
// run covers t.
//
// Grid (utterance, channel slice of CPB): each block builds the durations'
// inclusive prefix sum in LDS (a fixed-order scan; negative durations count
// as zero), then every (channel, frame) of its slice reads its column
// through a binary search of that scan. Frames at or past the utterance's
// total are zero.
#include "kdec_internal.hpp"

namespace kdec {
namespace {

constexpr int PT = 256;
constexpr int MAX_TOK = 4096;
constexpr int CPB = 8;  // channels per block

__global__ __launch_bounds__(PT) void length_regulate_k(const float* te, long te_bs, const int* dur, long dur_bs,
                                                        int C, int L, float* out, long out_bs, int T, int* totals) {
    __shared__ int cum[MAX_TOK];
    const int n = blockIdx.x;
    const int* d = dur + n * dur_bs;
    // inclusive scan: per-thread runs, then the thread totals in order
    __shared__ int part[PT];
    const int per = (L + PT - 1) / PT;
    const int a = threadIdx.x * per, b = min(L, a + per);
    int s = 0;
    for (int i = a; i < b; ++i) {
        s += max(d[i], 0);
        cum[i] = s;
    }
    part[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int i = 1; i < PT; ++i) part[i] += part[i - 1];
    __syncthreads();
    const int base = threadIdx.x ? part[threadIdx.x - 1] : 0;
    for (int i = a; i < b; ++i) cum[i] += base;
    __syncthreads();
    const int total = L > 0 ? cum[L - 1] : 0;
    if (threadIdx.x == 0 && totals && blockIdx.y == 0) totals[n] = total;
    const int c0 = blockIdx.y * CPB, nc = min(CPB, C - c0);
    const float* x = te + n * te_bs;
    float* y = out + n * out_bs;
    for (long e = threadIdx.x; e < static_cast<long>(nc) * T; e += PT) {
        const int c = c0 + static_cast<int>(e / T), t = static_cast<int>(e % T);
        float v = 0.0f;
        if (t < total) {
            int lo = 0, hi = L - 1;  // first l with cum[l] > t
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (cum[mid] > t) hi = mid;
                else lo = mid + 1;
            }
            v = x[static_cast<long>(c) * L + lo];
        }
        y[static_cast<long>(c) * T + t] = v;
    }
}

}  // namespace
}  // namespace kdec

using namespace kdec;

extern "C" {

int kdec_length_regulate(kdec_ctx* ctx, const float* t_en, long te_bs, const int* dur, long dur_bs, int N, int C,
                         int L, float* asr, long asr_bs, int T, int* totals) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, t_en && dur && asr && N > 0 && C > 0 && L > 0 && T > 0, "kdec_length_regulate: bad arguments");
    KDEC_CHECK(ctx, L <= MAX_TOK, "kdec_length_regulate: more than 4096 tokens per utterance");
    KDEC_CHECK(ctx, te_bs >= static_cast<long>(C) * L && dur_bs >= L && asr_bs >= static_cast<long>(C) * T,
               "kdec_length_regulate: batch stride too small");
    ProfScope ps(ctx, "elementwise", 0.0);
    hipLaunchKernelGGL(length_regulate_k, dim3(N, static_cast<unsigned>(cdiv(C, CPB))), dim3(PT), 0, ctx->stream,
                       t_en, te_bs, dur, dur_bs, C, L, asr, asr_bs, T, totals);
    return launch_check(ctx, "kdec_length_regulate");
}

}  // extern "C"

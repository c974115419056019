// DecoderLora's conditioning gate and its Adam step on gfx950.
//
// The gate (ConditioningGate, decoder_lora.h:20-53, decoder_lora.cpp:56-80)
// is a bias-free two-layer MLP g(v) = W2 tanh(W1 v) from a small condition
// vector to the LoRA rank; one block evaluates it for every utterance (a few
// hundred FLOP each). Adam (bt::adam_step as DecoderLora::adam_step calls
// it, decoder_lora.cpp:305-314) is one elementwise pass over a parameter
// tensor, its grad and its two moments.
#include "kdec_internal.hpp"

#include <cmath>

namespace kdec {
namespace {

constexpr int GT = 256;  // gate block

// act[n, h] = tanh(sum_i W1[h, i] v[n, i]);  g[n, r] = sum_h W2[r, h] act[n, h]
// W1 (hidden, in_dim), W2 (rank, hidden), v at batch stride v_bs, g at g_bs.
// Sums run in index order. One block; act staged in LDS (N * hidden floats).
__global__ __launch_bounds__(GT) void gate_fwd_k(const float* W1, const float* W2, const float* v, long v_bs,
                                                 int N, int in_dim, int hidden, int rank, float* act, float* g,
                                                 long g_bs) {
    extern __shared__ float sact[];
    for (int idx = threadIdx.x; idx < N * hidden; idx += GT) {
        const int n = idx / hidden, h = idx - n * hidden;
        float s = 0.0f;
        for (int i = 0; i < in_dim; ++i) s += W1[h * in_dim + i] * v[n * v_bs + i];
        const float a = tanhf(s);
        sact[idx] = a;
        act[idx] = a;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < N * rank; idx += GT) {
        const int n = idx / rank, r = idx - n * rank;
        float s = 0.0f;
        for (int h = 0; h < hidden; ++h) s += W2[r * hidden + h] * sact[n * hidden + h];
        g[n * g_bs + r] = s;
    }
}

// The gate's adjoint (ConditioningGate::backward, decoder_lora.cpp:68-80):
//   dW2[r, h] += sum_n dG[n, r] act[n, h]
//   dpre[n, h] = (1 - act[n, h]^2) sum_r W2[r, h] dG[n, r]
//   dW1[h, i] += sum_n dpre[n, h] v[n, i]
// (the condition is an input, not a trainable: no dv). Sums in index order.
__global__ __launch_bounds__(GT) void gate_bwd_k(const float* W2, const float* v, long v_bs, const float* act,
                                                 const float* dG, long dg_bs, int N, int in_dim, int hidden,
                                                 int rank, float* dW1, float* dW2) {
    extern __shared__ float sdpre[];
    for (int idx = threadIdx.x; idx < N * hidden; idx += GT) {
        const int n = idx / hidden, h = idx - n * hidden;
        float s = 0.0f;
        for (int r = 0; r < rank; ++r) s += W2[r * hidden + h] * dG[n * dg_bs + r];
        const float a = act[idx];
        sdpre[idx] = s * (1.0f - a * a);
    }
    for (int idx = threadIdx.x; idx < rank * hidden; idx += GT) {
        const int r = idx / hidden, h = idx - r * hidden;
        float s = 0.0f;
        for (int n = 0; n < N; ++n) s += dG[n * dg_bs + r] * act[n * hidden + h];
        dW2[idx] += s;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < hidden * in_dim; idx += GT) {
        const int h = idx / in_dim, i = idx - h * in_dim;
        float s = 0.0f;
        for (int n = 0; n < N; ++n) s += sdpre[n * hidden + h] * v[n * v_bs + i];
        dW1[idx] += s;
    }
}

// Adam with bias correction (torch.optim.Adam's arithmetic):
//   m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2
//   p -= (lr / bc1) * m / (sqrt(v) / sqrt(bc2) + eps),  bc_k = 1 - b_k^step
__global__ void adam_k(float* p, const float* gr, float* m, float* v, long n, float lr_bc1, float b1, float b2,
                       float sqrt_bc2, float eps) {
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const float gi = gr[i];
        const float mi = b1 * m[i] + (1.0f - b1) * gi;
        const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
        m[i] = mi;
        v[i] = vi;
        p[i] -= lr_bc1 * mi / (sqrtf(vi) / sqrt_bc2 + eps);
    }
}

}  // namespace
}  // namespace kdec

using namespace kdec;

extern "C" {

int kdec_lora_gate_fwd(kdec_ctx* ctx, const float* W1, const float* W2, const float* v, long v_bs, int N,
                       int in_dim, int hidden, int rank, float* act, float* g, long g_bs) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W1 && W2 && v && act && g && N > 0 && in_dim > 0 && hidden > 0 && rank > 0,
               "kdec_lora_gate_fwd: bad arguments");
    KDEC_CHECK(ctx, v_bs >= in_dim && g_bs >= rank, "kdec_lora_gate_fwd: batch stride too small");
    KDEC_CHECK(ctx, static_cast<long>(N) * hidden <= 16384, "kdec_lora_gate_fwd: N * hidden above 16384");
    ProfScope ps(ctx, "lora", 0.0);
    hipLaunchKernelGGL(gate_fwd_k, dim3(1), dim3(GT), static_cast<size_t>(N) * hidden * sizeof(float), ctx->stream,
                       W1, W2, v, v_bs, N, in_dim, hidden, rank, act, g, g_bs);
    return launch_check(ctx, "kdec_lora_gate_fwd");
}

int kdec_lora_gate_bwd(kdec_ctx* ctx, const float* W2, const float* v, long v_bs, const float* act,
                       const float* dG, long dg_bs, int N, int in_dim, int hidden, int rank, float* dW1,
                       float* dW2) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W2 && v && act && dG && dW1 && dW2 && N > 0 && in_dim > 0 && hidden > 0 && rank > 0,
               "kdec_lora_gate_bwd: bad arguments");
    KDEC_CHECK(ctx, v_bs >= in_dim && dg_bs >= rank, "kdec_lora_gate_bwd: batch stride too small");
    KDEC_CHECK(ctx, static_cast<long>(N) * hidden <= 16384, "kdec_lora_gate_bwd: N * hidden above 16384");
    ProfScope ps(ctx, "lora", 0.0);
    hipLaunchKernelGGL(gate_bwd_k, dim3(1), dim3(GT), static_cast<size_t>(N) * hidden * sizeof(float), ctx->stream,
                       W2, v, v_bs, act, dG, dg_bs, N, in_dim, hidden, rank, dW1, dW2);
    return launch_check(ctx, "kdec_lora_gate_bwd");
}

int kdec_adam_step(kdec_ctx* ctx, float* p, const float* g, float* m, float* v, long n, float lr, float beta1,
                   float beta2, float eps, int step) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, p && g && m && v && n >= 0 && step >= 1, "kdec_adam_step: bad arguments");
    KDEC_CHECK(ctx, beta1 >= 0.0f && beta1 < 1.0f && beta2 >= 0.0f && beta2 < 1.0f && eps >= 0.0f,
               "kdec_adam_step: bad hyper-parameters");
    if (n == 0) return KDEC_OK;
    const double bc1 = 1.0 - std::pow(static_cast<double>(beta1), step);
    const double bc2 = 1.0 - std::pow(static_cast<double>(beta2), step);
    long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    ProfScope ps(ctx, "lora", 0.0);
    hipLaunchKernelGGL(adam_k, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx->stream, p, g, m, v, n,
                       static_cast<float>(lr / bc1), beta1, beta2, static_cast<float>(std::sqrt(bc2)), eps);
    return launch_check(ctx, "kdec_adam_step");
}

}  // extern "C"

// AdaIN (instance norm + per-utterance style affine) fused with its
// activation, forward and backward, plus the small elementwise ops of the
// decoder (leaky ReLU, axpby, reflect pad, nearest-2x).
//
// Everything here is HBM-bound, so each kernel reads its operands once per
// pass and writes one output: the reference's adain_affine_forward is five
// full-tensor passes (group_norm, two transposes, modulate, a unit-gamma
// upload), its backward seven (kokoro_decoder_backward.cpp:100-150).
//
// Statistics are per (utterance, channel) row over L, accumulated in double
// so the result does not depend on the row length or the thread count.
#include "kdec_buffer.hpp"
#include "kdec_internal.hpp"
#include "kdec_snake_math.hpp"

#include <algorithm>
#include <initializer_list>
#include <type_traits>
#include <mutex>
#include <string>
#include <utility>

namespace kdec {
namespace {

// The float4 buffer access is declared on the LLVM intrinsic itself: with
// this compiler, __builtin_amdgcn_raw_buffer_load_b128 (and _b64) whose
// elements are read one by one is narrowed to a single-dword load and every
// element then reads element 0.
using f32x4 = float __attribute__((ext_vector_type(4)));
__device__ f32x4 buf_ld_f4(__amdgpu_buffer_rsrc_t r, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v4f32");
__device__ void buf_st_f4(f32x4 v, __amdgpu_buffer_rsrc_t r, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.store.v4f32");

constexpr int RT = 256;  // threads per row block

__device__ inline double block_sum(double v, double* red) {
    // wave reduction via shuffles, then across the block's waves
    for (int o = 32; o > 0; o >>= 1) v += __shfl_down(v, o, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x < (blockDim.x >> 6)) t = red[threadIdx.x];
    if (wave == 0)
        for (int o = 32; o > 0; o >>= 1) t += __shfl_down(t, o, 64);
    if (threadIdx.x == 0) red[0] = t;
    __syncthreads();
    const double r = red[0];
    return r;
}

// Block-wide double sum over NTB threads in a fixed order (shuffle tree per
// wave, then wave 0 over the per-wave sums); every thread gets the total.
template <int NTB>
__device__ inline double block_sum_n(double v, double* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_down(v, o, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = threadIdx.x < NTB / 64 ? red[threadIdx.x] : 0.0;
    if (wave == 0)
        for (int o = 32; o > 0; o >>= 1) t += __shfl_down(t, o, 64);
    if (threadIdx.x == 0) red[0] = t;
    __syncthreads();
    return red[0];
}

// Rows are cut into chunks of CH elements (EPT per thread, all loads issued
// before use so each thread keeps EPT reads in flight); per-chunk partial
// sums are reduced per row in a fixed order.
constexpr int EPT = 16;
constexpr int CH = RT * EPT;

// part[row*nch + ch] = (sum(x - x0), sum((x - x0)^2)) over chunk ch, with the
// row's first element x0 as shift (a well-conditioned variance); row = n*C + c.
__global__ __launch_bounds__(RT) void instnorm_part_k(const float* X, long x_bs, int C, int L, int nch,
                                                     double2* part) {
    __shared__ double red[RT / 64];
    const int row = blockIdx.y, ch = blockIdx.x;
    const int n = row / C, c = row - n * C;
    const float* x = X + n * x_bs + static_cast<long>(c) * L;
    const float x0f = x[0];
    const double x0 = x0f;
    const int l0 = ch * CH + threadIdx.x;
    float v[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int l = l0 + j * RT;
        v[j] = l < L ? x[l] : x0f;  // padding adds exact zeros
    }
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const double d = static_cast<double>(v[j]) - x0;
        s1 += d;
        s2 += d * d;
    }
    s1 = block_sum(s1, red);
    s2 = block_sum(s2, red);
    if (threadIdx.x == 0) part[static_cast<long>(row) * nch + ch] = make_double2(s1, s2);
}

// stats[row] = (mean, 1/sqrt(var + eps)) from the row's chunk partials.
__global__ void instnorm_fin_k(const float* X, long x_bs, int C, int L, int rows, int nch, const double2* part,
                               float eps, float2* stats) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const int n = row / C, c = row - n * C;
    const double x0 = X[n * x_bs + static_cast<long>(c) * L];
    double s1 = 0.0, s2 = 0.0;
    for (int ch = 0; ch < nch; ++ch) {
        const double2 p = part[static_cast<long>(row) * nch + ch];
        s1 += p.x;
        s2 += p.y;
    }
    const double m = s1 / L;
    double var = s2 / L - m * m;
    if (var < 0.0) var = 0.0;
    stats[row] = make_float2(static_cast<float>(x0 + m), static_cast<float>(1.0 / sqrt(var + static_cast<double>(eps))));
}

struct AdainArgs {
    const float* X;
    long x_bs;
    const float2* stats;
    const float* gamma;
    const float* beta;
    long gb_bs;
    int act;
    float slope;
    const float* alpha;
    int C, L;
};

// ia = 1 / alpha, formed once per row
__device__ inline float act_fwd(int act, float s, float slope, float a, float ia) {
    if (act == KDEC_ACT_LEAKY) return s > 0.0f ? s : slope * s;
    if (act == KDEC_ACT_SNAKE) return s + snake_sin2(a * s) * ia;
    return s;
}

// ds = dY * act'(s), the grad at the affine output s = g1 * xh + beta. For
// Snake, y = s + sin^2(th) / a with th = a * s:
//   dy/ds = 1 + sin(2 th),   dy/da = (th * sin(2 th) - sin^2(th)) / a^2,
// and `sa` accumulates dY times the numerator (the row sum is scaled by 1/a^2
// once). sin^2 and sin 2th come from the forward's reduced argument
// (snake_sin2_sin2x), accurate for any |th| the forward handles.
__device__ inline float act_bwd(int act, float dy, float s, float slope, float a, float& sa) {
    if (act == KDEC_ACT_LEAKY) return s > 0.0f ? dy : slope * dy;
    if (act == KDEC_ACT_SNAKE) {
        const float th = a * s;
        float sq, s2;
        snake_sin2_sin2x(th, sq, s2);
        sa += dy * (th * s2 - sq);
        return dy * (1.0f + s2);
    }
    return dy;
}

// the 1/a^2 of the Snake alpha-grad, applied to a row (or chunk) sum
__device__ inline double alpha_scale(int act, float a) {
    return act == KDEC_ACT_SNAKE ? 1.0 / (static_cast<double>(a) * a) : 0.0;
}

// One row's constants of the AdaIN(+activation) forward apply.
struct FwdRow {
    float mean, rstd, g1, bt, a, ia;
};

__device__ inline FwdRow fwd_row(const AdainArgs& g, int row, int n, int c) {
    const float2 st = g.stats[row];
    FwdRow r;
    r.mean = st.x;
    r.rstd = st.y;
    r.g1 = 1.0f + g.gamma[n * g.gb_bs + c];
    r.bt = g.beta ? g.beta[n * g.gb_bs + c] : 0.0f;
    r.a = g.act == KDEC_ACT_SNAKE ? g.alpha[c] : 1.0f;
    r.ia = 1.0f / r.a;
    return r;
}

// s = (1 + gamma) * xhat + beta (returned in s) and the activation of s
__device__ inline float fwd_elem(const AdainArgs& g, const FwdRow& r, float xv, float& s) {
    const float xh = (xv - r.mean) * r.rstd;
    s = r.g1 * xh + r.bt;
    return act_fwd(g.act, s, g.slope, r.a, r.ia);
}

// grid (chunks of CH, N*C)
__global__ __launch_bounds__(RT) void adain_act_fwd_k(AdainArgs g, float* Y, long y_bs, float* Yp,
                                                     long yp_bs) {
    const int row = blockIdx.y;
    const int n = row / g.C, c = row - n * g.C;
    const FwdRow rc = fwd_row(g, row, n, c);
    const long off = static_cast<long>(c) * g.L;
    const float* x = g.X + n * g.x_bs + off;
    float* y = Y + n * y_bs + off;
    float* yp = Yp ? Yp + n * yp_bs + off : nullptr;
    const int l0 = blockIdx.x * CH + threadIdx.x;
    float v[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int l = l0 + j * RT;
        v[j] = l < g.L ? x[l] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int l = l0 + j * RT;
        if (l >= g.L) break;
        float s;
        const float yv = fwd_elem(g, rc, v[j], s);
        if (yp) yp[l] = s;
        y[l] = yv;
    }
}

// The 16-byte form of a row's chunked pass. Every operand of a row shares
// the row's offset modulo 4 floats (16-B aligned bases, batch strides equal
// modulo 4; the launcher checks), so a row splits into a head of up to 3
// elements, whole float4s and a tail of up to 3; block 0 of the row does
// the head and tail. grid (cdiv(float4s, RT * EPT / 4), N*C).
__device__ inline int row_head(const float* p, int L) {
    return min(static_cast<int>((4u - ((reinterpret_cast<unsigned long long>(p) >> 2) & 3u)) & 3u), L);
}

__global__ __launch_bounds__(RT) void adain_act_fwd_v4_k(AdainArgs g, float* Y, long y_bs, float* Yp,
                                                        long yp_bs) {
    // a raised wave priority: beside the weight-grad GEMMs of another stream,
    // this pass sits on the conv chain, and its loads and stores win
    // issue slots over their MFMA waves on a shared SIMD
    __builtin_amdgcn_s_setprio(2);
    constexpr int Q = EPT / 4;  // float4s per thread
    const int row = blockIdx.y;
    const int n = row / g.C, c = row - n * g.C;
    const long off = static_cast<long>(c) * g.L;
    const float* x = g.X + n * g.x_bs + off;
    float* y = Y + n * y_bs + off;
    float* yp = Yp ? Yp + n * yp_bs + off : nullptr;
    const int head = row_head(x, g.L);
    const int nq = (g.L - head) >> 2;
    // the data loads go out before the row's constants are fetched, as
    // 16-byte buffer loads issued unconditionally (past the row's float4
    // body they read 0)
    const __amdgpu_buffer_rsrc_t xr = uniform_rsrc(x + head, nq * 16);
    float4* y4 = reinterpret_cast<float4*>(y + head);
    float4* yp4 = yp ? reinterpret_cast<float4*>(yp + head) : nullptr;
    const int q0 = blockIdx.x * (RT * Q) + threadIdx.x;
    float4 v[Q];
#pragma unroll
    for (int j = 0; j < Q; ++j)
        v[j] = __builtin_bit_cast(float4, buf_ld_f4(xr, (q0 + j * RT) * 16, 0, 0));
    const FwdRow rc = fwd_row(g, row, n, c);
    if (blockIdx.x == 0) {
        const int t = threadIdx.x;
        const int l = t < 4 ? t : head + 4 * nq + (t - 4);
        if ((t < 4 && l < head) || (t >= 4 && t < 8 && l < g.L)) {
            float s;
            const float yv = fwd_elem(g, rc, x[l], s);
            if (yp) yp[l] = s;
            y[l] = yv;
        }
    }
#pragma unroll
    for (int j = 0; j < Q; ++j) {
        const int q = q0 + j * RT;
        if (q >= nq) break;
        float4 s, o;
        o.x = fwd_elem(g, rc, v[j].x, s.x);
        o.y = fwd_elem(g, rc, v[j].y, s.y);
        o.z = fwd_elem(g, rc, v[j].z, s.z);
        o.w = fwd_elem(g, rc, v[j].w, s.w);
        if (yp4) yp4[q] = s;
        y4[q] = o;
    }
}

// part[(row*nch + ch)*3 + {0,1,2}] = chunk sums of ds, ds*xh and (SNAKE) the
// alpha-grad integrand; dgamma = sum(ds*xh), dbeta = sum(ds).
__global__ __launch_bounds__(RT) void adain_bwd_part_k(AdainArgs g, const float* dY, long dy_bs, int nch,
                                                      double* part) {
    __shared__ double red[RT / 64];
    const int row = blockIdx.y, ch = blockIdx.x;
    const int n = row / g.C, c = row - n * g.C;
    const float2 st = g.stats[row];
    const float g1 = 1.0f + g.gamma[n * g.gb_bs + c];
    const float bt = g.beta ? g.beta[n * g.gb_bs + c] : 0.0f;
    const float a = g.act == KDEC_ACT_SNAKE ? g.alpha[c] : 0.0f;
    const long off = static_cast<long>(c) * g.L;
    const float* x = g.X + n * g.x_bs + off;
    const float* dy = dY + n * dy_bs + off;
    const int l0 = ch * CH + threadIdx.x;
    float xv[EPT], dv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int l = l0 + j * RT;
        const bool in = l < g.L;
        xv[j] = in ? x[l] : st.x;   // xh = 0 and ds = 0 past the row: no contribution
        dv[j] = in ? dy[l] : 0.0f;
    }
    // per-thread sums of EPT terms in float, across the block in double
    float fsd = 0.0f, fsdx = 0.0f, fsa = 0.0f;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const float xh = (xv[j] - st.x) * st.y;
        const float s = g1 * xh + bt;
        const float ds = act_bwd(g.act, dv[j], s, g.slope, a, fsa);
        fsd += ds;
        fsdx += ds * xh;
    }
    const double sd = block_sum(fsd, red);
    const double sdx = block_sum(fsdx, red);
    const double sa = g.act == KDEC_ACT_SNAKE ? block_sum(fsa, red) * alpha_scale(g.act, a) : 0.0;
    if (threadIdx.x == 0) {
        double* p = part + (static_cast<long>(row) * nch + ch) * 3;
        p[0] = sd;
        p[1] = sdx;
        p[2] = sa;
    }
}

// Per row: dgamma / dbeta (overwritten), the row's alpha-grad share, and the
// two means the input grad needs.
__global__ void adain_bwd_fin_k(const double* part, int rows, int nch, int C, int L, float* dgamma, float* dbeta,
                                long dgb_bs, float* dalpha_part, float2* rowv) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const int n = row / C, c = row - n * C;
    double sd = 0.0, sdx = 0.0, sa = 0.0;
    for (int ch = 0; ch < nch; ++ch) {
        const double* p = part + (static_cast<long>(row) * nch + ch) * 3;
        sd += p[0];
        sdx += p[1];
        sa += p[2];
    }
    if (dgamma) dgamma[n * dgb_bs + c] = static_cast<float>(sdx);
    if (dbeta) dbeta[n * dgb_bs + c] = static_cast<float>(sd);
    if (dalpha_part) dalpha_part[row] = static_cast<float>(sa);
    rowv[row] = make_float2(static_cast<float>(sd / L), static_cast<float>(sdx / L));
}

// One row's constants of the AdaIN(+activation) backward apply.
struct BwdRow {
    float mean, rstd, g1, bt, a, k1, mds, mdsx;
};

__device__ inline BwdRow bwd_row(const AdainArgs& g, const float2* rowv, int row, int n, int c) {
    const float2 st = g.stats[row];
    const float2 mv = rowv[row];
    BwdRow r;
    r.mean = st.x;
    r.rstd = st.y;
    r.g1 = 1.0f + g.gamma[n * g.gb_bs + c];
    r.bt = g.beta ? g.beta[n * g.gb_bs + c] : 0.0f;
    r.a = g.act == KDEC_ACT_SNAKE ? g.alpha[c] : 0.0f;
    r.k1 = st.y * r.g1;
    r.mds = mv.x;
    r.mdsx = mv.y;
    return r;
}

// dx = rstd * g1 * (ds - mean(ds) - xh * mean(ds*xh)) (+ the residual grad)
__device__ inline float bwd_elem(const AdainArgs& g, const BwdRow& r, float xv, float dv, bool has_r, float rv) {
    const float xh = (xv - r.mean) * r.rstd;
    const float s = r.g1 * xh + r.bt;
    float unused = 0.0f;
    const float ds = act_bwd(g.act, dv, s, g.slope, r.a, unused);
    float v = r.k1 * (ds - r.mds - xh * r.mdsx);
    if (has_r) v += rv;
    return v;
}

// grid (chunks, N*C)
// With `ap`, the block of row (0, c), chunk 0, also adds dalpha[c] +=
// sum_n ap[n*C + c] in that order (as dalpha_reduce would).
__device__ inline void dalpha_fold(const float* ap, float* dalpha, int N, int C, int n, int c) {
    if (ap && n == 0 && blockIdx.x == 0 && threadIdx.x == 0) {
        double acc = 0.0;
        for (int k = 0; k < N; ++k) acc += ap[k * C + c];
        dalpha[c] += static_cast<float>(acc);
    }
}

__global__ __launch_bounds__(RT) void adain_bwd_apply_k(AdainArgs g, const float* dY, long dy_bs,
                                                       const float* R, long r_bs, float* dX, long dx_bs,
                                                       const float2* rowv, const float* ap, float* dalpha,
                                                       int N) {
    const int row = blockIdx.y;
    const int n = row / g.C, c = row - n * g.C;
    dalpha_fold(ap, dalpha, N, g.C, n, c);
    const BwdRow rc = bwd_row(g, rowv, row, n, c);
    const long off = static_cast<long>(c) * g.L;
    const float* x = g.X + n * g.x_bs + off;
    const float* dy = dY + n * dy_bs + off;
    const float* r = R ? R + n * r_bs + off : nullptr;
    float* dx = dX + n * dx_bs + off;
    const int l0 = blockIdx.x * CH + threadIdx.x;
    float xv[EPT], dv[EPT], rv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int l = l0 + j * RT;
        const bool in = l < g.L;
        xv[j] = in ? x[l] : 0.0f;
        dv[j] = in ? dy[l] : 0.0f;
        rv[j] = (in && r) ? r[l] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int l = l0 + j * RT;
        if (l >= g.L) break;
        dx[l] = bwd_elem(g, rc, xv[j], dv[j], r != nullptr, rv[j]);
    }
}

// The 16-byte form (head / float4s / tail as adain_act_fwd_v4_k), with
// BWD_Q float4s of each operand per thread: two rather than four gives twice
// the blocks at the same bytes in flight per CU, so blocks that start late
// (beside the weight-grad GEMMs) hold less of the pass (one-stream family
// 5.20 -> 5.12 ms/step, overlapped 16.1 -> 12.7; eight: 5.50).
constexpr int BWD_Q = 2;
unsigned v4_blocks_bwd(int L) { return static_cast<unsigned>(std::max(1L, cdiv(static_cast<long>(L) / 4, RT * BWD_Q))); }
__global__ __launch_bounds__(RT) void adain_bwd_apply_v4_k(AdainArgs g, const float* dY, long dy_bs,
                                                          const float* R, long r_bs, float* dX, long dx_bs,
                                                          const float2* rowv, const float* ap, float* dalpha,
                                                          int N) {
    // a raised wave priority: beside the weight-grad GEMMs of another stream,
    // this pass sits on the conv chain, and its loads and stores win
    // issue slots over their MFMA waves on a shared SIMD
    __builtin_amdgcn_s_setprio(2);
    constexpr int Q = BWD_Q;
    const int row = blockIdx.y;
    const int n = row / g.C, c = row - n * g.C;
    const long off = static_cast<long>(c) * g.L;
    const float* x = g.X + n * g.x_bs + off;
    const float* dy = dY + n * dy_bs + off;
    const float* r = R ? R + n * r_bs + off : nullptr;
    float* dx = dX + n * dx_bs + off;
    const bool has_r = r != nullptr;
    const int head = row_head(x, g.L);
    const int nq = (g.L - head) >> 2;
    // The data loads go out before the row's constants are fetched, as
    // 16-byte buffer loads over the row's float4 body issued unconditionally
    // (past the body, or with no residual grad, they read 0): written as
    // guarded float4 loads they were split into four exec-masked 4-byte
    // loads each, a quarter of the bytes per request.
    const __amdgpu_buffer_rsrc_t xr = uniform_rsrc(x + head, nq * 16);
    const __amdgpu_buffer_rsrc_t dr = uniform_rsrc(dy + head, nq * 16);
    const __amdgpu_buffer_rsrc_t rr = uniform_rsrc(has_r ? r + head : x + head, has_r ? nq * 16 : 0);
    float4* o4 = reinterpret_cast<float4*>(dx + head);
    const int q0 = blockIdx.x * (RT * Q) + threadIdx.x;
    float4 xv[Q], dv[Q], rv[Q];
#pragma unroll
    for (int j = 0; j < Q; ++j) {
        const int o = (q0 + j * RT) * 16;
        xv[j] = __builtin_bit_cast(float4, buf_ld_f4(xr, o, 0, 0));
        dv[j] = __builtin_bit_cast(float4, buf_ld_f4(dr, o, 0, 0));
        rv[j] = __builtin_bit_cast(float4, buf_ld_f4(rr, o, 0, 0));
    }
    dalpha_fold(ap, dalpha, N, g.C, n, c);
    const BwdRow rc = bwd_row(g, rowv, row, n, c);
    if (blockIdx.x == 0) {
        const int t = threadIdx.x;
        const int l = t < 4 ? t : head + 4 * nq + (t - 4);
        if ((t < 4 && l < head) || (t >= 4 && t < 8 && l < g.L))
            dx[l] = bwd_elem(g, rc, x[l], dy[l], has_r, has_r ? r[l] : 0.0f);
    }
#pragma unroll
    for (int j = 0; j < Q; ++j) {
        const int q = q0 + j * RT;
        if (q >= nq) break;
        float4 o;
        o.x = bwd_elem(g, rc, xv[j].x, dv[j].x, has_r, rv[j].x);
        o.y = bwd_elem(g, rc, xv[j].y, dv[j].y, has_r, rv[j].y);
        o.z = bwd_elem(g, rc, xv[j].z, dv[j].z, has_r, rv[j].z);
        o.w = bwd_elem(g, rc, xv[j].w, dv[j].w, has_r, rv[j].w);
        o4[q] = o;
    }
}

// Whether the 16-byte row passes apply: every base 16-B aligned and every
// batch stride equal to the first modulo 4 floats (then a row's operands all
// start at the same offset modulo 4).
bool rows_v4(std::initializer_list<std::pair<const void*, long>> ops) {
    long bs0 = -1;
    for (const auto& o : ops) {
        if (!o.first) continue;
        if (reinterpret_cast<unsigned long long>(o.first) & 15u) return false;
        if (bs0 < 0) bs0 = o.second & 3;
        else if ((o.second & 3) != bs0) return false;
    }
    return true;
}

unsigned v4_blocks(int L) { return static_cast<unsigned>(std::max(1L, cdiv(static_cast<long>(L) / 4, RT * EPT / 4))); }

// ─── one block per row, the row held in registers ───────────────────────
// For rows of up to NTB*EPR elements: the forward reads x once (statistics
// and the affine+activation in one pass, 8 B/elem), the backward reads x and
// dY once (12 B/elem + the residual) when both fit (BOTH), else keeps x and
// reads dY twice. Rows go through raw buffer loads / stores over exactly the
// row: element j of a thread is voffset + j*NTB*4 with the j term a scalar
// offset, so no per-element address registers are needed, and lanes past the
// row read zeros and drop their stores.

__device__ inline __amdgpu_buffer_rsrc_t row_rsrc(const float* base, int L) { return uniform_rsrc(base, L * 4); }

__device__ inline float row_ld(__amdgpu_buffer_rsrc_t r, int voff, int j, int ntb) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, j * ntb * 4, 0));
}

__device__ inline void row_st(__amdgpu_buffer_rsrc_t r, float v, int voff, int j, int ntb) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff, j * ntb * 4, 0);
}

// Element e of a thread's row share: with V = 1, element e*NTB + t; with
// V = 4 (rows of a multiple of 4 floats on 16-B aligned bases), element
// 4*((e/4)*NTB + t) + e%4, one 16-B access per four elements. Past the row
// the descriptor reads 0 and drops stores, a float4 wholly in either case.

template <int V, int NTB>
__device__ inline void row_ld_grp(__amdgpu_buffer_rsrc_t r, int j, float* v) {
    if constexpr (V == 1) {
        v[0] = row_ld(r, threadIdx.x * 4, j, NTB);
    } else {
        const f32x4 q = buf_ld_f4(r, threadIdx.x * 16, j * NTB * 16, 0);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    }
}
template <int V, int NTB>
__device__ inline void row_st_grp(__amdgpu_buffer_rsrc_t r, int j, const float* v) {
    if constexpr (V == 1) {
        row_st(r, v[0], threadIdx.x * 4, j, NTB);
    } else {
        buf_st_f4(f32x4{v[0], v[1], v[2], v[3]}, r, threadIdx.x * 16, j * NTB * 16, 0);
    }
}

// Rows longer than the register part (TT > 0): registers hold the NTB*EPR
// elements [head, head + NTB*EPR), 16-B aligned when V = 4 (head: the 0..3
// elements before the row's first 16-B boundary, given 16-B aligned bases and
// batch strides), and the rest of the row -- the head elements, then the
// elements past the register part -- is dealt out as i = tid + j*NTB, i < the
// rest's length, element rest_elem(i).
__device__ inline int row_head(int c, int L) { return (4 - (((c & 3) * (L & 3)) & 3)) & 3; }
__device__ inline int rest_elem(int i, int head, int rb) { return i < head ? i : i + rb; }

// stats[row] = (mean, rstd); Y = act((1 + gamma) * xhat + beta), the row held
// in registers between the statistics and the affine pass (V as for the
// backward: 16-B groups on aligned rows of a multiple of 4 floats, or past
// the head of a long row). TT > 0: up to TT rest elements per thread, also
// held in registers.
template <int NTB, int EPR, int V, int TT>
__global__ __launch_bounds__(NTB) void adain_fwd_row_k(AdainArgs g, float eps, float2* stats, float* Y, long y_bs,
                                                      float* Yp, long yp_bs) {
    static_assert(EPR % V == 0, "whole groups per thread");
    __shared__ double red[NTB / 64];
    constexpr int RB = NTB * EPR;
    const int row = blockIdx.x;
    const int n = row / g.C, c = row - n * g.C;
    const long off = static_cast<long>(c) * g.L;
    const float* x = g.X + n * g.x_bs + off;
    const int head = (TT > 0 && V == 4) ? row_head(c, g.L) : 0;
    const int Lr = TT > 0 ? RB : g.L;      // register-part length
    const int nrest = TT > 0 ? g.L - RB : 0;
    const __amdgpu_buffer_rsrc_t xr = row_rsrc(x + head, Lr);
    const double x0 = x[0];  // shift for a well-conditioned variance
    float v[EPR];
#pragma unroll
    for (int j = 0; j < EPR / V; ++j) row_ld_grp<V, NTB>(xr, j, v + V * j);
    // the rest through a descriptor over the whole row: one offset register
    // per element, and lanes past the rest read 0
    const __amdgpu_buffer_rsrc_t xw = row_rsrc(x, TT > 0 ? g.L : 0);
    float t[TT > 0 ? TT : 1];
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int i = threadIdx.x + j * NTB;
        t[j] = row_ld(xw, i < nrest ? rest_elem(i, head, RB) * 4 : g.L * 4, 0, NTB);
    }
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int j = 0; j < EPR / V; ++j) {
        if (V * (j * NTB + threadIdx.x) >= Lr) continue;  // past the row (a group lies wholly in or out)
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const double d = static_cast<double>(v[V * j + e]) - x0;
            s1 += d;
            s2 += d * d;
            // one difference live at a time (else all EPR + TT of them are
            // kept in double between a sum pass and a square pass)
            asm volatile("" : "+v"(s1), "+v"(s2));
        }
    }
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        if (threadIdx.x + j * NTB >= nrest) continue;
        const double d = static_cast<double>(t[j]) - x0;
        s1 += d;
        s2 += d * d;
        asm volatile("" : "+v"(s1), "+v"(s2));
    }
    s1 = block_sum_n<NTB>(s1, red);
    s2 = block_sum_n<NTB>(s2, red);
    const double m = s1 / g.L;
    double var = s2 / g.L - m * m;
    if (var < 0.0) var = 0.0;
    const float2 st = make_float2(static_cast<float>(x0 + m), static_cast<float>(1.0 / sqrt(var + static_cast<double>(eps))));
    if (threadIdx.x == 0) stats[row] = st;
    const float g1 = 1.0f + g.gamma[n * g.gb_bs + c];
    const float bt = g.beta ? g.beta[n * g.gb_bs + c] : 0.0f;
    const float a = g.act == KDEC_ACT_SNAKE ? g.alpha[c] : 1.0f;
    const float ia = 1.0f / a;
    float* yrow = Y + n * y_bs + off;
    float* prow = Yp ? Yp + n * yp_bs + off : nullptr;
    const __amdgpu_buffer_rsrc_t yr = row_rsrc(yrow + head, Lr);
    const __amdgpu_buffer_rsrc_t pr = row_rsrc(prow ? prow + head : Y, prow ? Lr : 0);
#pragma unroll
    for (int j = 0; j < EPR / V; ++j) {
        float yv[V], sv[V];
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const float xh = (v[V * j + e] - st.x) * st.y;
            sv[e] = g1 * xh + bt;
            yv[e] = act_fwd(g.act, sv[e], g.slope, a, ia);
        }
        row_st_grp<V, NTB>(yr, j, yv);
        row_st_grp<V, NTB>(pr, j, sv);  // dropped without a pre-activation output
    }
    const __amdgpu_buffer_rsrc_t yw = row_rsrc(yrow, TT > 0 ? g.L : 0);
    const __amdgpu_buffer_rsrc_t pw = row_rsrc(prow ? prow : Y, (TT > 0 && prow) ? g.L : 0);
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int i = threadIdx.x + j * NTB;
        if (i >= nrest) continue;
        const int lo = rest_elem(i, head, RB) * 4;
        const float xh = (t[j] - st.x) * st.y;
        const float sv = g1 * xh + bt;
        row_st(yw, act_fwd(g.act, sv, g.slope, a, ia), lo, 0, NTB);
        row_st(pw, sv, lo, 0, NTB);  // dropped without a pre-activation output
    }
}

// TT > 0: a long row (layout as adain_fwd_row_k); the rest's x and ds stay
// in dynamic LDS, [0, nrest) and [nrest, 2*nrest), each thread touching only
// its own elements.
template <int NTB, int EPR, bool BOTH, int V, int TT>
__global__ __launch_bounds__(NTB) void adain_bwd_row_k(AdainArgs g, const float* dY, long dy_bs, const float* R,
                                                      long r_bs, float* dX, long dx_bs, float* dgamma,
                                                      float* dbeta, long dgb_bs, float* dalpha_part,
                                                      float* dalpha_acc) {
    __shared__ double red[NTB / 64];
    extern __shared__ float rest[];
    constexpr int RB = NTB * EPR;
    const int row = blockIdx.x;
    const int n = row / g.C, c = row - n * g.C;
    const float2 st = g.stats[row];
    const float g1 = 1.0f + g.gamma[n * g.gb_bs + c];
    const float bt = g.beta ? g.beta[n * g.gb_bs + c] : 0.0f;
    const float a = g.act == KDEC_ACT_SNAKE ? g.alpha[c] : 0.0f;
    const long off = static_cast<long>(c) * g.L;
    const float* xrow = g.X + n * g.x_bs + off;
    const float* dyrow = dY + n * dy_bs + off;
    const int head = (TT > 0 && V == 4) ? row_head(c, g.L) : 0;
    const int Lr = TT > 0 ? RB : g.L;      // register-part length
    const int nrest = TT > 0 ? g.L - RB : 0;
    const __amdgpu_buffer_rsrc_t xr = row_rsrc(xrow + head, Lr);
    const __amdgpu_buffer_rsrc_t dr = row_rsrc(dyrow + head, Lr);
    static_assert(V == 1 || (BOTH && EPR % 4 == 0), "16-B row access holds both rows");
    static_assert(TT == 0 || BOTH, "long rows hold both rows");
    const int vo = threadIdx.x * 4;
    float xv[EPR], dv[BOTH ? EPR : 1];
#pragma unroll
    for (int j = 0; j < EPR / V; ++j) {
        row_ld_grp<V, NTB>(xr, j, xv + V * j);
        if (BOTH) row_ld_grp<V, NTB>(dr, j, dv + V * j);  // zero past the row: no contribution
    }
    // per-thread sums of at most EPR + TT terms in float, across the block in double
    float fsd = 0.0f, fsdx = 0.0f, fsa = 0.0f;
    const __amdgpu_buffer_rsrc_t xw = row_rsrc(xrow, TT > 0 ? g.L : 0);
    const __amdgpu_buffer_rsrc_t dw = row_rsrc(dyrow, TT > 0 ? g.L : 0);
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int i = threadIdx.x + j * NTB;
        if (i >= nrest) continue;
        const int lo = rest_elem(i, head, RB) * 4;
        const float xl = row_ld(xw, lo, 0, NTB);
        const float xh = (xl - st.x) * st.y;
        const float ds = act_bwd(g.act, row_ld(dw, lo, 0, NTB), g1 * xh + bt, g.slope, a, fsa);
        rest[i] = xl;
        rest[nrest + i] = ds;
        fsd += ds;
        fsdx += ds * xh;
    }
#pragma unroll
    for (int j = 0; j < EPR; ++j) {
        const float dyj = BOTH ? dv[j] : row_ld(dr, vo, j, NTB);
        const float xh = (xv[j] - st.x) * st.y;
        const float s = g1 * xh + bt;
        const float ds = act_bwd(g.act, dyj, s, g.slope, a, fsa);
        if (BOTH) dv[j] = ds;
        fsd += ds;
        fsdx += ds * xh;
    }
    const double sd = block_sum_n<NTB>(fsd, red);
    const double sdx = block_sum_n<NTB>(fsdx, red);
    const double sa = g.act == KDEC_ACT_SNAKE ? block_sum_n<NTB>(fsa, red) * alpha_scale(g.act, a) : 0.0;
    if (threadIdx.x == 0) {
        if (dgamma) dgamma[n * dgb_bs + c] = static_cast<float>(sdx);
        if (dbeta) dbeta[n * dgb_bs + c] = static_cast<float>(sd);
        if (dalpha_part) dalpha_part[row] = static_cast<float>(sa);
        if (dalpha_acc) dalpha_acc[c] += static_cast<float>(sa);  // one utterance: one row per channel
    }
    const float mds = static_cast<float>(sd / g.L);
    const float mdsx = static_cast<float>(sdx / g.L);
    const float k1 = st.y * g1;
    float* dxrow = dX + n * dx_bs + off;
    const float* rrow = R ? R + n * r_bs + off : nullptr;
    const __amdgpu_buffer_rsrc_t xo = row_rsrc(dxrow + head, Lr);
    // without a residual the descriptor covers nothing and its loads read 0
    const __amdgpu_buffer_rsrc_t rr = row_rsrc(rrow ? rrow + head : dY, rrow ? Lr : 0);
    const __amdgpu_buffer_rsrc_t ow = row_rsrc(dxrow, TT > 0 ? g.L : 0);
    const __amdgpu_buffer_rsrc_t rw = row_rsrc(rrow ? rrow : dY, (TT > 0 && rrow) ? g.L : 0);
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int i = threadIdx.x + j * NTB;
        if (i >= nrest) continue;
        const int lo = rest_elem(i, head, RB) * 4;
        const float xh = (rest[i] - st.x) * st.y;
        const float val = k1 * (rest[nrest + i] - mds - xh * mdsx) + row_ld(rw, lo, 0, NTB);  // R or 0
        row_st(ow, val, lo, 0, NTB);
    }
#pragma unroll
    for (int j = 0; j < EPR / V; ++j) {
        float val[V];
        row_ld_grp<V, NTB>(rr, j, val);
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const int i = V * j + e;
            const float xh = (xv[i] - st.x) * st.y;
            float ds;
            if (BOTH) {
                ds = dv[i];
            } else {
                float unused = 0.0f;
                ds = act_bwd(g.act, row_ld(dr, vo, j, NTB), g1 * xh + bt, g.slope, a, unused);
            }
            val[e] += k1 * (ds - mds - xh * mdsx);
        }
        row_st_grp<V, NTB>(xo, j, val);
    }
}

// dalpha[c] += sum_n part[n*C + c] (fixed order)
__global__ void dalpha_reduce(const float* part, float* dalpha, int N, int C) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    double acc = 0.0;
    for (int n = 0; n < N; ++n) acc += part[n * C + c];
    dalpha[c] += static_cast<float>(acc);
}

// Elementwise passes over rows of `len` floats per utterance (blockIdx.y);
// V = 4: whole float4s (every row base 16-B aligned, len a multiple of 4),
// the same per-element arithmetic as V = 1 with a quarter of the memory
// instructions.
template <int V>
using vec_t = typename std::conditional<V == 4, float4, float>::type;

template <class F>
__device__ inline float4 map4(float4 a, F f) {
    return make_float4(f(a.x), f(a.y), f(a.z), f(a.w));
}
template <class F>
__device__ inline float map4(float a, F f) {
    return f(a);
}
template <class F>
__device__ inline float4 map4(float4 a, float4 b, F f) {
    return make_float4(f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w));
}
template <class F>
__device__ inline float map4(float a, float b, F f) {
    return f(a, b);
}

template <int V>
__global__ void leaky_fwd_k(const float* X, long x_bs, float* Y, long y_bs, long len, float slope) {
    const int n = blockIdx.y;
    const vec_t<V>* x = reinterpret_cast<const vec_t<V>*>(X + n * x_bs);
    vec_t<V>* y = reinterpret_cast<vec_t<V>*>(Y + n * y_bs);
    const long nv = len / V;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < nv;
         i += static_cast<long>(gridDim.x) * blockDim.x)
        y[i] = map4(x[i], [slope](float v) { return v > 0.0f ? v : slope * v; });
}

// dx = (x > 0 ? dy : slope * dy) * scale (scale 1: the plain backward; any
// other: the same two roundings as the backward and a separate scaling pass)
template <int V>
__global__ void leaky_bwd_k(const float* X, long x_bs, const float* dY, long dy_bs, float* dX,
                            long dx_bs, long len, float slope, float scale) {
    const int n = blockIdx.y;
    const vec_t<V>* x = reinterpret_cast<const vec_t<V>*>(X + n * x_bs);
    const vec_t<V>* dy = reinterpret_cast<const vec_t<V>*>(dY + n * dy_bs);
    vec_t<V>* dx = reinterpret_cast<vec_t<V>*>(dX + n * dx_bs);
    const long nv = len / V;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < nv;
         i += static_cast<long>(gridDim.x) * blockDim.x)
        dx[i] = map4(x[i], dy[i], [slope, scale](float xv, float d) {
            const float g = xv > 0.0f ? d : slope * d;
            return scale * g;
        });
}

template <int V>
__global__ void axpby_k(float a, const float* A, long a_bs, float b, const float* B, long b_bs,
                        float* Y, long y_bs, long len) {
    const int n = blockIdx.y;
    const vec_t<V>* pa = reinterpret_cast<const vec_t<V>*>(A + n * a_bs);
    const vec_t<V>* pb = B ? reinterpret_cast<const vec_t<V>*>(B + n * b_bs) : nullptr;
    vec_t<V>* y = reinterpret_cast<vec_t<V>*>(Y + n * y_bs);
    const long nv = len / V;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < nv;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        if (pb)  // uniform
            y[i] = map4(pa[i], pb[i], [a, b](float u, float w) {
                float v = a * u;
                v += b * w;
                return v;
            });
        else
            y[i] = map4(pa[i], [a](float u) { return a * u; });
    }
}

// Y = (A + B) + C, the two float adds in that order; V = 4: whole float4s
// (every row base 16-B aligned, len a multiple of 4).
template <int V>
__global__ void add3_k(const float* A, long a_bs, const float* B, long b_bs, const float* C, long c_bs, float* Y,
                       long y_bs, long len) {
    const int n = blockIdx.y;
    const long nv = len / V;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < nv;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        if constexpr (V == 4) {
            const float4 a = reinterpret_cast<const float4*>(A + n * a_bs)[i];
            const float4 b = reinterpret_cast<const float4*>(B + n * b_bs)[i];
            const float4 c = reinterpret_cast<const float4*>(C + n * c_bs)[i];
            reinterpret_cast<float4*>(Y + n * y_bs)[i] =
                make_float4((a.x + b.x) + c.x, (a.y + b.y) + c.y, (a.z + b.z) + c.z, (a.w + b.w) + c.w);
        } else {
            Y[n * y_bs + i] = (A[n * a_bs + i] + B[n * b_bs + i]) + C[n * c_bs + i];
        }
    }
}

// add3_k that also writes Z = leaky_relu(Y, slope): the generator stage's
// resblock sum and the next layer's activation in one pass.
template <int V>
__global__ void add3_leaky_k(const float* A, long a_bs, const float* B, long b_bs, const float* C, long c_bs,
                             float* Y, long y_bs, float* Z, long z_bs, long len, float slope) {
    const int n = blockIdx.y;
    const long nv = len / V;
    auto lk = [slope](float v) { return v > 0.0f ? v : slope * v; };
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < nv;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        if constexpr (V == 4) {
            const float4 a = reinterpret_cast<const float4*>(A + n * a_bs)[i];
            const float4 b = reinterpret_cast<const float4*>(B + n * b_bs)[i];
            const float4 c = reinterpret_cast<const float4*>(C + n * c_bs)[i];
            const float4 y = make_float4((a.x + b.x) + c.x, (a.y + b.y) + c.y, (a.z + b.z) + c.z, (a.w + b.w) + c.w);
            reinterpret_cast<float4*>(Y + n * y_bs)[i] = y;
            reinterpret_cast<float4*>(Z + n * z_bs)[i] = make_float4(lk(y.x), lk(y.y), lk(y.z), lk(y.w));
        } else {
            const float y = (A[n * a_bs + i] + B[n * b_bs + i]) + C[n * c_bs + i];
            Y[n * y_bs + i] = y;
            Z[n * z_bs + i] = lk(y);
        }
    }
}

// y[c][0] = x[c][1]; y[c][j+1] = x[c][j]
__global__ void pad_fwd_k(const float* X, long x_bs, float* Y, long y_bs, int C, int L) {
    const int n = blockIdx.y;
    const long tot = static_cast<long>(C) * (L + 1);
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < tot;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int c = static_cast<int>(i / (L + 1));
        const int j = static_cast<int>(i - static_cast<long>(c) * (L + 1));
        const float* x = X + n * x_bs + static_cast<long>(c) * L;
        Y[n * y_bs + i] = j == 0 ? x[1] : x[j - 1];
    }
}

// dx[c][j] = dy[c][j+1] (+ dy[c][0] at j = 1)
__global__ void pad_bwd_k(const float* dY, long dy_bs, float* dX, long dx_bs, int C, int L) {
    const int n = blockIdx.y;
    const long tot = static_cast<long>(C) * L;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < tot;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int c = static_cast<int>(i / L);
        const int j = static_cast<int>(i - static_cast<long>(c) * L);
        const float* dy = dY + n * dy_bs + static_cast<long>(c) * (L + 1);
        float v = dy[j + 1];
        if (j == 1) v += dy[0];
        dX[n * dx_bs + i] = v;
    }
}

// add3_k over rows of L + 1 that also writes the left reflect pad's adjoint:
// Y = (A + B) + C, and Z[c][j] = Y[c][j + 1] (+ Y[c][0] at j = 1), rows of L.
// Block (row, x): positions [x * 1024, x * 1024 + 1024) of row `row` (of N*C),
// four per thread. Y may alias A, so Y[c][0] reaches the lane that forms
// Z[c][1] (lane 2 of block x = 0's first wave) by a shuffle from lane 0,
// never by a read of A after lane 0 has stored over it.
__global__ __launch_bounds__(256) void add3_unpad_k(const float* A, long a_bs, const float* B, long b_bs,
                                                    const float* Cc, long c_bs, float* Y, long y_bs, float* Z,
                                                    long z_bs, int C, int L) {
    const int row = blockIdx.x;
    const int n = row / C, c = row - n * C;
    const long ro = static_cast<long>(c) * (L + 1);
    const float* a = A + n * a_bs + ro;
    const float* b = B + n * b_bs + ro;
    const float* cc = Cc + n * c_bs + ro;
    float* y = Y + n * y_bs + ro;
    float* z = Z + n * z_bs + static_cast<long>(c) * L;
    const int j0 = blockIdx.y * 1024 + threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int j = j0 + q * 256;
        const bool in = j <= L;
        const float v = in ? (a[j] + b[j]) + cc[j] : 0.0f;
        float vz = v;
        if (q == 0 && blockIdx.y == 0) {
            const float y0 = __shfl(v, 0);
            if (j == 2) vz = v + y0;
        }
        if (in) {
            y[j] = v;
            if (j >= 1) z[j - 1] = vz;
        }
    }
}

__global__ void near2_fwd_k(const float* X, long x_bs, float* Y, long y_bs, int C, int L) {
    const int n = blockIdx.y;
    const long tot = static_cast<long>(C) * 2 * L;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < tot;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const long c = i / (2 * L);
        const long j = i - c * 2 * L;
        Y[n * y_bs + i] = X[n * x_bs + c * L + (j >> 1)];
    }
}

__global__ void near2_bwd_k(const float* dY, long dy_bs, float* dX, long dx_bs, int C, int L,
                            float scale, float beta) {
    const int n = blockIdx.y;
    const long tot = static_cast<long>(C) * L;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < tot;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const long c = i / L;
        const long l = i - c * L;
        const float* dy = dY + n * dy_bs + c * 2 * L;
        float v = scale * (dy[2 * l] + dy[2 * l + 1]);
        if (beta != 0.0f) v += beta * dX[n * dx_bs + i];
        dX[n * dx_bs + i] = v;
    }
}

__global__ void fill_k(float* Y, long n, float v) {
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * blockDim.x)
        Y[i] = v;
}

// Row-kernel shape for a row of L elements: {threads, elements per thread};
// {0, 0} where the chunked multi-block kernels are faster (measured on the
// decoder's shapes: the forward up to 4096 with 4-byte accesses, up to 49152
// with 16-byte ones; the backward up to 49152 with x and dY both held).
struct RowShape {
    int ntb, epr, tt = 0;
};
// Long rows: 1024 threads, each with EPR register elements and up to TT
// rest elements (the forward keeps them in registers, the backward holds x
// and dY for its register part and stores the rest's x and ds in LDS).
constexpr int FWD_LONG_EPR = 48, FWD_LONG_TT = 13;
constexpr int BWD_LONG_EPR = 44, BWD_LONG_TT = 17;
static_assert(FWD_LONG_EPR + FWD_LONG_TT == BWD_LONG_EPR + BWD_LONG_TT, "one long-row limit");
// A long row holds its register part [head, head + 1024*EPR) with a head of
// up to 3 elements, so it is at least 1024*EPR + 3 long (both shapes' first
// long length, 49155, lies past the register-only kernels), and at most the
// register part plus 1024*TT rest elements, the head among them.
constexpr int ROW_LONG_MIN = 1024 * FWD_LONG_EPR + 3;
constexpr int ROW_LONG_MAX = 1024 * (FWD_LONG_EPR + FWD_LONG_TT);
static_assert(ROW_LONG_MIN >= 1024 * BWD_LONG_EPR + 3, "the backward's register part fits every long row");
bool aligned16(const void* p) { return (reinterpret_cast<unsigned long long>(p) & 15) == 0; }

// v4: 16-B accesses are possible (every row starts on 16 B); v4_long: every
// row's register part does (16-B aligned bases and batch strides, any L).
RowShape row_shape_fwd(int L, bool v4, bool v4_long) {
    if (L <= 1024) return {256, 4};
    if (L <= 4096) return {256, 16};
    if (L > 49152)
        return (v4_long && L >= ROW_LONG_MIN && L <= ROW_LONG_MAX) ? RowShape{1024, FWD_LONG_EPR, FWD_LONG_TT}
                                                                    : RowShape{0, 0};
    if (!v4) return {0, 0};
    if (L <= 16384) return {1024, 16};
    return {1024, 48};
}
bool fwd_v4_long(const AdainArgs& g, const float* Y, long y_bs, const float* Yp, long yp_bs) {
    return g.x_bs % 4 == 0 && y_bs % 4 == 0 && aligned16(g.X) && aligned16(Y) &&
           (!Yp || (yp_bs % 4 == 0 && aligned16(Yp)));
}
bool fwd_v4(const AdainArgs& g, const float* Y, long y_bs, const float* Yp, long yp_bs) {
    return g.L % 4 == 0 && fwd_v4_long(g, Y, y_bs, Yp, yp_bs);
}
RowShape row_shape_fwd(const AdainArgs& g, const float* Y, long y_bs, const float* Yp, long yp_bs) {
    return row_shape_fwd(g.L, fwd_v4(g, Y, y_bs, Yp, yp_bs), fwd_v4_long(g, Y, y_bs, Yp, yp_bs));
}
bool bwd_v4_long(const AdainArgs& g, const float* dY, long dy_bs, const float* R, long r_bs, const float* dX,
                 long dx_bs) {
    return g.x_bs % 4 == 0 && dy_bs % 4 == 0 && dx_bs % 4 == 0 && aligned16(g.X) && aligned16(dY) &&
           aligned16(dX) && (!R || (r_bs % 4 == 0 && aligned16(R)));
}
// long rows need the 16-B register part (v4_long)
RowShape row_shape_bwd(int L, bool v4_long) {
    if (L <= 1024) return {256, 4};
    if (L <= 4096) return {256, 16};
    if (L <= 16384) return {1024, 16};
    if (L <= 49152) return {1024, 48};
    if (v4_long && L >= ROW_LONG_MIN && L <= ROW_LONG_MAX) return {1024, BWD_LONG_EPR, BWD_LONG_TT};
    return {0, 0};
}

int launch_fwd_row(kdec_ctx* ctx, RowShape rsh, unsigned rows, const AdainArgs& g, float eps, float2* st, float* Y,
                   long y_bs, float* Yp, long yp_bs) {
    const bool v4 = rsh.tt ? true : fwd_v4(g, Y, y_bs, Yp, yp_bs);
#define KDEC_FWD_ROW(T, E, V, TT)                                                                              \
    if (rsh.ntb == T && rsh.epr == E && rsh.tt == TT && (V == 4) == v4) {                                      \
        hipLaunchKernelGGL((adain_fwd_row_k<T, E, V, TT>), dim3(rows), dim3(T), 0, ctx->stream, g, eps, st, Y,  \
                           y_bs, Yp, yp_bs);                                                                   \
        return launch_check(ctx, "adain_fwd_row");                                                            \
    }
    KDEC_FWD_ROW(256, 4, 1, 0)
    KDEC_FWD_ROW(256, 16, 1, 0)
    KDEC_FWD_ROW(256, 4, 4, 0)
    KDEC_FWD_ROW(256, 16, 4, 0)
    KDEC_FWD_ROW(1024, 16, 4, 0)
    KDEC_FWD_ROW(1024, 48, 4, 0)
    KDEC_FWD_ROW(1024, FWD_LONG_EPR, 4, FWD_LONG_TT)
#undef KDEC_FWD_ROW
    return fail(ctx, KDEC_EINVAL, "adain forward: no row kernel for this length");
}

int launch_bwd_row(kdec_ctx* ctx, RowShape rsh, unsigned rows, const AdainArgs& g, const float* dY, long dy_bs,
                   const float* R, long r_bs, float* dX, long dx_bs, float* dgamma, float* dbeta, long dgb_bs,
                   float* apart, float* aacc) {
    if (rsh.tt) {  // long rows: the 16-B register part, the rest in LDS
        if (rsh.ntb != 1024 || rsh.epr != BWD_LONG_EPR || rsh.tt != BWD_LONG_TT)
            return fail(ctx, KDEC_EINVAL, "adain backward: no row kernel for this length");
        const void* kern =
            reinterpret_cast<const void*>(&adain_bwd_row_k<1024, BWD_LONG_EPR, true, 4, BWD_LONG_TT>);
        const size_t lds = 2 * static_cast<size_t>(g.L - 1024 * BWD_LONG_EPR) * sizeof(float);
        static std::once_flag once;
        std::call_once(once, [&] {
            (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      2 * 1024 * BWD_LONG_TT * static_cast<int>(sizeof(float)));
        });
        hipLaunchKernelGGL((adain_bwd_row_k<1024, BWD_LONG_EPR, true, 4, BWD_LONG_TT>), dim3(rows), dim3(1024), lds,
                           ctx->stream, g, dY, dy_bs, R, r_bs, dX, dx_bs, dgamma, dbeta, dgb_bs, apart, aacc);
        return launch_check(ctx, "adain_bwd_row");
    }
    // 16-B accesses when every row of every tensor starts on 16 B
    const bool v4 = g.L % 4 == 0 && bwd_v4_long(g, dY, dy_bs, R, r_bs, dX, dx_bs);
#define KDEC_BWD_ROW(T, E, B)                                                                                  \
    if (rsh.ntb == T && rsh.epr == E) {                                                                        \
        if (v4)                                                                                                \
            hipLaunchKernelGGL((adain_bwd_row_k<T, E, B, 4, 0>), dim3(rows), dim3(T), 0, ctx->stream, g, dY,    \
                               dy_bs, R, r_bs, dX, dx_bs, dgamma, dbeta, dgb_bs, apart, aacc);                 \
        else                                                                                                   \
            hipLaunchKernelGGL((adain_bwd_row_k<T, E, B, 1, 0>), dim3(rows), dim3(T), 0, ctx->stream, g, dY,    \
                               dy_bs, R, r_bs, dX, dx_bs, dgamma, dbeta, dgb_bs, apart, aacc);                 \
        return launch_check(ctx, "adain_bwd_row");                                                            \
    }
    KDEC_BWD_ROW(256, 4, true)
    KDEC_BWD_ROW(256, 16, true)
    KDEC_BWD_ROW(1024, 16, true)
    KDEC_BWD_ROW(1024, 48, true)
#undef KDEC_BWD_ROW
    return fail(ctx, KDEC_EINVAL, "adain backward: no row kernel for this length");
}

// Scratch of the AdaIN backward: the per-row alpha-grad shares, and for rows
// longer than the row kernels take the chunk partial sums and the per-row
// means. Every word a launch reads is written earlier in the same call, so
// a reused buffer needs no clearing.
struct BwdScratchLayout {
    size_t apart = 0, part = 0, rowv = 0, total = 0;  // byte offsets, total size
};
size_t round256(size_t b) { return (b + 255) & ~size_t(255); }
BwdScratchLayout bwd_scratch_layout(int N, int C, int L, bool want_alpha, bool v4_long) {
    const size_t rows = static_cast<size_t>(N) * C;
    const bool chunked = !row_shape_bwd(L, v4_long).ntb;
    BwdScratchLayout s;
    size_t off = 0;
    s.apart = off;
    // the row kernels add one utterance's alpha grads directly; shares are
    // kept for N > 1 and for the chunked passes
    off += want_alpha && (N > 1 || chunked) ? round256(rows * sizeof(float)) : 0;
    if (chunked) {
        s.part = off;
        off += round256(rows * static_cast<size_t>(cdiv(L, CH)) * 3 * sizeof(double));
        s.rowv = off;
        off += round256(rows * sizeof(float2));
    }
    s.total = off;
    return s;
}
struct BwdScratch {
    float* apart;
    double* part;
    float2* rowv;
};
BwdScratch bwd_scratch(void* base, const BwdScratchLayout& s) {
    char* b = static_cast<char*>(base);
    return {reinterpret_cast<float*>(b + s.apart), reinterpret_cast<double*>(b + s.part),
            reinterpret_cast<float2*>(b + s.rowv)};
}

unsigned chunks(long len, long cap = 1024) {
    long g = (len + 255) / 256;
    if (g > cap) g = cap;
    if (g < 1) g = 1;
    return static_cast<unsigned>(g);
}

// Whether an elementwise pass may run on whole float4s: len a multiple of 4
// and every (non-null) row base 16-B aligned with a batch stride that keeps
// it so.
bool ew_v4(long len, std::initializer_list<std::pair<const void*, long>> ops) {
    if (len % 4) return false;
    for (const auto& o : ops)
        if (o.first && (((reinterpret_cast<unsigned long long>(o.first) & 15u) != 0) || (o.second & 3) != 0))
            return false;
    return true;
}

int bwd_check(kdec_ctx* ctx, const AdainArgs& g, const float* dY, const float* dX, int N, const char* where) {
    const std::string w(where);
    KDEC_CHECK(ctx, g.X && g.stats && g.gamma && dY && dX && N > 0 && g.C > 0 && g.L > 0, w + ": bad arguments");
    KDEC_CHECK(ctx, g.beta || g.act == KDEC_ACT_NONE, w + ": beta needed to recompute the activation input");
    KDEC_CHECK(ctx, g.act >= KDEC_ACT_NONE && g.act <= KDEC_ACT_SNAKE && (g.act != KDEC_ACT_SNAKE || g.alpha),
               w + ": bad activation");
    return KDEC_OK;
}

// The AdaIN(+activation) backward over caller-provided scratch (laid out by
// bwd_scratch_layout for the same N, C, L, alpha-grad flag and bwd_v4_long).
int bwd_run(kdec_ctx* ctx, const AdainArgs& g, const float* dY, long dy_bs, const float* R, long r_bs, float* dX,
            long dx_bs, float* dgamma, float* dbeta, long dgb_bs, float* dalpha, int N, BwdScratch sc, bool prof) {
    const int C = g.C, L = g.L;
    const int rows = N * C;
    const int nch = static_cast<int>(cdiv(L, CH));
    const bool want_alpha = dalpha && g.act == KDEC_ACT_SNAKE;
    const RowShape rsh = row_shape_bwd(L, bwd_v4_long(g, dY, dy_bs, R, r_bs, dX, dx_bs));
    const double bytes = 4.0 * static_cast<double>(rows) * L * 3 +
                         (R ? 4.0 * static_cast<double>(rows) * L : 0.0);
    if (rsh.ntb) {
        // one utterance: each channel's alpha grad comes from one row, which
        // adds it directly; otherwise per-row shares are summed in order
        const bool direct = want_alpha && N == 1;
        {
            ProfScope ps(prof ? ctx : nullptr, "adain_bwd", 0, bytes);
            if (int rc = launch_bwd_row(ctx, rsh, static_cast<unsigned>(rows), g, dY, dy_bs, R, r_bs, dX, dx_bs,
                                        dgamma, dbeta, dgb_bs, want_alpha && !direct ? sc.apart : nullptr,
                                        direct ? dalpha : nullptr))
                return rc;
        }
        if (want_alpha && !direct) {
            hipLaunchKernelGGL(dalpha_reduce, dim3(static_cast<unsigned>(cdiv(C, 256))), dim3(256), 0, ctx->stream,
                               sc.apart, dalpha, N, C);
            return launch_check(ctx, "dalpha_reduce");
        }
        return KDEC_OK;
    }
    {
        ProfScope ps(prof ? ctx : nullptr, "adain_bwd", 0, 4.0 * static_cast<double>(rows) * L * 5);
        hipLaunchKernelGGL(adain_bwd_part_k, dim3(nch, rows), dim3(RT), 0, ctx->stream, g, dY, dy_bs, nch, sc.part);
        if (int rc = launch_check(ctx, "adain_bwd_part")) return rc;
        hipLaunchKernelGGL(adain_bwd_fin_k, dim3(static_cast<unsigned>(cdiv(rows, 256))), dim3(256), 0,
                           ctx->stream, sc.part, rows, nch, C, L, dgamma, dbeta, dgb_bs,
                           want_alpha ? sc.apart : nullptr, sc.rowv);
        if (int rc = launch_check(ctx, "adain_bwd_fin")) return rc;
        // the apply also folds the per-row alpha shares into dalpha
        const float* ap = want_alpha ? sc.apart : nullptr;
        if (rows_v4({{g.X, g.x_bs}, {dY, dy_bs}, {R, r_bs}, {dX, dx_bs}}))
            hipLaunchKernelGGL(adain_bwd_apply_v4_k, dim3(v4_blocks_bwd(L), rows), dim3(RT), 0, ctx->stream, g, dY,
                               dy_bs, R, r_bs, dX, dx_bs, sc.rowv, ap, dalpha, N);
        else
            hipLaunchKernelGGL(adain_bwd_apply_k, dim3(nch, rows), dim3(RT), 0, ctx->stream, g, dY, dy_bs, R, r_bs,
                               dX, dx_bs, sc.rowv, ap, dalpha, N);
        if (int rc = launch_check(ctx, "adain_bwd_apply")) return rc;
    }
    return KDEC_OK;
}

// adain_bwd_fin_k for many slots per row (the partials of a GEMM epilogue):
// one wave per row, lane j summing slots j, j + 64, ... in double, the lanes'
// sums then added in a fixed tree.
__global__ __launch_bounds__(64) void adain_bwd_fin_wide_k(const double* part, int nch, int C, int L,
                                                           float* dgamma, float* dbeta, long dgb_bs,
                                                           float* dalpha_part, float2* rowv) {
    // a raised wave priority: beside the weight-grad GEMMs of another stream,
    // this pass sits on the conv chain, and its loads and stores win
    // issue slots over their MFMA waves on a shared SIMD
    __builtin_amdgcn_s_setprio(2);
    const int row = blockIdx.x;
    const int n = row / C, c = row - n * C;
    const double* p = part + static_cast<long>(row) * nch * 3;
    double sd = 0.0, sdx = 0.0, sa = 0.0;
    // slots j, j + 64, ... in order, eight slots' loads in flight (issued
    // unconditionally from clamped indices)
    for (int j0 = threadIdx.x; j0 < nch; j0 += 8 * 64) {
        double a[8], b[8], c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = min(j0 + 64 * u, nch - 1);
            a[u] = p[j * 3];
            b[u] = p[j * 3 + 1];
            c[u] = p[j * 3 + 2];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (j0 + 64 * u < nch) {
                sd += a[u];
                sdx += b[u];
                sa += c[u];
            }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        sd += __shfl_xor(sd, o, 64);
        sdx += __shfl_xor(sdx, o, 64);
        sa += __shfl_xor(sa, o, 64);
    }
    if (threadIdx.x == 0) {
        if (dgamma) dgamma[n * dgb_bs + c] = static_cast<float>(sdx);
        if (dbeta) dbeta[n * dgb_bs + c] = static_cast<float>(sd);
        if (dalpha_part) dalpha_part[row] = static_cast<float>(sa);
        rowv[row] = make_float2(static_cast<float>(sd / L), static_cast<float>(sdx / L));
    }
}

}  // namespace

// The AdaIN backward after a GEMM epilogue produced ds = dY * act'(s) and the
// per-row partial sums (see store_tile_adain): dgamma / dbeta overwritten,
// dalpha accumulated (Snake, when non-null), and
//   dX = rstd (1 + gamma) (ds - mean(ds) - xh mean(ds xh)) + R.
// ds and dX may be the same buffer (each element is read before it is written).
int adain_bwd_finish(kdec_ctx* ctx, const float* X, long x_bs, const float* stats, const float* gamma, long gb_bs,
                     int act, const double* part, int nch, const float* ds, long ds_bs, const float* R, long r_bs,
                     float* dX, long dx_bs, float* dgamma, float* dbeta, long dgb_bs, float* dalpha, int N, int C,
                     int L) {
    const int rows = N * C;
    const bool want_alpha = dalpha && act == KDEC_ACT_SNAKE;
    Workspace rv(ctx, static_cast<size_t>(rows) * sizeof(float2));
    Workspace ap(ctx, want_alpha ? static_cast<size_t>(rows) * sizeof(float) : 0);
    if (!rv.p || (want_alpha && !ap.p)) return KDEC_ENOMEM;
    ProfScope ps(ctx, "adain_bwd", 0, 4.0 * static_cast<double>(rows) * L * (R ? 4 : 3));
    hipLaunchKernelGGL(adain_bwd_fin_wide_k, dim3(static_cast<unsigned>(rows)), dim3(64), 0, ctx->stream, part, nch,
                       C, L, dgamma, dbeta, dgb_bs, want_alpha ? ap.as<float>() : nullptr, rv.as<float2>());
    if (int rc = launch_check(ctx, "adain_bwd_fin")) return rc;
    // the apply with no activation: ds already carries act'
    const AdainArgs ga{X, x_bs, reinterpret_cast<const float2*>(stats), gamma, nullptr, gb_bs, KDEC_ACT_NONE, 0.0f,
                       nullptr, C, L};
    // (and dalpha += the per-row alpha shares, summed over utterances in order)
    const float* apf = want_alpha ? ap.as<float>() : nullptr;
    if (rows_v4({{X, x_bs}, {ds, ds_bs}, {R, r_bs}, {dX, dx_bs}}))
        hipLaunchKernelGGL(adain_bwd_apply_v4_k, dim3(v4_blocks_bwd(L), static_cast<unsigned>(rows)), dim3(RT), 0,
                           ctx->stream, ga, ds, ds_bs, R, r_bs, dX, dx_bs, rv.as<float2>(), apf, dalpha, N);
    else
        hipLaunchKernelGGL(adain_bwd_apply_k, dim3(static_cast<unsigned>(cdiv(L, CH)), static_cast<unsigned>(rows)),
                           dim3(RT), 0, ctx->stream, ga, ds, ds_bs, R, r_bs, dX, dx_bs, rv.as<float2>(), apf, dalpha,
                           N);
    return launch_check(ctx, "adain_bwd_apply");
}

}  // namespace kdec

using namespace kdec;

// Scratch of kdec_adain_act_bwd_noalloc: a file-scope device array, one copy
// per GPU (each at its own address), held until the process ends. Host code
// never uses its name as an address: at context creation, with the device
// current, hipGetSymbolAddress gives this GPU's copy, kept per device.
static __device__ __align__(256) unsigned char scratch[KDEC_NOALLOC_SCRATCH_BYTES];

namespace kdec {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int noalloc_scratch_setup(kdec_ctx* ctx) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return fail(ctx, KDEC_EINVAL, "no-allocation scratch: device index out of range");
    if (g_scratch_ptr[ctx->device]) return KDEC_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(ctx, KDEC_EHIP, "hipGetSymbolAddress(scratch) returned no address");
    g_scratch_ptr[ctx->device] = p;
    return KDEC_OK;
}

void* noalloc_scratch(kdec_ctx* ctx) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return ctx->device >= 0 && ctx->device < kMaxDevices ? g_scratch_ptr[ctx->device] : nullptr;
}

}  // namespace kdec

extern "C" {

int kdec_instnorm_stats(kdec_ctx* ctx, const float* X, long x_bs, int N,
                        int C, int L, float eps, float* stats) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && stats && N > 0 && C > 0 && L > 0 && x_bs >= static_cast<long>(C) * L,
               "kdec_instnorm_stats: bad arguments");
    const int rows = N * C;
    const int nch = static_cast<int>(cdiv(L, CH));
    Workspace part(ctx, static_cast<size_t>(rows) * nch * sizeof(double2));
    if (!part.p) return KDEC_ENOMEM;
    ProfScope ps(ctx, "adain_fwd", 0);
    hipLaunchKernelGGL(instnorm_part_k, dim3(nch, rows), dim3(RT), 0, ctx->stream, X, x_bs, C, L, nch,
                       part.as<double2>());
    if (int rc = launch_check(ctx, "instnorm_part")) return rc;
    hipLaunchKernelGGL(instnorm_fin_k, dim3(static_cast<unsigned>(cdiv(rows, 256))), dim3(256), 0, ctx->stream, X,
                       x_bs, C, L, rows, nch, part.as<double2>(), eps, reinterpret_cast<float2*>(stats));
    return launch_check(ctx, "instnorm_fin");
}

int kdec_adain_act_fwd(kdec_ctx* ctx, const float* X, long x_bs,
                       const float* stats, const float* gamma,
                       const float* beta, long gb_bs, int act,
                       float slope, const float* alpha, float* Y, long y_bs,
                       float* Ypre, long ypre_bs, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && stats && gamma && Y && N > 0 && C > 0 && L > 0,
               "kdec_adain_act_fwd: bad arguments");
    KDEC_CHECK(ctx, act >= KDEC_ACT_NONE && act <= KDEC_ACT_SNAKE && (act != KDEC_ACT_SNAKE || alpha),
               "kdec_adain_act_fwd: bad activation");
    AdainArgs g{X, x_bs, reinterpret_cast<const float2*>(stats), gamma, beta, gb_bs, act, slope, alpha, C, L};
    ProfScope ps(ctx, "adain_fwd", 0);
    if (rows_v4({{X, x_bs}, {Y, y_bs}, {Ypre, ypre_bs}}))
        hipLaunchKernelGGL(adain_act_fwd_v4_k, dim3(v4_blocks(L), N * C), dim3(RT), 0, ctx->stream, g, Y, y_bs, Ypre,
                           ypre_bs);
    else
        hipLaunchKernelGGL(adain_act_fwd_k, dim3(static_cast<unsigned>(cdiv(L, CH)), N * C), dim3(RT), 0,
                           ctx->stream, g, Y, y_bs, Ypre, ypre_bs);
    return launch_check(ctx, "adain_act_fwd");
}

int kdec_adain_act_fwd_stats(kdec_ctx* ctx, const float* X, long x_bs, float eps, float* stats,
                             const float* gamma, const float* beta, long gb_bs, int act, float slope,
                             const float* alpha, float* Y, long y_bs, float* Ypre, long ypre_bs, int N, int C,
                             int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && stats && gamma && Y && N > 0 && C > 0 && L > 0 && x_bs >= static_cast<long>(C) * L,
               "kdec_adain_act_fwd_stats: bad arguments");
    KDEC_CHECK(ctx, act >= KDEC_ACT_NONE && act <= KDEC_ACT_SNAKE && (act != KDEC_ACT_SNAKE || alpha),
               "kdec_adain_act_fwd_stats: bad activation");
    AdainArgs g{X, x_bs, reinterpret_cast<const float2*>(stats), gamma, beta, gb_bs, act, slope, alpha, C, L};
    const RowShape rsh = row_shape_fwd(g, Y, y_bs, Ypre, ypre_bs);
    if (!rsh.ntb) {  // rows the row kernels do not hold: statistics pass, then the affine pass
        if (int rc = kdec_instnorm_stats(ctx, X, x_bs, N, C, L, eps, stats)) return rc;
        return kdec_adain_act_fwd(ctx, X, x_bs, stats, gamma, beta, gb_bs, act, slope, alpha, Y, y_bs, Ypre, ypre_bs,
                                  N, C, L);
    }
    ProfScope ps(ctx, "adain_fwd", 0, 4.0 * static_cast<double>(N) * C * L * (Ypre ? 3 : 2));
    return launch_fwd_row(ctx, rsh, static_cast<unsigned>(N * C), g, eps, reinterpret_cast<float2*>(stats), Y, y_bs,
                          Ypre, ypre_bs);
}

int kdec_adain_act_bwd(kdec_ctx* ctx, const float* X, long x_bs,
                       const float* stats, const float* gamma,
                       const float* beta, long gb_bs, int act, float slope,
                       const float* alpha, const float* dY, long dy_bs,
                       const float* R, long r_bs, float* dX, long dx_bs,
                       float* dgamma, float* dbeta, long dgb_bs,
                       float* dalpha, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    AdainArgs g{X, x_bs, reinterpret_cast<const float2*>(stats), gamma, beta, gb_bs, act, slope, alpha, C, L};
    if (int rc = bwd_check(ctx, g, dY, dX, N, "kdec_adain_act_bwd")) return rc;
    const BwdScratchLayout lay = bwd_scratch_layout(N, C, L, dalpha && act == KDEC_ACT_SNAKE,
                                                    bwd_v4_long(g, dY, dy_bs, R, r_bs, dX, dx_bs));
    Workspace ws(ctx, lay.total);
    if (lay.total && !ws.p) return KDEC_ENOMEM;
    return bwd_run(ctx, g, dY, dy_bs, R, r_bs, dX, dx_bs, dgamma, dbeta, dgb_bs, dalpha, N,
                   bwd_scratch(ws.p, lay), true);
}

int kdec_adain_act_bwd_noalloc(kdec_ctx* ctx, const float* X, long x_bs,
                               const float* stats, const float* gamma,
                               const float* beta, long gb_bs, int act, float slope,
                               const float* alpha, const float* dY, long dy_bs,
                               const float* R, long r_bs, float* dX, long dx_bs,
                               float* dgamma, float* dbeta, long dgb_bs,
                               float* dalpha, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    AdainArgs g{X, x_bs, reinterpret_cast<const float2*>(stats), gamma, beta, gb_bs, act, slope, alpha, C, L};
    if (int rc = bwd_check(ctx, g, dY, dX, N, "kdec_adain_act_bwd_noalloc")) return rc;
    const BwdScratchLayout lay = bwd_scratch_layout(N, C, L, dalpha && act == KDEC_ACT_SNAKE,
                                                    bwd_v4_long(g, dY, dy_bs, R, r_bs, dX, dx_bs));
    if (lay.total > static_cast<size_t>(KDEC_NOALLOC_SCRATCH_BYTES))
        return fail(ctx, KDEC_EINVAL,
                    "kdec_adain_act_bwd_noalloc: N*C = " + std::to_string(static_cast<long>(N) * C) + ", L = " +
                        std::to_string(L) + " needs " + std::to_string(lay.total) +
                        " bytes of scratch; the limit is " + std::to_string(KDEC_NOALLOC_SCRATCH_BYTES));
    void* base = noalloc_scratch(ctx);
    if (!base) return fail(ctx, KDEC_EHIP,
                                "kdec_adain_act_bwd_noalloc: no scratch on this device: " + ctx->scratch_err);
    // the profiling bracket creates events, so it stays off here
    return bwd_run(ctx, g, dY, dy_bs, R, r_bs, dX, dx_bs, dgamma, dbeta, dgb_bs, dalpha, N, bwd_scratch(base, lay),
                   false);
}

int kdec_fill(kdec_ctx* ctx, float* Y, long n, float value) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, Y && n >= 0, "kdec_fill: bad arguments");
    if (n == 0) return KDEC_OK;
    hipLaunchKernelGGL(fill_k, dim3(chunks(n, 4096)), dim3(256), 0, ctx->stream, Y, n, value);
    return launch_check(ctx, "fill");
}

int kdec_leaky_fwd(kdec_ctx* ctx, const float* X, long x_bs, float* Y,
                   long y_bs, int N, long len, float slope) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && Y && N > 0 && len > 0, "kdec_leaky_fwd: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    if (ew_v4(len, {{X, x_bs}, {Y, y_bs}}))
        hipLaunchKernelGGL(leaky_fwd_k<4>, dim3(chunks(len / 4), N), dim3(256), 0, ctx->stream, X, x_bs, Y, y_bs, len,
                           slope);
    else
        hipLaunchKernelGGL(leaky_fwd_k<1>, dim3(chunks(len), N), dim3(256), 0, ctx->stream, X, x_bs, Y, y_bs, len,
                           slope);
    return launch_check(ctx, "leaky_fwd");
}

int kdec_leaky_bwd(kdec_ctx* ctx, const float* X, long x_bs, const float* dY,
                   long dy_bs, float* dX, long dx_bs, int N, long len,
                   float slope) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && dY && dX && N > 0 && len > 0, "kdec_leaky_bwd: bad arguments");
    return kdec_leaky_bwd_scaled(ctx, X, x_bs, dY, dy_bs, dX, dx_bs, N, len, slope, 1.0f);
}

int kdec_leaky_bwd_scaled(kdec_ctx* ctx, const float* X, long x_bs, const float* dY, long dy_bs, float* dX,
                          long dx_bs, int N, long len, float slope, float scale) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && dY && dX && N > 0 && len > 0, "kdec_leaky_bwd_scaled: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    if (ew_v4(len, {{X, x_bs}, {dY, dy_bs}, {dX, dx_bs}}))
        hipLaunchKernelGGL(leaky_bwd_k<4>, dim3(chunks(len / 4), N), dim3(256), 0, ctx->stream, X, x_bs, dY, dy_bs,
                           dX, dx_bs, len, slope, scale);
    else
        hipLaunchKernelGGL(leaky_bwd_k<1>, dim3(chunks(len), N), dim3(256), 0, ctx->stream, X, x_bs, dY, dy_bs,
                           dX, dx_bs, len, slope, scale);
    return launch_check(ctx, "leaky_bwd");
}

int kdec_axpby(kdec_ctx* ctx, float a, const float* A, long a_bs, float b,
               const float* B, long b_bs, float* Y, long y_bs, int N,
               long len) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, A && Y && N > 0 && len > 0, "kdec_axpby: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    if (ew_v4(len, {{A, a_bs}, {B, b_bs}, {Y, y_bs}}))
        hipLaunchKernelGGL(axpby_k<4>, dim3(chunks(len / 4), N), dim3(256), 0, ctx->stream, a, A, a_bs, b, B, b_bs,
                           Y, y_bs, len);
    else
        hipLaunchKernelGGL(axpby_k<1>, dim3(chunks(len), N), dim3(256), 0, ctx->stream, a, A, a_bs, b, B, b_bs, Y,
                           y_bs, len);
    return launch_check(ctx, "axpby");
}

int kdec_add3(kdec_ctx* ctx, const float* A, long a_bs, const float* B, long b_bs, const float* C, long c_bs,
              float* Y, long y_bs, int N, long len) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, A && B && C && Y && N > 0 && len > 0, "kdec_add3: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    auto al = [](const float* p, long bs) { return (reinterpret_cast<unsigned long long>(p) & 15) == 0 && bs % 4 == 0; };
    if (len % 4 == 0 && al(A, a_bs) && al(B, b_bs) && al(C, c_bs) && al(Y, y_bs))
        hipLaunchKernelGGL(add3_k<4>, dim3(chunks(len / 4), N), dim3(256), 0, ctx->stream, A, a_bs, B, b_bs, C, c_bs,
                           Y, y_bs, len);
    else
        hipLaunchKernelGGL(add3_k<1>, dim3(chunks(len), N), dim3(256), 0, ctx->stream, A, a_bs, B, b_bs, C, c_bs, Y,
                           y_bs, len);
    return launch_check(ctx, "add3");
}

int kdec_add3_leaky(kdec_ctx* ctx, const float* A, long a_bs, const float* B, long b_bs, const float* C, long c_bs,
                    float* Y, long y_bs, float* Z, long z_bs, int N, long len, float slope) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, A && B && C && Y && Z && N > 0 && len > 0, "kdec_add3_leaky: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    auto al = [](const float* p, long bs) { return (reinterpret_cast<unsigned long long>(p) & 15) == 0 && bs % 4 == 0; };
    if (len % 4 == 0 && al(A, a_bs) && al(B, b_bs) && al(C, c_bs) && al(Y, y_bs) && al(Z, z_bs))
        hipLaunchKernelGGL(add3_leaky_k<4>, dim3(chunks(len / 4), N), dim3(256), 0, ctx->stream, A, a_bs, B, b_bs, C,
                           c_bs, Y, y_bs, Z, z_bs, len, slope);
    else
        hipLaunchKernelGGL(add3_leaky_k<1>, dim3(chunks(len), N), dim3(256), 0, ctx->stream, A, a_bs, B, b_bs, C,
                           c_bs, Y, y_bs, Z, z_bs, len, slope);
    return launch_check(ctx, "add3_leaky");
}

int kdec_add3_unpad_left1(kdec_ctx* ctx, const float* A, long a_bs, const float* B, long b_bs, const float* C,
                          long c_bs, float* Y, long y_bs, float* Z, long z_bs, int N, int Cn, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, A && B && C && Y && Z && N > 0 && Cn > 0 && L > 1, "kdec_add3_unpad_left1: bad arguments");
    KDEC_CHECK(ctx, y_bs >= static_cast<long>(Cn) * (L + 1) && z_bs >= static_cast<long>(Cn) * L &&
                        a_bs >= static_cast<long>(Cn) * (L + 1) && b_bs >= static_cast<long>(Cn) * (L + 1) &&
                        c_bs >= static_cast<long>(Cn) * (L + 1),
               "kdec_add3_unpad_left1: batch stride too small");
    KDEC_CHECK(ctx, static_cast<long>(N) * Cn < (1L << 31) && cdiv(L + 1, 1024) <= 65535,
               "kdec_add3_unpad_left1: too many rows or too long a row");
    ProfScope ps(ctx, "elementwise", 0, 4.0 * static_cast<double>(N) * Cn * (4.0 * (L + 1) + L));
    hipLaunchKernelGGL(add3_unpad_k, dim3(static_cast<unsigned>(N * Cn), static_cast<unsigned>(cdiv(L + 1, 1024))),
                       dim3(256), 0, ctx->stream, A, a_bs, B, b_bs, C, c_bs, Y, y_bs, Z, z_bs, Cn, L);
    return launch_check(ctx, "add3_unpad");
}

int kdec_pad_reflect_left1_fwd(kdec_ctx* ctx, const float* X, long x_bs,
                               float* Y, long y_bs, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && Y && N > 0 && C > 0 && L > 1, "kdec_pad_reflect_left1_fwd: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    hipLaunchKernelGGL(pad_fwd_k, dim3(chunks(static_cast<long>(C) * (L + 1)), N), dim3(256), 0, ctx->stream,
                       X, x_bs, Y, y_bs, C, L);
    return launch_check(ctx, "pad_fwd");
}

int kdec_pad_reflect_left1_bwd(kdec_ctx* ctx, const float* dY, long dy_bs,
                               float* dX, long dx_bs, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, dY && dX && N > 0 && C > 0 && L > 1, "kdec_pad_reflect_left1_bwd: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    hipLaunchKernelGGL(pad_bwd_k, dim3(chunks(static_cast<long>(C) * L), N), dim3(256), 0, ctx->stream, dY,
                       dy_bs, dX, dx_bs, C, L);
    return launch_check(ctx, "pad_bwd");
}

int kdec_nearest2x_fwd(kdec_ctx* ctx, const float* X, long x_bs, float* Y,
                       long y_bs, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && Y && N > 0 && C > 0 && L > 0, "kdec_nearest2x_fwd: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    hipLaunchKernelGGL(near2_fwd_k, dim3(chunks(static_cast<long>(C) * 2 * L), N), dim3(256), 0, ctx->stream,
                       X, x_bs, Y, y_bs, C, L);
    return launch_check(ctx, "nearest2x_fwd");
}

int kdec_nearest2x_bwd(kdec_ctx* ctx, const float* dY, long dy_bs, float* dX,
                       long dx_bs, int N, int C, int L, float scale,
                       float beta) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, dY && dX && N > 0 && C > 0 && L > 0, "kdec_nearest2x_bwd: bad arguments");
    ProfScope ps(ctx, "elementwise", 0);
    hipLaunchKernelGGL(near2_bwd_k, dim3(chunks(static_cast<long>(C) * L), N), dim3(256), 0, ctx->stream, dY,
                       dy_bs, dX, dx_bs, C, L, scale, beta);
    return launch_check(ctx, "nearest2x_bwd");
}

}  // extern "C"

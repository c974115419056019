// Conv1d / ConvTranspose1d forward, input-grad and weight-grad on gfx950 as
// implicit GEMMs on FP32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Forward family (one kernel, `conv_gemm`):
//   Y[n, m, q] = sum_{c, t} A[(c, t), m] * X[n, c, q*s + t*d - p]
// with A the weights packed K-major ([C_in_pad * k][M_pad], zero padded so
// tiles never test bounds on the A side). It serves
//   - conv1d forward (A = W^T),
//   - conv1d input-grad at stride 1 (A = the flipped transpose of W,
//     p' = d(k-1) - p: the adjoint of a correlation is a correlation),
//   - conv-transpose input-grad (a strided correlation of dY with W viewed as
//     (C_in, C_out*k)),
//   - conv-transpose forward, polyphase: output phase r = (j + p) mod s sees
//     only taps t = r + m*s, so each phase is a stride-1 correlation with
//     ceil(k/s) taps whose outputs land at j = Q*s + r - p.
// A 256-thread block owns a 128 (m) x 128 (q) output tile as 2x2 waves of
// 64x64 (2x2 MFMA tiles each). Per K chunk the block stages CK input rows of
// the haloed window [q0*s - p, (q0+127)*s + (k-1)d - p] and the matching
// CK*k weight rows in LDS; every tap then reads a shifted window of the same
// staged rows, so X is fetched once per chunk instead of k times. Staging is
// direct global->LDS (global_load_lds_dwordx4 for the weight panel,
// buffer_load_dword ... lds for the input rows, whose buffer range turns
// out-of-row positions into zeros), double-buffered so the next chunk's loads
// fly during the current chunk's MFMAs; no VGPRs hold staged data, which keeps
// the kernel at ~80 VGPRs and 4-6 waves per SIMD.
//
// Weight-grad (`wgrad_gemm`): dW[m, (c, t)] = sum_{n, l} dY[n, m, l] *
// X[n, c, l*s + t*d - p], a GEMM with the huge position axis as K. It is
// split over K into deterministic partial tiles that a second kernel sums in
// a fixed order; the bias grad (row sums of dY) rides along in the same pass.
#include "kdec_buffer.hpp"
#include "kdec_internal.hpp"
#include "kdec_snake_math.hpp"

#include <algorithm>
#include <cmath>
#include <map>
#include <type_traits>
#include <mutex>
#include <string>
#include <utility>

namespace kdec {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;   // output-channel tile
constexpr int BN = 128;   // output-position tile
constexpr int NT = 256;   // threads per block (4 waves)
__device__ inline int floordiv_i(int a, int b) {
    int q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
    return q;
}

struct GemmArgs {
    const float* X;
    long x_bs;
    const float* A;          // packed weights [cin_pad*k][m_pad] per phase
    long a_phase_stride;     // elements between phases
    const float* bias;       // [C_out] or null
    float* Y;
    long y_bs;
    const float* R;          // residual [n][m][j] or null
    long r_bs;
    int C_in, L_in, C_out, L_y;   // L_y: length of a Y row
    int cin_pad, m_pad;
    int k, s, d, p;          // correlation geometry (plain mode)
    int n_q;                 // output columns (plain mode)
    int CK;                  // input channels per K chunk (even)
    float scale, beta;
    // polyphase transposed-conv mode when n_phase > 1
    int n_phase, ph_s, ph_p, ph_kt;
    int m_tiles, q_tiles;
    int nz;                  // N * n_phase
    // Tiles in logical order: the first `full_tiles` run over all channel
    // chunks; the remaining `split_tiles` run as `fsplit` chunk ranges each,
    // whose raw sums go to P[(tile - full_tiles) * fsplit + part][BM * BN]
    // and are summed, in part order, by tile_reduce.
    int full_tiles, split_tiles, fsplit;
    int full_per_xcd, parts_per_xcd;  // block slots per XCD for each kind
    float* P;
    int ybuf;                // (C_out + BM) * L_y * 4 < 2^31: the epilogue addresses Y through a descriptor
    // octet mode (corr_gemm): K chunk = one input-channel octet x up to G taps
    int G, n_tg, n_oct, span8;  // taps per chunk, tap groups, octets, staged positions
    int quad;                // conv_gemm_q: weights packed in quads of k-steps (stride 1, k = KT)
    // Output placement (polyphase transposed convs): every column lands y_off
    // positions on (a left pad of the output rows, whose length L_y counts
    // it), and with refl the column of unpadded index 1 is also stored, with
    // the residual of column 0, at column 0 (a one-sample left reflect pad).
    int y_off, refl;
    int single;              // conv_gemm: one LDS stage (where two would leave at most two blocks per CU)
    // AdaIN backward epilogue (conv input grads that feed an AdaIN +
    // activation backward; off when part is null): Y receives
    // ds = dY * act'(s) of the AdaIN whose input rows x have Y's layout, and
    // part[((n*C_out + m)*nch + 2*q_tile + half)*3 + j] the tile half's sums
    // of ds, ds * xh and (Snake) dY (th sin 2th - sin^2 th) / a^2.
    struct {
        const float* x;
        long x_bs;
        const float2* st;    // (mean, rstd) per n*C_out + m
        const float* gam;    // gamma / beta at n*gb_bs + m; beta may be null
        const float* bet;
        long gb_bs;
        const float* alpha;  // per m (Snake)
        int act;
        float slope;
        double* part;
        int nch;             // partial slots per row: 2 per q-tile
    } ad;
    // Instance-norm statistics epilogue (forward convs whose output feeds an
    // AdaIN; off when part is null, needs beta = 0): beside Y, per row and
    // tile half part[((n*C_out + m)*nch + 2*q_tile + half)*3 + {0, 1, 2}] =
    // (count, mean, sum of squared deviations from that mean) of the stored
    // values.
    struct {
        double* part;
        int nch;
    } fs;
};

// Logical block order with consecutive ids on one XCD: the dispatcher deals
// workgroups to the 8 XCDs round-robin, so without this remap the blocks that
// share an operand tile (one X tile across output-channel tiles, one dY tile
// across weight-grad column tiles) would each miss in a different L2.
__device__ inline int xcd_remap(int pid, int total) {
    constexpr int X = 8;
    const int per = (total + X - 1) / X;
    int tall = total % X;
    if (tall == 0) tall = X;
    const int xcd = pid % X, local = pid / X;
    if (xcd < tall) return xcd * per + local;
    return tall * per + (xcd - tall) * (per - 1) + local;
}

// Geometry of one output tile (wave-uniform).
struct TileGeo {
    int b, m0, q0, n_q, os, oo, k, s, d, p;
    const float* A;
};

// Logical tile order: m-tile fastest, then q-tile, then (utterance, phase),
// with every last q-tile (usually partly empty: its idle waves skip their
// MFMAs) moved to the end so that the short tiles come last. Polyphase
// transposed convs take the phase right after the m-tile: the s phase tiles
// of one q range store interleaved columns of the same output rows, and
// consecutive tiles run side by side on one XCD (block_work), so their
// partial cache lines meet in that XCD's L2 instead of each going to HBM.
__device__ inline void decode_tile(const GemmArgs& g, int tile, TileGeo& T) {
    const int full = (g.q_tiles - 1) * g.m_tiles * g.nz;
    int mt, qt, zz, lid = tile;
    if (g.n_phase > 1) {
        const bool last = lid >= full;
        if (last) lid -= full;
        mt = lid % g.m_tiles;
        lid /= g.m_tiles;
        const int r = lid % g.n_phase;
        lid /= g.n_phase;
        int b;
        if (last) {
            b = lid;
            qt = g.q_tiles - 1;
        } else {
            qt = lid % (g.q_tiles - 1);
            b = lid / (g.q_tiles - 1);
        }
        zz = b * g.n_phase + r;
    } else if (lid < full) {
        mt = lid % g.m_tiles;
        lid /= g.m_tiles;
        qt = lid % (g.q_tiles - 1);
        zz = lid / (g.q_tiles - 1);
    } else {
        lid -= full;
        mt = lid % g.m_tiles;
        zz = lid / g.m_tiles;
        qt = g.q_tiles - 1;
    }
    T.b = zz; T.k = g.k; T.s = g.s; T.d = g.d; T.p = g.p; T.n_q = g.n_q;
    T.os = 1; T.oo = 0;
    T.A = g.A;
    if (g.n_phase > 1) {
        const int r = zz % g.n_phase;
        T.b = zz / g.n_phase;
        const int qmin = -floordiv_i(r - g.ph_p, g.ph_s);          // ceil((p - r)/s)
        const int qmax = floordiv_i(g.L_y - g.y_off - 1 + g.ph_p - r, g.ph_s);
        T.n_q = qmax - qmin + 1;
        T.k = g.ph_kt;
        T.s = 1;
        T.d = 1;
        T.p = g.ph_kt - 1 - qmin;
        T.os = g.ph_s;
        T.oo = qmin * g.ph_s + r - g.ph_p + g.y_off;
        T.A += static_cast<long>(r) * g.a_phase_stride;
    }
    T.m0 = mt * BM;
    T.q0 = qt * BN;
}

// Block -> work: the dispatcher deals workgroups to the 8 XCDs round-robin,
// so block i runs on XCD i % 8. Each XCD gets full_per_xcd slots for a
// contiguous range of whole tiles (neighbouring tiles share operand tiles in
// its L2) and then parts_per_xcd slots for split-tile parts; the whole-tile
// rounds and the short split-part round are thus the same on every XCD.
// Returns false for a padding slot.
__device__ inline bool block_work(const GemmArgs& g, int& tile, int& part) {
    const int x = blockIdx.x & 7, local = blockIdx.x >> 3;
    if (local < g.full_per_xcd) {
        tile = x * g.full_per_xcd + local;
        part = -1;
        return tile < g.full_tiles;
    }
    const int j = x * g.parts_per_xcd + (local - g.full_per_xcd);
    if (j >= g.split_tiles * g.fsplit) return false;
    tile = g.full_tiles + j % g.split_tiles;
    part = j / g.split_tiles;
    return true;
}

// Tile epilogue shared by the GEMM kernels: lane owns column l32 and rows
// 8*(e/4) + 4*hi + e%4 of each 32x32 MFMA tile. A split part writes its raw
// sums to its compact partial tile; a whole tile applies bias, residual,
// scale and beta and stores Y.
__device__ inline void store_tile(const GemmArgs& g, const TileGeo& T, int tile, int part, const f32x16 (&acc)[2][2],
                                  int wm, int wn, int hi, int l32) {
    const int b = T.b, n_q = T.n_q, os = T.os, oo = T.oo, m0 = T.m0, q0 = T.q0;
    if (part >= 0) {  // raw sums of this chunk range, tile-local [m][q]
        float* Pt = g.P + (static_cast<long>(tile - g.full_tiles) * g.fsplit + part) * (BM * BN);
#pragma unroll
        for (int tn = 0; tn < 2; ++tn)
#pragma unroll
            for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int ml = wm * 64 + tm * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
                    Pt[ml * BN + wn * 64 + tn * 32 + l32] = acc[tm][tn][e];
                }
        return;
    }
    float* Yb = g.Y + static_cast<long>(b) * g.y_bs;
    const float* Rb = g.R ? g.R + static_cast<long>(b) * g.r_bs : nullptr;
    if (g.ybuf) {
        // Y, R and the bias through descriptors over exactly their rows: rows
        // at or past C_out fall outside and their stores drop, their loads
        // read 0. The whole byte offset goes in the VGPR offset, since the
        // scalar offset of a buffer access is not range checked; ybuf keeps
        // it below 2^31 for every row of the tile.
        // L_y through an empty asm: the row offsets below are then formed
        // here, not hoisted to the kernel's start and held through the k-loop
        int Ly = g.L_y;
        asm volatile("" : "+s"(Ly));
        const int rowb = g.C_out * Ly * 4;
        const __amdgpu_buffer_rsrc_t yr = uniform_rsrc(Yb, rowb);
        const __amdgpu_buffer_rsrc_t rr = uniform_rsrc(Rb ? Rb : Yb, Rb ? rowb : 0);
        const __amdgpu_buffer_rsrc_t br = uniform_rsrc(g.bias ? g.bias : Yb, g.bias ? g.C_out * 4 : 0);
        const int mrow = m0 + wm * 64 + 4 * hi;  // the lane's first row
        // Operand loads go in runs of eight elements under one uniform branch
        // each (bias, residual, old Y), so a run costs one memory round trip:
        // a load under a branch of its own is waited for at the branch's
        // join. Eight, not all 32 of a tile's rows at once, so that the runs'
        // registers and the accumulators fit without spilling.
        const bool hb = g.bias != nullptr, hr = Rb != nullptr, hy = g.beta != 0.0f;
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int q = q0 + wn * 64 + tn * 32 + l32;
            if (q >= n_q) continue;
            const int vo = (mrow * Ly + q * os + oo) * 4;
#pragma unroll
            for (int tm = 0; tm < 2; ++tm) {
#pragma unroll
                for (int e0 = 0; e0 < 16; e0 += 8) {
                    float bv[8], rv[8], yv[8];
                    if (hb) {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            bv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                br, (mrow + tm * 32 + 8 * ((e0 + e) >> 2) + (e & 3)) * 4, 0, 0));
                    }
                    if (hr) {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            rv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                rr, vo + (tm * 32 + 8 * ((e0 + e) >> 2) + (e & 3)) * Ly * 4, 0, 0));
                    }
                    if (hy) {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            yv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                yr, vo + (tm * 32 + 8 * ((e0 + e) >> 2) + (e & 3)) * Ly * 4, 0, 0));
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int dm = tm * 32 + 8 * ((e0 + e) >> 2) + (e & 3);  // uniform row step
                        const int o = vo + dm * Ly * 4;
                        float v = acc[tm][tn][e0 + e];
                        if (hb) v += bv[e];
                        if (hr) v += rv[e];
                        v *= g.scale;
                        if (hy) v += g.beta * yv[e];
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), yr, o, 0, 0);
                    }
                }
            }
            if (g.refl && q * os + oo == 1 + g.y_off) {  // the reflected column 0 (beta = 0)
#pragma unroll
                for (int tm = 0; tm < 2; ++tm) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int dm = tm * 32 + 8 * (e >> 2) + (e & 3);
                        const int o0 = (mrow + dm) * Ly * 4;
                        float v = acc[tm][tn][e];
                        if (g.bias)
                            v += __builtin_bit_cast(float,
                                                    __builtin_amdgcn_raw_buffer_load_b32(br, (mrow + dm) * 4, 0, 0));
                        if (Rb) v += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, o0, 0, 0));
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v * g.scale), yr, o0, 0, 0);
                    }
                }
            }
        }
        return;
    }
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
        const int q = q0 + wn * 64 + tn * 32 + l32;
        if (q >= n_q) continue;
        const long j = static_cast<long>(q) * os + oo;
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * 64 + tm * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
                if (m >= g.C_out) continue;
                float v = acc[tm][tn][e];
                if (g.bias) v += g.bias[m];
                const long yi = static_cast<long>(m) * g.L_y + j;
                if (Rb) v += Rb[yi];
                v *= g.scale;
                if (g.beta != 0.0f) v += g.beta * Yb[yi];
                Yb[yi] = v;
                if (g.refl && j == 1 + g.y_off) {  // the reflected column 0 (beta = 0)
                    const long y0 = static_cast<long>(m) * g.L_y;
                    Yb[y0] = (acc[tm][tn][e] + (g.bias ? g.bias[m] : 0.0f) + (Rb ? Rb[y0] : 0.0f)) * g.scale;
                }
            }
        }
    }
}

// The activation derivative of the AdaIN backward: ds = dy * act'(s) with
// s the affine output; for Snake, sa takes dy (th sin 2th - sin^2 th), the
// alpha-grad integrand before its 1/a^2 (the same arithmetic as the AdaIN
// backward kernels).
__device__ inline float epi_act_bwd(int act, float dy, float s, float slope, float a, float& sa) {
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

// Lane l's value from lane l ^ K within its 32-lane half (ds_swizzle, bit mode).
template <int K>
__device__ inline float xor_lane(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (K << 10)));
}

// One halving step of a transpose-reduce over the 32 lanes of a half: each
// lane keeps the upper or lower half of its N values (by lane bit K) and adds
// the partner's copy of that half.
template <int K, int N, int S>
__device__ inline void halve(float (&v)[S], int l32) {
    const bool up = (l32 & K) != 0;
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const float send = up ? v[j] : v[j + N / 2];
        const float keep = up ? v[j + N / 2] : v[j];
        v[j] = keep + xor_lane<K>(send);
    }
}

// Sums of 16 values per lane over the 32 lanes of a half: afterwards lanes
// l and l ^ 1 both hold the total of value l >> 1 in v[0].
__device__ inline void reduce16(float (&v)[16], int l32) {
    halve<16, 16>(v, l32);
    halve<8, 8>(v, l32);
    halve<4, 4>(v, l32);
    halve<2, 2>(v, l32);
    v[0] += xor_lane<1>(v[0]);
}

// Sums of 8 values per lane over the 32 lanes of a half: afterwards lanes
// 4 i .. 4 i + 3 hold the total of value i in v[0].
__device__ inline void reduce8(float (&v)[8], int l32) {
    halve<16, 8>(v, l32);
    halve<8, 4>(v, l32);
    halve<4, 2>(v, l32);
    v[0] += xor_lane<2>(v[0]);
    v[0] += xor_lane<1>(v[0]);
}

// Whole-tile epilogue of an input-grad GEMM feeding an AdaIN backward (the
// g.ad fields): the rows' (mean, rstd, 1 + gamma, beta, alpha) pass through
// LDS, each output dY = scale * acc becomes ds = dY * act'(s) (stored in Y)
// with s = (1 + gamma) xh + beta, xh = (x - mean) rstd, and the sums of ds,
// ds * xh and the alpha-grad integrand over the wave's 64 columns go to the
// row's partial slot 2 * q_tile + wn. Every lane takes part in the
// cross-lane reduction; positions past n_q add nothing.
__device__ inline void store_tile_adain(const GemmArgs& g, const TileGeo& T, const f32x16 (&acc)[2][2], int wm,
                                        int wn, int hi, int l32, float* smem) {
    const int b = T.b, n_q = T.n_q, m0 = T.m0, q0 = T.q0;
    const int tid = threadIdx.x;
    float4* prm = reinterpret_cast<float4*>(smem);
    float* pal = smem + 4 * BM;
    __syncthreads();  // every wave is past its last read of the staged operands
    if (tid < BM) {
        const int m = m0 + tid;
        float4 v = make_float4(0.0f, 0.0f, 1.0f, 0.0f);
        float a = 1.0f;
        if (m < g.C_out) {
            const float2 st = g.ad.st[b * g.C_out + m];
            v.x = st.x;
            v.y = st.y;
            v.z = 1.0f + g.ad.gam[b * g.ad.gb_bs + m];
            v.w = g.ad.bet ? g.ad.bet[b * g.ad.gb_bs + m] : 0.0f;
            if (g.ad.act == KDEC_ACT_SNAKE) a = g.ad.alpha[m];
        }
        prm[tid] = v;
        pal[tid] = a;
    }
    __syncthreads();
    int Ly = g.L_y;  // through an empty asm, as in store_tile
    asm volatile("" : "+s"(Ly));
    const int rowb = g.C_out * Ly * 4;
    const __amdgpu_buffer_rsrc_t yr = uniform_rsrc(g.Y + static_cast<long>(b) * g.y_bs, rowb);
    const __amdgpu_buffer_rsrc_t xr = uniform_rsrc(g.ad.x + static_cast<long>(b) * g.ad.x_bs, rowb);
    const int mrow = m0 + wm * 64 + 4 * hi;
    const int slot = (q0 / BN) * 2 + wn;
    // Rows in halves of 8 values per lane (e = 8 h .. 8 h + 7): the sums of
    // one half and its x run stay within the register budget of the GEMM.
#pragma unroll
    for (int tm = 0; tm < 2; ++tm) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float sd[8], sdx[8], sa[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) sd[j] = sdx[j] = sa[j] = 0.0f;
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const int q = q0 + wn * 64 + tn * 32 + l32;
                if (q >= n_q) continue;
                const int vo = (mrow * Ly + q) * 4;
                // x ahead of the stores: a load placed after a store to a
                // buffer that may alias waits for that store too.
                float xv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int e = 8 * h + j;
                    const int o = vo + (tm * 32 + 8 * (e >> 2) + (e & 3)) * Ly * 4;
                    xv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, o, 0, 0));
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int e = 8 * h + j;
                    const int dm = tm * 32 + 8 * (e >> 2) + (e & 3);
                    const int o = vo + dm * Ly * 4;
                    const int rl = wm * 64 + 4 * hi + dm;
                    const float4 pr = prm[rl];
                    const float dy = acc[tm][tn][e] * g.scale;
                    const float xh = (xv[j] - pr.x) * pr.y;
                    const float ds = epi_act_bwd(g.ad.act, dy, pr.z * xh + pr.w, g.ad.slope, pal[rl], sa[j]);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, ds), yr, o, 0, 0);
                    sd[j] += ds;
                    sdx[j] += ds * xh;
                }
            }
            reduce8(sd, l32);
            reduce8(sdx, l32);
            if (g.ad.act == KDEC_ACT_SNAKE) reduce8(sa, l32);  // uniform
            if ((l32 & 3) == 0) {
                const int e = 8 * h + (l32 >> 2);
                const int rl = wm * 64 + tm * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
                const int m = m0 + rl;
                if (m < g.C_out) {
                    double* pp = g.ad.part + ((static_cast<long>(b) * g.C_out + m) * g.ad.nch + slot) * 3;
                    const double a = pal[rl];
                    pp[0] = sd[0];
                    pp[1] = sdx[0];
                    pp[2] = g.ad.act == KDEC_ACT_SNAKE ? static_cast<double>(sa[0]) / (a * a) : 0.0;
                }
            }
        }
    }
}

// Lane `src`'s float, read by every lane.
__device__ inline float lane_value(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// Whole-tile epilogue of a forward conv whose output rows feed an instance
// norm (g.fs): Y stored as store_tile stores it (bias, residual, scale;
// beta = 0), and per row and wave (64 columns) the count, mean and sum of
// squared deviations of the stored values go to slot 2 * q_tile + wn: the
// row sums by a transpose-reduce, the means read back from the two lanes
// that hold them, then the squared deviations likewise. Every lane takes part
// in the cross-lane steps; positions past n_q add nothing.
__device__ inline void store_tile_stats(const GemmArgs& g, const TileGeo& T, f32x16 (&acc)[2][2], int wm, int wn,
                                        int hi, int l32) {
    const int b = T.b, n_q = T.n_q, m0 = T.m0, q0 = T.q0;
    int Ly = g.L_y;  // through an empty asm, as in store_tile
    asm volatile("" : "+s"(Ly));
    const int rowb = g.C_out * Ly * 4;
    const float* Rb = g.R ? g.R + static_cast<long>(b) * g.r_bs : nullptr;
    const __amdgpu_buffer_rsrc_t yr = uniform_rsrc(g.Y + static_cast<long>(b) * g.y_bs, rowb);
    const __amdgpu_buffer_rsrc_t rr = uniform_rsrc(Rb ? Rb : g.Y, Rb ? rowb : 0);
    const __amdgpu_buffer_rsrc_t br = uniform_rsrc(g.bias ? g.bias : g.Y, g.bias ? g.C_out * 4 : 0);
    const int mrow = m0 + wm * 64 + 4 * hi;
    const int cnt = min(max(n_q - (q0 + wn * 64), 0), 64);  // wave-uniform
    const float inv = cnt > 0 ? 1.0f / static_cast<float>(cnt) : 0.0f;
    const int slot = (q0 / BN) * 2 + wn;
    // operand loads in runs under one uniform branch each, as in store_tile
    // (the residual of a column past n_q reads whatever lies there and is
    // not used)
    const bool hb = g.bias != nullptr, hr = Rb != nullptr;
#pragma unroll
    for (int tm = 0; tm < 2; ++tm) {
        float sx[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) sx[e] = 0.0f;
        float bv[16];
        if (hb) {
#pragma unroll
            for (int e = 0; e < 16; ++e)
                bv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                      br, (mrow + tm * 32 + 8 * (e >> 2) + (e & 3)) * 4, 0, 0));
        }
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int q = q0 + wn * 64 + tn * 32 + l32;
            const bool qin = q < n_q;
            const int vo = (mrow * Ly + q) * 4;
            float rv[16];
            if (hr) {
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    rv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                          rr, vo + (tm * 32 + 8 * (e >> 2) + (e & 3)) * Ly * 4, 0, 0));
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int dm = tm * 32 + 8 * (e >> 2) + (e & 3);
                const int o = vo + dm * Ly * 4;
                float v = acc[tm][tn][e];
                if (hb) v += bv[e];
                if (hr && qin) v += rv[e];
                v *= g.scale;
                if (qin) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), yr, o, 0, 0);
                v = qin ? v : 0.0f;
                acc[tm][tn][e] = v;
                sx[e] += v;
            }
        }
        reduce16(sx, l32);  // lanes 2e, 2e + 1 of each half: the sum of row e
        const float my_mean = sx[0] * inv;
        float mean[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float lo = lane_value(sx[0], 2 * e), up = lane_value(sx[0], 32 + 2 * e);
            mean[e] = (hi ? up : lo) * inv;
        }
        float sq[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) sq[e] = 0.0f;
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const bool qin = q0 + wn * 64 + tn * 32 + l32 < n_q;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float dv = acc[tm][tn][e] - mean[e];
                sq[e] += qin ? dv * dv : 0.0f;
            }
        }
        reduce16(sq, l32);
        if ((l32 & 1) == 0) {
            const int e = l32 >> 1;
            const int m = m0 + wm * 64 + tm * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
            if (m < g.C_out) {
                double* pp = g.fs.part + ((static_cast<long>(b) * g.C_out + m) * g.fs.nch + slot) * 3;
                pp[0] = cnt;
                pp[1] = my_mean;
                pp[2] = sq[0];
            }
        }
    }
}

// Grid of 8 * (full_per_xcd + parts_per_xcd) blocks. Two LDS stages;
// weights arrive packed chunk-major (row ((chunk*k + t)*CK + c_local)), so a
// chunk's KR = CK*k rows are one contiguous slab of the panel.
//
// Inner loop: the chunk's KR/2 k-steps (2 packed rows each) run as a
// ping-pong over two register sets, each step's LDS reads issued between the
// MFMAs of the step before, so the read latency hides behind matrix work.
#ifndef CG_WPE
#define CG_WPE 4  // 128 VGPRs: no spills (at five waves the tile spilled 8-11 registers, for no speed)
#endif
template <int CK>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(CG_WPE)))
void conv_gemm(GemmArgs g) {
    extern __shared__ float smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, hi = lane >> 5;

    int tile, part;
    if (!block_work(g, tile, part)) return;  // uniform per block
    TileGeo T;
    decode_tile(g, tile, T);
    const int b = T.b, k = T.k, s = T.s, d = T.d, p = T.p, n_q = T.n_q, os = T.os, oo = T.oo;
    const float* A = T.A;
    const int m0 = T.m0;
    const int q0 = T.q0;
    if (q0 >= n_q) return;  // uniform per block

    const int KR = CK * k;                            // weight rows per chunk
    const int span = (BN - 1) * s + (k - 1) * d + 1;  // staged input window
    // Input rows are staged 16 B per lane (256 positions per instruction) at
    // a row stride that is a multiple of 256.
    const int span_p = (span + 3 + 255) & ~255;  // LDS row stride
    const int segs = span_p >> 6;
    const int stage = KR * BM + CK * span_p;
    const float* Xb = g.X + static_cast<long>(b) * g.x_bs;
    const int x0 = q0 * s - p;
    const int a_lane = (lane >> 5) * g.m_pad + (lane & 31) * 4;
    const int nitems = CK * segs;
    // one descriptor for this utterance's input; rows, positions out of range
    // get an out-of-bounds offset and stage as zeros
    const __amdgpu_buffer_rsrc_t xrs = uniform_rsrc(Xb, g.C_in * g.L_in * 4);
    // Interior tiles (window inside the row, x0 >= 3) take the 16-B path: row c
    // is staged from the 16-B aligned position x0 - dc, dc = (c*L_in + x0 +
    // the base's float offset) mod 4, and its reads shift by dc. Lm = xm = 0
    // elsewhere makes every shift 0.
    const bool x4 = x0 >= 3 && x0 + span <= g.L_in;  // uniform per tile
    const int base_f = static_cast<int>((reinterpret_cast<unsigned long long>(Xb) >> 2) & 3);
    const int Lm = x4 ? (g.L_in & 3) : 0;
    const int xm = x4 ? ((base_f + x0) & 3) : 0;

    // Stage chunk `ch` at LDS float offset `sb`: the weight slab two rows
    // (1 KB) per instruction, the input window 256 (16-B path) or 64 positions
    // per instruction.
    auto issue_a = [&](int ch, int sb) {
        const float* Ag = A + static_cast<long>(ch) * KR * g.m_pad + m0;
        for (int pr = wave; pr < KR / 2; pr += 4)
            __builtin_amdgcn_global_load_lds(Ag + static_cast<long>(2 * pr) * g.m_pad + a_lane,
                                             smem + sb + pr * 256, 16, 0, 0);
    };
    auto issue = [&](int ch, int sb) {
        issue_a(ch, sb);
        if (x4) {
            const int seg4 = span_p >> 8;
            for (int it = wave; it < CK * seg4; it += 4) {
                const int r = it / seg4, sg = it - r * seg4;
                const int c = ch * CK + r;
                const int pos = x0 - ((c * Lm + xm) & 3) + sg * 256 + lane * 4;
                const unsigned off = c < g.C_in ? static_cast<unsigned>(c * g.L_in + pos) * 4u : 0x80000000u;
                if (sg * 256 + lane * 4 < span + 3)  // lanes past the window stay idle
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, smem + sb + KR * BM + r * span_p + sg * 256, 16,
                                                             static_cast<int>(off), 0, 0, 0);
            }
            return;
        }
        for (int it = wave; it < nitems; it += 4) {
            const int r = it / segs, sg = it - r * segs;
            const int c = ch * CK + r;
            const int pos = x0 + sg * 64 + lane;
            const unsigned off = (c < g.C_in && pos >= 0 && pos < g.L_in)
                                     ? static_cast<unsigned>(c * g.L_in + pos) * 4u : 0x80000000u;
            if (sg * 64 + lane < span)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, smem + sb + KR * BM + r * span_p + sg * 64, 4,
                                                         static_cast<int>(off), 0, 0, 0);
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int am = wm * 64 + l32;         // A column (m) for tm = 0
    const int bq = (wn * 64 + l32) * s;   // B column offset for tn = 0
    const int nchunks = g.cin_pad / CK;
    const int nparts = part < 0 ? 1 : g.fsplit;
    const int pp = part < 0 ? 0 : part;
    const int ch0 = pp * nchunks / nparts;
    const int ch1 = (pp + 1) * nchunks / nparts;
    const int S = KR / 2;                 // k-steps per chunk
    const bool live = q0 + wn * 64 < n_q;  // wave-uniform
    constexpr int HS = CK / 2;

    // Two stages: chunk ch + 1 lands while ch is multiplied. One stage (where
    // two would fit only two blocks per CU, the long strided windows): each
    // chunk is staged after every wave has read the previous one, and the
    // other resident blocks' MFMA work covers the wait.
    const bool single = g.single != 0;  // uniform
    if (ch0 < ch1) issue(ch0, 0);
    __builtin_amdgcn_s_waitcnt(0);  // staging loads landed in LDS
    __syncthreads();
    for (int ch = ch0; ch < ch1; ++ch) {
        const int sb = single ? 0 : ((ch - ch0) & 1) * stage;
        if (!single && ch + 1 < ch1) issue(ch + 1, stage - sb);
        const int wb = sb + hi * BM + am;
        const int xb = sb + KR * BM + hi * span_p + bq;
        const int dl = (ch * CK + hi) * Lm + xm;  // row shift of the 16-B path: (dl + cc*Lm) mod 4
        // step u reads packed rows 2u + hi: tap t = u / HS, channel 2(u % HS) + hi
        auto ld = [&](int u, float& a0, float& a1, float& b0, float& b1) {
            u = min(u, S - 1);
            const int t = u / HS;
            const int cc = (u - t * HS) * 2;
            int wo = wb + u * 2 * BM;
            int xo = xb + cc * span_p + t * d + ((dl + cc * Lm) & 3);
            // opaque offsets keep each step's reads where they are placed
            asm volatile("" : "+v"(wo), "+v"(xo));
            a0 = smem[wo];
            a1 = smem[wo + 32];
            b0 = smem[xo];
            b1 = smem[xo + 32 * s];
        };
        auto mm = [&](float a0, float a1, float b0, float b1) {
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        };
        float pa0, pa1, pb0, pb1, qa0, qa1, qb0, qb1;
        ld(0, pa0, pa1, pb0, pb1);
        int u = live ? 0 : S;  // a wave whose columns all lie past n_q only stages
        for (; u + 1 < S; u += 2) {
            ld(u + 1, qa0, qa1, qb0, qb1);
            mm(pa0, pa1, pb0, pb1);
            ld(u + 2, pa0, pa1, pb0, pb1);
            mm(qa0, qa1, qb0, qb1);
            // 1 MFMA, the next step's reads, 3 MFMAs (twice)
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
        }
        if (live && u < S) mm(pa0, pa1, pb0, pb1);
        if (single && ch + 1 < ch1) {
            __syncthreads();  // every wave has read the stage
            issue(ch + 1, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's staging loads landed
        __syncthreads();
    }

    store_tile(g, T, tile, part, acc, wm, wn, hi, l32);
}

// Stride-1 correlation of KT taps with the weights read 16 B per lane.
//
// As conv_gemm (tile plan, input staging, epilogue), but the chunk's weight
// slab is stored in LDS as quads of k-steps: quad g holds k-steps 4g..4g+3 as
// [hi][m (128)][j (4)], element j being packed row 2(4g + j) + hi of the
// chunk (tap (2(4g+j)+hi) / CK, channel (2(4g+j)+hi) % CK). One ds_read_b128
// then gives a lane its A operand for four MFMA steps, so a wave issues two
// weight reads per 16 MFMAs instead of eight; the input operand stays one
// ds_read2 per k-step. The global panel is the LDS image of each chunk,
// m-tile major ([m_tile][chunk][quad][hi][128][4], see pack_quad), so a
// chunk's slab is one contiguous copy. The last quad of a chunk is partial
// when CK*KT/2 is not a multiple of 4; its unused slots are zeros that no
// MFMA reads.
#ifndef CGQ_WPE
#define CGQ_WPE 4
#endif
#ifndef CGQ_PF
#define CGQ_PF 2
#endif
// EPI picks the whole tiles' epilogue at compile time (split tiles always
// store partials): QEPI_STORE the plain store, QEPI_ADAIN_BWD the AdaIN
// backward row sums (store_tile_adain), QEPI_STATS the instance-norm moments
// (store_tile_stats). One epilogue per instantiation keeps the live ranges of
// the others out of the k-loop's register allocation.
enum { QEPI_STORE = 0, QEPI_ADAIN_BWD = 1, QEPI_STATS = 2 };

// Where a conv_gemm_q tile stages its operands from (wave-uniform): the
// m-tile's weight panel, the utterance's input rows and the input window.
struct QSrc {
    const float* A;
    __amdgpu_buffer_rsrc_t xrs;
    int x0;      // first staged position
    int Lm, xm;  // 16-B staging: row length and window start, mod 4 (0 otherwise)
    bool x4;     // the window lies inside the row: staged 16 B per lane
};

__device__ inline QSrc q_src(const GemmArgs& g, const TileGeo& T, int span, int chunk_floats) {
    QSrc s;
    const float* Xb = g.X + static_cast<long>(T.b) * g.x_bs;
    s.A = g.A + static_cast<long>(T.m0 / BM) * (g.cin_pad / g.CK) * chunk_floats;
    s.xrs = uniform_rsrc(Xb, g.C_in * g.L_in * 4);
    s.x0 = T.q0 - T.p;
    s.x4 = s.x0 >= 3 && s.x0 + span <= g.L_in;
    const int base_f = static_cast<int>((reinterpret_cast<unsigned long long>(Xb) >> 2) & 3);
    s.Lm = s.x4 ? (g.L_in & 3) : 0;
    s.xm = s.x4 ? ((base_f + s.x0) & 3) : 0;
    return s;
}

template <int CK, int KT, int EPI>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(CGQ_WPE)))
void conv_gemm_q(GemmArgs g) {
    constexpr int S = CK * KT / 2;  // k-steps per chunk
    constexpr int Q = (S + 3) / 4;  // weight quads per chunk
    constexpr int QA = Q * 1024;    // LDS floats of a chunk's weights
    constexpr int HS = CK / 2;      // k-steps per tap
    extern __shared__ float smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = wave & 1, wn0 = wave >> 1;
    const int l320 = lane & 31, hi0 = lane >> 5;

    int tile, part;
    if (!block_work(g, tile, part)) return;  // uniform per block

    const int span = BN + (KT - 1) * g.d;  // staged input window (stride 1)
    const int span_p0 = (span + 3 + 255) & ~255;
    const int segs = span_p0 >> 6;
    const int stage = QA + CK * span_p0;
    const int nchunks = g.cin_pad / CK;
    const int nparts = part < 0 ? 1 : g.fsplit;
    const int pp = part < 0 ? 0 : part;
    const int ch0 = pp * nchunks / nparts;
    const int ch1 = (pp + 1) * nchunks / nparts;

    // Stage chunk `ch` of tile Tg at LDS float offset `sb`: the weight slab
    // 1 KB per instruction, the input window as conv_gemm stages it.
    auto issue = [&](const TileGeo& Tg, int ch, int sb) {
        const QSrc s = q_src(g, Tg, span, QA);
        const float* Ag = s.A + static_cast<long>(ch) * QA + lane * 4;
        for (int i = wave; i < QA / 256; i += 4)
            __builtin_amdgcn_global_load_lds(Ag + i * 256, smem + sb + i * 256, 16, 0, 0);
        if (s.x4) {
            const int seg4 = span_p0 >> 8;
            for (int it = wave; it < CK * seg4; it += 4) {
                const int r = it / seg4, sg = it - r * seg4;
                const int c = ch * CK + r;
                const int pos = s.x0 - ((c * s.Lm + s.xm) & 3) + sg * 256 + lane * 4;
                const unsigned off = c < g.C_in ? static_cast<unsigned>(c * g.L_in + pos) * 4u : 0x80000000u;
                if (sg * 256 + lane * 4 < span + 3)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(s.xrs, smem + sb + QA + r * span_p0 + sg * 256, 16,
                                                             static_cast<int>(off), 0, 0, 0);
            }
            return;
        }
        for (int it = wave; it < CK * segs; it += 4) {
            const int r = it / segs, sg = it - r * segs;
            const int c = ch * CK + r;
            const int pos = s.x0 + sg * 64 + lane;
            const unsigned off = (c < g.C_in && pos >= 0 && pos < g.L_in)
                                     ? static_cast<unsigned>(c * g.L_in + pos) * 4u : 0x80000000u;
            if (sg * 64 + lane < span)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(s.xrs, smem + sb + QA + r * span_p0 + sg * 64, 4,
                                                         static_cast<int>(off), 0, 0, 0);
        }
    };

    TileGeo T;
    decode_tile(g, tile, T);
    if (T.q0 >= T.n_q) return;  // uniform per block (stride-1 plain tiles never are)
    if (ch0 < ch1) issue(T, ch0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // The lane coordinates and the staging geometry pass through an empty asm
    // after the prologue, the tile is decoded again for the epilogue from a
    // laundered index, and the staging source is formed at each issue: what
    // the MFMA loop and the epilogue derive from these (per-step LDS offsets,
    // per-element row offsets, descriptors) is then formed where it is used,
    // not hoisted to the kernel's start and held live through the MFMA loop
    // (measured: 2-3% on the stride-1 decoder convs).
    int wm = wm0, wn = wn0, hi = hi0, l32 = l320, span_p = span_p0, d = g.d;
    asm volatile("" : "+s"(wm), "+s"(wn), "+v"(hi), "+v"(l32), "+s"(span_p), "+s"(d));
    int sb = 0;  // LDS stage of the chunk in hand
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int am = wm * 64 + l32;
    const int bq = wn * 64 + l32;
    const bool live = T.q0 + wn * 64 < T.n_q;  // wave-uniform
    for (int ch = ch0; ch < ch1; ++ch) {
        // the next chunk's staging issued at a raised wave priority: a wave
        // that reaches it gets its DMA instructions out ahead of the other
        // waves' MFMAs and LDS reads on the SIMD, so the loads start early
        // (one-stream conv and weight-grad families 0.5 % faster)
        __builtin_amdgcn_s_setprio(1);
        if (ch + 1 < ch1) issue(T, ch + 1, stage - sb);
        __builtin_amdgcn_s_setprio(0);
        if (live) {
            const QSrc cur = q_src(g, T, span, QA);
            const f32x4* Aq = reinterpret_cast<const f32x4*>(smem + sb) + hi * BM + am;
            const int xb = sb + QA + hi * span_p + bq;
            const int dl = (ch * CK + hi) * cur.Lm + cur.xm;
            const int Lm = cur.Lm;
            auto ldb = [&](int u, float& b0, float& b1) {
                const int t = u / HS;
                const int cc = (u - t * HS) * 2;
                int xo = xb + cc * span_p + t * d + ((dl + cc * Lm) & 3);
                asm volatile("" : "+v"(xo));
                b0 = smem[xo];
                b1 = smem[xo + 32];
            };
            // the input operand is read CGQ_PF k-steps ahead (a ring of
            // CGQ_PF + 1 register pairs), the next weight quad at the first
            // step of the current one; each step issues one MFMA, its reads,
            // then three MFMAs
            constexpr int PF = CGQ_PF;
            f32x4 qa[2][2];
            float bb[PF + 1][2];
            qa[0][0] = Aq[0];
            qa[0][1] = Aq[32];
#pragma unroll
            for (int u = 0; u < PF && u < S; ++u) ldb(u, bb[u][0], bb[u][1]);
#pragma unroll
            for (int u = 0; u < S; ++u) {
                const int gq = u / 4, j = u % 4;
                const float a0 = qa[gq & 1][0][j], a1 = qa[gq & 1][1][j];
                const float b0 = bb[u % (PF + 1)][0], b1 = bb[u % (PF + 1)][1];
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
                if (j == 0 && gq + 1 < Q) {
                    qa[(gq + 1) & 1][0] = Aq[(gq + 1) * 2 * BM];
                    qa[(gq + 1) & 1][1] = Aq[(gq + 1) * 2 * BM + 32];
                }
                if (u + PF < S) ldb(u + PF, bb[(u + PF) % (PF + 1)][0], bb[(u + PF) % (PF + 1)][1]);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (j == 0 && gq + 1 < Q) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                if (u + PF < S) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
                __builtin_amdgcn_sched_barrier(0);  // nothing crosses into the next step
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's staging loads landed
        __syncthreads();
        sb = stage - sb;
    }

    int te = tile;
    asm volatile("" : "+s"(te));
    TileGeo Te;
    decode_tile(g, te, Te);
    if constexpr (EPI == QEPI_ADAIN_BWD) {
        if (part < 0) {  // uniform per block
            store_tile_adain(g, Te, acc, wm, wn, hi, l32, smem);
        } else {
            store_tile(g, Te, te, part, acc, wm, wn, hi, l32);
        }
    } else if constexpr (EPI == QEPI_STATS) {
        if (part < 0)
            store_tile_stats(g, Te, acc, wm, wn, hi, l32);
        else
            store_tile(g, Te, te, part, acc, wm, wn, hi, l32);
    } else {
        store_tile(g, Te, te, part, acc, wm, wn, hi, l32);
    }
}

// Stride-1 correlation (conv forward, conv input-grad, each transposed-conv
// phase) as an implicit GEMM whose operands are read 16 B per lane.
//
// K runs over (input channel c, tap t). A chunk is one channel octet
// o (c = 8o + 4h + e, h in {0, 1}, e in 0..3) times a group of up to G taps.
// In one 32x32x2 MFMA step e of tap t, lanes of half h contribute
// k = (8o + 4h + e, t), so each lane needs, per tap, four consecutive
// channels: the weights are packed as [o][t][h][m_pad][4] (a chunk's rows
// are whole 2 KB runs per (t, h) and a block's 128 columns), and the input
// window is staged channels-last, [h][position][4], by a gathering DMA
// (lane i of a 64-lane load fetches channel 4h + i%4 at position i/4 and
// lands at LDS float i of the block). One ds_read_b128 then feeds four
// MFMA steps: per tap a wave reads 2 A and 2 B vectors for 16 MFMAs.
// Grid, tile order, split parts and epilogue as conv_gemm.
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4)))
void corr_gemm(GemmArgs g) {
    extern __shared__ float smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, hi = lane >> 5;

    int tile, part;
    if (!block_work(g, tile, part)) return;  // uniform per block
    TileGeo T;
    decode_tile(g, tile, T);
    const int k = T.k, d = T.d;
    if (T.q0 >= T.n_q) return;  // uniform per block

    const int G = g.G, n_tg = g.n_tg, span8 = g.span8;
    const int a_st = G * 1024;             // A floats per stage: G taps x 2 halves x 128 x 4
    const int stage = a_st + 8 * span8;    // + input window: 2 halves x span8 positions x 4
    const float* Xb = g.X + static_cast<long>(T.b) * g.x_bs;
    const __amdgpu_buffer_rsrc_t xrs = uniform_rsrc(Xb, g.C_in * g.L_in * 4);
    const int x0 = T.q0 - T.p;             // input position of column q0 at tap 0
    // weight staging: wave w copies quarter w of every (tap, half) run:
    // half w>>1, 256-float piece w&1 of the block's 512 floats
    const long a_row = 8L * g.m_pad;       // floats per (octet, tap) = 2 halves x m_pad x 4
    const float* Aw = T.A + static_cast<long>(T.m0) * 4 + (wave >> 1) * g.m_pad * 4 + (wave & 1) * 256 + lane * 4;
    const int a_lds = (wave >> 1) * 512 + (wave & 1) * 256;
    // input staging: wave w fetches half w&1, 16-position blocks (w>>1) + 2j
    const int nb = span8 >> 4;
    const int lane_c = (wave & 1) * 4 + (lane & 3);
    const int lane_p = lane >> 2;
    const int x_lds = a_st + (wave & 1) * span8 * 4;

    auto issue = [&](int o, int tg, int sb) {
        const int t0 = tg * G;
        const int gt = min(G, k - t0);
        const float* Ag = Aw + (static_cast<long>(o) * k + t0) * a_row;
        for (int j = 0; j < gt; ++j)
            __builtin_amdgcn_global_load_lds(Ag + j * a_row, smem + sb + j * 1024 + a_lds, 16, 0, 0);
        const int xs = x0 + t0 * d;
        const int c = o * 8 + lane_c;
        const bool inner = o * 8 + 8 <= g.C_in && xs >= 0 && xs + span8 <= g.L_in;  // uniform
        for (int blk = wave >> 1; blk < nb; blk += 2) {
            const int pos = xs + blk * 16 + lane_p;
            const unsigned off = (inner || (c < g.C_in && pos >= 0 && pos < g.L_in))
                                     ? static_cast<unsigned>(c * g.L_in + pos) * 4u : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, smem + sb + x_lds + blk * 64, 4,
                                                     static_cast<int>(off), 0, 0, 0);
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int nchunks = g.n_oct * n_tg;
    const int nparts = part < 0 ? 1 : g.fsplit;
    const int pp = part < 0 ? 0 : part;
    const int ch0 = pp * nchunks / nparts;
    const int ch1 = (pp + 1) * nchunks / nparts;
    const bool live = T.q0 + wn * 64 < T.n_q;  // wave-uniform
    // lane reads: A at m = wm*64 + tm*32 + l32, B at column n = wn*64 + tn*32 + l32 (+ tap shift)
    const int a_rd = hi * 512 + (wm * 64 + l32) * 4;
    const int b_rd = a_st + hi * span8 * 4 + (wn * 64 + l32) * 4;

    int o = ch0 / n_tg, tg = ch0 - (ch0 / n_tg) * n_tg;  // chunk ch = o * n_tg + tg
    if (ch0 < ch1) issue(o, tg, 0);
    __builtin_amdgcn_s_waitcnt(0);  // staging loads landed in LDS
    __syncthreads();
    for (int ch = ch0; ch < ch1; ++ch) {
        const int sb = ((ch - ch0) & 1) * stage;
        const int no = tg + 1 == n_tg ? o + 1 : o, ntg = tg + 1 == n_tg ? 0 : tg + 1;
        if (ch + 1 < ch1) issue(no, ntg, stage - sb);
        const int gt = min(G, k - tg * G);
        const int ab = sb + a_rd, bb = sb + b_rd;
        auto ld = [&](int tl, float4 (&a)[2], float4 (&bv)[2]) {
            tl = min(tl, gt - 1);
            int ao = ab + tl * 1024, bo = bb + tl * d * 4;
            // opaque offsets keep each tap's reads where they are placed
            asm volatile("" : "+v"(ao), "+v"(bo));
            a[0] = *reinterpret_cast<const float4*>(smem + ao);
            a[1] = *reinterpret_cast<const float4*>(smem + ao + 128);
            bv[0] = *reinterpret_cast<const float4*>(smem + bo);
            bv[1] = *reinterpret_cast<const float4*>(smem + bo + 128);
        };
        auto mm = [&](const float4 (&a)[2], const float4 (&bv)[2]) {
            const float a0[4] = {a[0].x, a[0].y, a[0].z, a[0].w};
            const float a1[4] = {a[1].x, a[1].y, a[1].z, a[1].w};
            const float b0[4] = {bv[0].x, bv[0].y, bv[0].z, bv[0].w};
            const float b1[4] = {bv[1].x, bv[1].y, bv[1].z, bv[1].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], b0[e], acc[0][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], b1[e], acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], b0[e], acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], b1[e], acc[1][1], 0, 0, 0);
            }
        };
        float4 pa[2], pb[2], qa[2], qb[2];
        ld(0, pa, pb);
        int tl = live ? 0 : gt;  // a wave whose columns all lie past n_q only stages
        for (; tl + 1 < gt; tl += 2) {
            ld(tl + 1, qa, qb);
            mm(pa, pb);
            ld(tl + 2, pa, pb);
            mm(qa, qb);
            // (1 MFMA, 1 read) x 4, then 12 MFMAs; twice
            for (int r = 0; r < 2; ++r) {
                for (int i = 0; i < 4; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 12, 0);
            }
        }
        if (live && tl < gt) mm(pa, pb);
        o = no;
        tg = ntg;
        __builtin_amdgcn_s_waitcnt(0);  // this wave's staging loads landed
        __syncthreads();
    }

    store_tile(g, T, tile, part, acc, wm, wn, hi, l32);
}

// Split tiles: Y = scale * (sum of the parts in order + bias + R) + beta * Y.
// Grid (BM * BN / 1024, split_tiles).
// The split parts of one float4 of a tile summed in part order (the bits of
// a sequential loop), their loads issued eight at a time: a loop that loads
// one part per trip waits for each before the next.
__device__ inline float4 sum_parts(const float4* Pt, int e4, int fsplit) {
    float4 v = Pt[e4];
    for (int sp = 1; sp < fsplit; sp += 8) {
        float4 w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = Pt[min(sp + u, fsplit - 1) * (BM * BN / 4) + e4];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (sp + u < fsplit) {
                v.x += w[u].x;
                v.y += w[u].y;
                v.z += w[u].z;
                v.w += w[u].w;
            }
    }
    return v;
}

__global__ void tile_reduce(GemmArgs g) {
    __builtin_amdgcn_s_setprio(2);  // on the conv chain: as the AdaIN passes
    const int ti = blockIdx.y;
    TileGeo T;
    decode_tile(g, g.full_tiles + ti, T);
    if (T.q0 >= T.n_q) return;
    // four consecutive columns per thread: the parts are read 16 B per lane
    const float4* Pt = reinterpret_cast<const float4*>(g.P + static_cast<long>(ti) * g.fsplit * (BM * BN));
    float* Yb = g.Y + static_cast<long>(T.b) * g.y_bs;
    const float* Rb = g.R ? g.R + static_cast<long>(T.b) * g.r_bs : nullptr;
    for (int e4 = blockIdx.x * blockDim.x + threadIdx.x; e4 < BM * BN / 4; e4 += gridDim.x * blockDim.x) {
        const int m = T.m0 + (e4 * 4) / BN, qb = T.q0 + (e4 * 4) % BN;
        if (m >= g.C_out || qb >= T.n_q) continue;
        const float4 v = sum_parts(Pt, e4, g.fsplit);
        const float vv[4] = {v.x, v.y, v.z, v.w};
        const float bs = g.bias ? g.bias[m] : 0.0f;
        // the four columns' residual and old Y in one run each (a column
        // past n_q reads the last valid one and is not stored)
        float rv[4], yv[4];
        if (Rb) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                rv[j] = Rb[static_cast<long>(m) * g.L_y + static_cast<long>(min(qb + j, T.n_q - 1)) * T.os + T.oo];
        }
        if (g.beta != 0.0f) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                yv[j] = Yb[static_cast<long>(m) * g.L_y + static_cast<long>(min(qb + j, T.n_q - 1)) * T.os + T.oo];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int q = qb + j;
            if (q >= T.n_q) break;
            float x = vv[j] + bs;
            const long col = static_cast<long>(q) * T.os + T.oo;
            const long yi = static_cast<long>(m) * g.L_y + col;
            if (g.refl && col == 1 + g.y_off) {  // the reflected column 0 (beta = 0)
                const long y0 = static_cast<long>(m) * g.L_y;
                Yb[y0] = (x + (Rb ? Rb[y0] : 0.0f)) * g.scale;
            }
            if (Rb) x += rv[j];
            x *= g.scale;
            if (g.beta != 0.0f) x += g.beta * yv[j];
            Yb[yi] = x;
        }
    }
}

// Split tiles whose GEMM feeds an AdaIN backward: the parts summed in order
// (as tile_reduce), then the epilogue of store_tile_adain on the tile's
// values. One float4 of the tile per thread (grid (BM * BN / 1024,
// split_tiles) of 256 threads), so the 32 lanes of a half-wave hold one
// row's 128 columns: their sums go to slot 2 * q_tile, zeros to the other.
__global__ __launch_bounds__(256) void tile_reduce_adain(GemmArgs g) {
    __builtin_amdgcn_s_setprio(2);  // on the conv chain: as the AdaIN passes
    const int ti = blockIdx.y;
    TileGeo T;
    decode_tile(g, g.full_tiles + ti, T);
    if (T.q0 >= T.n_q) return;  // uniform per block
    const int e4 = blockIdx.x * blockDim.x + threadIdx.x;
    const int l32 = threadIdx.x & 31;
    const int m = T.m0 + e4 / (BN / 4), qb = T.q0 + (e4 % (BN / 4)) * 4;
    const float4* Pt = reinterpret_cast<const float4*>(g.P + static_cast<long>(ti) * g.fsplit * (BM * BN));
    float sd = 0.0f, sdx = 0.0f, sa = 0.0f, a = 1.0f;
    if (m < g.C_out) {
        const float4 v = sum_parts(Pt, e4, g.fsplit);
        const int row = T.b * g.C_out + m;
        const float2 st = g.ad.st[row];
        const float g1 = 1.0f + g.ad.gam[T.b * g.ad.gb_bs + m];
        const float bt = g.ad.bet ? g.ad.bet[T.b * g.ad.gb_bs + m] : 0.0f;
        if (g.ad.act == KDEC_ACT_SNAKE) a = g.ad.alpha[m];
        const float vv[4] = {v.x, v.y, v.z, v.w};
        float* Yb = g.Y + static_cast<long>(T.b) * g.y_bs;
        const float* xb = g.ad.x + static_cast<long>(T.b) * g.ad.x_bs;
        float xv[4];  // one run of loads (a column past n_q reads the last valid one)
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[j] = xb[static_cast<long>(m) * g.L_y + min(qb + j, T.n_q - 1)];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int q = qb + j;
            if (q >= T.n_q) break;
            const long yi = static_cast<long>(m) * g.L_y + q;
            const float xh = (xv[j] - st.x) * st.y;
            const float ds = epi_act_bwd(g.ad.act, vv[j] * g.scale, g1 * xh + bt, g.ad.slope, a, sa);
            Yb[yi] = ds;
            sd += ds;
            sdx += ds * xh;
        }
    }
    sd += xor_lane<16>(sd);
    sd += xor_lane<8>(sd);
    sd += xor_lane<4>(sd);
    sd += xor_lane<2>(sd);
    sd += xor_lane<1>(sd);
    sdx += xor_lane<16>(sdx);
    sdx += xor_lane<8>(sdx);
    sdx += xor_lane<4>(sdx);
    sdx += xor_lane<2>(sdx);
    sdx += xor_lane<1>(sdx);
    sa += xor_lane<16>(sa);
    sa += xor_lane<8>(sa);
    sa += xor_lane<4>(sa);
    sa += xor_lane<2>(sa);
    sa += xor_lane<1>(sa);
    if (l32 == 0 && m < g.C_out) {
        double* pp = g.ad.part + ((static_cast<long>(T.b) * g.C_out + m) * g.ad.nch + (T.q0 / BN) * 2) * 3;
        pp[0] = sd;
        pp[1] = sdx;
        pp[2] = g.ad.act == KDEC_ACT_SNAKE ? static_cast<double>(sa) / (static_cast<double>(a) * a) : 0.0;
        pp[3] = 0.0;
        pp[4] = 0.0;
        pp[5] = 0.0;
    }
}

// Split tiles of a forward conv with the statistics epilogue: the parts
// summed in order and stored as tile_reduce stores them, then per row the
// count, mean and sum of squared deviations over the tile's columns (the 32
// lanes of a half-wave hold one row's 128 columns) into slot 2 * q_tile, an
// empty record into the other. Grid (BM * BN / 1024, split_tiles) x 256.
__global__ __launch_bounds__(256) void tile_reduce_stats(GemmArgs g) {
    __builtin_amdgcn_s_setprio(2);  // on the conv chain: as the AdaIN passes
    const int ti = blockIdx.y;
    TileGeo T;
    decode_tile(g, g.full_tiles + ti, T);
    if (T.q0 >= T.n_q) return;  // uniform per block
    const int e4 = blockIdx.x * blockDim.x + threadIdx.x;
    const int l32 = threadIdx.x & 31;
    const int m = T.m0 + e4 / (BN / 4), qb = T.q0 + (e4 % (BN / 4)) * 4;
    const int cnt = min(T.n_q - T.q0, BN);
    const float4* Pt = reinterpret_cast<const float4*>(g.P + static_cast<long>(ti) * g.fsplit * (BM * BN));
    float vv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (m < g.C_out) {
        const float4 v = sum_parts(Pt, e4, g.fsplit);
        const float raw[4] = {v.x, v.y, v.z, v.w};
        const float bs = g.bias ? g.bias[m] : 0.0f;
        float* Yb = g.Y + static_cast<long>(T.b) * g.y_bs;
        const float* Rb = g.R ? g.R + static_cast<long>(T.b) * g.r_bs : nullptr;
        float rv[4];  // one run of loads (a column past n_q reads the last valid one)
        if (Rb) {
#pragma unroll
            for (int j = 0; j < 4; ++j) rv[j] = Rb[static_cast<long>(m) * g.L_y + min(qb + j, T.n_q - 1)];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int q = qb + j;
            if (q >= T.n_q) break;
            const long yi = static_cast<long>(m) * g.L_y + q;
            float x = raw[j] + bs;
            if (Rb) x += rv[j];
            x *= g.scale;
            Yb[yi] = x;
            vv[j] = x;
        }
    }
    float s = vv[0] + vv[1] + vv[2] + vv[3];
    s += xor_lane<16>(s);
    s += xor_lane<8>(s);
    s += xor_lane<4>(s);
    s += xor_lane<2>(s);
    s += xor_lane<1>(s);
    const float mean = s / static_cast<float>(cnt);
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float dv = vv[j] - mean;
        d += qb + j < T.n_q ? dv * dv : 0.0f;
    }
    d += xor_lane<16>(d);
    d += xor_lane<8>(d);
    d += xor_lane<4>(d);
    d += xor_lane<2>(d);
    d += xor_lane<1>(d);
    if (l32 == 0 && m < g.C_out) {
        double* pp = g.fs.part + ((static_cast<long>(T.b) * g.C_out + m) * g.fs.nch + (T.q0 / BN) * 2) * 3;
        pp[0] = cnt;
        pp[1] = mean;
        pp[2] = d;
        pp[3] = 0.0;
        pp[4] = 0.0;
        pp[5] = 0.0;
    }
}

// Merges (count, mean, sum of squared deviations) records (Chan et al.'s
// pairwise update, in double): a at b's side, in place.
__device__ inline void chan_merge(double& n, double& mean, double& m2, double nb, double mb, double m2b) {
    if (nb <= 0.0) return;
    const double nt = n + nb;
    const double delta = mb - mean;
    mean += delta * (nb / nt);
    m2 += m2b + delta * delta * (n * nb / nt);
    n = nt;
}

// stats[row] = (mean, 1 / sqrt(var + eps)) from the row's slot records: one
// wave per row, lane j merging slots j, j + 64, ... in order (eight slots'
// loads in flight, issued unconditionally from clamped indices), then the
// lanes in a fixed tree.
__global__ __launch_bounds__(64) void instnorm_fin_slots_k(const double* part, int nch, float eps, float2* stats) {
    __builtin_amdgcn_s_setprio(2);  // on the conv chain: as the AdaIN passes
    const int row = blockIdx.x;
    const double* p = part + static_cast<long>(row) * nch * 3;
    double n = 0.0, mean = 0.0, m2 = 0.0;
    for (int j0 = threadIdx.x; j0 < nch; j0 += 8 * 64) {
        double a[8], b[8], c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = min(j0 + 64 * u, nch - 1);
            a[u] = p[3 * j];
            b[u] = p[3 * j + 1];
            c[u] = p[3 * j + 2];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (j0 + 64 * u < nch) chan_merge(n, mean, m2, a[u], b[u], c[u]);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double n2 = __shfl_xor(n, o, 64), mean2 = __shfl_xor(mean, o, 64), m22 = __shfl_xor(m2, o, 64);
        chan_merge(n, mean, m2, n2, mean2, m22);
    }
    if (threadIdx.x == 0) {
        const double var = n > 0.0 ? m2 / n : 0.0;
        stats[row] = make_float2(static_cast<float>(mean), static_cast<float>(1.0 / sqrt(var + static_cast<double>(eps))));
    }
}

// ─── weight packing ──────────────────────────────────────────────────────
// All packers write the zero-padded panel A[row][m_pad] in chunk-major row
// order: row = ((c / CK) * kk + t) * CK + c % CK for input channel c and
// tap t, so that one K chunk (CK channels x kk taps) is a contiguous slab.

__device__ inline void panel_row(long row, int CK, int kk, int& c, int& t) {
    const int cl = static_cast<int>(row % CK);
    const long r2 = row / CK;
    t = static_cast<int>(r2 % kk);
    c = static_cast<int>(r2 / kk) * CK + cl;
}

// conv1d forward: A[(ci, t), co] = W[co, ci*k + t]
__global__ void pack_fwd(const float* W, float* A, int C_in, int C_out, int k,
                         int cin_pad, int m_pad, int CK) {
    const long total = static_cast<long>(cin_pad) * k * m_pad;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int m = static_cast<int>(i % m_pad);
        int c, t;
        panel_row(i / m_pad, CK, k, c, t);
        float v = 0.0f;
        if (m < C_out && c < C_in) v = W[(static_cast<long>(m) * C_in + c) * k + t];
        A[i] = v;
    }
}

// conv1d input-grad (stride 1): the correlation over dY (C_out channels) with
// A[(co, t'), ci] = W[co, ci*k + (k-1-t')]
__global__ void pack_dgrad(const float* W, float* A, int C_in, int C_out, int k,
                           int cout_pad, int m_pad, int CK) {
    const long total = static_cast<long>(cout_pad) * k * m_pad;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int m = static_cast<int>(i % m_pad);  // ci
        int c, t;                                   // c = co
        panel_row(i / m_pad, CK, k, c, t);
        float v = 0.0f;
        if (m < C_in && c < C_out) v = W[(static_cast<long>(c) * C_in + m) * k + (k - 1 - t)];
        A[i] = v;
    }
}

// The quad panel of conv_gemm_q: A[m_tile][chunk][quad][hi][128][4], element
// j of (quad g, hi, m) being packed row r = 2(4g + j) + hi of the chunk, i.e.
// tap r / CK of channel chunk*CK + r % CK; zero past the chunk's CK*k/2
// k-steps, past the channels or past the output rows. mode 0: conv1d forward
// (A[(ci, t), co] = W[co, ci*k + t]); mode 1: conv1d input-grad at stride 1
// (A[(co, t'), ci] = W[co, ci*k + k-1-t']). One thread writes one 16-B run.
__global__ void pack_quad(const float* W, float* A, int mode, int C_in, int C_out, int k, int CK, int nchunks,
                          int Q, long total4) {
    const int S = CK * k / 2;
    const int Cg = mode == 0 ? C_in : C_out;   // GEMM input channels
    const int Mg = mode == 0 ? C_out : C_in;   // GEMM output rows
    for (long e = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; e < total4;
         e += static_cast<long>(gridDim.x) * blockDim.x) {
        const int ml = static_cast<int>(e % BM);
        long r2 = e / BM;
        const int hi = static_cast<int>(r2 & 1);
        r2 >>= 1;
        const int gq = static_cast<int>(r2 % Q);
        r2 /= Q;
        const int ch = static_cast<int>(r2 % nchunks);
        const int m = static_cast<int>(r2 / nchunks) * BM + ml;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int u = 4 * gq + j;
            const int r = 2 * u + hi;
            const int t = r / CK, c = ch * CK + r % CK;
            float x = 0.0f;
            if (u < S && c < Cg && m < Mg)
                x = mode == 0 ? W[(static_cast<long>(m) * C_in + c) * k + t]
                              : W[(static_cast<long>(c) * C_in + m) * k + (k - 1 - t)];
            v[j] = x;
        }
        reinterpret_cast<float4*>(A)[e] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// conv-transpose input-grad: correlation over dY (C_out channels) with
// A[(co, t), ci] = W[ci, co*k + t]
__global__ void pack_convt_dgrad(const float* W, float* A, int C_in, int C_out,
                                 int k, int cout_pad, int m_pad, int CK) {
    const long total = static_cast<long>(cout_pad) * k * m_pad;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int m = static_cast<int>(i % m_pad);  // ci
        int c, t;                                   // c = co
        panel_row(i / m_pad, CK, k, c, t);
        float v = 0.0f;
        if (m < C_in && c < C_out) v = W[(static_cast<long>(m) * C_out + c) * k + t];
        A[i] = v;
    }
}

// The panel row of (channel c, tap t) for CK-channel chunks, the inverse of
// panel_row: row = ((c / CK) * kk + t) * CK + c % CK.
__device__ inline long panel_index(int c, int t, int CK, int kk) {
    return (static_cast<long>(c / CK) * kk + t) * CK + (c % CK);
}

// A[panel_index(c, t)][m] = W[m][c*k + t] (0 unless m < Mv and c < Cv): the
// conv1d forward panel (m = co, c = ci) and the conv-transpose input-grad
// panel (m = ci, c = co). A 32 (m) x 32 (j = c*k + t) tile passes through LDS:
// W is read along its rows (j), A written along its rows (m). 32-square tiles
// rather than 64: a single round of larger blocks spends most of its time
// waiting on one load and one store round trip, and four times as many
// blocks overlap one block's stores with others' loads (1.2-1.9x faster on
// the decoder's panels). Grid (cdiv(cpad*k, 32), m_pad / 32); cpad a
// multiple of CK, m_pad of 32.
__global__ __launch_bounds__(256) void pack_rows_t(const float* W, float* A, int Mv, int Cv, int k, int cpad,
                                                   int m_pad, int CK) {
    __shared__ float tile[32][33];
    const int j0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    const long ld = static_cast<long>(Cv) * k;  // W row length
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = m0 + ty + 8 * r, j = j0 + tx;
        v[r] = (m < Mv && j < ld) ? W[m * ld + j] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) tile[tx][ty + 8 * r] = v[r];
    __syncthreads();
    const long rows = static_cast<long>(cpad) * k;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = ty + 8 * r, j = j0 + i;
        if (j < rows) {
            const int c = j / k, t = j - c * k;
            A[panel_index(c, t, CK, k) * m_pad + m0 + tx] = tile[i][tx];
        }
    }
}

// A[panel_index(c, t)][m] = W[c][m*k + k-1-t] (0 unless m < C_in, c < C_out):
// the conv1d input-grad panel. Each wave takes one output channel c and a
// 64-column m slice: it reads that slice's contiguous 64*k floats of W[c]
// into LDS, then writes its k panel rows along m. Grid (cdiv(cpad, 4),
// m_pad / 64), dynamic LDS 4 * 64 * k floats; cpad a multiple of CK.
__global__ __launch_bounds__(256) void pack_dgrad_t(const float* W, float* A, int C_in, int C_out, int k,
                                                    int cpad, int m_pad, int CK) {
    extern __shared__ float seg_all[];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int c = blockIdx.x * 4 + ty, m0 = blockIdx.y * 64;
    float* seg = seg_all + ty * 64 * k;
    const long base = static_cast<long>(c) * C_in * k + static_cast<long>(m0) * k;
    const long lim = static_cast<long>(C_in) * k;  // valid part of row c
    // k <= 32: a fixed trip count, unrolled, so the loads overlap
    float v[32];
#pragma unroll
    for (int r = 0; r < 32; ++r) {
        const int e = tx + 64 * r;
        v[r] = (r < k && c < C_out && static_cast<long>(m0) * k + e < lim) ? W[base + e] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 32; ++r)
        if (r < k) seg[tx + 64 * r] = v[r];
    __syncthreads();
    if (c >= cpad) return;
    for (int t = 0; t < k; ++t)
        A[panel_index(c, t, CK, k) * m_pad + m0 + tx] = seg[tx * k + (k - 1 - t)];
}

// conv-transpose forward, phase r of s: tap t' of kt covers original tap
// t = r + (kt-1-t')*s.  A_r[(ci, t'), co] = W[ci, co*k + t] (0 if t >= k)
__global__ void pack_convt_fwd(const float* W, float* A, int C_in, int C_out,
                               int k, int s, int kt, int cin_pad, int m_pad,
                               long phase_stride, int CK) {
    const long total = phase_stride * s;
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<long>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(i / phase_stride);
        const long w = i - r * phase_stride;
        const int m = static_cast<int>(w % m_pad);  // co
        int c, tp;                                  // c = ci
        panel_row(w / m_pad, CK, kt, c, tp);
        const int t = r + (kt - 1 - tp) * s;
        float v = 0.0f;
        if (m < C_out && c < C_in && t < k) v = W[(static_cast<long>(c) * C_out + m) * k + t];
        A[i] = v;
    }
}

// corr_gemm panel [o][t][h][m_pad][4] for channel c = 8o + 4h + e and tap
// t < kt (per phase, phase_stride floats each). `mode` is the weight map:
// 0 conv forward            A[(c, t), m] = W[m, c*k + t]       (m < C_out, c < C_in)
// 1 conv input-grad         A[(c, t), m] = W[c, m*k + k-1-t]   (m < C_in, c < C_out)
// 2 conv-transpose forward, phase r of s: tap t covers original tap
//   r + (kt-1-t)*s, A_r[(c, t), m] = W[c, m*k + that] or 0   (m < C_out, c < C_in)
__global__ void pack_octet(const float* W, float* A, int mode, int C_in, int C_out, int k, int s, int kt,
                           int m_pad, int phase_stride, int n_phase) {
    // 32-bit index math: the host keeps phase_stride * n_phase below 2^31
    const unsigned total = static_cast<unsigned>(phase_stride) * n_phase;
    const unsigned mp = static_cast<unsigned>(m_pad);
    for (unsigned i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const unsigned r = i / static_cast<unsigned>(phase_stride);
        const unsigned w = i - r * static_cast<unsigned>(phase_stride);
        const int e = static_cast<int>(w & 3);
        const unsigned w4 = w >> 2;
        const unsigned rest = w4 / mp;
        const int m = static_cast<int>(w4 - rest * mp);
        const int h = static_cast<int>(rest & 1);
        const unsigned ot = rest >> 1;
        const int o = static_cast<int>(ot / static_cast<unsigned>(kt));
        const int t = static_cast<int>(ot) - o * kt;
        const int c = o * 8 + h * 4 + e;
        float v = 0.0f;
        if (mode == 0) {
            if (m < C_out && c < C_in) v = W[(m * C_in + c) * k + t];
        } else if (mode == 1) {
            if (m < C_in && c < C_out) v = W[(c * C_in + m) * k + (k - 1 - t)];
        } else {
            const int tt = static_cast<int>(r) + (kt - 1 - t) * s;
            if (m < C_out && c < C_in && tt < k) v = W[(c * C_out + m) * k + tt];
        }
        A[i] = v;
    }
}

// ─── weight grad ─────────────────────────────────────────────────────────

constexpr int KC = 32;       // positions per K chunk
// Waves along n (2 along m): 4 (256 columns per block) or 2 (128 columns,
// for column counts C_x * k that 256-wide tiles would leave partly idle).
constexpr int WG_WN = 4;
constexpr int WG_NT = 128 * WG_WN;       // threads per wide wgrad block
constexpr int WG_BN = 64 * WG_WN;        // n columns per wide wgrad block
// G tile in LDS: 64 row pairs (m, m + 64) of 2*KC positions at a pair stride
// of 2*KC + 4 floats: one 64-lane load fills a whole pair, rows stay 16-B
// aligned for ds_read_b128, and 16 consecutive m of one such read cover all
// 64 banks once.
constexpr int GP = 2 * KC + 4;
// Held packed input-window offsets per wave on the stride-1 fast path.
constexpr int WG_XI = 8;

struct WgradArgs {
    const float* X;      // correlation input  [n][C_x][L_x]
    long x_bs;
    const float* G;      // grad rows (A side) [n][M][L_g]
    long g_bs;
    float* P;            // partials [split][M][NN]
    float* Pb;           // bias partials [split][M] (sum of G), or null
    int M, C_x, L_x, L_g, k, s, d, p;
    int NN;              // C_x * k
    int chunks_per_n, total_chunks, splits;
    int n_tiles, m_tiles;
    int XR;              // staged input rows per n-tile
    int span, segs;      // input-row staging: `span` positions as segs loads of up to 64
    int rs;              // LDS row stride of the staged input rows
    int blk4;            // P in row quads: [split][M / 4][NN][4] (M a multiple of 4)
};

// P[z, m, c*k + t] = sum over this split's positions l of
//   G[n, m, l] * X[n, c, l*s + t*d - p]
// (and Pb[z, m] = sum of G over the same positions, from the n-tile-0 blocks).
// 1-D grid of n_tiles * m_tiles * splits blocks. Both operands run along the
// position axis in memory, so they are staged row by row straight into LDS
// (buffer_load_dword ... lds, zero past each row's end): G as 128 rows of KC
// positions at an odd row stride, the input window as XR channel rows at a
// stride rs chosen so that column n = c*k + t lands on bank n*d.
template <bool S1, int WN>  // S1: stride 1 (the four input values of a group are adjacent)
__global__ __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(4)))
void wgrad_gemm(WgradArgs g) {
    extern __shared__ float smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, hi = lane >> 5;

    int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int nt = lid % g.n_tiles;
    lid /= g.n_tiles;
    const int mt = lid % g.m_tiles;
    const int z = lid / g.m_tiles;
    const int m0 = mt * BM;
    const int n0 = nt * (64 * WN);
    const int k = g.k, s = S1 ? 1 : g.s, d = g.d;
    const int ci_lo = n0 / k;
    const int gsz = 64 * GP;
    const int stage = gsz + (g.XR * g.rs + 63) / 64 * 64;  // as wgrad_layout
    const bool do_bias = g.Pb && nt == 0;
    // a wave whose 64 columns all lie past NN (the last n-tile) only stages
    const bool live = n0 + wn * 64 < g.NN;
    constexpr unsigned OOB = 0x80000000u;  // any offset >= the buffer size reads 0

    // this lane's two B columns: staged row offset of (c - ci_lo, t)
    int xcol[2];
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
        const int n = n0 + wn * 64 + tn * 32 + l32;
        const int c = n / k;
        xcol[tn] = (c - ci_lo) * g.rs + (n - c * k) * d;
    }
    const int g_row_lane = lane >> 5;      // 0: row m0 + i, 1: row m0 + i + 64
    const int g_pos_lane = lane & 31;

    // One buffer descriptor per utterance; rows, positions and channels out
    // of range get an out-of-bounds offset and stage as zeros. Wave w stages
    // G row pairs w, w + 8, ... and input rows w, w + 8, ... (all segments of
    // each), with the range checks skipped for chunks wholly inside.
    // Fast staging plan for chunks wholly inside their rows: per-lane byte
    // offsets at chunk position 0, fixed for the block, with the chunk's start
    // in the scalar offset, so one DMA costs one M0 write and the load. The
    // input window is staged packed: instruction j fills LDS floats
    // [64j, 64j + 64) of the [row][rs] window, lanes past a row's span (and
    // rows past C_x) read out of range and stage zeros.
    constexpr int GI = 64 / (2 * WN);  // G pair rows per wave
    const bool g_rows_in = m0 + BM <= g.M;  // uniform: whole m-tile (else the checked path)
    // pair row wave + 8j of this lane: g_off + j * 8 * L_g * 4
    const unsigned g_off = static_cast<unsigned>((m0 + wave + 64 * g_row_lane) * g.L_g + g_pos_lane) * 4u;
    const int g_step = 2 * WN * g.L_g * 4;
    // Stride 1: the wave's packed-instruction offsets are held (windows of up
    // to WG_XI * 8 * 64 floats; larger ones take the checked path). Strided:
    // this lane's slot of the wave's first instruction as (row, position),
    // each further instruction of the wave 8 * 64 slots on.
    const int nxi = (g.XR * g.rs + 63) / 64;  // packed-window instructions
    const bool fast_x = !S1 || nxi <= WG_XI * 2 * WN;  // uniform per launch
    unsigned x_off[S1 ? WG_XI : 1];
    if (S1) {
#pragma unroll
        for (int j = 0; j < WG_XI; ++j) {
            const int slot = (wave + 2 * WN * j) * 64 + lane;
            const int r = slot / g.rs, pos = slot - r * g.rs;
            const int c = ci_lo + r;
            x_off[S1 ? j : 0] = (r < g.XR && pos < g.span && c < g.C_x)
                                    ? static_cast<unsigned>(c * g.L_x + pos) * 4u : OOB;
        }
    }
    const int xs0 = wave * 64 + lane;
    const int xr0 = xs0 / g.rs, xp0 = xs0 - xr0 * g.rs;
    const int xqd = (2 * WN * 64) / g.rs, xrd = (2 * WN * 64) - xqd * g.rs;
    auto issue = [&](int ch, int sb) {
        const int b = ch / g.chunks_per_n;
        const int l0 = (ch - b * g.chunks_per_n) * KC;
        const __amdgpu_buffer_rsrc_t grs = uniform_rsrc(g.G + static_cast<long>(b) * g.g_bs, g.M * g.L_g * 4);
        const __amdgpu_buffer_rsrc_t xrs = uniform_rsrc(g.X + static_cast<long>(b) * g.x_bs, g.C_x * g.L_x * 4);
        const int x0 = l0 * s - g.p;
        if (S1 && fast_x && x0 >= 0 && x0 + g.span <= g.L_x) {  // uniform
#pragma unroll
            for (int j = 0; j < WG_XI; ++j)
                if (wave + 2 * WN * j < nxi)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, smem + sb + gsz + (wave + 2 * WN * j) * 64, 4,
                                                             static_cast<int>(x_off[S1 ? j : 0]), x0 * 4, 0, 0);
        } else if (!S1 && x0 >= 0 && x0 + g.span <= g.L_x) {  // uniform
            int r = xr0, pp = xp0;
            for (int jj = wave; jj < nxi; jj += 2 * WN) {
                const int c = ci_lo + r;
                const unsigned off = (r < g.XR && pp < g.span && c < g.C_x)
                                         ? static_cast<unsigned>(c * g.L_x + pp) * 4u : OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, smem + sb + gsz + jj * 64, 4, static_cast<int>(off),
                                                         x0 * 4, 0, 0);
                pp += xrd;
                r += xqd;
                if (pp >= g.rs) {
                    pp -= g.rs;
                    ++r;
                }
            }
        } else {
            const bool x_in = x0 >= 0 && x0 + g.span <= g.L_x;  // uniform
            for (int r = wave; r < g.XR; r += 2 * WN) {
                const int c = ci_lo + r;
                const bool c_in = c < g.C_x;  // uniform
                int pos = x0 + lane;
                for (int sg = 0; sg < g.segs; ++sg, pos += 64) {
                    const unsigned off = (c_in && (x_in || (pos >= 0 && pos < g.L_x)))
                                             ? static_cast<unsigned>(c * g.L_x + pos) * 4u : OOB;
                    if (sg * 64 + lane < g.span)  // exactly the row's span: rows pack at stride rs >= span
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, smem + sb + gsz + r * g.rs + sg * 64, 4,
                                                                 static_cast<int>(off), 0, 0, 0);
                }
            }
        }
        if (g_rows_in && l0 + KC <= g.L_g) {  // uniform
            // the row step rides in the scalar offset: one lane offset for all
#pragma unroll
            for (int j = 0; j < GI; ++j)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(grs, smem + sb + (wave + 2 * WN * j) * GP, 4,
                                                         static_cast<int>(g_off), l0 * 4 + j * g_step, 0, 0);
            return;
        }
        const int l = l0 + g_pos_lane;  // a partial m-tile or the last chunk of a row: checked
        for (int i = wave; i < 64; i += 2 * WN) {
            const int m = m0 + i + 64 * g_row_lane;
            const unsigned off = (m < g.M && l < g.L_g) ? static_cast<unsigned>(m * g.L_g + l) * 4u : OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(grs, smem + sb + i * GP, 4, static_cast<int>(off), 0, 0, 0);
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    double bsum = 0.0;

    // split z: chunks [z * total / splits, (z + 1) * total / splits)
    const int ch0 = static_cast<int>(static_cast<long>(z) * g.total_chunks / g.splits);
    const int ch1 = static_cast<int>(static_cast<long>(z + 1) * g.total_chunks / g.splits);
    if (ch0 < ch1) issue(ch0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int ch = ch0; ch < ch1; ++ch) {
        const int sb = ((ch - ch0) & 1) * stage;
        __builtin_amdgcn_s_setprio(1);  // as in conv_gemm_q
        if (ch + 1 < ch1) issue(ch + 1, stage - sb);
        __builtin_amdgcn_s_setprio(0);
        if (do_bias && tid < BM) {
            float t = 0.0f;
            const int row = sb + (tid & 63) * GP + (tid >> 6) * KC;
            for (int kc = 0; kc < KC; ++kc) t += smem[row + kc];
            bsum += t;
        }
        // group gi covers positions l0 + 8*gi + 4*h + e (e = 0..3) for lanes of
        // half h: one ds_read_b128 per A row, four adjacent (stride s) input
        // values per B column, then 16 MFMAs
        const int ga = sb + l32 * GP + wm * KC + hi * 4;
        const int xa0 = sb + gsz + xcol[0] + hi * 4 * s;
        const int xa1 = sb + gsz + xcol[1] + hi * 4 * s;
        auto ld = [&](int gi, float4 (&a)[2], float (&bv)[2][4]) {
            gi = min(gi, KC / 8 - 1);
            int go = ga + gi * 8;
            int xo0 = xa0 + gi * 8 * s;
            int xo1 = xa1 + gi * 8 * s;
            asm volatile("" : "+v"(go), "+v"(xo0), "+v"(xo1));
            a[0] = *reinterpret_cast<const float4*>(smem + go);
            a[1] = *reinterpret_cast<const float4*>(smem + go + 32 * GP);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bv[0][e] = smem[xo0 + e * s];
                bv[1][e] = smem[xo1 + e * s];
            }
        };
        auto mm = [&](const float4 (&a)[2], const float (&bv)[2][4]) {
            const float a0[4] = {a[0].x, a[0].y, a[0].z, a[0].w};
            const float a1[4] = {a[1].x, a[1].y, a[1].z, a[1].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], bv[0][e], acc[0][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], bv[1][e], acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], bv[0][e], acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], bv[1][e], acc[1][1], 0, 0, 0);
            }
        };
        if (live) {
            constexpr int NR = S1 ? 6 : 10;  // LDS reads per group
            float4 pa[2], qa[2];
            float pb[2][4], qb[2][4];
            ld(0, pa, pb);
#pragma unroll
            for (int gi = 0; gi < KC / 8; gi += 2) {
                ld(gi + 1, qa, qb);
                mm(pa, pb);
                ld(gi + 2, pa, pb);
                mm(qa, qb);
                // (1 MFMA, 1 read) x NR, then the group's other MFMAs; twice
                for (int r = 0; r < 2; ++r) {
                    for (int i = 0; i < NR; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    }
                    __builtin_amdgcn_sched_group_barrier(0x008, 16 - NR, 0);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's staging loads landed
        __syncthreads();
    }

    float* Pz = g.P + static_cast<long>(z) * g.M * g.NN;
    if (g.blk4) {  // uniform: a lane's four consecutive rows of a column as one 16-byte store
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int n = n0 + wn * 64 + tn * 32 + l32;
            if (n >= g.NN) continue;
#pragma unroll
            for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int m = m0 + wm * 64 + tm * 32 + 8 * j + 4 * hi;  // a multiple of 4
                    if (m < g.M)
                        reinterpret_cast<float4*>(Pz)[static_cast<long>(m >> 2) * g.NN + n] =
                            make_float4(acc[tm][tn][4 * j], acc[tm][tn][4 * j + 1], acc[tm][tn][4 * j + 2],
                                        acc[tm][tn][4 * j + 3]);
                }
        }
    } else {
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int n = n0 + wn * 64 + tn * 32 + l32;
            if (n >= g.NN) continue;
#pragma unroll
            for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = m0 + wm * 64 + tm * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
                    if (m < g.M) Pz[static_cast<long>(m) * g.NN + n] = acc[tm][tn][e];
                }
        }
    }
    if (do_bias && tid < BM && m0 + tid < g.M)
        g.Pb[static_cast<long>(z) * g.M + m0 + tid] = static_cast<float>(bsum);
}

// db[m] += sum_y part[y*M + m] (one wave per row, four rows per 256-thread
// block `blk`; double sums in a fixed lane order)
__device__ inline void bias_rows(const float* part, float* db, int M, int S, int blk) {
    const int m = blk * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (m >= M) return;
    double acc = 0.0;
    for (int y = lane; y < S; y += 64) acc += part[static_cast<long>(y) * M + m];
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_down(acc, o, 64);
    if (lane == 0) db[m] += static_cast<float>(acc);
}

// out[i] += sum_z P[z][i] over the splits z, for V-float columns i (V = 4:
// 16-byte accesses, MN a multiple of 4 and both arrays 16-B aligned; BLK:
// the partials in the row-quad layout the GEMM stores 16 bytes at a time,
// each column's four sums added to four rows of out). A
// 256-thread block takes 256 / ZG columns and ZG split groups: thread (q, c)
// sums its group's contiguous range of z in order, eight loads in flight
// (each issued unconditionally from a clamped z, only its use bounded), and
// the groups' sums are added in group order. The stage-1 weight grads have
// hundreds of splits over a few thousand columns: the split groups turn one
// long chain of memory round trips per column into ZG shorter ones. Blocks at
// and past `main_blocks` (when Pb is given) sum the bias partials
// Pb[splits][M] into db instead, as bias_reduce would.
template <int V, int ZG, bool BLK = false>
__global__ __launch_bounds__(256) void wgrad_reduce(const float* P, float* out, long MN, int splits, int M,
                                                    const float* Pb, float* db, unsigned main_blocks) {
    if (blockIdx.x >= main_blocks) {
        bias_rows(Pb, db, M, splits, static_cast<int>(blockIdx.x - main_blocks));
        return;
    }
    using T = typename std::conditional<V == 4, float4, float>::type;
    constexpr int CW = 256 / ZG;
    const T* Pv = reinterpret_cast<const T*>(P);
    T* ov = reinterpret_cast<T*>(out);
    const long MV = MN / V;
    const int c = threadIdx.x % CW, q = threadIdx.x / CW;
    const long i = static_cast<long>(blockIdx.x) * CW + c;
    const long ic = i < MV ? i : MV - 1;
    const int z0 = static_cast<int>(static_cast<long>(q) * splits / ZG);
    const int z1 = static_cast<int>(static_cast<long>(q + 1) * splits / ZG);
    T acc{};
    for (int z = z0; z < z1; z += 8) {
        T v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = Pv[min(z + j, z1 - 1) * MV + ic];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (z + j < z1) acc += v[j];
    }
    // BLK: P in row quads, column i = (m / 4) * NN + n holds rows m .. m + 3
    auto put = [&](const T& t) {
        if constexpr (BLK) {
            const long NN = MN / M;
            const long mq = i / NN, n = i - mq * NN;
            float* o = out + 4 * mq * NN + n;
            o[0] += t.x;
            o[NN] += t.y;
            o[2 * NN] += t.z;
            o[3 * NN] += t.w;
        } else {
            ov[i] += t;
        }
    };
    if constexpr (ZG == 1) {
        if (i < MV) put(acc);
    } else {
        __shared__ T red[ZG][CW];
        red[q][c] = acc;
        __syncthreads();
        if (q == 0 && i < MV) {
            T t = red[0][c];
#pragma unroll
            for (int g = 1; g < ZG; ++g) t += red[g][c];
            put(t);
        }
    }
}

// part[y, m] = sum of G[n, m, l] over every utterance n and the y-th slice
// [y*per, (y+1)*per) of the positions; grid (M, S). Each thread walks its
// positions of each row with a fixed stride (no per-element index division)
// and the block sums the thread partials in a fixed tree; bias_reduce then
// adds the slices in order.
// V = 4: rows of a multiple of 4 floats on a 16-B aligned base and slices of
// a multiple of 4 positions, read as float4.
template <int V>
__global__ void bias_partial(const float* G, long g_bs, float* part, int N, int M, int L, int per) {
    const int m = blockIdx.x, y = blockIdx.y;
    const int l0 = y * per, l1 = min(L, l0 + per);
    double acc = 0.0;
    for (int n = 0; n < N; ++n) {
        const float* row = G + n * g_bs + static_cast<long>(m) * L;
        float t = 0.0f;
        if constexpr (V == 4) {
            const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll 4
            for (int l = l0 / 4 + threadIdx.x; l < l1 / 4; l += blockDim.x) {
                const float4 q = r4[l];
                t += (q.x + q.y) + (q.z + q.w);
            }
        } else {
#pragma unroll 8
            for (int l = l0 + threadIdx.x; l < l1; l += blockDim.x) t += row[l];
        }
        acc += t;
    }
    __shared__ double red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[static_cast<long>(y) * M + m] = static_cast<float>(red[0]);
}

// db[m] += sum over (n, l) of G[n, m, l] in one pass for rows of at most
// 128 K positions over all utterances: one 1024-thread block per row m;
// thread i sums, in float and in order, the vectors i, i + 1024, ... of the
// row's N * L / V (V = 4: float4 on 16-B aligned rows of a multiple of 4
// floats), eight loads in flight (each issued unconditionally from a clamped
// index, only its use is bounded), and the block adds the thread sums in
// double in a fixed tree.
template <int V>
__global__ __launch_bounds__(1024) void bias_rows_direct(const float* G, long g_bs, float* db, int N, int L) {
    const int m = blockIdx.x;
    const int Lv = L / V;
    const int tot = N * Lv;
    float acc = 0.0f;
    for (int f0 = threadIdx.x; f0 < tot; f0 += 8 * 1024) {
        float v[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int f = min(f0 + s * 1024, tot - 1);
            const int n = f / Lv, l = f - n * Lv;
            const float* row = G + n * g_bs + static_cast<long>(m) * L;
            if constexpr (V == 4) {
                const float4 q = reinterpret_cast<const float4*>(row)[l];
                v[s] = (q.x + q.y) + (q.z + q.w);
            } else {
                v[s] = row[l];
            }
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
            if (f0 + s * 1024 < tot) acc += v[s];
    }
    double d = acc;
    for (int o = 32; o > 0; o >>= 1) d += __shfl_down(d, o, 64);
    __shared__ double wsum[16];
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = d;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < 16; ++w) t += wsum[w];
        db[m] += static_cast<float>(t);
    }
}

// db[m] += sum_y part[y, m]: one wave per m; lane j sums y = j, j+64, ... in
// order, then a fixed shuffle tree adds the 64 lane sums.
__global__ void bias_reduce(const float* part, float* db, int M, int S) {
    bias_rows(part, db, M, S, static_cast<int>(blockIdx.x));
}

// ─── depthwise pool: ConvTranspose1d k3 s2 p1 op1, groups = C ──────────────
// y[2m] = b + W1 x[m];  y[2m+1] = b + W0 x[m+1] + W2 x[m]
__global__ void pool_fwd(const float* X, long x_bs, const float* W, const float* bias,
                         float* Y, long y_bs, int C, int L) {
    const int row = blockIdx.y;  // n*C + c
    const int n = row / C, c = row - n * C;
    const float* x = X + n * x_bs + static_cast<long>(c) * L;
    float* y = Y + n * y_bs + static_cast<long>(c) * 2 * L;
    const float w0 = W[c * 3], w1 = W[c * 3 + 1], w2 = W[c * 3 + 2];
    const float bb = bias ? bias[c] : 0.0f;
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < 2 * L; j += gridDim.x * blockDim.x) {
        const int m = j >> 1;
        float v;
        if ((j & 1) == 0) v = w1 * x[m];
        else v = w2 * x[m] + (m + 1 < L ? w0 * x[m + 1] : 0.0f);
        y[j] = v + bb;
    }
}

// dx[l] = W0 dy[2l-1] + W1 dy[2l] + W2 dy[2l+1]
__global__ void pool_dgrad(const float* W, const float* dY, long dy_bs, float* dX,
                           long dx_bs, int C, int L) {
    const int row = blockIdx.y;
    const int n = row / C, c = row - n * C;
    const float* dy = dY + n * dy_bs + static_cast<long>(c) * 2 * L;
    float* dx = dX + n * dx_bs + static_cast<long>(c) * L;
    const float w0 = W[c * 3], w1 = W[c * 3 + 1], w2 = W[c * 3 + 2];
    for (int l = blockIdx.x * blockDim.x + threadIdx.x; l < L; l += gridDim.x * blockDim.x) {
        float v = w1 * dy[2 * l] + w2 * dy[2 * l + 1];
        if (l > 0) v += w0 * dy[2 * l - 1];
        dx[l] = v;
    }
}

// dW[c][t] += sum_{n,l} x[l] dy[2l + t - 1];  db[c] += sum dy. Block per c.
__global__ void pool_wgrad(const float* X, long x_bs, const float* dY, long dy_bs,
                           float* dW, float* db, int N, int C, int L) {
    const int c = blockIdx.x;
    double a0 = 0, a1 = 0, a2 = 0, ab = 0;
    for (int n = 0; n < N; ++n) {
        const float* x = X + n * x_bs + static_cast<long>(c) * L;
        const float* dy = dY + n * dy_bs + static_cast<long>(c) * 2 * L;
        for (int l = threadIdx.x; l < L; l += blockDim.x) {
            const double xv = x[l];
            if (l > 0) a0 += xv * dy[2 * l - 1];
            a1 += xv * dy[2 * l];
            a2 += xv * dy[2 * l + 1];
            ab += static_cast<double>(dy[2 * l]) + dy[2 * l + 1];
        }
    }
    __shared__ double red[4][256];
    red[0][threadIdx.x] = a0;
    red[1][threadIdx.x] = a1;
    red[2][threadIdx.x] = a2;
    red[3][threadIdx.x] = ab;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w)
            for (int q = 0; q < 4; ++q) red[q][threadIdx.x] += red[q][threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        dW[c * 3 + 0] += static_cast<float>(red[0][0]);
        dW[c * 3 + 1] += static_cast<float>(red[1][0]);
        dW[c * 3 + 2] += static_cast<float>(red[2][0]);
        if (db) db[c] += static_cast<float>(red[3][0]);
    }
}

// LDS bytes of one conv_gemm block (two stages) for chunk CK and an effective
// correlation of kk taps at stride ss and dilation dd.
size_t conv_lds_bytes(int CK, int kk, int ss, int dd) {
    const long span = static_cast<long>(BN - 1) * ss + static_cast<long>(kk - 1) * dd + 1;
    const long span_p = (span + 3 + 255) / 256 * 256;  // as conv_gemm
    return 2 * (static_cast<size_t>(CK) * kk * BM + static_cast<size_t>(CK) * span_p) * sizeof(float);
}

// LDS bytes of one conv_gemm_q block (two stages): the chunk's weight quads
// and its CK input rows.
size_t quad_lds_bytes(int CK, int k, int d) {
    const long S = static_cast<long>(CK) * k / 2, Q = (S + 3) / 4;
    const long span = BN + static_cast<long>(k - 1) * d;
    const long span_p = (span + 3 + 255) / 256 * 256;
    return 2 * (static_cast<size_t>(Q) * 1024 + static_cast<size_t>(CK) * span_p) * sizeof(float);
}

#ifndef CGQ_CK3
#define CGQ_CK3 8
#endif
#ifndef CGQ_CK7
#define CGQ_CK7 4
#endif
#ifndef CGQ_CK11
#define CGQ_CK11 2
#endif
// Channel chunk of conv_gemm_q for a k-tap stride-1 correlation, or 0 where
// no instance exists (conv_gemm serves those).
int pick_ck_q(int k) {
    switch (k) {
        case 3: return CGQ_CK3;
        case 7: return CGQ_CK7;
        case 11: return CGQ_CK11;
        default: return 0;
    }
}

template <int CK, int KT, int EPI>
const void* conv_q_kernel() {
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_gemm_q<CK, KT, EPI>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    return reinterpret_cast<const void*>(&conv_gemm_q<CK, KT, EPI>);
}

template <int CK, int KT>
const void* conv_q_kernel_epi(int epi) {
    if (epi == QEPI_ADAIN_BWD) return conv_q_kernel<CK, KT, QEPI_ADAIN_BWD>();
    if (epi == QEPI_STATS) return conv_q_kernel<CK, KT, QEPI_STATS>();
    return conv_q_kernel<CK, KT, QEPI_STORE>();
}

const void* conv_q_kernel_for(int CK, int k, int epi) {
    if (k == 3 && CK == CGQ_CK3) return conv_q_kernel_epi<CGQ_CK3, 3>(epi);
    if (k == 7 && CK == CGQ_CK7) return conv_q_kernel_epi<CGQ_CK7, 7>(epi);
    if (k == 11 && CK == CGQ_CK11) return conv_q_kernel_epi<CGQ_CK11, 11>(epi);
    return nullptr;
}

// Input channels per K chunk: a power of two in [2, 32] so that it divides
// the 32-padded channel count of the packed weights (no chunk runs past them),
// at most 32 weight rows (CK*k) per chunk, and the largest such chunk whose two
// stages fit 32 KB of LDS, well inside the 40 KB per block that four blocks
// per CU (the kernel's 128-VGPR budget) leave. Only when even CK = 2 is larger
// does the stage size set occupancy.
int pick_ck(int k, int s, int d) {
    int ck = 32;
    while (ck > 2 && (ck * k > 32 || conv_lds_bytes(ck, k, s, d) > 32 * 1024)) ck >>= 1;
    return ck;
}

int grid1d(long n) {
    long g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    if (g < 1) g = 1;
    return static_cast<int>(g);
}

template <int CK>
const void* conv_kernel() {
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_gemm<CK>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    return reinterpret_cast<const void*>(&conv_gemm<CK>);
}

const void* conv_kernel_for(int CK) {
    switch (CK) {
        case 2: return conv_kernel<2>();
        case 4: return conv_kernel<4>();
        case 8: return conv_kernel<8>();
        case 16: return conv_kernel<16>();
        case 32: return conv_kernel<32>();
        default: return nullptr;
    }
}

// Resident blocks per CU of GEMM kernel `kern` with `lds` bytes (cached).
int blocks_per_cu(const void* kern, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void*, size_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(kern, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, NT, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    cache[key] = per_cu;
    return per_cu;
}

const void* corr_kernel() {
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&corr_gemm),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    return reinterpret_cast<const void*>(&corr_gemm);
}

// Octet-mode geometry for a stride-1 correlation of k taps at dilation d
// over C channels: chunks of up to 4 taps (three for k = 3), the staged
// window of a 4-tap chunk rounded to 16 positions.
void octet_setup(GemmArgs& g, int C, int k, int d) {
    g.G = k < 4 ? k : 4;
    g.n_tg = static_cast<int>(cdiv(k, g.G));
    g.span8 = static_cast<int>(cdiv(BN + (g.G - 1) * d, 16) * 16);
    g.n_oct = static_cast<int>(cdiv(C, 8));
    g.cin_pad = g.n_oct * 8;
    g.CK = 0;
}

// K chunking for a stride-1 correlation over C channels, kk taps at dilation
// dd, `tiles` output tiles. corr_gemm (octet chunks, 16-B operand reads) is
// the faster kernel where the grid is smaller than one round of conv_gemm's
// resident blocks (where conv_gemm would need a split plan); on larger grids
// conv_gemm is (the decoder's transposed-conv forwards: 1.23 vs 1.30 ms per
// step with corr_gemm).
void choose_chunks(kdec_ctx* ctx, GemmArgs& g, int C, int kk, int dd, long tiles) {
    const int ck = pick_ck(kk, 1, dd);
    const long slots = static_cast<long>(blocks_per_cu(conv_kernel_for(ck), conv_lds_bytes(ck, kk, 1, dd))) *
                       ctx->num_cus;
    if (tiles < slots) {
        octet_setup(g, C, kk, dd);
        return;
    }
    g.G = 0;
    g.CK = ck;
    g.cin_pad = static_cast<int>(cdiv(C, 32) * 32);
}

// Launches conv_gemm over an already packed A.
//
// Work plan: with S resident blocks, T tiles take T / S whole rounds plus a
// last round of r = T mod S tiles. When r is well below S, the last r tiles
// (in logical order) are split over their channel chunks into f parts,
// f <= S / r, so that the last round costs about 1/f of a tile instead of a
// whole one; their partial sums are reduced by tile_reduce.
int run_gemm(kdec_ctx* ctx, GemmArgs g, int N, int m_tiles, const char* fam,
             double flops) {
    const int CK = g.CK;
    const bool octet = g.G > 0;
    const int kk = g.n_phase > 1 ? g.ph_kt : g.k;
    const int ss = g.n_phase > 1 ? 1 : g.s;
    const int dd = g.n_phase > 1 ? 1 : g.d;
    if (octet ? (ss != 1 || g.G > kk || g.span8 < BN + (g.G - 1) * dd || g.span8 % 16)
              : (CK * kk > 64 || (CK * kk) % 2))
        return fail(ctx, KDEC_EINVAL, "conv: bad chunk geometry");
    const bool quad = g.quad != 0;
    const int epi = g.ad.part ? QEPI_ADAIN_BWD : g.fs.part ? QEPI_STATS : QEPI_STORE;
    if (!quad && epi != QEPI_STORE) return fail(ctx, KDEC_EINVAL, "conv: fused epilogue needs the quad kernel");
    if (quad && (octet || g.n_phase > 1 || g.s != 1 || !conv_q_kernel_for(CK, g.k, epi)))
        return fail(ctx, KDEC_EINVAL, "conv: bad quad geometry");
    size_t lds = octet ? 2 * (static_cast<size_t>(g.G) * 1024 + 8 * static_cast<size_t>(g.span8)) * sizeof(float)
               : quad ? quad_lds_bytes(CK, g.k, g.d)
                      : conv_lds_bytes(CK, kk, ss, dd);
    if (static_cast<long>(g.C_in) * g.L_in * 4 > 0x7fffffffL)
        return fail(ctx, KDEC_EINVAL, "conv: input too large for one buffer descriptor");
    g.ybuf = (static_cast<long>(g.C_out) + BM) * g.L_y * 4 < 0x7fffffffL ? 1 : 0;
    const void* kern = octet ? corr_kernel() : quad ? conv_q_kernel_for(CK, g.k, epi) : conv_kernel_for(CK);
    if (!kern) return fail(ctx, KDEC_EINVAL, "conv: unsupported channel chunk");
    // conv_gemm with one LDS stage where two leave at most two blocks per CU
    // and one leaves more (the long windows of large strides)
    g.single = 0;
    if (!octet && !quad && blocks_per_cu(kern, lds) <= 2 && blocks_per_cu(kern, lds / 2) > blocks_per_cu(kern, lds)) {
        g.single = 1;
        lds /= 2;
    }
    if (lds > 160 * 1024) return fail(ctx, KDEC_EINVAL, "conv: tile does not fit LDS");
    int max_q = g.n_q;
    if (g.n_phase > 1) max_q = static_cast<int>(cdiv(g.L_y + g.ph_s, g.ph_s)) + 1;
    g.m_tiles = m_tiles;
    g.q_tiles = static_cast<int>(cdiv(max_q, BN));
    g.nz = N * g.n_phase;
    const long tiles = static_cast<long>(g.m_tiles) * g.q_tiles * g.nz;
    if (tiles > 0x7fffffffL / 16) return fail(ctx, KDEC_EINVAL, "conv: grid too large");
    const long slots = static_cast<long>(blocks_per_cu(kern, lds)) * ctx->num_cus;
    const int nchunks = octet ? g.n_oct * g.n_tg : g.cin_pad / CK;
    const long rem = tiles % slots;
    long f = 1;
    if (rem > 0) f = std::min(std::min(slots / rem, static_cast<long>(nchunks / 4)), 16L);
    if (f < 2) f = 1;
    g.fsplit = static_cast<int>(f);
    g.split_tiles = f > 1 ? static_cast<int>(rem) : 0;
    g.full_tiles = static_cast<int>(tiles - g.split_tiles);
    g.full_per_xcd = static_cast<int>(cdiv(g.full_tiles, 8));
    g.parts_per_xcd = static_cast<int>(cdiv(static_cast<long>(g.split_tiles) * g.fsplit, 8));
    const long blocks = 8L * (g.full_per_xcd + g.parts_per_xcd);
    Workspace part(ctx, static_cast<size_t>(g.split_tiles) * g.fsplit * BM * BN * sizeof(float));
    if (g.split_tiles > 0) {
        if (!part.p) return KDEC_ENOMEM;
        g.P = part.as<float>();
    }
    // algorithmic HBM bytes: input and weights read once, output written once
    // (read too when accumulating), residual read once
    const int kk_all = g.n_phase > 1 ? g.ph_kt * g.n_phase : g.k;
    double bytes = 4.0 * (static_cast<double>(N) * g.C_in * g.L_in + static_cast<double>(g.C_in) * kk_all * g.C_out +
                          static_cast<double>(N) * g.C_out * g.L_y * (g.beta != 0.0f ? 2 : 1));
    if (g.R) bytes += 4.0 * static_cast<double>(N) * g.C_out * g.L_y;
    // fused epilogues: the AdaIN backward reads the normalised layer's input
    // x; both write (count / sum, mean / sum, m2) slot records per row
    if (g.ad.part) bytes += 4.0 * static_cast<double>(N) * g.C_out * g.L_y;
    if (g.ad.part || g.fs.part)
        bytes += 24.0 * static_cast<double>(N) * g.C_out * (g.ad.part ? g.ad.nch : g.fs.nch);
    {  // the GEMM kernel alone (the profile's FLOP rate is this launch's)
        ProfScope ps(ctx, fam, flops, bytes);
        void* args[] = {&g};
        if (hipLaunchKernel(kern, dim3(static_cast<unsigned>(blocks)), dim3(NT), args, lds, ctx->stream) !=
            hipSuccess)
            return fail(ctx, KDEC_EHIP, std::string(fam) + ": launch failed");
        if (int rc = launch_check(ctx, fam)) return rc;
    }
    if (g.split_tiles > 0) {
        ProfScope ps(ctx, "tile_reduce", 0.0);
        if (g.ad.part)
            hipLaunchKernelGGL(tile_reduce_adain, dim3(BM * BN / 1024, g.split_tiles), dim3(256), 0, ctx->stream, g);
        else if (g.fs.part)
            hipLaunchKernelGGL(tile_reduce_stats, dim3(BM * BN / 1024, g.split_tiles), dim3(256), 0, ctx->stream, g);
        else
            hipLaunchKernelGGL(tile_reduce, dim3(BM * BN / 1024, g.split_tiles), dim3(256), 0, ctx->stream, g);
        return launch_check(ctx, "tile_reduce");
    }
    return KDEC_OK;
}

}  // namespace
}  // namespace kdec

using namespace kdec;

extern "C" {

}  // extern "C"

namespace kdec {
namespace {
// The conv1d forward; with `part` (only where the GEMM runs conv_gemm_q and
// beta = 0) its epilogue also writes the output rows' statistics records
// (2 * q_tiles slots per row, see store_tile_stats).
int conv_fwd_impl(kdec_ctx* ctx, const float* X, long x_bs, const float* W, const float* bias, float* Y, long y_bs,
                  int N, int C_in, int L, int C_out, int k, int stride, int pad, int dil, const float* R, long r_bs,
                  float scale, float beta, double* part, int nch) {
    KDEC_CHECK(ctx, X && W && Y && N > 0 && C_in > 0 && C_out > 0 && k > 0 && stride > 0 && dil > 0 && pad >= 0,
               "kdec_conv1d_fwd: bad arguments");
    const int L_out = (L + 2 * pad - dil * (k - 1) - 1) / stride + 1;
    KDEC_CHECK(ctx, L > 0 && L_out > 0, "kdec_conv1d_fwd: empty output");
    KDEC_CHECK(ctx, x_bs >= static_cast<long>(C_in) * L && y_bs >= static_cast<long>(C_out) * L_out,
               "kdec_conv1d_fwd: batch stride too small");
    const int m_pad = static_cast<int>(cdiv(C_out, BM) * BM);
    GemmArgs g{};
    g.X = X; g.x_bs = x_bs; g.a_phase_stride = 0;
    g.bias = bias; g.Y = Y; g.y_bs = y_bs; g.R = R; g.r_bs = r_bs;
    g.C_in = C_in; g.L_in = L; g.C_out = C_out; g.L_y = L_out;
    g.m_pad = m_pad;
    g.k = k; g.s = stride; g.d = dil; g.p = pad; g.n_q = L_out;
    g.scale = scale; g.beta = beta; g.n_phase = 1;
    if (stride == 1) {
        choose_chunks(ctx, g, C_in, k, dil, cdiv(C_out, BM) * cdiv(L_out, BN) * N);
        if (g.G == 0 && pick_ck_q(k) > 0) {
            g.quad = 1;
            g.CK = pick_ck_q(k);
        }
    } else {
        g.CK = pick_ck(k, stride, dil);
        g.cin_pad = static_cast<int>(cdiv(C_in, 32) * 32);
    }
    if (part) {
        if (!g.quad || beta != 0.0f) return fail(ctx, KDEC_EINVAL, "conv forward: no statistics epilogue here");
        g.fs.part = part;
        g.fs.nch = nch;
    }
    const int nq = static_cast<int>(cdiv(static_cast<long>(g.CK) * k / 2, 4));
    const long tot = g.quad ? (m_pad / BM) * static_cast<long>(g.cin_pad / g.CK) * nq * 1024
                            : static_cast<long>(g.cin_pad) * k * m_pad;
    Workspace A(ctx, static_cast<size_t>(tot) * sizeof(float));
    if (!A.p) return KDEC_ENOMEM;
    g.A = A.as<float>();
    KDEC_CHECK(ctx, tot <= 0x7fffffffL && static_cast<long>(C_out) * C_in * k <= 0x7fffffffL,
               "kdec_conv1d_fwd: weights too large");
    if (g.quad)
        hipLaunchKernelGGL(pack_quad, dim3(grid1d(tot / 4)), dim3(256), 0, ctx->stream, W, A.as<float>(), 0, C_in,
                           C_out, k, g.CK, g.cin_pad / g.CK, nq, tot / 4);
    else if (g.G > 0)
        hipLaunchKernelGGL(pack_octet, dim3(grid1d(tot)), dim3(256), 0, ctx->stream, W, A.as<float>(), 0, C_in,
                           C_out, k, 1, k, m_pad, static_cast<int>(tot), 1);
    else
        if (g.cin_pad % g.CK == 0 && m_pad % 32 == 0)
            hipLaunchKernelGGL(pack_rows_t, dim3(static_cast<unsigned>(cdiv(static_cast<long>(g.cin_pad) * k, 32)),
                                                 static_cast<unsigned>(m_pad / 32)),
                               dim3(256), 0, ctx->stream, W, A.as<float>(), C_out, C_in, k, g.cin_pad, m_pad, g.CK);
        else
            hipLaunchKernelGGL(pack_fwd, dim3(grid1d(tot)), dim3(256), 0, ctx->stream, W, A.as<float>(), C_in,
                               C_out, k, g.cin_pad, m_pad, g.CK);
    if (int rc = launch_check(ctx, "pack_fwd")) return rc;
    return run_gemm(ctx, g, N, m_pad / BM, "conv_fwd",
                    2.0 * N * C_out * static_cast<double>(L_out) * C_in * k);
}


// Whether a forward conv of this geometry runs conv_gemm_q.
bool fwd_is_quad(kdec_ctx* ctx, int N, int C_in, int L, int C_out, int k, int dil) {
    if (pick_ck_q(k) <= 0) return false;
    GemmArgs g{};
    choose_chunks(ctx, g, C_in, k, dil, cdiv(C_out, BM) * cdiv(L, BN) * N);
    return g.G == 0;
}
}  // namespace
}  // namespace kdec

extern "C" {

int kdec_conv1d_fwd(kdec_ctx* ctx, const float* X, long x_bs, const float* W,
                    const float* bias, float* Y, long y_bs, int N, int C_in,
                    int L, int C_out, int k, int stride, int pad, int dil,
                    const float* R, long r_bs, float scale, float beta) {
    if (!ctx) return KDEC_EINVAL;
    return conv_fwd_impl(ctx, X, x_bs, W, bias, Y, y_bs, N, C_in, L, C_out, k, stride, pad, dil, R, r_bs, scale,
                         beta, nullptr, 0);
}

int kdec_conv1d_fwd_stats_fused(kdec_ctx* ctx, int N, int C_in, int L, int C_out, int k, int stride, int pad,
                                int dil) {
    if (!ctx || N <= 0 || C_in <= 0 || C_out <= 0 || k <= 0 || stride <= 0 || dil <= 0 || L <= 0) return 0;
    const int L_out = (L + 2 * pad - dil * (k - 1) - 1) / stride + 1;
    return stride == 1 && L_out == L && (static_cast<long>(C_out) + BM) * L_out * 4 < 0x7fffffffL &&
           fwd_is_quad(ctx, N, C_in, L, C_out, k, dil);
}

int kdec_conv1d_fwd_stats(kdec_ctx* ctx, const float* X, long x_bs, const float* W,
                          const float* bias, float* Y, long y_bs, int N, int C_in,
                          int L, int C_out, int k, int stride, int pad, int dil,
                          const float* R, long r_bs, float scale, float eps, float* stats) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, stats && Y && N > 0 && C_out > 0, "kdec_conv1d_fwd_stats: bad arguments");
    const int L_out = (L + 2 * pad - dil * (k - 1) - 1) / stride + 1;
    if (!kdec_conv1d_fwd_stats_fused(ctx, N, C_in, L, C_out, k, stride, pad, dil)) {
        if (int rc = kdec_conv1d_fwd(ctx, X, x_bs, W, bias, Y, y_bs, N, C_in, L, C_out, k, stride, pad, dil, R, r_bs,
                                     scale, 0.0f))
            return rc;
        return kdec_instnorm_stats(ctx, Y, y_bs, N, C_out, L_out, eps, stats);
    }
    const int nch = 2 * static_cast<int>(cdiv(L_out, BN));
    Workspace part(ctx, static_cast<size_t>(N) * C_out * nch * 3 * sizeof(double));
    if (!part.p) return KDEC_ENOMEM;
    if (int rc = conv_fwd_impl(ctx, X, x_bs, W, bias, Y, y_bs, N, C_in, L, C_out, k, stride, pad, dil, R, r_bs, scale,
                               0.0f, part.as<double>(), nch))
        return rc;
    ProfScope ps(ctx, "adain_fwd", 0, 0.0);
    hipLaunchKernelGGL(instnorm_fin_slots_k, dim3(static_cast<unsigned>(N * C_out)), dim3(64), 0, ctx->stream,
                       part.as<double>(), nch, eps, reinterpret_cast<float2*>(stats));
    return launch_check(ctx, "instnorm_fin_slots");
}

}  // extern "C"

namespace kdec {
namespace {
// Per-call inputs of the AdaIN backward epilogue of an input-grad GEMM.
struct AdainBwdIn {
    const float* X;
    long x_bs;
    const float* stats;
    const float* gamma;
    const float* beta;
    long gb_bs;
    int act;
    float slope;
    const float* alpha;
};

// Whether an input-grad GEMM of this geometry runs conv_gemm_q (whose
// epilogue, and tile_reduce_adain's, can apply an AdaIN backward).
bool dgrad_is_quad(kdec_ctx* ctx, int N, int C_in, int L, int C_out, int k, int dil) {
    if (pick_ck_q(k) <= 0) return false;
    GemmArgs g{};
    choose_chunks(ctx, g, C_out, k, dil, cdiv(C_in, BM) * cdiv(L, BN) * N);
    return g.G == 0;
}

// The input grad as a correlation of dY with the flipped weights; with `ad`
// (only where dgrad_is_quad) dX receives ds = dX * act'(s) of that AdaIN and
// `part` its row partial sums (2 * q_tiles slots per row).
int conv_dgrad_impl(kdec_ctx* ctx, const float* W, const float* dY, long dy_bs, float* dX, long dx_bs, int N,
                    int C_in, int L, int C_out, int k, int stride, int pad, int dil, float scale, float beta,
                    const AdainBwdIn* ad, double* part, int nch) {
    KDEC_CHECK(ctx, W && dY && dX && N > 0 && C_in > 0 && C_out > 0 && k > 0 && dil > 0 && pad >= 0,
               "kdec_conv1d_dgrad: bad arguments");
    KDEC_CHECK(ctx, stride == 1, "kdec_conv1d_dgrad: only stride 1 is on the decoder path");
    const int L_out = L + 2 * pad - dil * (k - 1);
    KDEC_CHECK(ctx, L > 0 && L_out > 0, "kdec_conv1d_dgrad: empty output");
    const int pp = dil * (k - 1) - pad;
    KDEC_CHECK(ctx, pp >= 0, "kdec_conv1d_dgrad: padding larger than the receptive field");
    KDEC_CHECK(ctx, dy_bs >= static_cast<long>(C_out) * L_out && dx_bs >= static_cast<long>(C_in) * L,
               "kdec_conv1d_dgrad: batch stride too small");
    const int m_pad = static_cast<int>(cdiv(C_in, BM) * BM);
    GemmArgs g{};
    g.X = dY; g.x_bs = dy_bs;
    g.Y = dX; g.y_bs = dx_bs;
    g.C_in = C_out; g.L_in = L_out; g.C_out = C_in; g.L_y = L;
    g.m_pad = m_pad;
    g.k = k; g.s = 1; g.d = dil; g.p = pp; g.n_q = L;
    g.scale = scale; g.beta = beta; g.n_phase = 1;
    choose_chunks(ctx, g, C_out, k, dil, cdiv(C_in, BM) * cdiv(L, BN) * N);
    if (g.G == 0 && pick_ck_q(k) > 0) {
        g.quad = 1;
        g.CK = pick_ck_q(k);
    }
    if (ad) {
        if (!g.quad || beta != 0.0f) return fail(ctx, KDEC_EINVAL, "conv dgrad: no AdaIN epilogue for this geometry");
        g.ad.x = ad->X;
        g.ad.x_bs = ad->x_bs;
        g.ad.st = reinterpret_cast<const float2*>(ad->stats);
        g.ad.gam = ad->gamma;
        g.ad.bet = ad->beta;
        g.ad.gb_bs = ad->gb_bs;
        g.ad.alpha = ad->alpha;
        g.ad.act = ad->act;
        g.ad.slope = ad->slope;
        g.ad.part = part;
        g.ad.nch = nch;
    }
    const int nq = static_cast<int>(cdiv(static_cast<long>(g.CK) * k / 2, 4));
    const long tot = g.quad ? (m_pad / BM) * static_cast<long>(g.cin_pad / g.CK) * nq * 1024
                            : static_cast<long>(g.cin_pad) * k * m_pad;
    Workspace A(ctx, static_cast<size_t>(tot) * sizeof(float));
    if (!A.p) return KDEC_ENOMEM;
    g.A = A.as<float>();
    KDEC_CHECK(ctx, tot <= 0x7fffffffL && static_cast<long>(C_out) * C_in * k <= 0x7fffffffL,
               "kdec_conv1d_dgrad: weights too large");
    if (g.quad)
        hipLaunchKernelGGL(pack_quad, dim3(grid1d(tot / 4)), dim3(256), 0, ctx->stream, W, A.as<float>(), 1, C_in,
                           C_out, k, g.CK, g.cin_pad / g.CK, nq, tot / 4);
    else if (g.G > 0)
        hipLaunchKernelGGL(pack_octet, dim3(grid1d(tot)), dim3(256), 0, ctx->stream, W, A.as<float>(), 1, C_in,
                           C_out, k, 1, k, m_pad, static_cast<int>(tot), 1);
    else
        if (g.cin_pad % g.CK == 0 && m_pad % 64 == 0 && k <= 32)
            hipLaunchKernelGGL(pack_dgrad_t, dim3(static_cast<unsigned>(cdiv(g.cin_pad, 4)),
                                                  static_cast<unsigned>(m_pad / 64)),
                               dim3(256), 4 * 64 * k * sizeof(float), ctx->stream, W, A.as<float>(), C_in, C_out, k,
                               g.cin_pad, m_pad, g.CK);
        else
            hipLaunchKernelGGL(pack_dgrad, dim3(grid1d(tot)), dim3(256), 0, ctx->stream, W, A.as<float>(), C_in,
                               C_out, k, g.cin_pad, m_pad, g.CK);
    if (int rc = launch_check(ctx, "pack_dgrad")) return rc;
    return run_gemm(ctx, g, N, m_pad / BM, "conv_dgrad",
                    2.0 * N * C_out * static_cast<double>(L_out) * C_in * k);
}

}  // namespace
}  // namespace kdec

extern "C" {

int kdec_conv1d_dgrad(kdec_ctx* ctx, const float* W, const float* dY,
                      long dy_bs, float* dX, long dx_bs, int N, int C_in,
                      int L, int C_out, int k, int stride, int pad, int dil,
                      float scale, float beta) {
    if (!ctx) return KDEC_EINVAL;
    return conv_dgrad_impl(ctx, W, dY, dy_bs, dX, dx_bs, N, C_in, L, C_out, k, stride, pad, dil, scale, beta, nullptr,
                           nullptr, 0);
}

int kdec_conv1d_dgrad_adain_bwd(kdec_ctx* ctx, const float* W, const float* dY, long dy_bs, int N, int C_in, int L,
                                int C_out, int k, int stride, int pad, int dil, const float* X, long x_bs,
                                const float* stats, const float* gamma, const float* beta, long gb_bs, int act,
                                float slope, const float* alpha, const float* R, long r_bs, float* dX, long dx_bs,
                                float* dgamma, float* dbeta, long dgb_bs, float* dalpha) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W && dY && X && stats && gamma && dX && N > 0 && C_in > 0 && C_out > 0 && k > 0 && L > 0,
               "kdec_conv1d_dgrad_adain_bwd: bad arguments");
    KDEC_CHECK(ctx, act == KDEC_ACT_NONE || act == KDEC_ACT_LEAKY || act == KDEC_ACT_SNAKE,
               "kdec_conv1d_dgrad_adain_bwd: unknown activation");
    KDEC_CHECK(ctx, act != KDEC_ACT_SNAKE || alpha, "kdec_conv1d_dgrad_adain_bwd: snake needs alpha");
    KDEC_CHECK(ctx, act == KDEC_ACT_NONE || beta, "kdec_conv1d_dgrad_adain_bwd: the activation needs beta");
    KDEC_CHECK(ctx, x_bs >= static_cast<long>(C_in) * L && dx_bs >= static_cast<long>(C_in) * L &&
                        (!R || r_bs >= static_cast<long>(C_in) * L),
               "kdec_conv1d_dgrad_adain_bwd: batch stride too small");
    // fused where the input grad runs conv_gemm_q and dX aliases neither the
    // AdaIN input nor R (ds is staged in dX); else the two calls it replaces
    const bool fuse = stride == 1 && dX != X && dX != R &&
                      (static_cast<long>(C_in) + BM) * L * 4 < 0x7fffffffL &&
                      dgrad_is_quad(ctx, N, C_in, L, C_out, k, dil);
    if (!fuse) {
        Workspace t(ctx, static_cast<size_t>(N) * C_in * L * sizeof(float));
        if (!t.p) return KDEC_ENOMEM;
        if (int rc = kdec_conv1d_dgrad(ctx, W, dY, dy_bs, t.as<float>(), static_cast<long>(C_in) * L, N, C_in, L,
                                       C_out, k, stride, pad, dil, 1.0f, 0.0f))
            return rc;
        return kdec_adain_act_bwd(ctx, X, x_bs, stats, gamma, beta, gb_bs, act, slope, alpha, t.as<float>(),
                                  static_cast<long>(C_in) * L, R, r_bs, dX, dx_bs, dgamma, dbeta, dgb_bs, dalpha, N,
                                  C_in, L);
    }
    const int nch = 2 * static_cast<int>(cdiv(L, BN));
    Workspace part(ctx, static_cast<size_t>(N) * C_in * nch * 3 * sizeof(double));
    if (!part.p) return KDEC_ENOMEM;
    const AdainBwdIn ad{X, x_bs, stats, gamma, beta, gb_bs, act, slope, alpha};
    if (int rc = conv_dgrad_impl(ctx, W, dY, dy_bs, dX, dx_bs, N, C_in, L, C_out, k, stride, pad, dil, 1.0f, 0.0f,
                                 &ad, part.as<double>(), nch))
        return rc;
    return adain_bwd_finish(ctx, X, x_bs, stats, gamma, gb_bs, act, part.as<double>(), nch, dX, dx_bs, R, r_bs, dX,
                            dx_bs, dgamma, dbeta, dgb_bs, dalpha, N, C_in, L);
}

// LDS bytes of one wgrad_gemm block (two stages) and its input-row layout.
struct WgradLayout {
    int XR, span, segs, rs;
    size_t lds;
};

WgradLayout wgrad_layout(int k, int s, int d, int wn) {
    WgradLayout w{};
    w.XR = (64 * wn - 1) / k + 2;
    w.span = static_cast<int>(static_cast<long>(KC - 1) * s + static_cast<long>(k - 1) * d + 1);
    w.segs = static_cast<int>(cdiv(w.span, 64));
    // Column n = c*k + t sits at c*rs + t*d: with rs = k*d (mod 32) that is
    // n*d (mod 32), distinct banks across 32 lanes for odd d; for k = 1 any
    // odd rs. The smallest such rs >= span keeps the stage small (two blocks
    // per CU for the k = 3 dilated convs).
    long rs = w.span;
    if (k == 1) {
        if (rs % 2 == 0) ++rs;
    } else {
        const long want = (static_cast<long>(k) * d) % 32;
        rs += ((want - rs % 32) % 32 + 32) % 32;
    }
    w.rs = static_cast<int>(rs);
    // the packed staging writes whole 64-float runs: round the window up
    const size_t xsz = (static_cast<size_t>(w.XR) * w.rs + 63) / 64 * 64;
    w.lds = 2 * (static_cast<size_t>(64) * GP + xsz) * sizeof(float);
    return w;
}

size_t wgrad_lds_bytes(int k, int s, int d, int wn) { return wgrad_layout(k, s, d, wn).lds; }

#ifndef WG_ROUNDS
#define WG_ROUNDS 2
#endif
const void* wgrad_kernel(bool s1, int wn) {
    static bool done = false;
    const void* k[2][2] = {{reinterpret_cast<const void*>(&wgrad_gemm<false, 2>),
                            reinterpret_cast<const void*>(&wgrad_gemm<false, 4>)},
                           {reinterpret_cast<const void*>(&wgrad_gemm<true, 2>),
                            reinterpret_cast<const void*>(&wgrad_gemm<true, 4>)}};
    if (!done) {
        for (auto& r : k)
            for (const void* f : r)
                (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        done = true;
    }
    return k[s1 ? 1 : 0][wn == 4 ? 1 : 0];
}

// Waves along the column axis (C_x * k columns): the narrow 128-column tile
// where it leaves fewer idle columns than the 256-column one (the stage-1
// convs' 128 * {3, 7, 11} columns), else the wide tile.
int wgrad_wn(int NN) {
    const long w4 = cdiv(NN, 256) * 256 - NN, w2 = cdiv(NN, 128) * 128 - NN;
    return w2 < w4 ? 2 : 4;
}

int wgrad_splits(kdec_ctx* ctx, int total_chunks, long tiles, size_t lds, bool s1, int wn) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, wgrad_kernel(s1, wn), 128 * wn, lds) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    // The most whole rounds of resident blocks, up to WG_ROUNDS, whose splits
    // keep at least 8 chunks each (shorter runs spend more on the partial
    // tile's write-out and reduction than on the GEMM); never a block past the
    // last whole round: blocks carry equal work (within one chunk), so one
    // more would cost a whole extra round.
    const long slots = static_cast<long>(ctx->num_cus) * per_cu;
    for (int r = WG_ROUNDS; r >= 1; --r) {
        const long splits = r * slots / tiles;
        if (splits >= 1 && total_chunks / splits >= 8) return static_cast<int>(splits);
    }
    return static_cast<int>(std::max(1L, std::min(slots / tiles, static_cast<long>(total_chunks / 8))));
}

// out (M x C_x*k) += the weight grad; db (M) += the row sums of G when
// non-null (fused into the GEMM's n-tile-0 blocks).
static int wgrad_common(kdec_ctx* ctx, const float* X, long x_bs, const float* G,
                        long g_bs, int N, int M, int C_x, int L_x, int L_g, int k,
                        int s, int d, int p, float* out, float* db, const char* fam) {
    const int NN = C_x * k;
    const int wn = wgrad_wn(NN);
    const int m_tiles = static_cast<int>(cdiv(M, BM));
    const int n_tiles = static_cast<int>(cdiv(NN, 64 * wn));
    const int chunks_per_n = static_cast<int>(cdiv(L_g, KC));
    const int total_chunks = chunks_per_n * N;
    // split the position chunks so that the blocks fill WG_ROUNDS rounds of
    // the resident slots
    const int splits = wgrad_splits(ctx, total_chunks, static_cast<long>(m_tiles) * n_tiles,
                                    wgrad_lds_bytes(k, s, d, wn), s == 1, wn);
    const long MN = static_cast<long>(M) * NN;
    Workspace P(ctx, static_cast<size_t>(splits) * MN * sizeof(float));
    Workspace Pb(ctx, db ? static_cast<size_t>(splits) * M * sizeof(float) : 0);
    if (!P.p || (db && !Pb.p)) return KDEC_ENOMEM;
    WgradArgs a{};
    a.X = X; a.x_bs = x_bs; a.G = G; a.g_bs = g_bs; a.P = P.as<float>();
    a.Pb = db ? Pb.as<float>() : nullptr;
    a.M = M; a.C_x = C_x; a.L_x = L_x; a.L_g = L_g; a.k = k; a.s = s; a.d = d; a.p = p;
    a.NN = NN; a.chunks_per_n = chunks_per_n; a.total_chunks = total_chunks;
    a.splits = splits;
    a.n_tiles = n_tiles;
    a.m_tiles = m_tiles;
    const WgradLayout lay = wgrad_layout(k, s, d, wn);
    a.XR = lay.XR;
    a.span = lay.span;
    a.segs = lay.segs;
    a.rs = lay.rs;
    a.blk4 = M % 4 == 0 ? 1 : 0;
    if (static_cast<long>(L_x) * 4 > 0x7fffffffL || static_cast<long>(L_g) * 4 > 0x7fffffffL)
        return fail(ctx, KDEC_EINVAL, "wgrad: rows too long");
    if (static_cast<long>(M) * L_g * 4 > 0x7fffffffL || static_cast<long>(C_x) * L_x * 4 > 0x7fffffffL)
        return fail(ctx, KDEC_EINVAL, "wgrad: operand too large for one buffer descriptor");
    const size_t lds = lay.lds;
    if (lds > 160 * 1024) return fail(ctx, KDEC_EINVAL, "wgrad: tile does not fit LDS");
    const long blocks = static_cast<long>(n_tiles) * m_tiles * splits;
    {
        ProfScope ps(ctx, fam, 2.0 * N * M * static_cast<double>(L_g) * NN,
                     4.0 * (static_cast<double>(N) * C_x * L_x + static_cast<double>(N) * M * L_g +
                            static_cast<double>(M) * NN));
        void* args[] = {&a};
        if (hipLaunchKernel(wgrad_kernel(s == 1, wn), dim3(static_cast<unsigned>(blocks)), dim3(128 * wn), args, lds,
                            ctx->stream) != hipSuccess)
            return fail(ctx, KDEC_EHIP, std::string(fam) + ": launch failed");
        if (int rc2 = launch_check(ctx, fam)) return rc2;
    }
    // the weight-grad partials and, in extra blocks, the bias partials
    ProfScope ps(ctx, "wgrad_reduce", 0.0);
    const bool blk = a.blk4 != 0;
    const bool v4 = blk || (MN % 4 == 0 && ((reinterpret_cast<unsigned long long>(P.p) |
                                             reinterpret_cast<unsigned long long>(out)) & 15) == 0);
    const int zg = splits >= 64 ? 8 : splits >= 16 ? 4 : 1;
    const long cols = v4 ? MN / 4 : MN;
    const unsigned mb = static_cast<unsigned>(cdiv(cols, 256 / zg));
    const unsigned bb = db ? static_cast<unsigned>(cdiv(M, 4)) : 0u;
    const void* kern = blk ? (zg == 8   ? reinterpret_cast<const void*>(&wgrad_reduce<4, 8, true>)
                              : zg == 4 ? reinterpret_cast<const void*>(&wgrad_reduce<4, 4, true>)
                                        : reinterpret_cast<const void*>(&wgrad_reduce<4, 1, true>))
                       : v4 ? (zg == 8   ? reinterpret_cast<const void*>(&wgrad_reduce<4, 8>)
                             : zg == 4 ? reinterpret_cast<const void*>(&wgrad_reduce<4, 4>)
                                       : reinterpret_cast<const void*>(&wgrad_reduce<4, 1>))
                          : (zg == 8   ? reinterpret_cast<const void*>(&wgrad_reduce<1, 8>)
                             : zg == 4 ? reinterpret_cast<const void*>(&wgrad_reduce<1, 4>)
                                       : reinterpret_cast<const void*>(&wgrad_reduce<1, 1>));
    const float* Pp = P.as<float>();
    const float* Pbp = db ? Pb.as<float>() : nullptr;
    long mn = MN;
    int sp = splits, mrows = M;
    unsigned mbk = mb;
    void* args[] = {&Pp, &out, &mn, &sp, &mrows, &Pbp, &db, &mbk};
    if (hipLaunchKernel(kern, dim3(mb + bb), dim3(256), args, 0, ctx->stream) != hipSuccess)
        return fail(ctx, KDEC_EHIP, "wgrad_reduce: launch failed");
    return launch_check(ctx, "wgrad_reduce");
}

// db (M) += sum over (n, l) of G[n, m, l]
static int bias_grad_only(kdec_ctx* ctx, const float* G, long g_bs, float* db, int N, int M, int L) {
    const bool v4 = L % 4 == 0 && g_bs % 4 == 0 && (reinterpret_cast<unsigned long long>(G) & 15) == 0;
    if (2L * M >= ctx->num_cus && static_cast<long>(N) * L <= 128L * 1024) {
        // a row per block on at least half the CUs, each row short enough for one block
        if (v4)
            hipLaunchKernelGGL(bias_rows_direct<4>, dim3(static_cast<unsigned>(M)), dim3(1024), 0, ctx->stream, G,
                               g_bs, db, N, L);
        else
            hipLaunchKernelGGL(bias_rows_direct<1>, dim3(static_cast<unsigned>(M)), dim3(1024), 0, ctx->stream, G,
                               g_bs, db, N, L);
        return launch_check(ctx, "bias_rows_direct");
    }
    // slices of at least 1024 positions, enough of them for ~4 blocks per CU
    long S = std::min(cdiv(4L * ctx->num_cus, M), cdiv(L, 1024));
    if (S > 256) S = 256;
    if (S < 1) S = 1;
    int per = static_cast<int>(cdiv(L, S));
    if (v4) per = (per + 3) & ~3;
    S = cdiv(L, per);
    Workspace part(ctx, static_cast<size_t>(S) * M * sizeof(float));
    if (!part.p) return KDEC_ENOMEM;
    if (v4)
        hipLaunchKernelGGL(bias_partial<4>, dim3(M, static_cast<unsigned>(S)), dim3(256), 0, ctx->stream, G, g_bs,
                           part.as<float>(), N, M, L, per);
    else
        hipLaunchKernelGGL(bias_partial<1>, dim3(M, static_cast<unsigned>(S)), dim3(256), 0, ctx->stream, G, g_bs,
                           part.as<float>(), N, M, L, per);
    if (int rc = launch_check(ctx, "bias_partial")) return rc;
    hipLaunchKernelGGL(bias_reduce, dim3(static_cast<unsigned>(cdiv(M, 4))), dim3(256), 0, ctx->stream,
                       part.as<float>(), db, M, static_cast<int>(S));
    return launch_check(ctx, "bias_reduce");
}

int kdec_conv1d_wgrad(kdec_ctx* ctx, const float* X, long x_bs,
                      const float* dY, long dy_bs, float* dW, float* db, int N,
                      int C_in, int L, int C_out, int k, int stride, int pad,
                      int dil) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && dY && N > 0 && C_in > 0 && C_out > 0 && k > 0 && stride > 0 && dil > 0,
               "kdec_conv1d_wgrad: bad arguments");
    const int L_out = (L + 2 * pad - dil * (k - 1) - 1) / stride + 1;
    KDEC_CHECK(ctx, L > 0 && L_out > 0, "kdec_conv1d_wgrad: empty output");
    if (dW)
        return wgrad_common(ctx, X, x_bs, dY, dy_bs, N, C_out, C_in, L, L_out, k, stride, dil, pad, dW, db,
                            "conv_wgrad");
    if (db) return bias_grad_only(ctx, dY, dy_bs, db, N, C_out, L_out);
    return KDEC_OK;
}

namespace kdec {
namespace {
// The transposed-conv forward; with pad_left = 1 the output rows are
// L_out + 1 long, column 0 the reflection of column 2 (reflection_pad
// (1, 0) of the result), and R (same layout as Y, or null) is added to
// every stored column.
int convt_fwd_impl(kdec_ctx* ctx, const float* X, long x_bs, const float* W, const float* bias, float* Y, long y_bs,
                   int N, int C_in, int L, int C_out, int k, int stride, int pad, int op, const float* R, long r_bs,
                   int pad_left, const char* where) {
    if (!ctx) return KDEC_EINVAL;
    const std::string w(where);
    KDEC_CHECK(ctx, X && W && Y && N > 0 && C_in > 0 && C_out > 0 && k > 0 && stride > 0 && pad >= 0 && op >= 0 &&
                        (pad_left == 0 || pad_left == 1),
               w + ": bad arguments");
    const int L_out = (L - 1) * stride - 2 * pad + (k - 1) + op + 1;
    KDEC_CHECK(ctx, L > 0 && L_out > 0, w + ": empty output");
    KDEC_CHECK(ctx, pad_left == 0 || (stride > 1 && L_out >= 2), w + ": the reflect pad needs a strided output of 2+");
    const long L_y = L_out + pad_left;
    KDEC_CHECK(ctx, y_bs >= static_cast<long>(C_out) * L_y && x_bs >= static_cast<long>(C_in) * L &&
                        (!R || r_bs >= static_cast<long>(C_out) * L_y),
               w + ": batch stride too small");
    const int kt = static_cast<int>(cdiv(k, stride));
    const int m_pad = static_cast<int>(cdiv(C_out, BM) * BM);
    GemmArgs g{};
    // output tiles: per phase at most L_out / stride + 2 columns (as run_gemm)
    const long q_tiles = stride > 1 ? cdiv(cdiv(L_out + stride, stride) + 1, BN) : cdiv(L_out, BN);
    choose_chunks(ctx, g, C_in, kt, 1, cdiv(C_out, BM) * q_tiles * N * stride);
    const long ph = static_cast<long>(g.cin_pad) * kt * m_pad;
    Workspace A(ctx, static_cast<size_t>(ph) * stride * sizeof(float));
    if (!A.p) return KDEC_ENOMEM;
    KDEC_CHECK(ctx, ph * stride <= 0x7fffffffL && static_cast<long>(C_out) * C_in * k <= 0x7fffffffL,
               "kdec_convt1d_fwd: weights too large");
    if (g.G > 0)
        hipLaunchKernelGGL(pack_octet, dim3(grid1d(ph * stride)), dim3(256), 0, ctx->stream, W, A.as<float>(), 2,
                           C_in, C_out, k, stride, kt, m_pad, static_cast<int>(ph), stride);
    else
        hipLaunchKernelGGL(pack_convt_fwd, dim3(grid1d(ph * stride)), dim3(256), 0, ctx->stream, W,
                           A.as<float>(), C_in, C_out, k, stride, kt, g.cin_pad, m_pad, ph, g.CK);
    if (int rc = launch_check(ctx, "pack_convt_fwd")) return rc;
    g.X = X; g.x_bs = x_bs; g.A = A.as<float>(); g.a_phase_stride = ph;
    g.bias = bias; g.Y = Y; g.y_bs = y_bs;
    g.R = R; g.r_bs = r_bs;
    g.C_in = C_in; g.L_in = L; g.C_out = C_out; g.L_y = static_cast<int>(L_y);
    g.y_off = pad_left; g.refl = pad_left;
    g.m_pad = m_pad;
    g.k = kt; g.s = 1; g.d = 1; g.p = 0; g.n_q = 0;
    g.scale = 1.0f; g.beta = 0.0f;
    g.n_phase = stride; g.ph_s = stride; g.ph_p = pad; g.ph_kt = kt;
    if (stride == 1) {  // plain correlation: taps reversed, p' = k-1-pad
        g.n_phase = 1; g.k = k; g.p = k - 1 - pad; g.n_q = L_out; g.a_phase_stride = 0;
        KDEC_CHECK(ctx, g.p >= 0, w + ": padding larger than the kernel");
    }
    return run_gemm(ctx, g, N, m_pad / BM, "convt_fwd",
                    2.0 * N * C_in * static_cast<double>(L) * C_out * k);
}
}  // namespace
}  // namespace kdec

int kdec_convt1d_fwd(kdec_ctx* ctx, const float* X, long x_bs, const float* W,
                     const float* bias, float* Y, long y_bs, int N, int C_in,
                     int L, int C_out, int k, int stride, int pad, int op) {
    return convt_fwd_impl(ctx, X, x_bs, W, bias, Y, y_bs, N, C_in, L, C_out, k, stride, pad, op, nullptr, 0, 0,
                          "kdec_convt1d_fwd");
}

int kdec_convt1d_fwd_res(kdec_ctx* ctx, const float* X, long x_bs, const float* W, const float* bias, float* Y,
                         long y_bs, int N, int C_in, int L, int C_out, int k, int stride, int pad, int op,
                         const float* R, long r_bs, int pad_left) {
    return convt_fwd_impl(ctx, X, x_bs, W, bias, Y, y_bs, N, C_in, L, C_out, k, stride, pad, op, R, r_bs, pad_left,
                          "kdec_convt1d_fwd_res");
}

int kdec_convt1d_dgrad(kdec_ctx* ctx, const float* W, const float* dY,
                       long dy_bs, float* dX, long dx_bs, int N, int C_in,
                       int L, int C_out, int k, int stride, int pad, int op) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W && dY && dX && N > 0 && C_in > 0 && C_out > 0 && k > 0 && stride > 0 && pad >= 0 && op >= 0,
               "kdec_convt1d_dgrad: bad arguments");
    const int L_out = (L - 1) * stride - 2 * pad + (k - 1) + op + 1;
    KDEC_CHECK(ctx, L > 0 && L_out > 0, "kdec_convt1d_dgrad: empty output");
    const int CK = pick_ck(k, stride, 1);
    const int cpad = static_cast<int>(cdiv(C_out, 32) * 32);
    const int m_pad = static_cast<int>(cdiv(C_in, BM) * BM);
    const long tot = static_cast<long>(cpad) * k * m_pad;
    Workspace A(ctx, static_cast<size_t>(tot) * sizeof(float));
    if (!A.p) return KDEC_ENOMEM;
    if (cpad % CK == 0 && m_pad % 32 == 0)
        hipLaunchKernelGGL(pack_rows_t, dim3(static_cast<unsigned>(cdiv(static_cast<long>(cpad) * k, 32)),
                                             static_cast<unsigned>(m_pad / 32)),
                           dim3(256), 0, ctx->stream, W, A.as<float>(), C_in, C_out, k, cpad, m_pad, CK);
    else
        hipLaunchKernelGGL(pack_convt_dgrad, dim3(grid1d(tot)), dim3(256), 0, ctx->stream, W, A.as<float>(),
                           C_in, C_out, k, cpad, m_pad, CK);
    if (int rc = launch_check(ctx, "pack_convt_dgrad")) return rc;
    GemmArgs g{};
    g.X = dY; g.x_bs = dy_bs; g.A = A.as<float>();
    g.Y = dX; g.y_bs = dx_bs;
    g.C_in = C_out; g.L_in = L_out; g.C_out = C_in; g.L_y = L;
    g.cin_pad = cpad; g.m_pad = m_pad;
    g.k = k; g.s = stride; g.d = 1; g.p = pad; g.n_q = L; g.CK = CK;
    g.scale = 1.0f; g.beta = 0.0f; g.n_phase = 1;
    return run_gemm(ctx, g, N, m_pad / BM, "convt_dgrad",
                    2.0 * N * C_in * static_cast<double>(L) * C_out * k);
}

int kdec_convt1d_wgrad(kdec_ctx* ctx, const float* X, long x_bs,
                       const float* dY, long dy_bs, float* dW, float* db,
                       int N, int C_in, int L, int C_out, int k, int stride,
                       int pad, int op) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && dY && N > 0 && C_in > 0 && C_out > 0 && k > 0 && stride > 0 && pad >= 0,
               "kdec_convt1d_wgrad: bad arguments");
    const int L_out = (L - 1) * stride - 2 * pad + (k - 1) + op + 1;
    KDEC_CHECK(ctx, L > 0 && L_out > 0, "kdec_convt1d_wgrad: empty output");
    // dW[ci, co*k + t] = sum_l X[ci, l] dY[co, l*s + t - p]: the conv weight
    // grad with the roles of input and output grad exchanged (M = C_in).
    if (dW)
        if (int rc = wgrad_common(ctx, dY, dy_bs, X, x_bs, N, C_in, C_out, L_out, L, k, stride, 1, pad, dW,
                                  nullptr, "convt_wgrad"))
            return rc;
    if (db) return bias_grad_only(ctx, dY, dy_bs, db, N, C_out, L_out);
    return KDEC_OK;
}

int kdec_pool_fwd(kdec_ctx* ctx, const float* X, long x_bs, const float* W,
                  const float* bias, float* Y, long y_bs, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && W && Y && N > 0 && C > 0 && L > 0, "kdec_pool_fwd: bad arguments");
    ProfScope ps(ctx, "pool", 0);
    hipLaunchKernelGGL(pool_fwd, dim3(static_cast<unsigned>(cdiv(2 * L, 256) > 64 ? 64 : cdiv(2 * L, 256)), N * C),
                       dim3(256), 0, ctx->stream, X, x_bs, W, bias, Y, y_bs, C, L);
    return launch_check(ctx, "pool_fwd");
}

int kdec_pool_dgrad(kdec_ctx* ctx, const float* W, const float* dY,
                    long dy_bs, float* dX, long dx_bs, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, W && dY && dX && N > 0 && C > 0 && L > 0, "kdec_pool_dgrad: bad arguments");
    ProfScope ps(ctx, "pool", 0);
    hipLaunchKernelGGL(pool_dgrad, dim3(static_cast<unsigned>(cdiv(L, 256) > 64 ? 64 : cdiv(L, 256)), N * C),
                       dim3(256), 0, ctx->stream, W, dY, dy_bs, dX, dx_bs, C, L);
    return launch_check(ctx, "pool_dgrad");
}

int kdec_pool_wgrad(kdec_ctx* ctx, const float* X, long x_bs, const float* dY,
                    long dy_bs, float* dW, float* db, int N, int C, int L) {
    if (!ctx) return KDEC_EINVAL;
    KDEC_CHECK(ctx, X && dY && dW && N > 0 && C > 0 && L > 0, "kdec_pool_wgrad: bad arguments");
    ProfScope ps(ctx, "pool", 0);
    hipLaunchKernelGGL(pool_wgrad, dim3(C), dim3(256), 0, ctx->stream, X, x_bs, dY, dy_bs, dW, db, N, C, L);
    return launch_check(ctx, "pool_wgrad");
}

}  // extern "C"

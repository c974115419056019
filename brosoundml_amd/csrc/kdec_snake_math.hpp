// sin^2 for the Snake activation y = s + sin^2(a s) / a on gfx950, and the
// sin / cos pair of the spectral head's polar map, from one reduction.
//
// Cody-Waite reduction of th by pi/2 with a three-part split of pi/2 (each
// product folded in by fma), then the Taylor series of sin or of cos on
// [-pi/4, pi/4], chosen by the parity of the quadrant (sin^2 needs no sign).
// The series' truncation is below 3e-9 relative (the r^11 / 11! and r^12 / 12!
// terms at pi/4), so the result is float-rounding limited for |th| < 2^15.
// About 20 VALU operations against the library sinf's reduction with its
// large-argument path.
#pragma once

#ifndef __HIPCC__
#include <cmath>
#define KDEC_HD
#else
#define KDEC_HD __host__ __device__
#endif

namespace kdec {

// th = q (pi/2) + r with |r| <= pi/4; sets sin r, cos r and returns whether
// q is odd. The parity test compares q / 2 with its rounding (exact in float), so
// no integer conversion of q is needed.
KDEC_HD inline bool snake_reduce(float th, float& sn, float& cs) {
    const float q = rintf(th * 0.636619746685028076f);  // nearest multiple of pi/2
    float r = fmaf(-q, 1.57079637050628662f, th);        // pi/2 = c1 + c2 + c3
    r = fmaf(-q, -4.37113882867379300e-08f, r);
    r = fmaf(-q, -1.71512451000588190e-15f, r);
    // |r| stays within pi/4 plus the rounding of th * 2/pi (a few 1e-3 at
    // |th| = 30000) wherever th carries its phase; far past that the split
    // cancels nothing, and clamping to [-1, 1] (where the series still holds
    // to 3e-8) keeps the results bounded
    r = fminf(fmaxf(r, -1.0f), 1.0f);
    const float w = r * r;
    // sin r = r + r w (-1/3! + w (1/5! + w (-1/7! + w / 9!)))
    const float ps = fmaf(w, fmaf(w, fmaf(w, 2.75573188e-06f, -1.98412701e-04f), 8.33333377e-03f), -1.66666672e-01f);
    sn = fmaf(r * w, ps, r);
    // cos r = 1 + w (-1/2! + w (1/4! + w (-1/6! + w (1/8! - w / 10!))))
    const float pc = fmaf(w, fmaf(w, fmaf(w, fmaf(w, -2.75573199e-07f, 2.48015876e-05f), -1.38888892e-03f),
                                  4.16666679e-02f),
                          -0.5f);
    cs = fmaf(w, pc, 1.0f);
    const float h = 0.5f * q;
    return h != rintf(h);
}

KDEC_HD inline float snake_sin2(float th) {
    float sn, cs;
    const float v = snake_reduce(th, sn, cs) ? cs : sn;
    return v * v;
}

// sin^2(th) and sin(2 th) from the same reduction: for odd q, sin th = +-cos r
// and cos th = -+sin r, so sin^2 th = cos^2 r and sin 2th = -sin 2r.
KDEC_HD inline void snake_sin2_sin2x(float th, float& s2, float& sin2x) {
    float sn, cs;
    const bool odd = snake_reduce(th, sn, cs);
    const float v = odd ? cs : sn;
    s2 = v * v;
    const float t = 2.0f * sn * cs;
    sin2x = odd ? -t : t;
}

// sin th and cos th from one reduction: with th = q (pi/2) + r, the quadrant
// q mod 4 (formed in float: q / 4, its floor and the difference are exact)
// rotates (sin r, cos r) by q quarter turns.
KDEC_HD inline void kdec_sincos(float th, float& s, float& c) {
    float sn, cs;
    snake_reduce(th, sn, cs);
    const float q = rintf(th * 0.636619746685028076f);
    const float qm = q - 4.0f * floorf(0.25f * q);  // 0, 1, 2 or 3
    const bool odd = qm == 1.0f || qm == 3.0f;
    const float s0 = odd ? cs : sn, c0 = odd ? sn : cs;
    s = qm >= 2.0f ? -s0 : s0;
    c = (qm == 1.0f || qm == 2.0f) ? -c0 : c0;
}

// sin x and cos x for |x| <= 1 (the spectral head's second map, whose
// argument is a sine), by their Taylor series without a reduction: through
// x^11 / 11! and x^12 / 12!, whose first omitted terms are below 1.7e-10 and
// 1.2e-11 at |x| = 1. About half the operations of kdec_sincos.
KDEC_HD inline void kdec_sincos_unit(float x, float& s, float& c) {
    const float w = x * x;
    const float ps = fmaf(w, fmaf(w, fmaf(w, fmaf(w, -2.50521084e-08f, 2.75573192e-06f), -1.98412698e-04f),
                                  8.33333333e-03f),
                          -1.66666667e-01f);
    s = fmaf(x * w, ps, x);
    const float pc = fmaf(w, fmaf(w, fmaf(w, fmaf(w, fmaf(w, 2.08767570e-09f, -2.75573192e-07f), 2.48015873e-05f),
                                            -1.38888889e-03f),
                                  4.16666667e-02f),
                          -0.5f);
    c = fmaf(w, pc, 1.0f);
}

}  // namespace kdec

#undef KDEC_HD

// Scalar math shared by the gfx950 kernels and by host-side checks.
//
// Every function here uses only IEEE-754 binary32/binary64 operations that
// are correctly rounded on both gfx950 and x86-64 (add, mul, fma, rint,
// ldexp, conversions), so one source gives the same bits on the device and
// in a host build. Kernels are compiled with -ffp-contract=off; any fused
// multiply-add below is an explicit fma().
#pragma once

#include <stdint.h>
#include <string.h>
#include <math.h>

#if defined(__HIPCC__)
#define CHELIS_HD __host__ __device__
#define CHELIS_TABLE_QUAL static __device__ __constant__ const
#include <hip/hip_runtime.h>
#else
#define CHELIS_HD
#define CHELIS_TABLE_QUAL static const
#endif

#include "exp2_table.h"

namespace chelis {

CHELIS_HD inline uint32_t f32_bits(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return b;
}
CHELIS_HD inline float f32_from(uint32_t b) {
    float v;
    memcpy(&v, &b, 4);
    return v;
}
CHELIS_HD inline uint64_t f64_bits(double v) {
    uint64_t b;
    memcpy(&b, &v, 8);
    return b;
}
CHELIS_HD inline double f64_from(uint64_t b) {
    double v;
    memcpy(&v, &b, 8);
    return v;
}

// [04-NUM-2]: an arithmetic result that is NaN is stored as the canonical
// quiet NaN of its dtype, whatever payload the hardware produced.
CHELIS_HD inline float canon(float v) { return v != v ? f32_from(0x7fc00000u) : v; }
CHELIS_HD inline double canon(double v) { return v != v ? f64_from(0x7ff8000000000000ull) : v; }

// Round the positive unevaluated sum s + e (|e| <= half an ulp of s) to
// binary32, nearest-even. (float)s is already the answer unless s lies
// exactly on a binary32 midpoint, where the sign of e breaks the tie.
CHELIS_HD inline float round_pos_dd_to_f32(double s, double e) {
    float f = (float)s;
    double fd = (double)f;
    if (fd == s || e == 0.0) return f;
    uint32_t fb = f32_bits(f);
    float g;
    if (fb == 0x7f800000u) {          // overflowed: the neighbour below is FLT_MAX
        g = f32_from(0x7f7fffffu);
    } else {
        g = f32_from(s > fd ? fb + 1u : fb - 1u);
    }
    double gd = (double)g;
    double mid = (fb == 0x7f800000u) ? ldexp(1.0, 128) - ldexp(1.0, 103) : 0.5 * (fd + gd);
    if (s != mid) return f;
    double hi = fd > gd ? fd : gd;
    return (e > 0.0) ? (float)hi : (float)(fd + gd - hi);
}

// Correctly rounded binary32 exp, double-double core (any input).
//
// x = k ln2/64 + r with k = rint(x * 64/ln2), |r| <= ln2/128; the reduction
// x - k*HI is exact (HI has 39 significant bits, |k| < 2^14, and Sterbenz
// applies), the tail -k*LO is carried separately. exp(x) =
// 2^(k>>6) * T[k&63] * (1 + expm1(r)) with T a double-double table and
// expm1(r) = r + r^2 P(r), P the degree-5 Taylor tail (truncation below
// 2^-74 on this interval). The product T*(1 + ...) is accumulated as an
// unevaluated double-double whose error is about 2^-66 relative, then
// rounded once to binary32 by round_pos_dd_to_f32. Checked against the
// CORE-MATH oracle over every binary32 input (tests/test_devmath.py).
CHELIS_HD inline float expf_cr_dd(float xf) {
    if (xf != xf) return f32_from(0x7fc00000u);
    if (xf > 89.0f) return f32_from(0x7f800000u);
    if (xf < -104.0f) return 0.0f;
    const double x = (double)xf;
    const double kd = rint(x * CHELIS_INV_LN2_64);
    const int k = (int)kd;
    const double rhi = x - kd * CHELIS_LN2_64_HI;   // exact
    const double rlo = -kd * CHELIS_LN2_64_LO;
    const double r = rhi + rlo;
    double p = fma(r, 1.0 / 5040.0, 1.0 / 720.0);
    p = fma(r, p, 1.0 / 120.0);
    p = fma(r, p, 1.0 / 24.0);
    p = fma(r, p, 1.0 / 6.0);
    p = fma(r, p, 0.5);
    p = (r * r) * p;
    const int j = k & 63;
    const int m = k >> 6;                             // floor division: k = 64m + j
    const double th = chelis_exp2_64_tab[j][0];
    const double tl = chelis_exp2_64_tab[j][1];
    const double ph = th * rhi;
    const double pl = fma(th, rhi, -ph);            // th*rhi = ph + pl exactly
    const double s1 = th + ph;                        // |ph| < |th|: Fast2Sum
    const double e1 = (th - s1) + ph;
    const double low = e1 + (pl + (tl + th * (rlo + p)));
    const double s = s1 + low;
    const double e = (s1 - s) + low;
    return round_pos_dd_to_f32(ldexp(s, m), ldexp(e, m));
}

// Binary32 exp, fast path, branch free. Returns (float)y and sets `slow`
// when y is not known to be the correctly rounded result.
//
// For -87 < x < 88 the result is a normal binary32: x = (64m + j) ln2/64 + r
// with k = 64m + j the integer nearest x * 64/ln2, |r| <= ln2/128 + 2^-40
// (two fma steps against a split ln2/64), exp(r) the degree-4 Taylor
// polynomial (truncation below r^5/120 < 2^-44.5), T[j] = 2^(j/64) rounded
// to binary64, and y = 2^m T[j] p(r) within 2^-44.4 relative: under 2^8.7
// units in the last place of the double y. (float)y is the correctly
// rounded result unless the exact value may lie across a binary32 rounding
// midpoint, i.e. unless the 29 bits below binary32 precision in y are
// within 2^11 units of the midpoint pattern 1 << 28 (about one input in
// 2^17). x <= -104 (with -inf) gives +0, exp(x) being below half the least
// subnormal. NaN, [-104, -87] and [88, inf] are left to the slow path; for
// them the arithmetic below runs on whatever the input is and its value is
// discarded.
//
// k is read from the low word of x * 64/ln2 + 1.5 * 2^52, rounded once by
// the fma: that sum's unit in the last place is 1, so its low 32 bits are k
// in two's complement and subtracting the shift gives k exactly (|k| < 2^14
// on the fast range). `tab(j)` supplies T[j]: a constant-memory table, or
// (inside a full wave) the lane-held copy of it. NONPOS instances serve
// arguments known to be <= 0 or NaN (softmax's x - max): the upper range
// test is dropped, and a positive argument would take the fast path
// unchecked, so callers must not pass one.
template <bool NONPOS = false, class Tab>
CHELIS_HD inline float expf_fast(float xf, const Tab &tab, bool &slow) {
    const bool zero = xf <= -104.0f;
    const bool fast = NONPOS ? xf > -87.0f : (xf > -87.0f && xf < 88.0f);
    const double x = (double)xf;
    const double shifted = fma(x, CHELIS_INV_LN2_64, 0x1.8p52);
    const double kd = shifted - 0x1.8p52;
    const int k = (int)(uint32_t)f64_bits(shifted);
    double r = fma(-kd, CHELIS_LN2_64_HI, x);
    r = fma(-kd, CHELIS_LN2_64_LO, r);
    double p = fma(r, 0x1.5555555555555p-5, 0x1.5555555555555p-3);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    const double y = ldexp(tab(k & 63) * p, k >> 6);
    // 29 bits below binary32 precision, offset so the midpoint pattern is 2047
    const uint32_t below = ((uint32_t)f64_bits(y) & 0x1fffffffu) - (0x10000000u - 2047u);
    slow = (!fast && !zero) || (fast && below < 4095u);
    return zero ? 0.0f : (float)y;
}

struct ExpTableConst {
    CHELIS_HD double operator()(int j) const { return chelis_exp2_64_tab[j][0]; }
};

// Correctly rounded binary32 exp (any input): the fast path, else the
// double-double core. Checked against the CORE-MATH oracle over every
// binary32 input (tests/test_devmath.py).
CHELIS_HD inline float expf_cr(float xf) {
    bool slow;
    const float y = expf_fast(xf, ExpTableConst{}, slow);
    return slow ? expf_cr_dd(xf) : y;
}

// expf_cr restricted to arguments <= 0 or NaN, through the NONPOS fast
// path. Checked against the CORE-MATH oracle over every binary32 input with
// the sign bit set, +0 and every positive NaN (tests/test_devmath.py).
CHELIS_HD inline float expf_cr_nonpos(float xf) {
    bool slow;
    const float y = expf_fast<true>(xf, ExpTableConst{}, slow);
    return slow ? expf_cr_dd(xf) : y;
}

// Correctly rounded binary32 v / t from a precomputed binary64 inv = 1 / t
// (t >= 1 or NaN, as for a softmax row total): the binary64 product is
// within 2^-52 relative of v / t, and the exact quotient of two binary32
// values is never within 2^-49 relative of a binary32 rounding midpoint, so
// one rounding to binary32 gives the correctly rounded quotient. Checked
// against IEEE division on the host (tests/test_devmath.py).
CHELIS_HD inline float quot_f32(float v, double inv) { return (float)((double)v * inv); }

}  // namespace chelis

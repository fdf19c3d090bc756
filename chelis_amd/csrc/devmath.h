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
#include "erfc_table.h"

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
// The same rule decided on the stored bits, for results the compiler treats
// as never NaN: after the device sqrt it folds `v != v` to false, so canon()
// would let the hardware's NaN (sign set, or the operand's payload) through.
// An integer test on the bits cannot be folded that way.
CHELIS_HD inline float canon_bits(float v) {
    return (f32_bits(v) & 0x7fffffffu) > 0x7f800000u ? f32_from(0x7fc00000u) : v;
}
CHELIS_HD inline double canon_bits(double v) {
    return (f64_bits(v) & 0x7fffffffffffffffull) > 0x7ff0000000000000ull ? f64_from(0x7ff8000000000000ull) : v;
}

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
    if constexpr (NONPOS) {
        // x <= 0 or NaN: arguments below -104.5 are raised to it (their exp,
        // like exp(-104.5) < 2^-150, rounds to +0 at any of the fast path's
        // errors), (-104, -87] (subnormal results) and NaN are flagged
        // (every comparison with NaN is false), and the midpoint test runs
        // on every other result; a flag on a raised argument only costs the
        // slow path.
        // Here |k| <= 9660, so one fma against ln2/64 rounded to binary64
        // (within 2^-60 of it) reduces x to within 2^-46.7 absolute: the
        // two-part constant of the general case is not needed.
        const float xc = xf > -104.5f ? xf : -104.5f;
        const double x = (double)xc;
        const double shifted = fma(x, CHELIS_INV_LN2_64, 0x1.8p52);
        const double kd = shifted - 0x1.8p52;
        const int k = (int)(uint32_t)f64_bits(shifted);
        const double r = fma(-kd, 0x1.62e42fefa39efp-7, x);  // ln2/64
        double p = fma(r, 0x1.5555555555555p-5, 0x1.5555555555555p-3);
        p = fma(p, r, 0.5);
        p = fma(p, r, 1.0);
        p = fma(p, r, 1.0);
        const double y = ldexp(tab(k & 63) * p, k >> 6);
        const uint32_t below = ((uint32_t)f64_bits(y) & 0x1fffffffu) - (0x10000000u - 2047u);
        slow = !(xf > -87.0f) && !(xf <= -104.0f);
        slow = slow || below < 4095u;
        return (float)y;
    }
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

// Binary32 erfc, fast path, branch free. Returns (float)y and sets `slow`
// when y is not known to be the correctly rounded result (and for NaN and
// 9.1 <= x < 10.1, left to the caller's fallback).
//
// For -4.5 < x < 9.1, y is erfc(x) in binary64 to about 2^-47 relative:
// exp(-x^2) erfcx(|x|) with erfcx a degree-9 fit on the intervals
// [i/4, (i + 1)/4) (2^-48; x^2 is exact, exp(-x^2) is reduced as in
// expf_fast with a degree-5 Taylor polynomial, truncation below 2^-54), and
// erfc(x) = 2 - erfc(-x) for x < 0 (a result in (1, 2], no cancellation).
// One branch-free evaluation serves every x: the interval 0 fit starts at
// x = 0, where a separate fit of erf(x)/x for |x| < 1/2 was evaluated for
// every argument beside the interval one and then mostly discarded. The coefficients are erfc_table.h's
// (gen_erfc_table.py). Every such result is a normal binary32 (erfc(9.1) >
// 2^-126), so (float)y is the correctly rounded result unless the 29 bits
// below binary32 precision in y lie within 2^9 units of the midpoint
// pattern 1 << 28: the error is below 2^6 units there. x <= -4.5 gives 2
// (erfc(-4.5) lies above 2 - 2^-24, the midpoint below 2), x >= 10.1 gives
// +0 (erfc(10.1) is below 2^-150, half the least subnormal), and +inf and
// -inf fall in those ranges. Checked against CORE-MATH over every binary32
// input (tests/test_devmath.py).
// erfcf_fast_t reads the erfcx coefficients B[i][d] and 2^(j/64) through
// `tb`: ErfcTablesConst (below) reads the constant-memory tables; a kernel
// that evaluates many erfc per lane stages the same values in LDS and passes
// an accessor reading them there (a per-lane index into constant memory is a
// vector memory load per coefficient: GELU over 16.7M binary32 values 82-85
// us from constant memory, 65-72 us from LDS, same bits).
// exp_neg_sq, when given, receives the binary64 exp(-x^2) of the exact
// square that the evaluation uses (within 2^-51.2 relative while x^2 < 104:
// truncation 2^-54.5, the Horner polynomial's last rounding 1.1 * 2^-53,
// T[j] and the product 2^-53 each).
template <class Tabs>
CHELIS_HD inline float erfcf_fast_t(float xf, bool &slow, const Tabs &tb, double *exp_neg_sq = nullptr) {
    const double x = (double)xf;
    const double ax = fabs(x);
    const double s = x * x;  // exact
    // the interval, clamped before the conversion (NaN and the infinities
    // take the last one; their results are flagged or replaced below)
    const double q = ax * 4.0;
    const int i = q < 36.0 ? (int)q : 36;
    const double tv = (ax - 0.25 * i) * 8.0 - 1.0;  // exact
    double g = tb.b(i, 9);
#pragma unroll
    for (int d = 8; d >= 0; --d) g = fma(g, tv, tb.b(i, d));
    // exp(-s), -s = k ln2/64 + r, |k| < 2^11
    const double shifted = fma(-s, CHELIS_INV_LN2_64, 0x1.8p52);
    const double kd = shifted - 0x1.8p52;
    const int k = (int)(uint32_t)f64_bits(shifted);
    double r = fma(-kd, CHELIS_LN2_64_HI, -s);
    r = fma(-kd, CHELIS_LN2_64_LO, r);
    double p = fma(r, 0x1.1111111111111p-7, 0x1.5555555555555p-5);  // 1/5!, 1/4!
    p = fma(p, r, 0x1.5555555555555p-3);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    const double e = ldexp(tb.e(k & 63) * p, k >> 6);  // k = 64 (k >> 6) + (k & 63)
    if (exp_neg_sq) *exp_neg_sq = e;
    const double yb = e * g;
    double y = x > 0.0 ? yb : 2.0 - yb;
    y = x <= -4.5 ? 2.0 : (x >= 10.1 ? 0.0 : y);
    const uint32_t below = ((uint32_t)f64_bits(y) & 0x1fffffffu) - (0x10000000u - 512u);
    slow = (x != x) || (x >= 9.1 && x < 10.1) || below < 1024u;
    return (float)y;
}

// Correctly rounded binary32 exp(-fl(t * t)) for a binary32 t, derived from
// E = exp(-t^2) in binary64 for the exact square (erfcf_fast_t's exp_neg_sq
// for x = t, within 2^-51.2 relative), so GELU's correction term needs no
// exp evaluation of its own. d = t^2 - fl(t^2) is exact in binary64 and
// |d| <= 2^-18 wherever the result is not +0 (fl(t^2) < 104), so
// exp(-fl(t^2)) = E exp(d) = E (1 + d + d^2/2) to 2^-56.6; with the two
// fma and the product, y is within 2^-50.5 relative: under 6 units of the
// rounding test's 2^-29 binary32-ulp grid, whose window is 2047 units (the
// test and the ranges are expf_fast's: arguments at or below -104 give +0,
// (-104, -87] - subnormal results - are flagged). t must be finite.
CHELIS_HD inline float expf_neg_square_from(float t, double E, bool &slow) {
    const float s32 = t * t;
    const double d = (double)t * (double)t - (double)s32;
    const double y = E * fma(d, fma(d, 0.5, 1.0), 1.0);
    const float xf = -s32;
    const bool zero = xf <= -104.0f;
    const uint32_t below = ((uint32_t)f64_bits(y) & 0x1fffffffu) - (0x10000000u - 2047u);
    slow = !zero && (!(xf > -87.0f) || below < 4095u);
    return zero ? 0.0f : (float)y;
}

// The constant-memory tables (also the 2^(j/64) accessor of expf_fast).
struct ErfcTablesConst {
    CHELIS_HD double b(int i, int d) const { return chelis_erfcx_b[i][d]; }
    CHELIS_HD double e(int j) const { return chelis_exp2_64_tab[j][0]; }
    CHELIS_HD double operator()(int j) const { return chelis_exp2_64_tab[j][0]; }
};

// The same values staged in LDS (stage_erfc_tables).
struct ErfcTablesLds {
    const double (*bt)[10];
    const double *et;
    CHELIS_HD double b(int i, int d) const { return bt[i][d]; }
    CHELIS_HD double e(int j) const { return et[j]; }
    CHELIS_HD double operator()(int j) const { return et[j]; }
};

CHELIS_HD inline float erfcf_fast(float xf, bool &slow) { return erfcf_fast_t(xf, slow, ErfcTablesConst{}); }

// ------------------------------------------------------------ binary64 exp
//
// Correctly rounded binary64 exp in two stages, both on the reduction
// x = k ln2/64 + r, k the integer nearest x * 64/ln2 (|k| < 2^17 on the
// finite range), exp(x) = 2^m * 2^(j/64) * exp(r), k = 64m + j, |r| <= ln2/128
// (plus 2^-30 relative for the rounding of x * 64/ln2).
//
// exp_fast: binary64 and double-double arithmetic to an error below 2^-73.7
// (bound derived at the function), then Ziv's rounding test: the
// result is returned when both ends of the error interval round to the same
// binary64 number (all but about one input in 2^19).
//
// exp_cr_fx: 128-bit fixed-point arithmetic to an error below 2^-124.4
// relative, rounded at the binary64 (or subnormal) grid of the result. The
// inputs whose exp lies closest to a binary64 rounding midpoint need about
// 2^-113 (Lefevre and Muller's worst cases for exp over the binary64
// domain), so this rounding is the correct one; the sampled worst cases of
// tests/golden/exp_worst_cases.txt and CORE-MATH on random inputs are
// checked on the host and on the device.

struct U128 {
    uint64_t hi, lo;
};

// 64 x 64 -> 128-bit product from 32-bit halves (the same integer result on
// host and device).
CHELIS_HD inline uint64_t mul64_wide(uint64_t a, uint64_t b, uint64_t *lo) {
    const uint64_t a0 = (uint32_t)a, a1 = a >> 32, b0 = (uint32_t)b, b1 = b >> 32;
    const uint64_t p00 = a0 * b0, p01 = a0 * b1, p10 = a1 * b0, p11 = a1 * b1;
    const uint64_t mid = (p00 >> 32) + (uint32_t)p01 + (uint32_t)p10;
    *lo = (mid << 32) | (uint32_t)p00;
    return p11 + (p01 >> 32) + (p10 >> 32) + (mid >> 32);
}

// floor(a * b / 2^128), exactly.
CHELIS_HD inline U128 mulhi128(U128 a, U128 b) {
    uint64_t l00, l01, l10, l11;
    const uint64_t h00 = mul64_wide(a.lo, b.lo, &l00);
    const uint64_t h01 = mul64_wide(a.lo, b.hi, &l01);
    const uint64_t h10 = mul64_wide(a.hi, b.lo, &l10);
    const uint64_t h11 = mul64_wide(a.hi, b.hi, &l11);
    uint64_t w1 = h00 + l01;
    uint64_t c1 = w1 < l01;
    w1 += l10;
    c1 += w1 < l10;
    uint64_t w2 = h01 + h10;
    uint64_t c2 = w2 < h10;
    w2 += l11;
    c2 += w2 < l11;
    w2 += c1;
    c2 += w2 < c1;
    return {h11 + c2, w2};
}

CHELIS_HD inline U128 add128(U128 a, U128 b) {
    U128 r;
    r.lo = a.lo + b.lo;
    r.hi = a.hi + b.hi + (r.lo < a.lo);
    return r;
}
CHELIS_HD inline U128 sub128(U128 a, U128 b) {
    U128 r;
    r.lo = a.lo - b.lo;
    r.hi = a.hi - b.hi - (a.lo < b.lo);
    return r;
}
CHELIS_HD inline U128 shr128(U128 a, int s) {  // 0 <= s
    if (s >= 128) return {0, 0};
    if (s >= 64) return {0, a.hi >> (s - 64)};
    if (s == 0) return a;
    return {a.hi >> s, (a.lo >> s) | (a.hi << (64 - s))};
}
CHELIS_HD inline U128 shl128(U128 a, int s) {  // 0 <= s < 128
    if (s >= 64) return {a.lo << (s - 64), 0};
    if (s == 0) return a;
    return {(a.hi << s) | (a.lo >> (64 - s)), a.lo << s};
}
CHELIS_HD inline bool less128(U128 a, U128 b) { return a.hi < b.hi || (a.hi == b.hi && a.lo < b.lo); }
CHELIS_HD inline U128 table128(const unsigned long long (&w)[2]) { return {w[0], w[1]}; }

// d * 2^s truncated toward zero, as a two's complement 128-bit integer;
// |d| 2^s < 2^127.
CHELIS_HD inline U128 fixed_scaled(double d, int s) {
    const uint64_t b = f64_bits(d);
    const int be = (int)((b >> 52) & 0x7ff);
    if (be == 0) return {0, 0};  // zero or subnormal: far below the 2^-s resolution here
    const U128 m = {0, (b & 0xfffffffffffffull) | (1ull << 52)};
    const int sh = be - 1075 + s;  // d = m * 2^(be - 1075)
    const U128 mag = sh >= 0 ? shl128(m, sh) : shr128(m, -sh);
    return (b >> 63) ? sub128(U128{0, 0}, mag) : mag;
}

// exp(x) = Y 2^(m - 126) for -745.2 <= x <= 709.79, Y within 5.9 units of
// the exact value, 2^-124.4 relative (Y >= 0.99 * 2^126).
//
// r = x - k (HI + LO + LO2): x - k HI is exact (HI has 36 significant bits),
// k LO and k LO2 are split exactly into double-double products, and the
// five terms are summed in fixed point at 2^-134 (truncation error below
// 4 * 2^-134; c - HI - LO - LO2 is below 2^-152, times |k| < 2^17).
// exp(r) by Horner over 1/n!, n = 0..13, at 2^-127 (the omitted terms are
// below 2^-141; each step's truncation adds at most 1.03 units of 2^-127 and
// earlier errors shrink by |r| < 2^-7.5, so the sum is within 1.7 units).
// Y = T[j] exp(r) at 2^-126 with T[j] within half a unit of 2^-127: within
// 0.5 + 2 * 1.7 + 2 = 5.9 units of 2^-127 of the exact product.
CHELIS_HD inline U128 exp_fx(double x, int &m) {
    const double kd = rint(x * CHELIS_INV_LN2_64);
    const int k = (int)kd;
    const double rhi = fma(-kd, CHELIS_LN2_64_HI36, x);  // exact
    const double t = kd * CHELIS_LN2_64_LO36;
    const double tl = fma(kd, CHELIS_LN2_64_LO36, -t);
    const double u = kd * CHELIS_LN2_64_LO36B;
    const double ul = fma(kd, CHELIS_LN2_64_LO36B, -u);
    U128 r = fixed_scaled(rhi, 134);
    r = sub128(r, fixed_scaled(t, 134));
    r = sub128(r, fixed_scaled(tl, 134));
    r = sub128(r, fixed_scaled(u, 134));
    r = sub128(r, fixed_scaled(ul, 134));
    const bool neg = (int64_t)r.hi < 0;
    const U128 ra = neg ? sub128(U128{0, 0}, r) : r;
    U128 p = table128(chelis_inv_fact_fx[13]);
    for (int n = 12; n >= 0; --n) {
        const U128 term = shr128(mulhi128(ra, p), 6);  // |r| p at 2^-127
        const U128 c = table128(chelis_inv_fact_fx[n]);
        p = neg ? sub128(c, term) : add128(c, term);
    }
    const int j = k & 63;
    m = (k - j) / 64;
    return mulhi128(table128(chelis_exp2_64_fx[j]), p);
}

// Correctly rounded exp for -745.2 <= x <= 709.79: Y of exp_fx rounded to
// nearest at the cut where the result keeps 53 bits, or at 2^-1074 in the
// subnormal range.
CHELIS_HD inline double exp_cr_fx(double x) {
    int m;
    const U128 y = exp_fx(x, m);
    const int lead = y.hi >> 63 ? 127 : (y.hi >> 62 ? 126 : 125);
    int cut = lead - 52;
    if (-948 - m > cut) cut = -948 - m;  // below 2^-1022: the subnormal grid 2^-1074
    if (cut > 128) return 0.0;           // below half the least subnormal
    const U128 kept = shr128(y, cut);
    const U128 rem = cut >= 128 ? y : sub128(y, shl128(kept, cut));
    const U128 half = shl128(U128{0, 1}, cut - 1);
    uint64_t q = kept.lo;
    if (less128(half, rem) || (!less128(rem, half) && (q & 1))) ++q;
    return ldexp((double)q, cut + m - 126);
}

// Binary64 exp, fast path, branch free: exp_dd evaluates exp(x) as
// (yh + yl) 2^m, exp_fast returns the rounded result and sets `slow` when it
// is not known to be the correctly rounded one (and for NaN, x <= -708 and,
// unless NONPOS, x >= 709; NONPOS instances serve arguments known to be <= 0
// or NaN, and a positive argument would take the fast path unchecked).
// `tab(j, hi, lo)` supplies 2^(j/64) as a double-double: a constant-memory
// table, or (inside a full wave) the lane-held copy of it.
//
// Error budget on -708 < x < 709 (|k| < 2^16, results normal, no overflow),
// absolute on y = T[j] exp(r) < 2.02:
// - r = rh + rl: x - k HI exact, k LO split exactly as t + tl; rh = rhi - t
//   with its rounding error recovered exactly when |rhi| >= |t| and to 2^-81
//   otherwise (then |r| < 2^-28); the omitted k (c - HI - LO) is below
//   2^16 * 2^-99 = 2^-83;
// - exp(r) - 1 = rh + rh^2/2 + rh^3 C(rh) + rl (1 + qh) with C the Taylor
//   coefficients 1/3! .. 1/8! (omitted degree 9: 2^-86.2; rl^2 and
//   rl rh^3/6: below 2^-86): rh^2 exact as sh + sl, qh + e1 = rh + sh/2
//   exactly (Fast2Sum); the cubic part P carries at most 4.2 roundings of
//   2^-53 relative on |P| < 2^-25.16 (2^-76.1) and is added, with the low
//   terms, into ql (|ql| < 2^-25; two roundings below 2^-78.2 each);
// - T[j] = th + tl within 2^-107; th qh split exactly (ph + pl), yh + e2 =
//   th + ph exactly (Fast2Sum); yl sums e2, pl, th ql and tl (1 + qh), of
//   magnitude below 2^-24, with three roundings below 2^-77.2 each; the
//   omitted tl ql is below 2^-78.
// Total below 2^-73.7 (2 * 2^-76.1 + 5 * 2^-77.2 + 2^-78 + smaller terms,
// times T[j] < 2 where the terms are relative to exp(r)); the host check
// measures the largest error over 2 * 10^7 inputs against the fixed-point
// value and requires it below that bound. The rounding test uses eps =
// 2^-72.
struct ExpDD {
    double yh, yl;
    int m;
};
template <class Tab2>
CHELIS_HD inline ExpDD exp_dd(double x, const Tab2 &tab) {
    const double shifted = fma(x, CHELIS_INV_LN2_64, 0x1.8p52);
    const double kd = shifted - 0x1.8p52;
    const int k = (int)(uint32_t)f64_bits(shifted);
    const double rhi = fma(-kd, CHELIS_LN2_64_HI36, x);  // exact on the fast range
    const double t = kd * CHELIS_LN2_64_LO36;
    const double tl = fma(kd, CHELIS_LN2_64_LO36, -t);
    const double rh = rhi - t;  // Fast2Sum when |rhi| >= |t|; else |r| < 2^-28
    const double rl = ((rhi - rh) - t) - tl;
    const double sh = rh * rh;
    const double sl = fma(rh, rh, -sh);
    double c = fma(rh, 0x1.a01a01a01a01ap-16, 0x1.a01a01a01a01ap-13);  // 1/8!, 1/7!
    c = fma(rh, c, 0x1.6c16c16c16c17p-10);                              // 1/6!
    c = fma(rh, c, 0x1.1111111111111p-7);                               // 1/5!
    c = fma(rh, c, 0x1.5555555555555p-5);                               // 1/4!
    c = fma(rh, c, 0x1.5555555555555p-3);                               // 1/3!
    const double P = (sh * rh) * c;
    const double half = 0.5 * sh;
    const double qh = rh + half;  // Fast2Sum: |rh| >= rh^2/2
    const double e1 = half - (qh - rh);
    const double ql = e1 + (P + (rl + fma(qh, rl, 0.5 * sl)));
    double th, tlo;
    tab(k & 63, th, tlo);
    const double ph = th * qh;
    const double pl = fma(th, qh, -ph);
    const double yh = th + ph;  // Fast2Sum: th >= 1 > |ph|
    const double e2 = ph - (yh - th);
    const double yl = e2 + (pl + fma(th, ql, fma(tlo, qh, tlo)));
    return {yh, yl, k >> 6};  // k = 64 (k >> 6) + (k & 63)
}

template <bool NONPOS = false, class Tab2>
CHELIS_HD inline double exp_fast(double x, const Tab2 &tab, bool &slow) {
    const bool fast = NONPOS ? x > -708.0 : (x > -708.0 && x < 709.0);
    const ExpDD d = exp_dd(x, tab);
    constexpr double eps = 0x1p-72;
    const double a = d.yh + (d.yl - eps);
    const double b = d.yh + (d.yl + eps);
    slow = !fast || a != b;
    return ldexp(a, d.m);
}

struct Exp2TableConst {
    CHELIS_HD void operator()(int j, double &hi, double &lo) const {
        hi = chelis_exp2_64_tab[j][0];
        lo = chelis_exp2_64_tab[j][1];
    }
};

// The binary64 exp's slow path with its special cases: NaN -> the canonical
// NaN; above 709.79 (with +inf) -> +inf; below -745.2 (with -inf) -> +0.
CHELIS_HD inline double exp_cr_slow(double x) {
    if (x != x) return f64_from(0x7ff8000000000000ull);
    if (x > 709.79) return f64_from(0x7ff0000000000000ull);
    if (x < -745.2) return 0.0;
    return exp_cr_fx(x);
}

// Correctly rounded binary64 exp (any input).
CHELIS_HD inline double exp_cr(double x) {
    bool slow;
    const double y = exp_fast(x, Exp2TableConst{}, slow);
    return slow ? exp_cr_slow(x) : y;
}

// Binary64 exp of an argument <= 0 or NaN, faithful rather than correctly
// rounded, for the default binary64 softmax row. One binary64 evaluation,
// branch free:
//   exp(x) = 2^m T[j] exp(r),  x = (64m + j) ln2/64 + r,  |r| <= ln2/128,
// r reduced with the two-part ln2/64 as in expf_fast; expm1(r) as its
// degree-5 Taylor polynomial r c(r) (omitted r^6/6!: below 2^-54.6);
// y = fma(T_hi, r c, T_hi), T_hi the binary64 rounding of 2^(j/64). On the
// normal range the error is below 0.5 ulp (the final rounding) plus
// 1.4 * 2^-53 relative (T_hi, the truncation, the Horner roundings), so
// under 2 ulp; below 2^-1022 ldexp rounds once into the subnormal grid.
// x < -746 (-inf included) is raised to -746, whose exp rounds to +0; a NaN
// fails the comparison and propagates (k & 63 stays in range).
// `tab(j)` supplies T_hi[j]. Checked against CORE-MATH on the host
// (tests/test_devmath.py).
template <class Tab1>
CHELIS_HD inline double exp_nonpos_faithful(double x, const Tab1 &tab) {
    const double xc = x < -746.0 ? -746.0 : x;
    const double shifted = fma(xc, CHELIS_INV_LN2_64, 0x1.8p52);
    const double kd = shifted - 0x1.8p52;
    const int k = (int)(uint32_t)f64_bits(shifted);
    double r = fma(-kd, CHELIS_LN2_64_HI, xc);
    r = fma(-kd, CHELIS_LN2_64_LO, r);
    double c = fma(r, 0x1.1111111111111p-7, 0x1.5555555555555p-5);  // 1/5!, 1/4!
    c = fma(r, c, 0x1.5555555555555p-3);                               // 1/3!
    c = fma(r, c, 0.5);
    c = fma(r, c, 1.0);
    const double th = tab(k & 63);
    return ldexp(fma(th, r * c, th), k >> 6);
}

}  // namespace chelis

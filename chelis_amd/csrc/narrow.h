// bfloat16 and IEEE binary16 storage: 16-bit carriers whose arithmetic runs
// at binary32 and is finalized back to 16 bits once per operation
// ([04-NUM-8]). The conversions are those of the C lane's runtime
// (crates/chelis-runtime/include/chelis_runtime.h:664-760): widening is
// exact; narrowing rounds to nearest even, overflows to infinity, keeps the
// subnormals of binary16, and stores every NaN as the canonical quiet NaN
// of the format ([04-NUM-2]: 0x7fc0 for bf16, 0x7e00 for f16). Integer
// code only, so host and device give the same bits.
#pragma once

#include "devmath.h"

namespace chelis {

enum class Narrow : int { Bf16 = 0, F16 = 1 };

CHELIS_HD inline float bf16_to_f32(uint16_t h) { return f32_from((uint32_t)h << 16); }

CHELIS_HD inline uint16_t f32_to_bf16(float v) {
    const uint32_t b = f32_bits(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    // nearest even on the 16 discarded bits; a carry moves into the exponent
    // (and past the largest finite value to infinity) as the rounding requires
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

CHELIS_HD inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1fu) return f32_from(sign | 0x7f800000u | (m << 13));
    if (e != 0) return f32_from(sign | ((e + 112u) << 23) | (m << 13));
    // zero or subnormal: m * 2^-24 exactly
    const float mag = (float)m * 0x1p-24f;
    return f32_from(sign | f32_bits(mag));
}

CHELIS_HD inline uint16_t f32_to_f16(float v) {
    const uint32_t b = f32_bits(v);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t be = (b >> 23) & 0xffu, mant = b & 0x7fffffu;
    if (be == 0xffu) return mant ? (uint16_t)0x7e00u : (uint16_t)(sign | 0x7c00u);
    const int e = (int)be - 127 + 15;  // binary16 biased exponent
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        // subnormal result (or zero): round the full significand once at
        // the quantum 2^-24; a carry into bit 10 is the least normal
        if (e < -10) return sign;
        const uint32_t full = mant | 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t kept = full >> shift;
        const uint32_t dropped = full & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (dropped > half || (dropped == half && (kept & 1u))) ++kept;
        return (uint16_t)(sign | kept);
    }
    // normal: nearest even on the 13 discarded bits; the carry may bump the
    // exponent, up to infinity
    const uint32_t r = ((uint32_t)e << 23 | mant) + 0xfffu + ((mant >> 13) & 1u);
    if ((r >> 23) >= 0x1fu) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (r >> 13));
}

template <Narrow K>
CHELIS_HD inline float narrow_to_f32(uint16_t h) {
    if constexpr (K == Narrow::Bf16) return bf16_to_f32(h);
    else return f16_to_f32(h);
}
template <Narrow K>
CHELIS_HD inline uint16_t f32_to_narrow(float v) {
    if constexpr (K == Narrow::Bf16) return f32_to_bf16(v);
    else return f32_to_f16(v);
}

// [05-OP-40] max_elem / min_elem on stored bits: the left operand when it
// is NaN, or when the right one is not NaN and left >= right (max) /
// left <= right (min); the selected operand's bits are returned unchanged
// (crates/chelis-backend-hip/src/kernels.rs:2291-2305).
template <Narrow K>
CHELIS_HD inline uint16_t narrow_max(uint16_t a, uint16_t b) {
    const float x = narrow_to_f32<K>(a), y = narrow_to_f32<K>(b);
    return (x != x || (y == y && x >= y)) ? a : b;
}
template <Narrow K>
CHELIS_HD inline uint16_t narrow_min(uint16_t a, uint16_t b) {
    const float x = narrow_to_f32<K>(a), y = narrow_to_f32<K>(b);
    return (x != x || (y == y && x <= y)) ? a : b;
}
// [05-OP-41] sub at the binary32 arithmetic width, finalized once.
template <Narrow K>
CHELIS_HD inline uint16_t narrow_sub(uint16_t a, uint16_t b) {
    return f32_to_narrow<K>(narrow_to_f32<K>(a) - narrow_to_f32<K>(b));
}
// [05-OP-43] relu: x < 0 ? +0 : x on the stored bits (NaN and -0 kept);
// its adjoint: g where 0 < x, else +0 (kernels.rs:1196-1260).
template <Narrow K>
CHELIS_HD inline uint16_t narrow_relu(uint16_t x) {
    return narrow_to_f32<K>(x) < 0.0f ? (uint16_t)0 : x;
}
template <Narrow K>
CHELIS_HD inline uint16_t narrow_relu_adjoint(uint16_t x, uint16_t g) {
    return 0.0f < narrow_to_f32<K>(x) ? g : (uint16_t)0;
}

}  // namespace chelis

// Per-element math shared by the elementwise, reduction and GEMM-epilogue
// kernels: keyed RNG, transcendental leaves, the GELU graph and the fused
// chain step evaluator. Each float result is finalized at its dtype with the
// canonical NaN ([04-NUM-2]) unless the operation is a bit-preserving
// selection ([05-OP-40], [05-OP-43]).
#pragma once

#include "gelu_poly.h"
#include "hip_common.h"

namespace chelis {

// ---------------------------------------------------------------- RNG
// [05-RNG-1] splitmix64 and [05-RNG-2] word/unit; identical integer
// arithmetic on every lane, so draws are bit-exact.
__device__ inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
__device__ inline uint64_t random_word(uint64_t key, uint64_t index) {
    const uint64_t e = splitmix64(index);
    return splitmix64(key ^ ((e << 41) | (e >> 23)));
}
__device__ inline double random_unit(uint64_t key, uint64_t index) {
    return (double)(random_word(key, index) >> 11) * 0x1p-53;
}

// ---------------------------------------------------------------- math leaves
template <typename T> __device__ inline T leaf_exp(T v);
template <> __device__ inline float leaf_exp<float>(float v) { return expf_cr(v); }
// Binary64 exp: the branch-free fast path, and for the rare flagged input
// (about one in 2^19, plus NaN and the saturated and subnormal ranges) the
// 128-bit fixed-point path out of line.
__device__ __noinline__ inline double exp_slow64(double v) { return exp_cr_slow(v); }
template <> __device__ inline double leaf_exp<double>(double v) {
    bool slow;
    const double y = exp_fast(v, Exp2TableConst{}, slow);
    return slow ? exp_slow64(v) : y;
}
template <typename T> __device__ inline T leaf_erfc(T v);
template <typename T> __device__ inline T leaf_log(T v);
template <typename T> __device__ inline T leaf_tanh(T v);
template <> __device__ inline double leaf_erfc<double>(double v) { return canon(erfc(v)); }
template <> __device__ inline double leaf_log<double>(double v) { return canon(log(v)); }
template <> __device__ inline double leaf_tanh<double>(double v) { return canon(tanh(v)); }

// Binary32 log, erfc and tanh: the binary64 device function rounded once to
// binary32 is the correctly rounded result (the same bits as CORE-MATH, the
// C backend's libm) on every binary32 input except the six below, where the
// binary64 value sits within its own error of a rounding midpoint. The
// inputs come from comparing all 2^32 inputs on the device; the results are
// the correctly rounded values (80-digit decimal arithmetic). tanh has no
// exception. A change of the device math library is caught by the
// exhaustive comparison, which runs over every input again.
__device__ inline float cr_exception(float y, uint32_t xb, uint32_t in, uint32_t out) {
    return xb == in ? f32_from(out) : y;
}
template <> __device__ inline float leaf_log<float>(float v) {
    const uint32_t b = f32_bits(v);
    float y = (float)log((double)v);
    y = cr_exception(y, b, 0x3c413d3au, 0xc08e158fu);
    y = cr_exception(y, b, 0x41178febu, 0x400fe5e7u);
    y = cr_exception(y, b, 0x4c5d65a5u, 0x418f034bu);
    y = cr_exception(y, b, 0x65d890d3u, 0x4254d1f9u);
    y = cr_exception(y, b, 0x6f31a8ecu, 0x42845a89u);
    return canon(y);
}
// expf_cr's correctly rounded core for the arguments its fast path flags.
__device__ __noinline__ inline float expf_slow_cr(float v) { return expf_cr_dd(v); }
__device__ __noinline__ inline float erfc_slow32(float v) {
    const float y = cr_exception((float)erfc((double)v), f32_bits(v), 0xb76c9f62u, 0x3f800085u);
    return canon(y);
}
// the branch-free fast path (devmath.h erfcf_fast), else the binary64
// device erfc rounded once with its exception (out of line)
template <> __device__ inline float leaf_erfc<float>(float v) {
    bool slow;
    const float y = erfcf_fast(v, slow);
    return slow ? erfc_slow32(v) : y;
}
template <> __device__ inline float leaf_tanh<float>(float v) { return canon((float)tanh((double)v)); }

template <typename T> struct Lim;
template <> struct Lim<float> {
    __device__ static float lowest() { return -3.4028234663852886e38f; }
};
template <> struct Lim<double> {
    __device__ static double lowest() { return -1.7976931348623157e308; }
};

// ---------------------------------------------------------------- GELU
// spec/05 section 3.3: gelu(x) = mul(m(x), Phi(x)) with the exact Phi graph
// (erfc leaf, Veltkamp-split correction, exp leaf); constants as in
// crates/chelis-numeric-core/src/activation.rs:41-56.
template <typename T> struct PhiK;
template <> struct PhiK<float> {
    static constexpr float c = (float)0.70710678118654752440, cl = (float)1.2101617485882343e-8,
                           k = (float)1.12837916709551257390, s = 4097.0f;
};
template <> struct PhiK<double> {
    static constexpr double c = 0.70710678118654752440, cl = -4.833646656726457e-17, k = 1.12837916709551257390,
                            s = 134217729.0;
};

//
// Every primitive of the graph rounds at T; only the final product is
// NaN-finalized. That gives the same bits as finalizing each primitive: for
// a non-NaN x no intermediate is NaN (z is finite with |z| < 64, so the
// split, the products and the exp argument are finite; erfc and exp of
// finite or infinite arguments are not NaN; m * phi is +-inf * 1 or
// -0 * 0 at the infinities), and a NaN x makes the product NaN, which the
// final step canonicalizes.
//
// gelu_one_t reads the binary32 erfc and exp tables through `tb`
// (ErfcTablesConst or ErfcTablesLds, same bits); binary64 uses none.
template <typename T, class Tabs>
__device__ inline T gelu_one_t(T x, const Tabs &tb) {
    const T c = PhiK<T>::c, cl = PhiK<T>::cl, k = PhiK<T>::k, s = PhiK<T>::s;
    T e;
    double e_neg_sq = 0.0;  // binary32: exp(-(x c)^2) in binary64 from the erfc fast path
    if constexpr (sizeof(T) == 4) {
        bool slow;
        e = erfcf_fast_t(-x * c, slow, tb, &e_neg_sq);
        if (slow) e = erfc_slow32(-x * c);
    } else {
        e = leaf_erfc<T>(-x * c);
    }
    const T z = (fabs(x) < T(64)) ? x : T(0);
    const T a = -z;
    const T th = a * c;
    const T ta = s * a;
    const T ah = ta - (ta - a);
    const T al = a - ah;
    const T tc = s * c;
    const T ch = tc - (tc - c);
    const T cr = c - ch;
    T t = ah * ch - th;
    t = t + ah * cr;
    t = t + al * ch;
    t = t + al * cr;
    const T tl = t + a * cl;
    T g;
    if constexpr (sizeof(T) == 4) {
        // |x| < 64: th is the erfc argument -x c itself, so exp(-fl(th^2))
        // comes from the erfc path's exp(-th^2); otherwise th = -0, g = 1
        const bool near = fabs(x) < T(64);
        bool slow;
        const float gf = expf_neg_square_from(th, e_neg_sq, slow);
        g = near ? gf : T(1);
        if (near && slow) g = expf_slow_cr(-(th * th));
    } else {
        g = leaf_exp<T>(-(th * th));
    }
    const T corr = (k * g) * tl;
    const T phi = T(0.5) * (e - corr);
    const T m = (x < Lim<T>::lowest()) ? T(-0.0) : x;
    return canon(m * phi);
}

template <typename T>
__device__ inline T gelu_one(T x) {
    return gelu_one_t<T>(x, ErfcTablesConst{});
}

// binary32 GELU for the default (not exact) mode: x Phi(x) directly, not
// the Phi graph primitive by primitive. Phi = 1 - E for x >= 0 and E for
// x < 0, E = erfc(|x| / sqrt 2) / 2 = q(|x|) exp(-x^2 / 2):
//   q = erfcx(|x| / sqrt 2) / 2, one degree-9 polynomial in
//       u = (|x| - K) / (|x| + K) (gelu_poly.h);
//   exp(-x^2 / 2) = 2^a, a = -x^2 log2(e) / 2 in binary64 (x^2 is exact
//       there, so the exponential's relative error does not grow with
//       x^2), split into floor(a) and a fraction in [0, 1) for one
//       v_exp_f32 and an exponent scaling;
//   x Phi(x) = fma(-|x| q, e, x) for x >= 0, fma(-|x| q, e, 0) for x < 0.
// About 30 instructions against about 110 for the graph (binary64 runs at
// the binary32 rate here, as packed binary32 is not used); within 7e-7
// relative of the graph on every binary32 input (the north star's binary32
// bar is 1e-5). `slow` marks what it does not serve - x < -12.5, where E
// and the result leave the normal range, +inf and NaN - for the graph.
__device__ inline float gelu_fast_f32(float x, bool &slow) {
    constexpr float kQ[CHELIS_GELU_DEG + 1] = CHELIS_GELU_Q;
    constexpr float kK = CHELIS_GELU_K;
    constexpr double kHalfLog2e = -0.72134752044448170368;  // -log2(e) / 2
    // x + 12.5 is +0, +subnormal or +normal exactly when -12.5 <= x < +inf
    slow = !__builtin_amdgcn_classf(x + 12.5f, (1 << 6) | (1 << 7) | (1 << 8));
    const float ax = fabsf(x);
    // u = (|x| - K) / (|x| + K) = 1 - 2K / (|x| + K)
    const float u = fmaf(-2.0f * kK, __builtin_amdgcn_rcpf(ax + kK), 1.0f);
    float q = kQ[CHELIS_GELU_DEG];
#pragma unroll
    for (int d = CHELIS_GELU_DEG - 1; d >= 0; --d) q = fmaf(q, u, kQ[d]);
    const double xd = (double)x;
    // beyond -1000, 2^a is 0 against 1 (and floor(a) stays an int)
    const double a = fmax((xd * kHalfLog2e) * xd, -1000.0);
    const double fl = floor(a);
    const float e = __builtin_ldexpf(__builtin_amdgcn_exp2f((float)(a - fl)), (int)fl);
    // x Phi(x) = x - |x| q e for x >= 0, -|x| q e for x < 0
    return fmaf(-(ax * q), e, x >= 0.0f ? x : 0.0f);
}

// A workgroup's copy of the binary32 erfc and exp tables in LDS; every
// thread of the NT-thread workgroup calls it, and the caller's next barrier
// publishes the copy.
struct ErfcLdsStore {
    double bt[37][10];
    double et[64];
    template <int NT>
    __device__ void fill() {
        for (int i = threadIdx.x; i < 37 * 10; i += NT) bt[i / 10][i % 10] = chelis_erfcx_b[i / 10][i % 10];
        for (int i = threadIdx.x; i < 64; i += NT) et[i] = chelis_exp2_64_tab[i][0];
    }
    __device__ ErfcTablesLds tabs() const { return ErfcTablesLds{bt, et}; }
};

// ---------------------------------------------------------------- chain ops
// The step fields are 32-bit words: the interpreter reads them at a
// run-time step index, and gfx950's scalar loads move whole dwords, so a
// byte field would be read with a vector load (a full memory round trip per
// step, queued behind the kernel's streaming loads).
struct ChainDev {
    int32_t n_steps;
    int32_t op[CHELIS_FUSED_MAX_STEPS];
    int32_t a0[CHELIS_FUSED_MAX_STEPS];
    int32_t a1[CHELIS_FUSED_MAX_STEPS];
    double imm[CHELIS_FUSED_MAX_STEPS];
};

// Transcendental leaves of the chain interpreter stay out of line: every
// unrolled step of every chain kernel would otherwise inline all of them.
template <typename T> __device__ __noinline__ T chain_exp(T a) { return leaf_exp<T>(a); }
template <typename T> __device__ __noinline__ T chain_log(T a) { return leaf_log<T>(a); }
template <typename T> __device__ __noinline__ T chain_tanh(T a) { return leaf_tanh<T>(a); }
template <typename T> __device__ __noinline__ T chain_erfc(T a) { return leaf_erfc<T>(a); }

template <typename T>
__device__ inline T apply_step(uint8_t op, T a, T b, double imm) {
    switch (op) {
        case CHELIS_FUSED_ADD: return canon(a + b);
        case CHELIS_FUSED_SUB: return canon(a - b);
        case CHELIS_FUSED_MUL: return canon(a * b);
        case CHELIS_FUSED_DIV: return canon(a / b);
        case CHELIS_FUSED_MAX_ELEM: return max_first(a, b);  // [05-OP-40] bit preserving
        case CHELIS_FUSED_MIN_ELEM: return min_first(a, b);
        case CHELIS_FUSED_NEG: return canon(-a);
        case CHELIS_FUSED_RECIP: return canon(T(1) / a);
        case CHELIS_FUSED_EXP: return chain_exp<T>(a);
        case CHELIS_FUSED_LOG: return chain_log<T>(a);
        case CHELIS_FUSED_SQRT: return canon_bits(sqrt(a));
        case CHELIS_FUSED_TANH: return chain_tanh<T>(a);
        case CHELIS_FUSED_ERFC: return chain_erfc<T>(a);
        case CHELIS_FUSED_ABS: return canon(fabs(a));
        case CHELIS_FUSED_FLOOR: return canon(floor(a));
        case CHELIS_FUSED_CEIL: return canon(ceil(a));
        case CHELIS_FUSED_ROUND: return canon(rint(a));
        case CHELIS_FUSED_RELU: return a < T(0) ? T(0) : a;          // [05-OP-43]
        case CHELIS_FUSED_RELU_ADJOINT: return T(0) < a ? b : T(0);  // a = x, b = g
        case CHELIS_FUSED_CONST: return (T)imm;
        default: return T(0);
    }
}


// ---------------------------------------------------------------- chain interpreter
// One element's inputs and step results live in a row of LDS slots (inputs
// first, then steps) and the steps run as a loop over the chain: a private
// array indexed by the run-time step arguments would live in scratch
// memory. The slot row stride is odd, so the lanes of a wave hit distinct
// LDS banks.
constexpr int kSlots = CHELIS_FUSED_MAX_INPUTS + CHELIS_FUSED_MAX_STEPS;
constexpr int kSlotStride = kSlots + 1;

template <typename T>
__device__ inline T run_chain(const ChainDev &ch, T *slot) {
    T v = T(0);
#pragma unroll 1
    for (int s = 0; s < ch.n_steps; ++s) {
        const int a0 = ch.a0[s], a1 = ch.a1[s];
        const T x = slot[a0 >= 0 ? a0 : CHELIS_FUSED_MAX_INPUTS - a0 - 1];
        const T y = slot[a1 >= 0 ? a1 : CHELIS_FUSED_MAX_INPUTS - a1 - 1];
        v = apply_step<T>(ch.op[s], x, y, ch.imm[s]);
        slot[CHELIS_FUSED_MAX_INPUTS + s] = v;
    }
    return v;
}


template <typename T>
struct Vec16F;
template <>
struct Vec16F<float> {
    using type = float4;
};
template <>
struct Vec16F<double> {
    using type = double2;
};

// 16-byte nontemporal load and store of a Vec16F value (the builtins take
// clang vector types, not HIP's float4 / double2): for operands read once
// or written once, which then do not displace reused lines in the caches.
template <typename T>
__device__ inline typename Vec16F<T>::type load_nt16(const T *p) {
    typedef T E __attribute__((ext_vector_type(16 / sizeof(T))));
    const E e = __builtin_nontemporal_load(reinterpret_cast<const E *>(p));
    typename Vec16F<T>::type q;
    __builtin_memcpy(&q, &e, 16);
    return q;
}
template <typename T>
__device__ inline void store_nt16(T *p, const typename Vec16F<T>::type &q) {
    typedef T E __attribute__((ext_vector_type(16 / sizeof(T))));
    E e;
    __builtin_memcpy(&e, &q, 16);
    __builtin_nontemporal_store(e, reinterpret_cast<E *>(p));
}

template <typename T, int V>
__device__ inline void apply_step_vec(uint8_t op, const T (&x)[V], const T (&y)[V], double imm, T (&r)[V]) {
    switch (op) {
#define CHELIS_STEP_CASE(OPC)                                                  \
    case OPC:                                                                  \
        _Pragma("unroll") for (int e = 0; e < V; ++e) r[e] = apply_step<T>(OPC, x[e], y[e], imm); \
        break;
        CHELIS_STEP_CASE(CHELIS_FUSED_ADD)
        CHELIS_STEP_CASE(CHELIS_FUSED_SUB)
        CHELIS_STEP_CASE(CHELIS_FUSED_MUL)
        CHELIS_STEP_CASE(CHELIS_FUSED_DIV)
        CHELIS_STEP_CASE(CHELIS_FUSED_MAX_ELEM)
        CHELIS_STEP_CASE(CHELIS_FUSED_MIN_ELEM)
        CHELIS_STEP_CASE(CHELIS_FUSED_NEG)
        CHELIS_STEP_CASE(CHELIS_FUSED_RECIP)
        CHELIS_STEP_CASE(CHELIS_FUSED_EXP)
        CHELIS_STEP_CASE(CHELIS_FUSED_LOG)
        CHELIS_STEP_CASE(CHELIS_FUSED_SQRT)
        CHELIS_STEP_CASE(CHELIS_FUSED_TANH)
        CHELIS_STEP_CASE(CHELIS_FUSED_ERFC)
        CHELIS_STEP_CASE(CHELIS_FUSED_ABS)
        CHELIS_STEP_CASE(CHELIS_FUSED_FLOOR)
        CHELIS_STEP_CASE(CHELIS_FUSED_CEIL)
        CHELIS_STEP_CASE(CHELIS_FUSED_ROUND)
        CHELIS_STEP_CASE(CHELIS_FUSED_RELU)
        CHELIS_STEP_CASE(CHELIS_FUSED_RELU_ADJOINT)
        CHELIS_STEP_CASE(CHELIS_FUSED_CONST)
#undef CHELIS_STEP_CASE
        default:
#pragma unroll
            for (int e = 0; e < V; ++e) r[e] = T(0);
    }
}

// The vector form of run_chain: V elements per thread, slots slot-major
// ([n_in + n_steps][256] 16-byte vectors, adjacent lanes on adjacent
// words), one op dispatch per step. r holds the last step's values.
template <typename T, int V, typename Q>
__device__ inline void run_chain_vec(const ChainDev &ch, Q *slots, int n_in, int tid, T (&r)[V]) {
#pragma unroll 1
    for (int st = 0; st < ch.n_steps; ++st) {
        const int a0 = ch.a0[st], a1 = ch.a1[st];
        const Q xq = slots[(a0 >= 0 ? a0 : n_in - a0 - 1) * 256 + tid];
        const Q yq = slots[(a1 >= 0 ? a1 : n_in - a1 - 1) * 256 + tid];
        T x[V], y[V];
#pragma unroll
        for (int j = 0; j < V; ++j) {
            x[j] = reinterpret_cast<const T *>(&xq)[j];
            y[j] = reinterpret_cast<const T *>(&yq)[j];
        }
        apply_step_vec<T, V>(ch.op[st], x, y, ch.imm[st], r);
        Q rq;
#pragma unroll
        for (int j = 0; j < V; ++j) reinterpret_cast<T *>(&rq)[j] = r[j];
        slots[(n_in + st) * 256 + tid] = rq;
    }
}

}  // namespace chelis
